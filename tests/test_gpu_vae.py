"""VAE convolution prologue on the GPU: GroupNorm statistics, GroupNorm + swish (per row
and gathered), and the conv_gn_swish / resnet compositions against the float64 oracle
(src/hi3d_mac/mlx_backend/vae.py:141-218, kernels.py:240-296). Gates: statistics to
fp32 rounding (rel 1e-5); activations 1e-5 (fp32) / 2e-3 (fp16), the reference test's
tolerances (tests/test_mlx_kernels.py:63-76); convolutions max-abs / RMS <= 1e-5 (fp32),
1e-2 (fp16); the residual block <= 1e-4 (fp32, two chained GroupNorms)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import conv as oconv
from oracle import vae as ovae

pytestmark = pytest.mark.gpu


def _level(cuda, side=16, density=0.5, seed=3):
    from hi3d_amd import sparse

    rng = np.random.default_rng(seed)
    idx = np.stack(np.meshgrid(*[np.arange(side)] * 3, indexing="ij"), -1).reshape(-1, 3)
    coords = idx[rng.random(idx.shape[0]) < density].astype(np.int32)
    return coords, sparse.Level.from_coords(torch.as_tensor(coords).to(cuda))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("c", [64, 128, 256])
def test_group_stats_matches_float64(cuda, dtype, c):
    from hi3d_amd import vae

    rng = np.random.default_rng(c)
    x = torch.as_tensor(rng.normal(0.5, 2.0, (20011, c)).astype(np.float32)).to(dtype)
    mean, inv = vae.group_stats(x.to(cuda))
    rm, ri = ovae.group_stats_f64(x.float().numpy())
    std = 1 / ri
    assert np.max(np.abs(mean.cpu().numpy() - rm) / std) <= 1e-5
    assert np.max(np.abs(inv.cpu().numpy() - ri) / ri) <= 1e-5


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.float16, 2e-3)])
def test_gather_group_norm_swish_matches_composed(cuda, dtype, tol):
    """The reference test's case: n = 300, C = 64, a [120, 27] table with n for absent."""
    from hi3d_amd import kernels

    rng = np.random.default_rng(10)
    n, c = 300, 64
    x = rng.normal(size=(n, c)).astype(np.float32)
    mean = rng.normal(size=c).astype(np.float32)
    inv = rng.uniform(0.5, 2.0, c).astype(np.float32)
    w, b = rng.normal(size=(1, c)).astype(np.float32), rng.normal(size=(1, c)).astype(np.float32)
    table = rng.integers(0, n + 1, (120, 27)).astype(np.int32)
    t = lambda a: torch.as_tensor(a).to(cuda)
    got = kernels.gather_group_norm_swish(t(x), t(table), t(mean), t(inv), t(w), t(b), dtype).float().cpu().numpy()
    ref = ovae.gather_group_norm_swish(x, table, mean, inv, w, b, np.float32).astype(np.float32)
    ref = torch.as_tensor(ref).to(dtype).float().numpy()
    assert got.shape == (120, 27 * c)
    assert np.allclose(got, ref, atol=tol, rtol=tol)
    assert np.all(got[np.repeat(table == n, c, axis=1)] == 0)


@pytest.mark.parametrize("din,dout", [(torch.float16, torch.float16), (torch.float32, torch.float32),
                                      (torch.bfloat16, torch.float32), (torch.float32, torch.float16)])
def test_group_norm_swish_rows(cuda, din, dout):
    from hi3d_amd import kernels, vae

    rng = np.random.default_rng(4)
    x = torch.as_tensor(rng.normal(0.2, 1.5, (3001, 128)).astype(np.float32)).to(din)
    w = rng.uniform(0.5, 1.5, (1, 128)).astype(np.float32)
    b = rng.normal(0, 0.1, (1, 128)).astype(np.float32)
    mean, inv = vae.group_stats(x.to(cuda))
    got = kernels.group_norm_swish(x.to(cuda), mean, inv, torch.as_tensor(w).to(cuda), torch.as_tensor(b).to(cuda),
                                   dout).float().cpu().numpy()
    ref = ovae.group_norm_swish(x.float().numpy(), mean.cpu().numpy(), inv.cpu().numpy(), w, b, np.float64)
    tol = 1e-5 if dout == torch.float32 else 2e-3
    assert np.allclose(got, ref, atol=tol, rtol=tol)


@pytest.mark.parametrize("dtype,gate", [(torch.float32, 1e-5), (torch.float16, 1e-2)])
def test_conv_gn_swish_matches_float64(cuda, dtype, gate):
    from hi3d_amd import vae

    coords, level = _level(cuda)
    table = level.table.cpu().numpy()
    rng = np.random.default_rng(5)
    c = 32
    x = rng.normal(0, 1, (len(coords), c)).astype(np.float32)
    gw, gb = rng.uniform(0.5, 1.5, (1, c)).astype(np.float32), rng.normal(0, 0.1, (1, c)).astype(np.float32)
    wt = rng.normal(0, 0.05, (27 * c, c)).astype(np.float32)
    bias = rng.normal(0, 0.1, c).astype(np.float32)
    res = rng.normal(0, 1, (len(coords), c)).astype(np.float32)
    t = lambda a, d=torch.float32: torch.as_tensor(a).to(cuda).to(d)
    got = vae.conv_gn_swish(t(x, dtype), level, t(gw), t(gb), t(wt, dtype), t(bias, dtype), residual=t(res, dtype))
    xr = t(x, dtype).float().cpu().numpy()
    ref = ovae.conv_gn_swish_f64(xr, table, gw, gb, t(wt, dtype).float().cpu().numpy(),
                                 t(bias, dtype).float().cpu().numpy(), residual=t(res, dtype).float().cpu().numpy())
    assert got.dtype == dtype
    assert oconv.rel_err(got.float().cpu().numpy(), ref) <= gate


@pytest.mark.parametrize("with_res_conv", [False, True])
def test_resnet_matches_float64(cuda, with_res_conv):
    """The reference's residual-block test geometry (16^3 cube at density 0.5, C = 32,
    tests/test_mlx_kernels.py:125-150) in fp32 against the float64 composition."""
    from hi3d_amd import vae

    coords, level = _level(cuda)
    table = level.table.cpu().numpy()
    rng = np.random.default_rng(3)
    c = 32
    p = {}
    for name in ("r.block.0", "r.block.3"):
        p[f"{name}.weights"] = rng.uniform(0.5, 1.5, (1, c)).astype(np.float32)
        p[f"{name}.bias"] = rng.normal(0, 0.1, (1, c)).astype(np.float32)
    for name in ("r.block.2", "r.block.5"):
        p[f"{name}.weight"] = rng.normal(0, 0.05, (27 * c, c)).astype(np.float32)
        p[f"{name}.bias"] = rng.normal(0, 0.1, (c,)).astype(np.float32)
    if with_res_conv:
        p["r.res_conv.weight"] = rng.normal(0, 0.2, (c, c)).astype(np.float32)
        p["r.res_conv.bias"] = rng.normal(0, 0.1, (c,)).astype(np.float32)
    x = rng.normal(0, 1, (len(coords), c)).astype(np.float32)
    gp = {k: torch.as_tensor(v).to(cuda) for k, v in p.items()}
    got = vae.resnet(torch.as_tensor(x).to(cuda), level, gp, "r").cpu().numpy()
    ref = ovae.resnet_f64(x, table, p, "r")
    assert oconv.rel_err(got, ref) <= 1e-4
