"""Empty and single-voxel sets through every convolution dispatch path, the stride-2
pair, the spconv-style modules, the refiner geometry and the VAE residual block, against
the float64 oracle: an empty set gives empty results of the right shape and dtype (the
reference's empty-geometry test, tests/test_empty_geometry.py:8-18, asks the same of
unique), and a single voxel sees only its own centre tap. Gates as in the convolution
tests: max-abs / RMS <= 1e-5 (fp32), 1e-2 (fp16), 3e-2 (bf16)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import conv as oconv
from oracle import vae as ovae

pytestmark = pytest.mark.gpu

GATE = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 3e-2}
EMPTY = np.zeros((0, 4), np.int32)
SINGLE = np.array([[0, 3, 4, 5]], np.int32)


def _weights(rng, n, cin, cout, dtype, kvol=27):
    x = torch.as_tensor(rng.standard_normal((n, cin), dtype=np.float32)).to(dtype)
    w = torch.as_tensor(rng.standard_normal((cout, kvol, cin), dtype=np.float32) / np.sqrt(kvol * cin)).to(dtype)
    b = torch.as_tensor(rng.standard_normal(cout, dtype=np.float32) * 0.1).to(dtype)
    return x, w, b


@pytest.mark.parametrize("dtype,cin,cout,path", [
    (torch.float16, 128, 128, "mfma"), (torch.float16, 64, 64, "mfma"), (torch.float32, 64, 64, "mfma"),
    (torch.bfloat16, 256, 256, "mfma"), (torch.float16, 256, 8, "narrow"), (torch.float32, 48, 5, "narrow"),
    (torch.float16, 12, 20, "simple"),
])
@pytest.mark.parametrize("idx", [EMPTY, SINGLE], ids=["empty", "single"])
def test_conv_empty_and_single_voxel(cuda, dtype, cin, cout, path, idx):
    """Each dispatch path (MFMA tile kernels, the narrow kernel, the simple kernel) on
    an empty set and on one voxel, with and without a residual added in place."""
    from hi3d_amd import conv, kmap

    assert {"narrow": conv.narrow_supported(dtype, cin, cout, 27),
            "mfma": conv.mfma_supported(dtype, cin, cout) and not conv.narrow_supported(dtype, cin, cout, 27),
            "simple": not conv.mfma_supported(dtype, cin, cout) and not conv.narrow_supported(dtype, cin, cout, 27),
            }[path]
    rng = np.random.default_rng(cin + cout)
    n = len(idx)
    km = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [8] * 3, 1)
    assert km.table.shape == (n, 27)
    x, w, b = _weights(rng, n, cin, cout, dtype)
    r = torch.as_tensor(rng.standard_normal((n, cout), dtype=np.float32)).to(dtype)
    xd, wd, bd, rd = x.to(cuda), w.to(cuda), b.to(cuda), r.to(cuda)
    plan = km.plan()
    y = conv.conv(xd, plan, wd, bd)
    assert y.shape == (n, cout) and y.dtype == dtype and y.device.type == "cuda"
    inplace = rd.clone()
    z = conv.conv(xd, plan, wd, bd, residual=inplace, out=inplace)
    assert z.shape == (n, cout) and z.data_ptr() == inplace.data_ptr()
    if n == 0:
        return
    ref = oconv.gather_conv_f64(x.float().numpy(), km.table.cpu().numpy(), w.float().numpy(), b.float().numpy())
    centre = x.double().numpy() @ w[:, 13, :].double().numpy().T + b.double().numpy()
    assert np.allclose(ref, centre, rtol=1e-12, atol=1e-12)
    assert oconv.rel_err(y.float().cpu().numpy(), ref) <= GATE[dtype]
    assert oconv.rel_err(z.float().cpu().numpy(), ref + r.double().numpy()) <= GATE[dtype]


@pytest.mark.parametrize("idx", [EMPTY, SINGLE], ids=["empty", "single"])
def test_spconv_modules_empty_and_single_voxel(cuda, idx):
    """SubMConv3d, SparseConv3d (2x2x2, stride 2) and SparseInverseConv3d in float64 on
    an empty set and on one voxel: coarse coordinates exact, features against the
    centre / slot taps."""
    from hi3d_amd import spconv

    rng = np.random.default_rng(4)
    n = len(idx)
    feats = torch.as_tensor(rng.standard_normal((n, 6))).to(cuda)
    x = spconv.SparseConvTensor(feats, torch.as_tensor(idx).to(cuda), [8] * 3, 1)
    subm = spconv.SubMConv3d(6, 6, 3, bias=True, indice_key="subm3").double().to(cuda)
    down = spconv.SparseConv3d(6, 10, 2, stride=2, bias=True, indice_key="s2").double().to(cuda)
    up = spconv.SparseInverseConv3d(10, 6, 2, bias=True, indice_key="s2").double().to(cuda)
    with torch.no_grad():
        h = subm(x)
        y = down(h)
        z = up(y)
    assert h.features.shape == (n, 6) and y.features.shape == (n, 10) and z.features.shape == (n, 6)
    assert y.spatial_shape == [4, 4, 4] and z.spatial_shape == [8, 8, 8]
    if n == 0:
        return
    assert y.indices.cpu().tolist() == [[0, 1, 2, 2]]
    f = feats.cpu().numpy()

    def taps(layer):  # [Cout, kvol, Cin] in float64
        wt = layer.weight.detach().cpu().numpy()
        return wt.reshape(wt.shape[0], -1, wt.shape[-1])

    def bias(layer):
        return layer.bias.detach().cpu().numpy()

    h_ref = f @ taps(subm)[:, 13].T + bias(subm)
    assert np.allclose(h.features.cpu().numpy(), h_ref, atol=1e-12)
    slot = 4 * (3 % 2) + 2 * (4 % 2) + (5 % 2)  # child (3, 4, 5) of parent (1, 2, 2)
    y_ref = h_ref @ taps(down)[:, slot].T + bias(down)
    assert np.allclose(y.features.cpu().numpy(), y_ref, atol=1e-12)
    z_ref = y_ref @ taps(up)[:, slot].T + bias(up)
    assert np.allclose(z.features.cpu().numpy(), z_ref, atol=1e-12)


@pytest.mark.parametrize("coords", [np.zeros((0, 3), np.int32), np.array([[3, 4, 5]], np.int32)],
                         ids=["empty", "single"])
def test_geometry_empty_and_single_voxel(cuda, coords):
    """The refiner geometry (transformer.py:234-266,449-473): one voxel has one parent
    with one child; the pool divides by children + 1, the parent copy returns the row,
    and the up convolution sees only the centre tap."""
    from hi3d_amd.geometry import Geometry

    rng = np.random.default_rng(9)
    n = len(coords)
    geo = Geometry(torch.as_tensor(coords).to(cuda))
    assert geo.full.n == n and geo.low.n == n
    assert geo.inverse.shape == (n,) and geo.counts.shape == (n,)
    x = torch.as_tensor(rng.standard_normal((n, 64), dtype=np.float32)).to(cuda)
    low = geo.downsample(x)
    back = geo.upsample(low)
    odd = geo.upsample(x[:, :3].contiguous())  # 12-byte rows
    w = torch.as_tensor(rng.standard_normal((32, 27 * 64), dtype=np.float32) / np.sqrt(27 * 64)).to(cuda)
    b = torch.as_tensor(rng.standard_normal(32, dtype=np.float32) * 0.1).to(cuda)
    y = geo.up_conv(low, w, b)
    assert low.shape == (n, 64) and back.shape == (n, 64) and odd.shape == (n, 3) and y.shape == (n, 32)
    if n == 0:
        return
    assert geo.low.coords.cpu().tolist() == [[1, 2, 2]] and geo.counts.cpu().tolist() == [1]
    assert torch.equal(low, x / 2)
    assert torch.equal(back, low) and torch.equal(odd, x[:, :3])
    ref = low.double().cpu().numpy() @ w.double().cpu().numpy().reshape(32, 27, 64)[:, 13].T + b.double().cpu().numpy()
    assert oconv.rel_err(y.cpu().numpy(), ref) <= GATE[torch.float32]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_group_stats_of_no_rows(cuda, dtype):
    """The reference divides by ``n * width + eps`` (vae.py:158-163), so no rows give
    mean 0 and ``1 / sqrt(eps)`` in fp32 rather than NaN."""
    from hi3d_amd import vae

    mean, inv = vae.group_stats(torch.empty((0, 64), dtype=dtype, device=cuda), 1e-6)
    ref_mean, ref_inv = ovae.group_stats_f64(np.zeros((0, 64)), 1e-6)
    assert np.array_equal(mean.cpu().numpy(), ref_mean.astype(np.float32))
    expected = np.float32(1.0) / np.sqrt(np.float32(1e-6))
    assert np.array_equal(inv.cpu().numpy(), np.full(64, expected, np.float32))
    assert np.allclose(inv.cpu().numpy(), ref_inv, rtol=1e-6)


@pytest.mark.parametrize("with_res_conv", [False, True])
@pytest.mark.parametrize("coords", [np.zeros((0, 3), np.int32), np.array([[3, 4, 5]], np.int32)],
                         ids=["empty", "single"])
def test_vae_resnet_empty_and_single_voxel(cuda, coords, with_res_conv):
    """The VAE residual block (vae.py:200-218), identity or 1x1 shortcut, fp32, out of
    place and in place: an empty set stays empty, one voxel against the float64
    oracle."""
    from hi3d_amd import sparse, vae

    rng = np.random.default_rng(11)
    c, n = 32, len(coords)
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
    gp = {k: torch.as_tensor(v).to(cuda) for k, v in p.items()}
    level = sparse.Level.from_coords(torch.as_tensor(coords).to(cuda))
    x = rng.normal(0, 1, (n, c)).astype(np.float32)
    got = vae.resnet(torch.as_tensor(x).to(cuda), level, gp, "r")
    inplace = vae.resnet([torch.as_tensor(x).to(cuda)], level, gp, "r")
    assert got.shape == (n, c) and inplace.shape == (n, c)
    if n == 0:
        return
    ref = ovae.resnet_f64(x, level.table.cpu().numpy(), p, "r")
    assert oconv.rel_err(got.cpu().numpy(), ref) <= 1e-4
    assert torch.equal(inplace, got)
