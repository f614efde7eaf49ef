"""LayerNorm + adaLN row kernel, the adaLN projection and the residual block on the GPU.

LayerNorm gate (the reference's own, tests/test_mlx_kernels.py:58-60): more than
99.9 % of outputs bit-equal to the oracle and all within atol 1e-2 / rtol 1e-3 (the rest
differ by one fp16 ulp from the fp32 summation order). Block gate: max|y - y_ref| /
rms(y_ref) <= 1e-2 against a float64 composition.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import conv as oconv
from oracle import norm as onorm

pytestmark = pytest.mark.gpu


def _ln_inputs(seed=5, rows=100, c=2112):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, c)) * 3 + 0.5).astype(np.float16)
    scale = (1 + 0.1 * rng.standard_normal(c)).astype(np.float16)
    shift = (0.1 * rng.standard_normal(c)).astype(np.float16)
    w = rng.standard_normal(c).astype(np.float32)
    b = rng.standard_normal(c).astype(np.float32)
    return x, scale, shift, w, b


def _check_ln(got, ref):
    got = np.asarray(got)
    equal = float(np.mean(got == ref))
    assert equal > 0.999, equal
    np.testing.assert_allclose(got.astype(np.float32), ref.astype(np.float32), atol=1e-2, rtol=1e-3)


@pytest.mark.parametrize("c", [2112, 256, 64, 8, 20, 4104])
def test_layer_norm_modulate_variants(cuda, c):
    from hi3d_amd import kernels

    x, scale, shift, w, b = _ln_inputs(c=c)
    xt = torch.as_tensor(x).to(cuda)
    for kw in ({"scale": scale, "shift": shift}, {"weight": w, "bias": b}, {}):
        got = kernels.layer_norm_modulate(xt, 1e-6, **{k: torch.as_tensor(v).to(cuda) for k, v in kw.items()})
        _check_ln(got.cpu().numpy(), onorm.layer_norm_modulate(x, 1e-6, **kw))


def test_layer_norm_golden_head(cuda):
    from hi3d_amd import kernels

    data = np.load(GOLDEN / "layer_norm.npz")
    x, scale, shift, _, _ = _ln_inputs()
    got = kernels.layer_norm_modulate(torch.as_tensor(x[:2]).to(cuda), 1e-6, scale=torch.as_tensor(scale).to(cuda),
                                      shift=torch.as_tensor(shift).to(cuda))
    _check_ln(got.cpu().numpy(), data["mod_head"])


def test_adaln_projection(cuda):
    from hi3d_amd import kernels

    rng = np.random.default_rng(3)
    w = (rng.standard_normal((512, 1024)) / 32).astype(np.float32)
    b = (rng.standard_normal(512) * 0.02).astype(np.float32)
    cond = rng.standard_normal(1024).astype(np.float32)
    for silu in (False, True):
        s1p, sh = kernels.adaln_projection(torch.as_tensor(w).to(cuda), torch.as_tensor(b).to(cuda),
                                           torch.as_tensor(cond).to(cuda), silu)
        rs, rh = onorm.adaln_projection(w, b, cond, silu)
        np.testing.assert_allclose(s1p.float().cpu().numpy(), rs.astype(np.float32), atol=2e-3, rtol=1e-3)
        np.testing.assert_allclose(sh.float().cpu().numpy(), rh.astype(np.float32), atol=2e-3, rtol=1e-3)
    # closed forms: W = 0, b = [s; t] gives exactly (fp16(1 + s), fp16(t)); W = [0; I]
    # gives (1, fp16(cond)) whatever the summation order
    s = np.linspace(-2, 2, 256).astype(np.float32)
    t = np.linspace(3, -1, 256).astype(np.float32)
    s1p, sh = kernels.adaln_projection(torch.zeros((512, 1024), device=cuda), torch.as_tensor(np.concatenate([s, t])).to(cuda),
                                       torch.as_tensor(cond).to(cuda))
    assert np.array_equal(s1p.cpu().numpy(), (1 + s.astype(np.float16).astype(np.float32)).astype(np.float16))
    assert np.array_equal(sh.cpu().numpy(), t.astype(np.float16))
    eye = np.zeros((512, 256), np.float32)
    eye[256:] = np.eye(256)
    s1p, sh = kernels.adaln_projection(torch.as_tensor(eye).to(cuda), None, torch.as_tensor(cond[:256]).to(cuda))
    assert np.array_equal(s1p.cpu().numpy(), np.ones(256, np.float16))
    assert np.array_equal(sh.cpu().numpy(), cond[:256].astype(np.float16))


def _block_weights(rng, c, d, cuda):
    from hi3d_amd.block import ResBlockWeights

    pw = (rng.standard_normal((2 * c, d)) / np.sqrt(d) * 0.3).astype(np.float32)
    pb = (rng.standard_normal(2 * c) * 0.02).astype(np.float32)
    w1 = (rng.standard_normal((c, 27, c)) / np.sqrt(27 * c)).astype(np.float16)
    w2 = (rng.standard_normal((c, 27, c)) / np.sqrt(27 * c)).astype(np.float16)
    weights = ResBlockWeights(*(torch.as_tensor(a).to(cuda) for a in (pw, pb)), torch.as_tensor(w1).to(cuda), None,
                              torch.as_tensor(w2).to(cuda), None)
    return weights, (pw, pb, w1, w2)


def test_residual_block_small(cuda):
    from hi3d_amd import block, kmap

    rng = np.random.default_rng(9)
    xyz = np.argwhere(rng.random((20, 20, 20)) < 0.2)
    idx = np.concatenate([np.zeros((len(xyz), 1)), xyz], 1).astype(np.int32)
    idx = idx[rng.permutation(len(idx))]
    c, d = 64, 96
    x = rng.standard_normal((len(idx), c)).astype(np.float16)
    cond = rng.standard_normal(d).astype(np.float32)
    weights, (pw, pb, w1, w2) = _block_weights(rng, c, d, cuda)
    km = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [20] * 3, 1)
    y = block.residual_block(torch.as_tensor(x).to(cuda), km.plan(), torch.as_tensor(cond).to(cuda), weights)
    ref = onorm.residual_block_f64(x, km.table.cpu().numpy(), cond, pw, pb, w1, None, w2, None)
    assert oconv.rel_err(y.float().cpu().numpy(), ref) <= 1e-2


def test_residual_block_workload5_sampled(cuda):
    """1024^3 shell (~4.4M voxels), C = 256, cond 1024 -> [512, 1024] projection."""
    from hi3d_amd import block, kmap, workloads

    idx = workloads.coords_for("resblock_c256_fp16", device=cuda)
    rng = np.random.default_rng(51)
    c, d = 256, 1024
    x = workloads.normal((len(idx), c), 1.0, seed=52, dtype=np.float16)
    cond = workloads.normal((d,), 1.0, seed=53)
    weights, (pw, pb, w1, w2) = _block_weights(rng, c, d, cuda)
    km = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [1024] * 3, 1)
    y = block.residual_block(torch.as_tensor(x).to(cuda), km.plan(), torch.as_tensor(cond).to(cuda), weights)
    rows = np.random.default_rng(0).choice(len(idx), 512, replace=False)
    table = km.table.cpu().numpy()
    ref = onorm.residual_block_f64(x, table, cond, pw, pb, w1, None, w2, None, rows=rows)
    assert oconv.rel_err(y.float().cpu().numpy()[rows], ref) <= 1e-2
    assert torch.isfinite(y).all()
