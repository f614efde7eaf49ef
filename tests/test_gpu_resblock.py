"""The transformer's sparse residual block (``resblock.SparseResBlock3d``) on the GPU
against the float64 composition of the reference's block (oracle ``res_block3d_f64``),
with and without the skip projection, with two batch elements of their own embeddings,
and with the paired factor-2 downsample / upsample in front.

Gate (fp16): max|y - y_ref| / rms(y_ref) <= 1e-2. The fused LayerNorm + SiLU kernel is
checked on its own at the LayerNorm gate (more than 99.9 % bit-equal to the oracle's
fp16 steps, all within atol 1e-2 / rtol 1e-3).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import conv as oconv
from oracle import kmap as okmap
from oracle import norm as onorm

pytestmark = pytest.mark.gpu


def _indices(rng, side, density, batches):
    """Batch-grouped coordinates (rows of one element contiguous, shuffled inside)."""
    parts = []
    for b in range(batches):
        xyz = np.argwhere(rng.random((side,) * 3) < density)
        xyz = xyz[rng.permutation(len(xyz))]
        parts.append(np.concatenate([np.full((len(xyz), 1), b), xyz], 1))
    return np.concatenate(parts).astype(np.int32)


def _spans(idx):
    spans, start = [], 0
    for b in range(int(idx[:, 0].max()) + 1):
        count = int((idx[:, 0] == b).sum())
        spans.append(slice(start, start + count))
        start += count
    return spans


def _block(rng, cuda, channels, emb, out=None, **kw):
    """A block with every parameter random (the zero-initialised linear too), in fp16,
    and its state dict as float64 arrays for the oracle."""
    from hi3d_amd.resblock import SparseResBlock3d

    m = SparseResBlock3d(channels, emb, out_channels=out, **kw)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if name.startswith("norm1.weight"):
                p.copy_(torch.as_tensor(rng.uniform(0.5, 1.5, p.shape)))
            elif name.endswith("bias"):
                p.copy_(torch.as_tensor(rng.normal(0, 0.1, p.shape)))
            else:
                fan_in = int(np.prod(p.shape[1:]))
                p.copy_(torch.as_tensor(rng.normal(0, 1 / np.sqrt(fan_in), p.shape)))
    m = m.half().to(cuda)
    params = {k: v.detach().float().cpu().numpy().astype(np.float64) for k, v in m.state_dict().items()}
    return m, params


def _sparse(cuda, idx, x):
    from hi3d_amd.nn import SparseTensor

    return SparseTensor(torch.as_tensor(x).to(cuda), torch.as_tensor(idx).to(cuda))


@pytest.mark.parametrize("c", [64, 256, 2112, 40])
def test_layer_norm_silu_kernel(cuda, c):
    """LayerNorm + affine + SiLU, LayerNorm + modulate + SiLU and plain LayerNorm + SiLU
    against the oracle's fp16 steps (LN as layer_norm_modulate, then silu_f16)."""
    from hi3d_amd import kernels

    rng = np.random.default_rng(c)
    x = (rng.standard_normal((300, c)) * 2 + 0.3).astype(np.float16)
    w = rng.uniform(0.5, 1.5, c).astype(np.float32)
    b = rng.normal(0, 0.3, c).astype(np.float32)
    scale = (1 + 0.2 * rng.standard_normal(c)).astype(np.float16)
    shift = (0.2 * rng.standard_normal(c)).astype(np.float16)
    xt = torch.as_tensor(x).to(cuda)
    for kw in ({"weight": w, "bias": b}, {"scale": scale, "shift": shift}, {}):
        got = kernels.layer_norm_modulate(xt, 1e-6, act="silu", **{k: torch.as_tensor(v).to(cuda)
                                                                     for k, v in kw.items()}).cpu().numpy()
        ref = onorm.silu_f16(onorm.layer_norm_modulate(x, 1e-6, **kw))
        assert float(np.mean(got == ref)) > 0.999
        np.testing.assert_allclose(got.astype(np.float32), ref.astype(np.float32), atol=1e-2, rtol=1e-3)


@pytest.mark.parametrize("channels,out,batches", [(64, None, 1), (64, 128, 2), (256, None, 1)])
def test_res_block_matches_float64(cuda, channels, out, batches):
    rng = np.random.default_rng(channels + batches)
    side = 18
    idx = _indices(rng, side, 0.15, batches)
    x = rng.standard_normal((len(idx), channels)).astype(np.float16)
    emb = rng.standard_normal((batches, 96)).astype(np.float16)
    m, p = _block(rng, cuda, channels, 96, out)
    st = _sparse(cuda, idx, x)
    y = m(st, torch.as_tensor(emb).to(cuda))
    assert y.feats.dtype == torch.float16 and tuple(y.feats.shape) == (len(idx), out or channels)
    assert torch.equal(y.coords, st.coords)
    table = okmap.neighbour_table(idx, [side] * 3)
    ref = onorm.res_block3d_f64(x, table, emb.astype(np.float64), p, _spans(idx))
    assert oconv.rel_err(y.feats.float().cpu().numpy(), ref) <= 1e-2
    # a second pass over the same rows reuses the cached maps and gives the same bits
    again = m(st.replace(torch.as_tensor(x).to(cuda)), torch.as_tensor(emb).to(cuda))
    assert torch.equal(again.feats, y.feats)


def test_res_block_downsample_then_upsample(cuda):
    """A downsampling block (mean of each coarse cell's rows with the reference's
    ``count + 1`` divisor, then the block on the coarse rows) followed by its paired
    upsampling block (parent rows copied back to the fine rows, then the block)."""
    rng = np.random.default_rng(77)
    side = 20
    idx = _indices(rng, side, 0.12, 2)
    x = rng.standard_normal((len(idx), 64)).astype(np.float16)
    emb = rng.standard_normal((2, 32)).astype(np.float16)
    down, pd = _block(rng, cuda, 64, 32, 128, downsample=True)
    up, pu = _block(rng, cuda, 128, 32, 64, upsample=True)
    st = _sparse(cuda, idx, x)
    coarse = down(st, torch.as_tensor(emb).to(cuda))
    low, inverse, counts, slot, table_down, table_up = okmap.stride2_structure(idx)
    assert np.array_equal(coarse.coords.cpu().numpy(), low)
    pooled = oconv.gather_mean(x.astype(np.float64), table_down, extra=1)
    ref_c = onorm.res_block3d_f64(pooled, okmap.neighbour_table(low, [side // 2] * 3), emb.astype(np.float64), pd,
                                  _spans(low))
    got_c = coarse.feats.float().cpu().numpy()
    assert oconv.rel_err(got_c, ref_c) <= 1e-2
    fine = up(coarse, torch.as_tensor(emb).to(cuda))
    assert torch.equal(fine.coords, st.coords)
    x_up = got_c[inverse]
    ref_f = onorm.res_block3d_f64(x_up, okmap.neighbour_table(idx, [side] * 3), emb.astype(np.float64), pu,
                                  _spans(idx))
    assert oconv.rel_err(fine.feats.float().cpu().numpy(), ref_f) <= 1e-2


def test_res_block_errors(cuda):
    from hi3d_amd.resblock import SparseResBlock3d

    with pytest.raises(ValueError, match="cannot downsample and upsample"):
        SparseResBlock3d(8, 8, downsample=True, upsample=True)
    rng = np.random.default_rng(5)
    idx = _indices(rng, 8, 0.3, 1)
    m = SparseResBlock3d(16, 8).to(cuda)
    with pytest.raises(NotImplementedError, match="fp16"):
        m(_sparse(cuda, idx, rng.standard_normal((len(idx), 16)).astype(np.float32)), torch.zeros(8, device=cuda))
    m = m.half()
    with pytest.raises(ValueError, match="embedding"):
        m(_sparse(cuda, idx, rng.standard_normal((len(idx), 16)).astype(np.float16)),
          torch.zeros((2, 8), device=cuda, dtype=torch.float16))


@pytest.mark.parametrize("n,cin,cout,with_bias,with_res", [
    (4429, 128, 256, True, True), (1000, 64, 128, True, False), (77, 16, 64, False, True),
    (5000, 112, 192, True, True), (33, 128, 256, False, False), (1, 48, 64, True, True)])
def test_dense_linear_bitwise_equals_identity_plan_conv(cuda, n, cin, cout, with_bias, with_res):
    """The row-wise linear kernel against the gather convolution over the one-offset
    identity plan (same MFMA sequence and rounding points): bitwise equal, ragged row
    counts included; in place over the residual too; and against float64 at the fp16
    gate."""
    from hi3d_amd import conv, kmap

    rng = np.random.default_rng(n + cin + cout)
    x = torch.as_tensor(rng.standard_normal((n, cin)).astype(np.float16)).to(cuda)
    w = torch.as_tensor((rng.standard_normal((cout, cin)) / np.sqrt(cin)).astype(np.float16)).to(cuda)
    b = torch.as_tensor(rng.normal(0, 0.1, cout).astype(np.float16)).to(cuda) if with_bias else None
    r = torch.as_tensor(rng.standard_normal((n, cout)).astype(np.float16)).to(cuda) if with_res else None
    got = conv.dense_linear(x, w, b, residual=r)
    want = conv.conv(x, kmap.identity_plan(n, x.device), w[:, None, :], b, residual=r)
    assert torch.equal(got, want)
    if with_res:
        inplace = r.clone()
        conv.dense_linear(x, w, b, residual=inplace, out=inplace)
        assert torch.equal(inplace, want)
    ref = x.double().cpu() @ w.double().cpu().T
    if with_bias:
        ref = ref + b.double().cpu()
    if with_res:
        ref = ref + r.double().cpu()
    assert oconv.rel_err(got.float().cpu().numpy(), ref.numpy()) <= 1e-2


def test_dense_linear_refuses_unsupported_shapes(cuda):
    from hi3d_amd import conv

    x = torch.zeros((8, 40), dtype=torch.float16, device=cuda)
    with pytest.raises(ValueError, match="Cin % 16"):
        conv.dense_linear(x, torch.zeros((64, 40), dtype=torch.float16, device=cuda))
    with pytest.raises(ValueError, match="input channels"):
        conv.dense_linear(x, torch.zeros((64, 48), dtype=torch.float16, device=cuda))
    with pytest.raises(ValueError, match="Cin % 16"):
        conv.dense_linear(x[:, :32], torch.zeros((96, 32), dtype=torch.float16, device=cuda))


@pytest.mark.parametrize("cin,batches,side", [(256, 1, 18), (128, 3, 14), (512, 2, 12), (192, 2, 16)])
def test_conv_ln_silu_bitwise_equals_conv_then_norm(cuda, cin, batches, side):
    """conv1 with norm2, each row's batch modulation and SiLU in its epilogue against the
    convolution followed by the LayerNorm + modulate + SiLU kernel on each batch's rows:
    bitwise equal (rows of several batch elements interleaved, so tiles mix batches)."""
    from hi3d_amd import conv, kernels, kmap

    rng = np.random.default_rng(cin + batches)
    idx = _indices(rng, side, 0.2, batches)
    idx = idx[rng.permutation(len(idx))]  # interleave the batch elements' rows
    n = len(idx)
    coords = torch.as_tensor(idx).to(cuda)
    km = kmap.build_kernel_map(coords, [side] * 3, batches)
    plan = km.plan()
    x = torch.as_tensor(rng.standard_normal((n, cin)).astype(np.float16)).to(cuda)
    w = torch.as_tensor((rng.standard_normal((128, 27, cin)) / np.sqrt(27 * cin)).astype(np.float16)).to(cuda)
    b = torch.as_tensor(rng.normal(0, 0.1, 128).astype(np.float16)).to(cuda)
    scale1p = torch.as_tensor((1 + 0.3 * rng.standard_normal((batches, 128))).astype(np.float16)).to(cuda)
    shift = torch.as_tensor((0.3 * rng.standard_normal((batches, 128))).astype(np.float16)).to(cuda)
    got = conv.conv_ln_silu(x, plan, w, b, coords, scale1p, shift, 1e-6)
    h = conv.gather_conv(x, plan, w, b)
    want = torch.empty_like(h)
    for bb in range(batches):
        sel = coords[:, 0] == bb
        want[sel] = kernels.layer_norm_modulate(h[sel].contiguous(), 1e-6, scale=scale1p[bb], shift=shift[bb],
                                                act="silu")
    assert torch.equal(got, want)


def test_conv_ln_silu_refuses_unsupported_shapes(cuda):
    from hi3d_amd import conv, kmap

    idx = _indices(np.random.default_rng(1), 8, 0.3, 1)
    coords = torch.as_tensor(idx).to(cuda)
    plan = kmap.build_kernel_map(coords, [8] * 3, 1).plan()
    x = torch.zeros((len(idx), 96), dtype=torch.float16, device=cuda)
    w = torch.zeros((128, 27, 96), dtype=torch.float16, device=cuda)
    s = torch.ones((1, 128), dtype=torch.float16, device=cuda)
    with pytest.raises(ValueError, match="128..512"):
        conv.conv_ln_silu(x, plan, w, None, coords, s, s, 1e-6)
    with pytest.raises(ValueError, match="coords"):
        conv.conv_ln_silu(x[:, :64].repeat(1, 2), plan, w[..., :64].repeat(1, 1, 2), None, coords[:5], s, s, 1e-6)
