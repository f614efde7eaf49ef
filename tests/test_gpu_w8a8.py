"""W8A8 on the GPU: quantiser codes and scales bit-exact against the oracle (both
rotations), int32 accumulators bit-exact, the fp16 epilogue bit-exact against the
unfused float32 formula, and the reference test's tolerance
(tests/test_w8a8_inference.py:8-20)."""

from __future__ import annotations

import hashlib

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import w8a8 as ow8a8

pytestmark = pytest.mark.gpu

SHAPES = ((3, 17, 64), (65, 131, 2112), (7, 33, 8448))


def _inputs(rows, cols, width):
    rng = np.random.default_rng(7)
    x = rng.normal(size=(rows, width)).astype(np.float16)
    w = rng.integers(-127, 128, size=(cols, width), dtype=np.int8)
    sw = rng.uniform(0.0001, 0.001, cols).astype(np.float32)
    bias = rng.normal(0, 0.01, cols).astype(np.float16)
    return x, w, sw, bias


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.mark.parametrize("rows,cols,width", SHAPES)
def test_reference_shapes_bit_exact(cuda, rows, cols, width):
    from hi3d_amd import w8a8

    golden = np.load(GOLDEN / "w8a8.npz")
    tag = f"{rows}_{cols}_{width}"
    x, w, sw, bias = _inputs(rows, cols, width)
    xt = torch.as_tensor(x).to(cuda)
    q, sa = w8a8.quantize_activation(xt)
    q, sa = q.cpu().numpy(), sa.cpu().numpy()
    assert _sha(q) == str(golden[f"q_{tag}"]) and _sha(sa) == str(golden[f"s_{tag}"])
    out, acc = w8a8.gemm(torch.as_tensor(q).to(cuda), torch.as_tensor(sa).to(cuda), torch.as_tensor(w).to(cuda),
                         torch.as_tensor(sw).to(cuda), torch.as_tensor(bias).to(cuda), return_acc=True)
    assert _sha(acc.cpu().numpy()) == str(golden[f"acc_{tag}"])
    assert _sha(out.cpu().numpy()) == str(golden[f"out_{tag}"])
    # the reference test's own check (rtol=5e-4, atol=2e-6) through linear()
    result = w8a8.linear(xt, torch.as_tensor(w).to(cuda), torch.as_tensor(sw).to(cuda),
                         torch.as_tensor(bias).to(cuda)).float().cpu().numpy()
    integer = np.asarray(q, np.int64) @ np.asarray(w, np.int64).T
    expected = integer.astype(np.float32) * sa[:, None] * sw[None, :] + bias.astype(np.float32)
    assert np.isfinite(result).all()
    np.testing.assert_allclose(result, expected, rtol=5e-4, atol=2e-6)


@pytest.mark.parametrize("rotation", ["h64", "none"])
def test_quantiser_with_outliers_bit_exact(cuda, rotation):
    from hi3d_amd import w8a8

    rng = np.random.default_rng(11)
    x = rng.standard_normal((1000, 1024)).astype(np.float32)
    out = rng.random(x.shape) < 0.01
    x[out] *= 20
    x = x.astype(np.float16)
    q, s = w8a8.quantize_activation(torch.as_tensor(x).to(cuda), rotation=rotation)
    rq, rs = ow8a8.quantize_activation(x, rotation=rotation)
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(q.cpu().numpy(), rq)


@pytest.mark.parametrize("m,k,rotation,custom", [
    (3000, 2048, "h64", False), (700, 8192, "h64", False), (700, 8192, "none", False),
    (513, 72, "none", False), (5000, 4096, "h64", True), (4099, 1024, "none", False),
])
def test_quantiser_paths_bit_exact(cuda, m, k, rotation, custom):
    """Every quantiser path against the oracle: one to eight 1024-column passes held in
    registers (with the next row prefetched up to four), widths that end inside a pass,
    more rows than waves, and a general float multiplier instead of the signs. Rows mix
    magnitudes from fp16 subnormals to 6e4, all-zero rows and one-hot rows, so the
    division by the row scale meets tiny and exact quotients."""
    from hi3d_amd import w8a8

    rng = np.random.default_rng(m + k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    mag = np.float32(10.0) ** rng.uniform(-7, 4.7, size=(m, 1)).astype(np.float32)
    x = x * mag
    x[::17] = 0.0
    x[5::23] = 0.0
    x[5::23, 3] = -2.5
    x[rng.random(x.shape) < 0.002] *= 50
    x = np.clip(x, -60000, 60000).astype(np.float16)
    mult = rng.standard_normal(k).astype(np.float32) if custom else None
    xt = torch.as_tensor(x).to(cuda)
    q, s = w8a8.quantize_activation(xt, None if mult is None else torch.as_tensor(mult).to(cuda), rotation=rotation)
    rq, rs = ow8a8.quantize_activation(x, mult, rotation=rotation)
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(q.cpu().numpy(), rq)


def test_zero_rows_and_small_k(cuda):
    from hi3d_amd import w8a8

    x = np.zeros((5, 64), np.float16)
    x[2, 7] = -3.5
    q, s = w8a8.quantize_activation(torch.as_tensor(x).to(cuda), rotation="none")
    rq, rs = ow8a8.quantize_activation(x, rotation="none")
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(s.cpu().numpy(), rs)
    q, s = w8a8.quantize_activation(torch.as_tensor(x).to(cuda))
    rq, rs = ow8a8.quantize_activation(x)
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(s.cpu().numpy(), rs)


@pytest.mark.parametrize("m,n,k", [(4096, 4096, 1024), (2048, 1024, 4096), (300, 200, 48), (129, 257, 2112)])
def test_gemm_accumulators_bit_exact(cuda, m, n, k):
    from hi3d_amd import w8a8

    rng = np.random.default_rng(m + n + k)
    q = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sa = rng.uniform(1e-3, 1e-2, m).astype(np.float32)
    sw = rng.uniform(1e-4, 1e-3, n).astype(np.float32)
    bias = rng.normal(0, 0.02, n).astype(np.float16)
    out, acc = w8a8.gemm(*(torch.as_tensor(a).to(cuda) for a in (q, sa, w, sw, bias)), return_acc=True)
    ref = (q.astype(np.float64) @ w.astype(np.float64).T).astype(np.int64)
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), ref)
    assert np.array_equal(out.cpu().numpy(), ow8a8.epilogue(ref.astype(np.int32), sa, sw, bias))


def test_workload4_shapes_sampled(cuda):
    """[65536, 1024] x [4096, 1024]^T and [65536, 4096] x [1024, 4096]^T with 1 % outliers
    x20: codes, scales and sampled outputs exact against the oracle."""
    from hi3d_amd import w8a8

    for m, k, n in ((65536, 1024, 4096), (65536, 4096, 1024)):
        rng = np.random.default_rng(k)
        x = rng.standard_normal((m, k), dtype=np.float32)
        x[rng.random((m, k)) < 0.01] *= 20
        x = x.astype(np.float16)
        wf = (rng.standard_normal((n, k), dtype=np.float32) / 32).astype(np.float16)
        bias = (rng.standard_normal(n, dtype=np.float32) * 0.02).astype(np.float16)
        for rotation in ("h64", "none"):
            wq, sw = w8a8.quantize_weight(torch.as_tensor(wf).to(cuda), rotation)
            xt = torch.as_tensor(x).to(cuda)
            q, sa = w8a8.quantize_activation(xt, rotation=rotation)
            out = w8a8.gemm(q, sa, wq, sw, torch.as_tensor(bias).to(cuda))
            rows = np.random.default_rng(5).choice(m, 256, replace=False)
            rq, rs = ow8a8.quantize_activation(x[rows], rotation=rotation)
            assert np.array_equal(q[torch.as_tensor(rows).to(cuda)].cpu().numpy(), rq)
            assert np.array_equal(sa.cpu().numpy()[rows], rs)
            wqn, swn = wq.cpu().numpy(), sw.cpu().numpy()
            ref = ow8a8.epilogue(ow8a8.int_gemm(rq, wqn).astype(np.int32), rs, swn, bias)
            assert np.array_equal(out[torch.as_tensor(rows).to(cuda)].cpu().numpy(), ref)
            # the int8 product approximates the fp16 projection
            y = x[rows].astype(np.float32) @ wf.astype(np.float32).T + bias.astype(np.float32)
            err = np.sqrt(np.mean((ref.astype(np.float32) - y) ** 2) / np.mean(y * y))
            assert err < 0.15


def test_workload4_every_row_accumulators_bit_exact(cuda):
    """Both workload shapes, [65536, 1024] x [4096, 1024]^T and [65536, 4096] x
    [1024, 4096]^T, on the codes of the outlier-laden activations and the quantised
    weights: every int32 accumulator equals the float64 product of the codes (exact:
    |acc| <= 127^2 * 4096 < 2^53), and every fp16 output equals the unfused float32
    epilogue of those accumulators. Both shapes run the persistent ping-pong kernel (K =
    1024: 16 stages per tile, 16 tiles per workgroup; K = 4096: 64 stages, 4 tiles); the
    accumulator dump comes from the same kernel as the fp16 output, whose bits must not
    change with it."""
    from hi3d_amd import w8a8

    for m, k, n in ((65536, 1024, 4096), (65536, 4096, 1024)):
        g = torch.Generator(device=cuda).manual_seed(k)
        x = torch.randn((m, k), device=cuda, generator=g)
        x = torch.where(torch.rand((m, k), device=cuda, generator=g) < 0.01, x * 20, x).half()
        wf = (torch.randn((n, k), device=cuda, generator=g) / 32).half()
        bias = (torch.randn(n, device=cuda, generator=g) * 0.02).half()
        wq, sw = w8a8.quantize_weight(wf)
        q, sa = w8a8.quantize_activation(x)
        del x, wf
        plain = w8a8.gemm(q, sa, wq, sw, bias)
        out, acc = w8a8.gemm(q, sa, wq, sw, bias, return_acc=True)
        assert torch.equal(plain, out)
        del plain
        wd = torch.as_tensor(wq.cpu().numpy().astype(np.float64))
        swn, bn = sw.cpu().numpy(), bias.cpu().numpy()
        for r0 in range(0, m, 8192):
            qd = torch.as_tensor(q[r0:r0 + 8192].cpu().numpy().astype(np.float64))
            ref = (qd @ wd.T).numpy().astype(np.int64)
            got = acc[r0:r0 + 8192].cpu().numpy()
            assert np.array_equal(got.astype(np.int64), ref), (m, k, n, r0)
            want = ow8a8.epilogue(ref.astype(np.int32), sa[r0:r0 + 8192].cpu().numpy(), swn, bn)
            assert np.array_equal(out[r0:r0 + 8192].cpu().numpy(), want), (m, k, n, r0)
        del out, acc


def test_gemm_non_contiguous_operands_and_scale_checks(cuda):
    """A transposed weight and a column-sliced activation give the bits of their
    contiguous copies; float16 or short scale vectors and a short bias are refused
    before any launch."""
    from hi3d_amd import w8a8

    rng = np.random.default_rng(31)
    m, n, k = 1000, 520, 320
    q_wide = torch.as_tensor(rng.integers(-127, 128, size=(m, k + 64), dtype=np.int8)).to(cuda)
    w_t = torch.as_tensor(rng.integers(-127, 128, size=(k, n), dtype=np.int8)).to(cuda)
    sa = torch.as_tensor(rng.uniform(1e-3, 1e-2, m).astype(np.float32)).to(cuda)
    sw = torch.as_tensor(rng.uniform(1e-4, 1e-3, n).astype(np.float32)).to(cuda)
    bias = torch.as_tensor(rng.normal(0, 0.02, n).astype(np.float16)).to(cuda)
    q, w = q_wide[:, 32:32 + k], w_t.T
    assert not q.is_contiguous() and not w.is_contiguous()
    got, acc = w8a8.gemm(q, sa, w, sw, bias, return_acc=True)
    want, acc_want = w8a8.gemm(q.contiguous(), sa, w.contiguous(), sw, bias, return_acc=True)
    assert torch.equal(got, want) and torch.equal(acc, acc_want)
    ref = q.cpu().numpy().astype(np.float64) @ w.cpu().numpy().astype(np.float64).T
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), ref.astype(np.int64))
    with pytest.raises(ValueError, match="float32 scales"):
        w8a8.gemm(q, sa.half(), w, sw, bias)
    with pytest.raises(ValueError, match="scales must be"):
        w8a8.gemm(q, sa, w, sw[:-1], bias)
    with pytest.raises(ValueError, match="bias must be"):
        w8a8.gemm(q, sa, w, sw, bias[:-1])


@pytest.mark.parametrize("m,n,k,with_bias", [(1000, 520, 320, True), (4096, 4096, 1024, True), (300, 264, 1984, False),
                                             (256, 256, 256, True), (2600, 1032, 1536, True), (1000, 520, 4096, True),
                                             (600, 300, 2112, False), (200, 264, 512, True), (513, 8, 768, False),
                                             (777, 1800, 2560, True)])
def test_gemm_full_output_bit_exact(cuda, m, n, k, with_bias):
    """Every output bit-equal to the oracle on every fused-output path: the persistent
    ping-pong kernel (k % 256 == 0, k >= 512, n % 8 == 0: ragged rows and channel tiles
    through its store descriptors, one tile per workgroup or several, k = 512 and 768
    with no middle stage loop), the ping-pong kernel (k = 256), the persistent four-wave
    kernel (k % 64 == 0, k < 2048, m, n >= 256: its edge tiles move back to overlap their
    neighbours) and the one-tile kernel (the rest), with and without bias; each also
    equals its accumulator-dump variant's output."""
    from hi3d_amd import w8a8

    rng = np.random.default_rng(m * 7 + n * 3 + k)
    q = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sa = rng.uniform(1e-3, 1e-2, m).astype(np.float32)
    sw = rng.uniform(1e-4, 1e-3, n).astype(np.float32)
    bias = rng.normal(0, 0.02, n).astype(np.float16)
    dev = [torch.as_tensor(a).to(cuda) for a in (q, sa, w, sw, bias)]
    bias_t = dev[4] if with_bias else None
    out = w8a8.gemm(dev[0], dev[1], dev[2], dev[3], bias_t)
    ref_acc = (q.astype(np.float64) @ w.astype(np.float64).T).astype(np.int64).astype(np.int32)
    ref = ow8a8.epilogue(ref_acc, sa, sw, bias if with_bias else np.zeros(n, np.float16))
    got = out.cpu().numpy()
    assert np.array_equal(got, ref), int((got != ref).sum())
    out2, _ = w8a8.gemm(dev[0], dev[1], dev[2], dev[3], bias_t, return_acc=True)
    assert torch.equal(out, out2)


def test_checkpoint_round_trip(cuda, tmp_path):
    """A ``hi3d-w8a8-h64`` safetensors file (written here: no released checkpoint is
    available offline) loads with its int8 rows and float32 scales and drives the same
    projection bits as the in-memory weights; files of another format, or without the
    first block's QKV scale, are refused with the reference's message
    (src/hi3d_mac/mlx_backend/transformer.py:289-301)."""
    from hi3d_amd import w8a8

    rng = np.random.default_rng(17)
    k, n = 1024, 3072
    dense = {
        "blocks.0.self_attn.to_qkv.weight": torch.as_tensor((rng.standard_normal((n, k)) / 32).astype(np.float16)).to(cuda),
        "blocks.0.self_attn.to_qkv.bias": torch.as_tensor((rng.standard_normal(n) * 0.02).astype(np.float16)).to(cuda),
        "blocks.0.norm1.weight": torch.as_tensor(rng.standard_normal(k).astype(np.float32)).to(cuda),
    }
    q = w8a8.quantize_checkpoint(dense, ["blocks.0.self_attn.to_qkv"])
    path = tmp_path / "w8a8.safetensors"
    w8a8.save_checkpoint(path, q)
    loaded = w8a8.load_checkpoint(path, cuda)
    assert set(loaded) == set(q)
    for key in q:
        assert loaded[key].dtype == q[key].dtype and torch.equal(loaded[key], q[key])
    wq, sw = loaded["blocks.0.self_attn.to_qkv.weight"], loaded["blocks.0.self_attn.to_qkv.w8_scale"]
    rq, rs = ow8a8.quantize_activation(dense["blocks.0.self_attn.to_qkv.weight"].cpu().numpy())
    assert np.array_equal(wq.cpu().numpy(), rq) and np.array_equal(sw.cpu().numpy(), rs)
    x = torch.as_tensor(rng.standard_normal((300, k)).astype(np.float16)).to(cuda)
    got = w8a8.linear_named(x, loaded, "blocks.0.self_attn.to_qkv")
    want = w8a8.linear(x, wq, sw, dense["blocks.0.self_attn.to_qkv.bias"])
    assert torch.equal(got, want)
    from safetensors.torch import save_file

    other = tmp_path / "fp16.safetensors"
    save_file({k: v.cpu() for k, v in dense.items()}, str(other), metadata={"format": "pt"})
    with pytest.raises(ValueError, match="released Hi3Dv1.0-mlx-w8a8"):
        w8a8.load_checkpoint(other, cuda)
    partial = tmp_path / "partial.safetensors"
    w8a8.save_checkpoint(partial, {"blocks.0.norm1.weight": dense["blocks.0.norm1.weight"]})
    with pytest.raises(ValueError, match="released Hi3Dv1.0-mlx-w8a8"):
        w8a8.load_checkpoint(partial, cuda)
    assert set(w8a8.load_checkpoint(partial, cuda, require_blocks=False)) == {"blocks.0.norm1.weight"}


def _norm_params(rng, c, affine, modulate):
    kw = {}
    if affine:
        kw["weight"] = rng.uniform(0.5, 1.5, c).astype(np.float32)
        kw["bias"] = rng.normal(0, 0.3, c).astype(np.float32)
    if modulate:
        kw["scale"] = (1 + 0.3 * rng.standard_normal(c)).astype(np.float16)
        kw["shift"] = (0.3 * rng.standard_normal(c)).astype(np.float16)
    return kw


@pytest.mark.parametrize("c,rotation", [(64, "h64"), (128, "none"), (1024, "h64"), (1024, "none"), (2112, "h64"),
                                        (4096, "h64"), (1000, "none"), (4160, "h64")])
def test_norm_quantize_bitwise_equals_norm_then_quantiser(cuda, c, rotation):
    """LayerNorm (plain, affine, modulate, both) fused with the quantiser: codes and
    scales bitwise equal to ``layer_norm_modulate`` then ``quantize_activation``, and to
    the oracle's quantiser on the norm's fp16 rows. One lane per 8 columns from 8 to 64
    lanes per row, two to eight chunks per lane, widths that leave lanes idle (1000,
    2112), and the composed path above 4096. Rows include all-equal rows (a zero
    norm), rows whose modulated values overflow fp16 (an infinite scale, compared with
    the composition only) and tiny and huge magnitudes."""
    from hi3d_amd import kernels, w8a8

    rng = np.random.default_rng(c + len(rotation))
    m = 777
    x = (rng.standard_normal((m, c)) * 10.0 ** rng.uniform(-3, 3, (m, 1)) + rng.normal(0, 2, (m, 1)))
    x[3] = 1.25  # constant row: every normalised value 0
    x[10, : c // 3] *= 40
    x = np.clip(x, -60000, 60000).astype(np.float16)
    xt = torch.as_tensor(x).to(cuda)
    for affine, modulate in ((False, False), (True, False), (False, True), (True, True)):
        kw = {k: torch.as_tensor(v).to(cuda) for k, v in _norm_params(rng, c, affine, modulate).items()}
        if modulate:
            kw["scale"][c // 2] = 60000.0  # column c/2 overflows to +-inf in most rows
        q, s = w8a8.norm_quantize(xt, 1e-6, rotation=rotation, **kw)
        h = kernels.layer_norm_modulate(xt, 1e-6, **kw)
        rq, rs = w8a8.quantize_activation(h, rotation=rotation)
        assert torch.equal(q, rq) and torch.equal(s, rs), (affine, modulate)
        # the oracle on the rows with a finite scale (its int8 cast of a NaN quotient is
        # the platform's, not the reference's clamp)
        fin = np.isfinite(s.cpu().numpy())
        assert fin.sum() >= m // 2
        oq, os_ = ow8a8.quantize_activation(h.cpu().numpy()[fin], rotation=rotation)
        assert np.array_equal(q.cpu().numpy()[fin], oq) and np.array_equal(s.cpu().numpy()[fin], os_)


def test_norm_quantize_custom_multiplier_and_views(cuda):
    """A float multiplier in place of the signs, a row-sliced input and leading batch
    dimensions give the composed bits."""
    from hi3d_amd import kernels, w8a8

    rng = np.random.default_rng(3)
    c = 1024
    x = torch.as_tensor(rng.standard_normal((2, 300, c)).astype(np.float16)).to(cuda)
    mult = torch.as_tensor(rng.standard_normal(c).astype(np.float32)).to(cuda)
    kw = {k: torch.as_tensor(v).to(cuda) for k, v in _norm_params(rng, c, False, True).items()}
    for xin in (x, x[:, 7:]):
        q, s = w8a8.norm_quantize(xin, 1e-6, multiplier=mult, **kw)
        rq, rs = w8a8.quantize_activation(kernels.layer_norm_modulate(xin, 1e-6, **kw), mult)
        assert tuple(q.shape) == (xin.numel() // c, c)
        assert torch.equal(q, rq) and torch.equal(s, rs)
    with pytest.raises(ValueError, match="fp16"):
        w8a8.norm_quantize(x.float(), 1e-6)
    with pytest.raises(ValueError, match="H64"):
        w8a8.norm_quantize(x[..., :72], 1e-6)
    with pytest.raises(ValueError, match="scale and shift"):
        w8a8.norm_quantize(x, 1e-6, scale=kw["scale"])


def test_norm_linear_workload4_shape_a(cuda):
    """The MLP's first projection as the transformer block runs it, on config 4's shape A
    (65,536 tokens, 1024 -> 4096): modulated norm fused with the quantiser, then the int8
    GEMM; every output bit equals the composition of the three kernels."""
    from hi3d_amd import kernels, w8a8

    m, k, n = 65536, 1024, 4096
    g = torch.Generator(device=cuda).manual_seed(41)
    x = (torch.randn((m, k), device=cuda, generator=g) * 3 + 0.5).half()
    scale = (1 + 0.2 * torch.randn(k, device=cuda, generator=g)).half()
    shift = (0.2 * torch.randn(k, device=cuda, generator=g)).half()
    wq, sw = w8a8.quantize_weight((torch.randn((n, k), device=cuda, generator=g) / 32).half())
    bias = (torch.randn(n, device=cuda, generator=g) * 0.02).half()
    fused = w8a8.norm_linear(x, 1e-6, wq, sw, bias, scale=scale, shift=shift)
    composed = w8a8.linear(kernels.layer_norm_modulate(x, 1e-6, scale=scale, shift=shift), wq, sw, bias)
    assert torch.equal(fused, composed)
