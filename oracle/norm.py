"""LayerNorm + adaLN and residual-block oracle (NumPy). Test infrastructure only."""

from __future__ import annotations

import numpy as np

from .conv import gather_conv_f64


def layer_norm_modulate(x, eps, weight=None, bias=None, scale=None, shift=None) -> np.ndarray:
    """Restates ``layer_norm_modulate`` (src/hi3d_mac/mlx_backend/kernels.py:162-201):
    fp32 two-pass mean / variance, ``inv = 1 / sqrt(var + eps)``,
    ``y = (x - mean) * inv`` (``* w + b``), ``h = fp16(y)``, then
    ``fp16(fp16(h * scale) + shift)`` (two roundings, no FMA)."""
    xf = np.asarray(x).astype(np.float32)
    c = xf.shape[-1]
    mean = (xf.sum(axis=-1, dtype=np.float32) / np.float32(c)).astype(np.float32)
    d = xf - mean[..., None]
    var = ((d * d).sum(axis=-1, dtype=np.float32) / np.float32(c)).astype(np.float32)
    inv = (np.float32(1.0) / np.sqrt(var + np.float32(eps))).astype(np.float32)
    y = d * inv[..., None]
    if weight is not None:
        y = y * np.asarray(weight, np.float32) + np.asarray(bias, np.float32)
    h = y.astype(np.float16)
    if scale is not None:
        p = (h.astype(np.float32) * np.asarray(scale).astype(np.float16).astype(np.float32)).astype(np.float16)
        h = (p.astype(np.float32) + np.asarray(shift).astype(np.float16).astype(np.float32)).astype(np.float16)
    return h


def adaln_projection(weight, bias, cond, apply_silu: bool = False):
    """``(fp16(1 + fp16(y[:C])), fp16(y[C:]))`` for ``y = W @ cond' + b`` (float64 sum,
    the (scale, shift) chunk order of src/hi3d_mac/mlx_backend/transformer.py:413-416)."""
    c = np.asarray(cond, np.float64).reshape(-1)
    if apply_silu:
        c = c / (1.0 + np.exp(-c))
    y = np.asarray(weight, np.float64) @ c
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    half = y.shape[0] // 2
    scale = y[:half].astype(np.float32).astype(np.float16)
    scale1p = (np.float32(1.0) + scale.astype(np.float32)).astype(np.float16)
    shift = y[half:].astype(np.float32).astype(np.float16)
    return scale1p, shift


def residual_block_f64(x, table, cond, proj_w, proj_b, w1, b1, w2, b2, eps=1e-6, rows=None, apply_silu=False):
    """Float64 composition of the block on fp16-rounded inputs:
    ``x + conv2(silu(conv1(LN(x) * (1 + scale) + shift)))``; conv2 and the residual are
    evaluated for ``rows`` only (all if None)."""
    scale1p, shift = adaln_projection(proj_w, proj_b, cond, apply_silu)
    t = np.asarray(table)
    n = int(np.asarray(x).shape[0])

    def modulated(sel):
        xf = np.asarray(x[sel]).astype(np.float64)
        mean = xf.mean(axis=1, keepdims=True)
        var = ((xf - mean) ** 2).mean(axis=1, keepdims=True)
        h = (xf - mean) / np.sqrt(var + eps)
        return h * scale1p.astype(np.float64) + shift.astype(np.float64)

    if rows is None:
        h = modulated(slice(None))
        h1 = gather_conv_f64(h, t, w1, b1, act="silu")
        return gather_conv_f64(h1, t, w2, b2, residual=np.asarray(x).astype(np.float64))
    # conv2 at `rows` needs conv1 at their neighbours, which needs LN two hops out;
    # rows outside the neighbourhood stay zero and are never gathered
    need1 = np.unique(t[rows].reshape(-1))
    need1 = need1[need1 < n]
    need2 = np.unique(t[need1].reshape(-1))
    need2 = need2[need2 < n]

    def compact(sel):  # row id -> position in `sel` (len(sel) for every other row)
        m = np.full(n + 1, len(sel), dtype=np.int64)
        m[sel] = np.arange(len(sel))
        return m

    h2 = modulated(need2)
    h1 = gather_conv_f64(h2, compact(need2)[t[need1]], w1, b1, act="silu")
    out = gather_conv_f64(h1, compact(need1)[t[rows]], w2, b2)
    return out + np.asarray(x[rows]).astype(np.float64)


def silu_f16(h) -> np.ndarray:
    """fp16 ``x * sigmoid(x)`` of the reference's res blocks
    (src/hi3d_mac/mlx_backend/transformer.py:172-173): the sigmoid rounded to fp16, then
    the product rounded to fp16."""
    hf = np.asarray(h).astype(np.float16).astype(np.float32)
    sig = (np.float32(1.0) / (np.float32(1.0) + np.exp(-hf))).astype(np.float16)
    return (hf * sig.astype(np.float32)).astype(np.float16)


def res_block3d_f64(x, table, embedding, p: dict, spans=None, eps: float = 1e-6) -> np.ndarray:
    """``SparseResBlock3d.forward`` after its resampling, in float64
    (src/sparc3d/models/transformers/sparc3d_transformer.py:132-144;
    src/hi3d_mac/mlx_backend/transformer.py:413-437) over the rows' ``[N, 27]`` table:
    ``scale, shift = Linear(SiLU(emb))`` per batch element, ``h = silu(LN(x) w1 + b1)``,
    ``h = conv1(h)``, ``h = silu(LN(h) (1 + scale) + shift)``, ``h = silu(conv2(h))``,
    ``linear(h) + skip(x)``. ``p`` holds the module's state-dict names
    (``conv*.conv.weight`` in spconv's ``[Cout, 3, 3, 3, Cin]``); ``spans`` are the batch
    elements' row ranges (one element when None)."""
    f = lambda k: np.asarray(p[k], np.float64)
    x64 = np.asarray(x, np.float64)
    emb = np.asarray(embedding, np.float64).reshape(-1, f("emb_layers.1.weight").shape[1])
    spans = spans or [slice(0, x64.shape[0])]
    silu = lambda v: v / (1.0 + np.exp(-v))

    def ln(v):
        mean = v.mean(axis=1, keepdims=True)
        var = ((v - mean) ** 2).mean(axis=1, keepdims=True)
        return (v - mean) / np.sqrt(var + eps)

    def taps(name):
        w = f(name)
        return w.reshape(w.shape[0], -1, w.shape[-1])

    h = silu(ln(x64) * f("norm1.weight") + f("norm1.bias"))
    h = gather_conv_f64(h, table, taps("conv1.conv.weight"), f("conv1.conv.bias"))
    hidden = h.shape[1]
    h2 = np.empty_like(h)
    for b, span in enumerate(spans):
        y = f("emb_layers.1.weight") @ silu(emb[b]) + f("emb_layers.1.bias")
        scale, shift = y[:hidden], y[hidden:]
        h2[span] = ln(h[span]) * (1.0 + scale) + shift
    h = gather_conv_f64(silu(h2), table, taps("conv2.conv.weight"), f("conv2.conv.bias"), act="silu")
    skip = x64 @ f("skip_connection.weight").T + f("skip_connection.bias") if "skip_connection.weight" in p else x64
    return h @ f("linear.weight").T + f("linear.bias") + skip
