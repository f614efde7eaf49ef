"""VAE decoder oracle (NumPy): GroupNorm statistics, GroupNorm + swish, the gathered
activation block, the residual block built from them, and one octree upsampling
(occupancy logits, child map, child projection, child coordinates). Test
infrastructure only.

Follows SparconvVAEDecoderMLX.group_stats / conv_gn_swish / resnet / children /
occupancy and the upsampling step of __call__ (src/hi3d_mac/mlx_backend/vae.py:141-244,
270-271,316-327) and gather_group_norm_swish (src/hi3d_mac/mlx_backend/kernels.py:240-296).
"""

from __future__ import annotations

import numpy as np

from .conv import gather_conv_f64
from .kmap import child_neighbour_table


def groups_for(c: int) -> int:
    """32 groups, or C / 4 below 128 channels (vae.py:152)."""
    return 32 if 4 * 32 <= c else c // 4


def group_stats_f64(x, eps: float = 1e-6):
    """Per-channel ``(mean, 1 / sqrt(var + eps))`` in float64 over ``groups_for(C)``
    groups of consecutive channels, with the reference's divisor ``n * width + eps``
    and ``var = E[x^2] - mean^2`` (vae.py:153-164)."""
    x = np.asarray(x, np.float64)
    n, c = x.shape
    g = groups_for(c)
    w = c // g
    xg = x.reshape(n, g, w)
    count = n * w + eps
    mean = xg.sum(axis=(0, 2)) / count
    var = (xg * xg).sum(axis=(0, 2)) / count - mean * mean
    inv = 1.0 / np.sqrt(var + eps)
    return np.repeat(mean, w), np.repeat(inv, w)


def swish_reference_form(u):
    """``u * sigmoid(u)`` with the reference's sigmoid ``e = 1 / (1 + exp(|u|))``,
    ``u < 0 ? e : 1 - e`` (kernels.py:254-255), in the dtype of ``u``."""
    u = np.asarray(u)
    e = 1 / (1 + np.exp(np.abs(u)))
    return u * np.where(u < 0, e, 1 - e)


def group_norm_swish(x, mean, inv, weight, bias, dtype=np.float64):
    """``swish(((x - mean) * inv) * weight + bias)`` evaluated in ``dtype``."""
    x = np.asarray(x).astype(dtype)
    mean, inv, weight, bias = (np.asarray(v, dtype).reshape(-1) for v in (mean, inv, weight, bias))
    u = ((x - mean) * inv) * weight + bias
    return swish_reference_form(u)


def gather_group_norm_swish(x, table, mean, inv, weight, bias, dtype=np.float64):
    """``[rows, kvol * C]`` block of activated rows ``table[o, k]`` (zeros where the table
    holds ``n``), as gather_group_norm_swish (kernels.py:261-296)."""
    a = group_norm_swish(x, mean, inv, weight, bias, dtype)
    n, c = a.shape
    padded = np.concatenate([a, np.zeros((1, c), a.dtype)])
    t = np.asarray(table)
    t = np.where((t >= 0) & (t < n), t, n)
    return padded[t].reshape(t.shape[0], -1)


def conv_gn_swish_f64(x, table, norm_weight, norm_bias, weight_t, bias, residual=None, eps: float = 1e-6):
    """``conv(swish(GN(x))) + bias (+ residual)`` in float64 with ``weight_t [27 Cin, Cout]``
    (vae.py:166-192)."""
    mean, inv = group_stats_f64(x, eps)
    a = group_norm_swish(x, mean, inv, norm_weight, norm_bias, np.float64)
    cin = a.shape[1]
    w = np.asarray(weight_t, np.float64).T.reshape(-1, 27, cin)
    return gather_conv_f64(a, table, w, bias, residual=residual)


def resnet_f64(x, table, p: dict, name: str, eps: float = 1e-6):
    """``shortcut + conv(swish(GN(conv(swish(GN(x))))))`` in float64 (vae.py:200-218)."""
    f = lambda k: np.asarray(p[k], np.float64)
    h = conv_gn_swish_f64(x, table, f(f"{name}.block.0.weights"), f(f"{name}.block.0.bias"),
                          f(f"{name}.block.2.weight"), f(f"{name}.block.2.bias"), eps=eps)
    x64 = np.asarray(x, np.float64)
    if f"{name}.res_conv.weight" in p:
        shortcut = x64 @ f(f"{name}.res_conv.weight").T + f(f"{name}.res_conv.bias")
    else:
        shortcut = x64
    return conv_gn_swish_f64(h, table, f(f"{name}.block.3.weights"), f(f"{name}.block.3.bias"),
                             f(f"{name}.block.5.weight"), f(f"{name}.block.5.bias"), residual=shortcut, eps=eps)


def children_f64(x, parent, slot, weight):
    """Kept children's features in float64 the reference's way (vae.py:220-244): project
    every parent to all eight children, ``(x @ weight.T).reshape(-1, C)`` with
    ``weight [8C, C]``, and take rows ``parent * 8 + slot``."""
    x = np.asarray(x, np.float64)
    c = x.shape[1]
    proj = (x @ np.asarray(weight, np.float64).T).reshape(-1, c)
    flat = np.asarray(parent, np.int64) * 8 + np.asarray(slot, np.int64)
    return proj[flat]


def child_coords(coords, parent, slot):
    """``coords[parent] * 2 + (s >> 2 & 1, s >> 1 & 1, s & 1)`` (vae.py:324-325)."""
    s = np.asarray(slot, np.int64)
    bits = np.stack([(s >> 2) & 1, (s >> 1) & 1, s & 1], 1)
    return (np.asarray(coords, np.int64)[np.asarray(parent, np.int64)] * 2 + bits).astype(np.int32)


def occupancy_f64(x, table, p: dict, name: str, eps: float = 1e-6):
    """``SparseClsHead`` logits ``[P, 8]`` in float64 (vae.py:270-271)."""
    f = lambda k: np.asarray(p[k], np.float64)
    return conv_gn_swish_f64(x, table, f(f"{name}.cls_head.fc.0.weights"), f(f"{name}.cls_head.fc.0.bias"),
                             f(f"{name}.cls_head.fc.2.weight"), f(f"{name}.cls_head.fc.2.bias"), eps=eps)


def upsample_f64(x, coords, table, p: dict, name: str, mask=None, eps: float = 1e-6):
    """One decoder upsampling (vae.py:316-327) in float64: ``mask = logits > 0`` unless
    given, then the child table, parent and slot, the children's features and
    coordinates. Returns ``(features, coords, table, parent, slot, mask)``."""
    if mask is None:
        mask = occupancy_f64(x, table, p, name, eps) > 0
    ctable, parent, slot = child_neighbour_table(np.asarray(table), np.asarray(mask, bool))
    feats = children_f64(x, parent, slot, p[f"{name}.proj.weight"])
    return feats, child_coords(coords, parent, slot), ctable, parent, slot, mask
