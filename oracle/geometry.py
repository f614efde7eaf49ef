"""Refiner transformer geometry oracle (NumPy, float64): mean-pool down, parent-copy up
and the up block's first convolution in the reference's projection form. Test
infrastructure only.

Follows Geometry.downsample / upsample and Sparc3DTransformerMLX._up_conv
(src/hi3d_mac/mlx_backend/transformer.py:261-266,449-473).
"""

from __future__ import annotations

import numpy as np


def downsample_f64(x, inverse, n_low):
    """``scatter_add(x) / (children + 1)`` in float64 (transformer.py:261-263)."""
    x = np.asarray(x, np.float64)
    inverse = np.asarray(inverse, np.int64)
    sums = np.zeros((n_low, x.shape[1]))
    np.add.at(sums, inverse, x)
    counts = np.bincount(inverse, minlength=n_low)
    return sums / (counts + 1)[:, None]


def upsample(x, inverse):
    """Each fine voxel's parent row (transformer.py:265-266)."""
    return np.asarray(x)[np.asarray(inverse, np.int64)]


def up_conv_index(full_table, inverse, n_low):
    """``parent(o + d_k) * 27 + k``, ``n_low * 27`` where the neighbour is absent
    (transformer.py:253-259)."""
    t = np.asarray(full_table, np.int64)
    n = t.shape[0]
    parent_of = np.append(np.asarray(inverse, np.int64), n_low)
    nb_parent = parent_of[np.where((t >= 0) & (t < n), t, n)]
    flat = nb_parent * 27 + np.arange(27)[None, :]
    flat[nb_parent == n_low] = n_low * 27
    return flat


def up_conv_f64(h_low, full_table, inverse, weight, bias):
    """``_up_conv`` in float64 the reference's way: project every coarse row through all
    27 taps (``[N_low * 27, Cout]`` plus a zero row) and sum the gathered projections
    per fine voxel, then add the bias (transformer.py:449-473). ``weight [Cout, 27 * Cin]``."""
    h = np.asarray(h_low, np.float64)
    w = np.asarray(weight, np.float64)
    cout, cin = w.shape[0], h.shape[1]
    w_taps = w.reshape(cout, 27, cin).transpose(2, 1, 0).reshape(cin, 27 * cout)
    proj = (h @ w_taps).reshape(-1, cout)
    proj = np.concatenate([proj, np.zeros((1, cout))], 0)
    idx = up_conv_index(full_table, inverse, h.shape[0])
    y = proj[idx].sum(axis=1)
    return y if bias is None else y + np.asarray(bias, np.float64)


def sparse_downsample(indices, feats, factor):
    """``SparseDownsample(factor).forward`` in float64 (src/sparc3d/nn/sparse/spatial.py:
    34-79): the coordinates divided per axis, packed with offsets from the cumulative
    product of the divided extents (batch most significant), ``unique`` with inverse,
    the features' mean per coarse row onto zeros (``scatter_reduce(mean)`` with the zero
    included: the sum over count + 1), the coarse coordinates unpacked. Returns
    ``(coords [Nc, 4], feats [Nc, C], inverse [N])``."""
    c = np.asarray(indices, np.int64)
    cols = [c[:, 0]] + [c[:, a + 1] // int(f) for a, f in enumerate(factor)]
    extents = [int(col.max()) + 1 for col in cols[1:]]
    offsets = list(np.cumprod(extents[::-1])[::-1]) + [1]
    codes = sum(col * int(off) for col, off in zip(cols, offsets))
    unique, inverse = np.unique(codes, return_inverse=True)
    inverse = inverse.reshape(-1)
    low = np.stack([unique // offsets[0]] + [(unique // offsets[a + 1]) % extents[a] for a in range(3)], 1)
    return low.astype(np.int32), downsample_f64(feats, inverse, len(unique)), inverse
