"""Unique-values oracle (NumPy): the reference's sort + run-mark + scatter restated on
the host. Test infrastructure only.

Follows unique_keys / _packed_keys / unique_rows (src/hi3d_mac/fast_unique.py:25-91):
argsort the keys, mark where a sorted key differs from its predecessor, number the runs
by a running sum, scatter each run number back to the key's position, and read counts
off the run boundaries. Rows become one int64 key each by mixed-radix packing of their
offsets from the column minima, which keeps their lexicographic order.
"""

from __future__ import annotations

import numpy as np


def unique_keys(keys, return_counts: bool = False):
    """``(values, inverse, counts)`` of a 1-D int64 array (fast_unique.py:25-56)."""
    keys = np.asarray(keys, dtype=np.int64)
    n = keys.shape[0]
    if n == 0:
        empty = np.empty(0, dtype=np.int64)
        return empty, empty.copy(), (empty.copy() if return_counts else None)
    order = np.argsort(keys, kind="stable")
    sorted_keys = keys[order]
    starts = np.concatenate([[True], sorted_keys[1:] != sorted_keys[:-1]])
    run = np.cumsum(starts.astype(np.int64)) - 1
    inverse = np.empty(n, dtype=np.int64)
    inverse[order] = run
    values = sorted_keys[starts]
    counts = None
    if return_counts:
        bounds = np.flatnonzero(starts)
        counts = np.diff(np.append(bounds, n)).astype(np.int64)
    return values, inverse, counts


def packed_keys(a):
    """``(keys, lo, extent)`` or ``None`` past 2^62 (fast_unique.py:59-71)."""
    a = np.asarray(a, dtype=np.int64)
    lo = a.min(axis=0)
    extent = a.max(axis=0) - lo + 1
    if float(np.prod(extent.astype(np.float64))) >= 2**62:
        return None
    key = a[:, 0] - lo[0]
    for j in range(1, a.shape[1]):
        key = key * int(extent[j]) + (a[:, j] - lo[j])
    return key, lo, extent


def unique_rows(rows, return_inverse: bool = False, return_counts: bool = False):
    """Sorted unique rows, inverse and counts as ``torch.unique(dim=0)`` gives them
    (fast_unique.py:74-91); rows too wide to pack are not handled here."""
    a = np.asarray(rows, dtype=np.int64)
    packed = packed_keys(a)
    if packed is None:
        raise ValueError("rows too wide to pack")
    key, lo, extent = packed
    values, inverse, counts = unique_keys(key, return_counts=return_counts)
    out = np.empty((values.shape[0], a.shape[1]), dtype=np.int64)
    rem = values.copy()
    for j in range(a.shape[1] - 1, 0, -1):
        out[:, j] = rem % extent[j] + lo[j]
        rem //= extent[j]
    out[:, 0] = rem + lo[0]
    return out, inverse, counts
