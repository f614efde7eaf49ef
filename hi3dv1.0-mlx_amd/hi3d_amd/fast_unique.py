"""``torch.unique(x, dim=0, ...)`` on integer rows and ``np.unique`` on int64 keys, on the
GPU through the HIP library.

Same names and results as src/hi3d_mac/fast_unique.py: ``unique_keys`` :25-56 (sorted
unique values, inverse, counts), ``_packed_keys`` :59-71 (one int64 key per row in the
rows' lexicographic order, ``None`` when the extents multiply past 2^62) and
``unique_rows`` :74-91 (the ``torch.unique(dim=0)`` drop-in). The reference sorts with
MLX and finishes on the host; here the sort, the run marks, the inverse scatter and the
row packing all run on the device and the results stay there.
"""

from __future__ import annotations

import math

import torch

from . import _lib

_INT_DTYPES = (torch.int16, torch.int32, torch.int64, torch.uint8)


def unique_keys(keys: torch.Tensor, return_counts: bool = False, key_bits: int = 0):
    """``(values, inverse, counts)`` of a 1-D int64 tensor, equal to
    ``np.unique(keys, return_inverse=True, return_counts=return_counts)`` (``counts`` is
    ``None`` without ``return_counts``). ``key_bits`` > 0 promises keys in
    ``[0, 2**key_bits)`` and sorts only those bits."""
    device = _lib.require_gpu(keys)
    if keys.dim() != 1:
        raise ValueError("keys must be 1-D")
    k = keys.to(torch.int64).contiguous()
    n = int(k.shape[0])
    uniq = torch.empty(n, dtype=torch.int64, device=device)
    inverse = torch.empty(n, dtype=torch.int64, device=device)
    counts = torch.empty(n, dtype=torch.int64, device=device) if return_counts else None
    n_unique = torch.empty(1, dtype=torch.int64, device=device)
    ws = _lib.workspace(_lib.query("hi3d_unique_keys_workspace", n), device)
    _lib.call("hi3d_unique_keys", _lib.ptr(k), n, int(key_bits), _lib.ptr(ws), ws.numel(), _lib.ptr(uniq),
              _lib.ptr(inverse), _lib.ptr(counts), _lib.ptr(n_unique), _lib.stream(device))
    u = int(n_unique.item())
    return uniq[:u], inverse, (counts[:u] if counts is not None else None)


def _packed_keys(a: torch.Tensor):
    """``(keys, lo, extent, bits)``: one int64 key per row of ``a [n, d]`` preserving the
    rows' lexicographic order, or ``None`` if the extents multiply to 2^62 or more."""
    d = int(a.shape[1])
    dtype = _lib.I64 if a.dtype == torch.int64 else _lib.I32
    lo = torch.empty(d, dtype=torch.int64, device=a.device)
    hi = torch.empty(d, dtype=torch.int64, device=a.device)
    _lib.call("hi3d_row_bounds", _lib.ptr(a), dtype, int(a.shape[0]), d, _lib.ptr(lo), _lib.ptr(hi),
              _lib.stream(a.device))
    extent = hi - lo + 1
    ext = [int(v) for v in extent.tolist()]
    span = math.prod(ext)
    if span >= 2**62:
        return None
    keys = torch.empty(a.shape[0], dtype=torch.int64, device=a.device)
    _lib.call("hi3d_pack_rows", _lib.ptr(a), dtype, int(a.shape[0]), int(a.shape[1]), _lib.ptr(lo),
              _lib.ptr(extent), _lib.ptr(keys), _lib.stream(a.device))
    return keys, lo, extent, max(1, (span - 1).bit_length())


def unique_rows(x: torch.Tensor, return_inverse: bool = False, return_counts: bool = False):
    """``torch.unique(x, dim=0, return_inverse=..., return_counts=...)`` for integer rows:
    sorted unique rows in ``x``'s dtype, int64 inverse and counts. Rows whose value
    ranges multiply past 2^62 go to ``torch.unique`` itself, as in the reference; so do
    empty inputs and rows of more than 8 columns (the packing kernels take up to 8)."""
    device = _lib.require_gpu(x)
    if x.dim() != 2 or x.dtype not in _INT_DTYPES:
        raise ValueError("x must be a 2-D integer tensor")
    n, d = int(x.shape[0]), int(x.shape[1])
    if n == 0 or d > 8:
        return torch.unique(x, dim=0, return_inverse=return_inverse, return_counts=return_counts)
    a = x.contiguous() if x.dtype in (torch.int32, torch.int64) else x.to(torch.int32).contiguous()
    packed = _packed_keys(a)
    if packed is None:
        return torch.unique(x, dim=0, return_inverse=return_inverse, return_counts=return_counts)
    keys, lo, extent, bits = packed
    uniq, inverse, counts = unique_keys(keys, return_counts=return_counts, key_bits=bits)
    u = int(uniq.shape[0])
    rows = torch.empty((u, d), dtype=a.dtype, device=device)
    n_dev = torch.full((1,), u, dtype=torch.int64, device=device)
    _lib.call("hi3d_unpack_rows", _lib.ptr(uniq), u, _lib.ptr(n_dev), d, _lib.ptr(lo), _lib.ptr(extent),
              _lib.ptr(rows), _lib.I64 if a.dtype == torch.int64 else _lib.I32, _lib.stream(device))
    out = [rows.to(x.dtype)]
    if return_inverse:
        out.append(inverse)
    if return_counts:
        out.append(counts)
    return out[0] if len(out) == 1 else tuple(out)


def unique(input, sorted=True, return_inverse=False, return_counts=False, dim=None):
    """``torch.unique`` with ``dim=0`` on 2-D integer GPU rows taken by
    :func:`unique_rows`; everything else goes to ``torch.unique`` (the reference's
    ``_unique`` dispatch, fast_unique.py:97-107)."""
    if (
        dim == 0
        and isinstance(input, torch.Tensor)
        and input.device.type == "cuda"
        and input.dtype in _INT_DTYPES
        and input.ndim == 2
        and sorted
    ):
        return unique_rows(input, return_inverse, return_counts)
    return torch.unique(input, sorted=sorted, return_inverse=return_inverse, return_counts=return_counts, dim=dim)
