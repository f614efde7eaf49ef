"""Device radix sort and scan (``hi3d_sort_pairs``, ``hi3d_scan``): the sort and prefix
sum behind the kernel-map, plan, stride-2 and unique builds, for callers that need them
directly. GPU tensors only."""

from __future__ import annotations

import ctypes

import torch

from . import _lib

_KEY_BYTES = {torch.int32: 4, torch.int64: 8}


def sort_pairs(keys: torch.Tensor, values: torch.Tensor, begin_bit: int = 0, end_bit: int | None = None):
    """Stable sort of ``(keys, values)`` by key bits ``[begin_bit, end_bit)`` (keys read
    as unsigned). Returns new ``(keys, values)`` tensors; the inputs are unchanged."""
    device = _lib.require_gpu(keys, values)
    if keys.dtype not in _KEY_BYTES or values.dtype != torch.int32:
        raise ValueError("keys must be int32 or int64 and values int32")
    if keys.ndim != 1 or values.shape != keys.shape:
        raise ValueError("keys and values must be 1-D of one length")
    kb = _KEY_BYTES[keys.dtype]
    end = 8 * kb if end_bit is None else int(end_bit)
    n = int(keys.shape[0])
    k0, v0 = keys.contiguous().clone(), values.contiguous().clone()
    k1, v1 = torch.empty_like(k0), torch.empty_like(v0)
    ws = _lib.workspace(_lib.query("hi3d_sort_pairs_workspace", n), device)
    in_alt = ctypes.c_int32(0)
    _lib.call(
        "hi3d_sort_pairs",
        _lib.ptr(k0), _lib.ptr(k1), _lib.ptr(v0), _lib.ptr(v1), n, kb, int(begin_bit), end, _lib.ptr(ws), ws.numel(),
        ctypes.byref(in_alt), _lib.stream(device),
    )
    return (k1, v1) if in_alt.value else (k0, v0)


def scan(x: torch.Tensor, inclusive: bool = False) -> torch.Tensor:
    """Exclusive (or inclusive) prefix sum of a 1-D int32 tensor, as int32."""
    device = _lib.require_gpu(x)
    if x.dtype != torch.int32 or x.ndim != 1:
        raise ValueError("scan takes a 1-D int32 tensor")
    x = x.contiguous()
    n = int(x.shape[0])
    out = torch.empty_like(x)
    ws = _lib.workspace(_lib.query("hi3d_sort_pairs_workspace", n), device)
    _lib.call("hi3d_scan", _lib.ptr(x), _lib.ptr(out), n, int(inclusive), _lib.ptr(ws), ws.numel(), _lib.stream(device))
    return out
