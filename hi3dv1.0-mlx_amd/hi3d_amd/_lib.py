"""ctypes binding of ``libhi3d_amd.so`` (the gfx950 HIP library, C ABI in
``include/hi3d_amd.h``).

Loading is lazy and fails loudly: there is no CPU fallback for any operation. Every
entry point takes raw device pointers and the current HIP stream of the tensors'
device, so launches are ordered with PyTorch's own work on that stream.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(os.environ.get("HI3D_AMD_LIB", Path(__file__).with_name("libhi3d_amd.so")))

OK, ERR_INVALID, ERR_HIP, ERR_UNSUPPORTED = 0, 1, 2, 3
MAP_DUPLICATE, MAP_OVERFLOW, MAP_RANGE = 1, 2, 4
F32, F16, BF16, F64, I32, I64 = 0, 1, 2, 3, 4, 5
ACT_NONE, ACT_SILU = 0, 1

DTYPES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.float64: F64}

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

# name -> argtypes (every entry point returns int status unless listed in _RESTYPES)
_SIGNATURES = {
    "hi3d_last_error": [],
    "hi3d_version": [],
    "hi3d_kmap_workspace": [_i64, _i64, _i32, _p],
    "hi3d_kmap_subm": [_p, _i64, _i32, _i32, _i32, _i32, _i32, _i64, _p, _i64, _p, _p, _p, _p],
    "hi3d_kmap_subm_noalloc": [_p, _i64, _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _p],
    "hi3d_kmap_pairs_workspace": [_i64, _i32, _p],
    "hi3d_kmap_pairs": [_p, _i64, _i32, _p, _i64, _p, _p, _p, _p],
    "hi3d_downsample_workspace": [_i64, _p],
    "hi3d_downsample_structure": [_p, _i64, _i32, _i32, _i32, _i32, _p, _i64, _p, _p, _p, _p, _p, _p, _p],
    "hi3d_stride2_tables": [_p, _p, _i64, _i64, _p, _p, _p],
    "hi3d_resample_structure": [_p, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p, _i64, _p, _p, _p, _p, _p, _p,
                                _p],
    "hi3d_resample_down_table": [_p, _p, _i64, _i64, _i32, _p, _p],
    "hi3d_child_table_workspace": [_i64, _p],
    "hi3d_child_neighbour_table": [_p, _p, _i64, _p, _i64, _p, _p, _p, _p, _p],
    "hi3d_conv_tile_rows": [],
    "hi3d_conv_plan_workspace": [_i64, _p],
    "hi3d_conv_plan": [_p, _i64, _i32, _i64, _p, _i32, _i32, _i64, _p, _i64, _p, _p, _p, _p],
    "hi3d_gather_conv": [_p, _i64, _i32, _p, _p, _i32, _i32, _p, _p, _p, _i64, _p, _i32, _i32, _p, _p],
    "hi3d_gather_conv_ln_silu": [_p, _i64, _i32, _p, _p, _i32, _i32, _p, _p, _p, _i64, _p, _i32, _p, _p, _f32, _p,
                                 _p],
    "hi3d_gather_conv_simple": [_p, _i64, _i32, _p, _p, _i32, _i32, _p, _i64, _p, _i32, _i32, _p, _p],
    "hi3d_kmap_dense_workspace": [_i32, _i32, _i32, _i32, _p],
    "hi3d_kmap_subm_dense": [_p, _i64, _i32, _i32, _i32, _i32, _i32, _p, _i64, _p, _p, _p, _p],
    "hi3d_kmap_dense_order_workspace": [_i64, _p],
    "hi3d_sort_pairs_workspace": [_i64, _p],
    "hi3d_sort_pairs": [_p, _p, _p, _p, _i64, _i32, _i32, _i32, _p, _i64, _p, _p],
    "hi3d_scan": [_p, _p, _i64, _i32, _p, _i64, _p],
    "hi3d_kmap_subm_dense_kept": [_p, _i64, _i32, _i32, _i32, _i32, _i32, _p, _i64, _p, _i64, _p, _p, _p, _p],
    "hi3d_parent_table": [_p, _i64, _i32, _p, _i64, _p, _p],
    "hi3d_gather_rows": [_p, _i64, _i32, _p, _i64, _p, _p],
    "hi3d_stride2_up_supported": [_i32, _i32, _i32],
    "hi3d_stride2_up_conv": [_p, _i64, _i32, _p, _p, _i32, _p, _i64, _i32, _p, _p],
    "hi3d_stride2_up_tile_rows": [],
    "hi3d_stride2_up_plan_workspace": [_i64, _p],
    "hi3d_stride2_up_plan": [_p, _i64, _i64, _i32, _p, _i64, _p, _p, _p],
    "hi3d_stride2_up_conv_sorted": [_p, _i64, _i32, _p, _p, _i32, _p, _p, _i64, _i32, _p, _p],
    "hi3d_unique_keys_workspace": [_i64, _p],
    "hi3d_unique_keys": [_p, _i64, _i32, _p, _i64, _p, _p, _p, _p, _p],
    "hi3d_pack_rows": [_p, _i32, _i64, _i32, _p, _p, _p, _p],
    "hi3d_row_bounds": [_p, _i32, _i64, _i32, _p, _p, _p],
    "hi3d_unpack_rows": [_p, _i64, _p, _i32, _p, _p, _p, _i32, _p],
    "hi3d_gather_conv_narrow": [_p, _i64, _i32, _p, _p, _i32, _i32, _p, _p, _p, _i64, _p, _i32, _i32, _p, _p],
    "hi3d_gather_mean": [_p, _i64, _i32, _p, _i32, _i64, _i32, _i32, _p, _p],
    "hi3d_halo_tile_rows": [],
    "hi3d_halo_capacity": [],
    "hi3d_halo_plan_workspace": [_i64, _p],
    "hi3d_halo_plan": [_p, _i64, _i32, _i64, _p, _i32, _i32, _p, _i64, _p, _p, _p, _p, _p, _p, _p],
    "hi3d_halo_conv": [_p, _i64, _i32, _p, _p, _i32, _p, _p, _p, _i64, _p, _i32, _i32, _p, _p],
    "hi3d_w8a8_quantize": [_p, _i64, _i32, _p, _p, _p, _p],
    "hi3d_w8a8_gemm": [_p, _p, _p, _p, _p, _i64, _i32, _i32, _p, _p, _p],
    "hi3d_layer_norm_modulate": [_p, _i64, _i32, _f32, _p, _p, _p, _p, _p, _p],
    "hi3d_layer_norm_act": [_p, _i64, _i32, _f32, _p, _p, _p, _p, _i32, _p, _p],
    "hi3d_layer_norm_quantize": [_p, _i64, _i32, _f32, _p, _p, _p, _p, _p, _p, _p, _p],
    "hi3d_dense_linear": [_p, _i64, _i32, _p, _p, _i32, _p, _p, _p],
    "hi3d_adaln_projection": [_p, _p, _p, _i32, _i32, _i32, _p, _p, _p],
    "hi3d_group_stats_workspace": [_i64, _i32, _p],
    "hi3d_group_stats": [_p, _i32, _i64, _i32, _i32, _f32, _p, _i64, _p, _p, _p],
    "hi3d_gn_swish": [_p, _i32, _i64, _i32, _p, _p, _p, _p, _p, _i32, _p],
    "hi3d_gather_gn_swish": [_p, _i32, _i64, _i32, _p, _i64, _p, _p, _p, _p, _p, _i32, _p],
}
_RESTYPES = {"hi3d_last_error": ctypes.c_char_p, "hi3d_version": ctypes.c_char_p, "hi3d_conv_tile_rows": _i32,
             "hi3d_stride2_up_tile_rows": _i32,
             "hi3d_halo_tile_rows": _i32, "hi3d_halo_capacity": _i32}

_LIB: ctypes.CDLL | None = None


class Hi3dError(RuntimeError):
    """A HIP runtime failure inside the library."""


def lib() -> ctypes.CDLL:
    """The loaded library; raises ``ImportError`` if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build the gfx950 HIP library first "
            "(python hi3dv1.0-mlx_amd/build.py, or __graft_entry__.build())"
        )
    handle = ctypes.CDLL(str(LIB_PATH))
    for name, args in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.argtypes = args
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
    _LIB = handle
    return handle


def exported_symbols() -> list[str]:
    """Names of every entry point the binding declares."""
    return list(_SIGNATURES)


def last_error() -> str:
    return lib().hi3d_last_error().decode()


def check(rc: int) -> None:
    """Map a status code onto the reference's exception types."""
    if rc == OK:
        return
    msg = last_error()
    if rc == ERR_INVALID:
        raise ValueError(msg)
    if rc == ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise Hi3dError(msg)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device) -> int:
    """Handle of the current HIP stream of ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors: torch.Tensor | None) -> torch.device:
    """Every tensor must live on one ROCm GPU; there is no host path."""
    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(
                f"hi3d_amd runs on a ROCm GPU only; got a tensor on {t.device} (move it with .cuda())"
            )
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError(f"tensors on different devices: {device} and {t.device}")
    if device is None:
        raise ValueError("no tensor given")
    lib()
    return device


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Caller-owned scratch for one call (the library never allocates)."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def query(name: str, *args) -> int:
    """Run a ``*_workspace`` size query and return the byte count."""
    out = ctypes.c_int64(0)
    check(getattr(lib(), name)(*args, ctypes.byref(out)))
    return int(out.value)
