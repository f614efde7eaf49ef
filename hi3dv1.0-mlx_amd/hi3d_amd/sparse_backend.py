"""``sparc3d.ops.sparse_backend`` on the gfx950 kernels: same functions, signatures,
dtype policy and errors as src/sparc3d/ops/sparse_backend.py:154-280.

``Conv3d`` builds a submanifold convolution that ignores autocast, runs the GEMM in the
weight's dtype (features are cast to it) and returns the features' dtype
(src/sparc3d/ops/sparse_backend.py:130-148). The reference switches to a chunked path
when the input matrix reaches 2^31 - 1 bytes (:14-15,132-145); the HIP kernels address
features with 64-bit offsets, so one path serves every size.
"""

from __future__ import annotations

from typing import Any, Optional, Tuple

import torch
from torch import nn

from . import kmap as _kmap
from . import spconv

_SPARSE_CONV_FLAG = "_sparc3d_sparse_conv"
"""Instance attribute marking a module that consumes and returns a sparse tensor."""


class SubMConv3d(spconv.SubMConv3d):
    """Submanifold convolution that ignores autocast and preserves the feature dtype."""

    def forward(self, input: Any) -> Any:
        feats_dtype = input.features.dtype
        with torch.autocast("cuda", enabled=False):
            if feats_dtype != self.weight.dtype:
                input = input.replace_feature(input.features.to(self.weight.dtype))
            out = super().forward(input)
            if out.features.dtype != feats_dtype:
                out = out.replace_feature(out.features.to(feats_dtype))
        return out


def Conv3d(
    in_channels: int,
    out_channels: int,
    kernel_size: int = 3,
    stride: int = 1,
    padding: Optional[int] = None,
    bias: bool = True,
) -> nn.Module:
    """Build a submanifold sparse convolution (keeps the input's coordinates and row
    order). Raises ``ValueError`` for an even ``kernel_size``, ``stride != 1`` or a
    non-submanifold ``padding``."""
    if kernel_size % 2 == 0:
        raise ValueError(f"kernel_size must be odd, got {kernel_size}")
    if stride != 1:
        raise ValueError(f"only stride 1 is supported, got {stride}")
    if padding is not None and padding != kernel_size // 2:
        raise ValueError(f"only submanifold padding {kernel_size // 2} is supported, got {padding}")
    conv = SubMConv3d(in_channels, out_channels, kernel_size=kernel_size, bias=bias, indice_key=f"subm{kernel_size}")
    setattr(conv, _SPARSE_CONV_FLAG, True)
    return conv


def is_sparse_conv(module: nn.Module) -> bool:
    """Return whether ``module`` was built by :func:`Conv3d`."""
    return getattr(module, _SPARSE_CONV_FLAG, False)


def sparse_tensor(
    feats: torch.Tensor,
    coords: torch.Tensor,
    spatial_shape: Optional[Tuple[int, int, int]] = None,
) -> Any:
    """Wrap features and ``[N, 4]`` ``(batch, x, y, z)`` coordinates in a sparse tensor.

    Raises ``ValueError`` when ``coords`` is not ``[N, 4]``, holds negative entries or
    exceeds ``spatial_shape``."""
    if coords.ndim != 2 or coords.shape[1] != 4:
        raise ValueError(f"expected coords [N, 4], got {tuple(coords.shape)}")
    coords = coords.int().contiguous()
    if coords.shape[0] == 0:
        lo, hi = [0] * 4, [0] * 4
    elif coords.is_cuda:
        lo, hi = _kmap.column_bounds(coords)
    else:  # a host-side container (validation only; the convolutions need the GPU)
        lo, hi = coords.min(dim=0).values.tolist(), coords.max(dim=0).values.tolist()
    if min(lo[1:]) < 0:
        raise ValueError("grid coordinates must be non-negative")
    extent = [v + 1 for v in hi[1:]]
    if spatial_shape is None:
        spatial_shape = tuple(extent)
    elif any(bound < size for bound, size in zip(spatial_shape, extent)):
        raise ValueError(f"grid coordinates reach {extent}, outside spatial_shape {spatial_shape}")
    return spconv.SparseConvTensor(
        features=feats,
        indices=coords,
        spatial_shape=list(spatial_shape),
        batch_size=hi[0] + 1,
    )


def get_feats(tensor: Any) -> torch.Tensor:
    """Return the feature matrix of a sparse tensor."""
    return tensor.features


def replace_feats(tensor: Any, feats: torch.Tensor) -> Any:
    """Return a sparse tensor with the same coordinates and new features; raises
    ``ValueError`` when the row count differs."""
    current = get_feats(tensor)
    if feats.shape[0] != current.shape[0]:
        raise ValueError(f"expected {current.shape[0]} rows to match the coordinates, got {feats.shape[0]}")
    return tensor.replace_feature(feats)
