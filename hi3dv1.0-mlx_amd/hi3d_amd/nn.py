"""``sparc3d.nn.sparse`` wrappers on the gfx950 kernels: ``SparseTensor``,
``SparseConv3d``, ``SparseDownsample`` and ``SparseUpsample``.

Same interface as src/sparc3d/nn/sparse/basic.py:16-177 (batch-first ``[N, 4]`` int32
coordinates, contiguous batches, per-scale spatial cache), src/sparc3d/nn/sparse/conv.py:
46-88 (coordinate-preserving convolution routed through ``sparse_backend``) and
src/sparc3d/nn/sparse/spatial.py:23-125 (paired mean downsample / cached upsample).
The downsample's coarse set, inverse map and the mean (which, like
``scatter_reduce(reduce="mean")`` onto zeros, divides by ``count + 1``) run on the GPU.
"""

from __future__ import annotations

from collections.abc import Callable, Sequence
from typing import Any

import torch
from torch import nn

from . import _lib
from . import kmap as _kmap
from . import sparse_backend


class SparseTensor:
    """Sparse features with batch-first coordinates and shared spatial caches."""

    def __init__(
        self,
        feats: torch.Tensor | None = None,
        coords: torch.Tensor | None = None,
        shape: torch.Size | None = None,
        layout: list[slice] | None = None,
        *,
        data: Any | None = None,
        scale: tuple[int, ...] = (1, 1, 1),
        spatial_cache: dict[str, dict[str, Any]] | None = None,
    ):
        if data is not None:
            if feats is not None or coords is not None:
                raise ValueError("provide either data or feats and coords")
            feats = sparse_backend.get_feats(data)
            coords = data.indices
        if feats is None or coords is None:
            raise ValueError("feats and coords are required")
        if coords.ndim != 2 or coords.shape[1] != 4:
            raise ValueError(f"expected coords [N, 4], got {tuple(coords.shape)}")
        if feats.shape[0] != coords.shape[0]:
            raise ValueError("features and coordinates must have the same row count")
        if coords.shape[0] == 0:
            raise ValueError("a SparseTensor cannot be empty")
        self._feats = feats
        self._coords = coords.int().contiguous()
        self.data = data
        batch_size = int(self._coords[:, 0].max().item()) + 1
        self._shape = shape or torch.Size((batch_size, *feats.shape[1:]))
        self._layout = layout or self._calculate_layout(self._coords, batch_size)
        self._scale = tuple(scale)
        self._spatial_cache = spatial_cache if spatial_cache is not None else {}
        self._validate_layout()

    @staticmethod
    def _calculate_layout(coords: torch.Tensor, batch_size: int) -> list[slice]:
        counts = torch.bincount(coords[:, 0].long(), minlength=batch_size)
        offsets = torch.cumsum(counts, dim=0)
        return [slice(int(offsets[i] - counts[i]), int(offsets[i])) for i in range(batch_size)]

    def _validate_layout(self) -> None:
        for batch, span in enumerate(self._layout):
            if not torch.all(self._coords[span, 0] == batch):
                raise ValueError("coordinates for each batch must be contiguous")

    def backend_data(self) -> Any:
        """Return the sparse-backend tensor, creating it lazily."""
        if self.data is None:
            self.data = sparse_backend.sparse_tensor(self._feats, self._coords)
        return self.data

    @property
    def shape(self) -> torch.Size:
        return self._shape

    @property
    def layout(self) -> list[slice]:
        return self._layout

    @property
    def feats(self) -> torch.Tensor:
        return self._feats

    @property
    def coords(self) -> torch.Tensor:
        return self._coords

    @property
    def dtype(self) -> torch.dtype:
        return self.feats.dtype

    @property
    def device(self) -> torch.device:
        return self.feats.device

    @property
    def scale(self) -> tuple[int, ...]:
        return self._scale

    def replace(self, feats: torch.Tensor) -> "SparseTensor":
        """Return a tensor sharing coordinates and caches with new features."""
        if feats.shape[0] != self.feats.shape[0]:
            raise ValueError("replacement features must preserve the sparse row count")
        data = None
        if self.data is not None and feats.ndim == 2:
            data = sparse_backend.replace_feats(self.data, feats)
        return SparseTensor(
            feats=feats if data is None else None,
            coords=self.coords if data is None else None,
            data=data,
            shape=torch.Size((self.shape[0], *feats.shape[1:])),
            layout=self.layout,
            scale=self._scale,
            spatial_cache=self._spatial_cache,
        )

    def reshape(self, *shape: int) -> "SparseTensor":
        return self.replace(self.feats.reshape(self.feats.shape[0], *shape))

    def type(self, dtype: torch.dtype) -> "SparseTensor":
        return self.replace(self.feats.to(dtype=dtype))

    def register_spatial_cache(self, key: str, value: Any) -> None:
        self._spatial_cache.setdefault(str(self._scale), {})[key] = value

    def get_spatial_cache(self, key: str) -> Any | None:
        return self._spatial_cache.get(str(self._scale), {}).get(key)

    def _elementwise(self, other, operation: Callable[[torch.Tensor, Any], torch.Tensor]) -> "SparseTensor":
        if isinstance(other, SparseTensor):
            if not torch.equal(self.coords, other.coords):
                raise ValueError("sparse operands must have identical coordinates")
            other = other.feats
        elif isinstance(other, torch.Tensor) and other.ndim >= 1:
            if other.shape[0] == self.shape[0] and other.shape != self.feats.shape:
                other = sparse_batch_broadcast(self, other)
        return self.replace(operation(self.feats, other))

    def __add__(self, other):
        return self._elementwise(other, torch.add)

    def __mul__(self, other):
        return self._elementwise(other, torch.mul)


def sparse_batch_broadcast(input: SparseTensor, other: torch.Tensor) -> torch.Tensor:
    """Broadcast per-batch rows of ``other`` to the rows of each batch element."""
    out = torch.empty((input.feats.shape[0], *other.shape[1:]), dtype=other.dtype, device=other.device)
    for batch, span in enumerate(input.layout):
        out[span] = other[batch]
    return out


class SparseConv3d(nn.Module):
    """Coordinate-preserving three-dimensional sparse convolution."""

    _sparc3d_convertible = True

    def __init__(self, in_channels: int, out_channels: int, kernel_size: int, bias: bool = True):
        super().__init__()
        self.conv = sparse_backend.Conv3d(in_channels, out_channels, kernel_size=kernel_size, bias=bias)
        self.out_channels = out_channels

    def forward(self, x: SparseTensor) -> SparseTensor:
        output = self.conv(x.backend_data())
        return SparseTensor(
            data=output,
            shape=x.shape[:1] + (self.out_channels,),
            layout=x.layout,
            scale=x.scale,
            spatial_cache=x._spatial_cache,
        )


def _factor_tuple(factor: int | Sequence[int], dimensions: int) -> tuple[int, ...]:
    values = tuple(factor) if isinstance(factor, Sequence) else (factor,) * dimensions
    if len(values) != dimensions or any(value <= 0 for value in values):
        raise ValueError("factor must provide one positive value per spatial dimension")
    return values


class SparseDownsample(nn.Module):
    """Average features that collapse onto the same downsampled coordinate (factor 2)."""

    def __init__(self, factor: int | Sequence[int]):
        super().__init__()
        self.factor = tuple(factor) if isinstance(factor, Sequence) else factor

    def forward(self, input: SparseTensor) -> SparseTensor:
        dimensions = input.coords.shape[-1] - 1
        factor = _factor_tuple(self.factor, dimensions)
        if factor != (2, 2, 2):
            raise NotImplementedError("the GPU downsample implements factor 2")
        coords = input.coords
        extent = [v + 1 for v in _kmap.column_bounds(coords.to(torch.int32))[1][1:]]
        s = _kmap.stride2_structure(coords, extent)
        feats = input.feats.contiguous()
        device = _lib.require_gpu(feats)
        out = torch.empty((s.n_coarse, feats.shape[1]), dtype=feats.dtype, device=device)
        _lib.call(
            "hi3d_gather_mean",
            _lib.ptr(feats), s.n_fine, int(feats.shape[1]), _lib.ptr(s.down), 8, s.n_coarse, 1,
            _lib.DTYPES[feats.dtype], _lib.ptr(out), _lib.stream(device),
        )
        output = SparseTensor(
            out,
            s.low,
            shape=input.shape,
            scale=tuple(scale * value for scale, value in zip(input.scale, factor)),
            spatial_cache=input._spatial_cache,
        )
        output.register_spatial_cache(f"upsample_{factor}_coords", input.coords)
        output.register_spatial_cache(f"upsample_{factor}_layout", input.layout)
        output.register_spatial_cache(f"upsample_{factor}_idx", s.inverse.long())
        return output


class SparseUpsample(nn.Module):
    """Restore coordinates from a paired downsample cache."""

    def __init__(self, factor: int | Sequence[int]):
        super().__init__()
        self.factor = tuple(factor) if isinstance(factor, Sequence) else factor

    def forward(self, input: SparseTensor) -> SparseTensor:
        dimensions = input.coords.shape[-1] - 1
        factor = _factor_tuple(self.factor, dimensions)
        if any(scale % value for scale, value in zip(input.scale, factor)):
            raise ValueError(
                f"cannot upsample by {factor} from scale {input.scale}; "
                "SparseUpsample must mirror its paired SparseDownsample"
            )
        coords = input.get_spatial_cache(f"upsample_{factor}_coords")
        layout = input.get_spatial_cache(f"upsample_{factor}_layout")
        inverse = input.get_spatial_cache(f"upsample_{factor}_idx")
        if coords is None or layout is None or inverse is None:
            raise ValueError("upsample cache not found; SparseUpsample must follow its paired SparseDownsample")
        return SparseTensor(
            input.feats[inverse],
            coords,
            shape=input.shape,
            layout=layout,
            scale=tuple(scale // value for scale, value in zip(input.scale, factor)),
            spatial_cache=input._spatial_cache,
        )
