"""``sparc3d.nn.sparse`` on the gfx950 kernels: ``SparseTensor``, ``SparseConv3d``,
``SparseDownsample`` and ``SparseUpsample``.

The public surface follows src/sparc3d/nn/sparse/basic.py:16-185 (constructor keywords,
properties, ``replace`` / ``reshape`` / ``type``, the per-scale spatial cache, ``+`` and
``*`` with per-batch broadcasting, the ValueError texts), conv.py:46-88 and
spatial.py:16-125 (factor parsing, paired resampling caches and their errors).

The container itself is this build's: a :class:`SparseTensor` is a feature matrix over
a shared :class:`_Rows` record (the int32 coordinates on the device, the batch spans
found with one device pass and one host read, and the spconv-layer tensor that owns the
kernel maps). ``replace`` keeps the record, so every tensor derived from one set of
coordinates reuses the same maps and tile plans. The downsample's coarse set, inverse
map and mean (which, like ``scatter_reduce(reduce="mean")`` onto zeros, divides by
``count + 1``) run on the GPU.
"""

from __future__ import annotations

from collections.abc import Sequence
from typing import Any

import torch
from torch import nn

from . import _lib
from . import kmap as _kmap
from . import sparse_backend


def _batch_layout(coords: torch.Tensor, batch_size: int) -> list[slice]:
    """Row span of each batch element when rows are grouped by ascending batch."""
    counts = torch.bincount(coords[:, 0].long(), minlength=batch_size)
    ends = counts.cumsum(0).tolist()
    starts = [0] + ends[:-1]
    return [slice(a, b) for a, b in zip(starts, ends)]


def _layout_holds(coords: torch.Tensor, layout: list[slice]) -> bool:
    """Whether every row inside span b carries batch index b (one device comparison)."""
    expected = torch.full((coords.shape[0],), -1, dtype=torch.int32, device=coords.device)
    for batch, span in enumerate(layout):
        expected[span] = batch
    covered = expected >= 0
    return bool(((expected == coords[:, 0]) | ~covered).all())


class _Rows:
    """What every tensor over one coordinate set shares: the coordinates, their batch
    layout and the spconv-layer tensor that caches kernel maps (built on first use)."""

    __slots__ = ("coords", "layout", "batch_size", "backend")

    def __init__(self, coords: torch.Tensor, layout: list[slice] | None, backend: Any | None):
        self.coords = coords
        self.batch_size = int(coords[:, 0].max()) + 1
        self.layout = list(layout) if layout else _batch_layout(coords, self.batch_size)
        if not _layout_holds(coords, self.layout):
            raise ValueError("coordinates for each batch must be contiguous")
        self.backend = backend


class SparseTensor:
    """Features ``[N, ...]`` over batch-first ``[N, 4]`` coordinates ``(batch, x, y, z)``
    whose batches occupy contiguous row ranges, with a spatial cache shared across the
    scales of one pyramid (the paired resampling modules keep their maps there)."""

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
        _rows: _Rows | None = None,
    ):
        if data is not None:
            if feats is not None or coords is not None:
                raise ValueError("provide either data or feats and coords")
            feats, coords = sparse_backend.get_feats(data), data.indices
        if feats is None or coords is None:
            raise ValueError("feats and coords are required")
        if coords.ndim != 2 or coords.shape[1] != 4:
            raise ValueError(f"expected coords [N, 4], got {tuple(coords.shape)}")
        if feats.shape[0] != coords.shape[0]:
            raise ValueError("features and coordinates must have the same row count")
        if coords.shape[0] == 0:
            raise ValueError("a SparseTensor cannot be empty")
        if _rows is None or _rows.coords.data_ptr() != coords.data_ptr():
            _rows = _Rows(coords.to(torch.int32).contiguous(), layout, None)
        self._rows = _rows
        self._feats = feats
        self.data = data
        self._shape = torch.Size(shape) if shape else torch.Size((_rows.batch_size, *feats.shape[1:]))
        self._scale = tuple(scale)
        self._spatial_cache = {} if spatial_cache is None else spatial_cache

    # -- the reference's read-only view ------------------------------------------------
    @property
    def feats(self) -> torch.Tensor:
        """Feature rows in coordinate order."""
        return self._feats

    @property
    def coords(self) -> torch.Tensor:
        """``[N, 4]`` int32 ``(batch, x, y, z)``."""
        return self._rows.coords

    @property
    def layout(self) -> list[slice]:
        """Row range of each batch element."""
        return self._rows.layout

    @property
    def shape(self) -> torch.Size:
        """``[batch, *feature shape]``."""
        return self._shape

    @property
    def scale(self) -> tuple[int, ...]:
        """Downsampling factor of this level relative to the finest grid."""
        return self._scale

    @property
    def dtype(self) -> torch.dtype:
        return self._feats.dtype

    @property
    def device(self) -> torch.device:
        return self._feats.device

    def backend_data(self) -> Any:
        """The spconv-layer tensor of these rows (built once per coordinate set; its
        ``indice_dict`` holds the kernel maps every convolution over the set reuses)."""
        if self.data is None:
            rows = self._rows
            if rows.backend is None:
                rows.backend = sparse_backend.sparse_tensor(self._feats, rows.coords)
                self.data = rows.backend
            else:
                self.data = sparse_backend.replace_feats(rows.backend, self._feats)
        return self.data

    # -- derived tensors ---------------------------------------------------------------
    def replace(self, feats: torch.Tensor) -> "SparseTensor":
        """New features over the same rows, layout, scale, spatial cache and kernel maps."""
        if feats.shape[0] != self._feats.shape[0]:
            raise ValueError("replacement features must preserve the sparse row count")
        data = sparse_backend.replace_feats(self.data, feats) if self.data is not None and feats.ndim == 2 else None
        return SparseTensor(
            feats if data is None else None,
            self.coords if data is None else None,
            torch.Size((self._shape[0], *feats.shape[1:])),
            data=data,
            scale=self._scale,
            spatial_cache=self._spatial_cache,
            _rows=self._rows,
        )

    def reshape(self, *shape: int) -> "SparseTensor":
        """Reshape each row's features; the rows stay."""
        return self.replace(self._feats.reshape(self._feats.shape[0], *shape))

    def type(self, dtype: torch.dtype) -> "SparseTensor":
        """Cast the features to ``dtype``."""
        return self.replace(self._feats.to(dtype=dtype))

    # -- spatial cache (keyed by scale) -------------------------------------------------
    def register_spatial_cache(self, key: str, value: Any) -> None:
        """Keep ``value`` under ``key`` at this tensor's scale."""
        self._spatial_cache.setdefault(str(self._scale), {})[key] = value

    def get_spatial_cache(self, key: str) -> Any | None:
        """The value kept under ``key`` at this tensor's scale, or None."""
        return self._spatial_cache.get(str(self._scale), {}).get(key)

    # -- arithmetic --------------------------------------------------------------------
    def _operand(self, other: Any) -> Any:
        if isinstance(other, SparseTensor):
            if other._rows is not self._rows and not torch.equal(self.coords, other.coords):
                raise ValueError("sparse operands must have identical coordinates")
            return other.feats
        if isinstance(other, torch.Tensor) and other.ndim >= 1:
            per_batch = other.shape[0] == self._shape[0] and other.shape != self._feats.shape
            if per_batch:
                return sparse_batch_broadcast(self, other)
        return other

    def __add__(self, other: Any) -> "SparseTensor":
        return self.replace(torch.add(self._feats, self._operand(other)))

    def __mul__(self, other: Any) -> "SparseTensor":
        return self.replace(torch.mul(self._feats, self._operand(other)))


def sparse_batch_broadcast(input: SparseTensor, other: torch.Tensor) -> torch.Tensor:
    """``other[b]`` on every row of batch element b, in the features' dtype: one gather
    by each row's batch index, then ``other[b]`` broadcast against the row's feature
    shape (trailing dimensions aligned, as an assignment would)."""
    feats = input.feats
    picked = other.to(feats.device).index_select(0, input.coords[:, 0].long())
    inner = other.ndim - 1
    if inner > feats.ndim - 1:
        raise ValueError(f"cannot broadcast {tuple(other.shape)} over feature rows {tuple(feats.shape)}")
    picked = picked.reshape(feats.shape[0], *([1] * (feats.ndim - 1 - inner)), *other.shape[1:])
    return torch.broadcast_to(picked, feats.shape).to(feats.dtype).contiguous()


class SparseConv3d(nn.Module):
    """Submanifold convolution of a :class:`SparseTensor` (output rows = input rows),
    through ``sparse_backend.Conv3d``, so the dtype policy and kernel-map cache apply."""

    _sparc3d_convertible = True

    def __init__(self, in_channels: int, out_channels: int, kernel_size: int, bias: bool = True):
        super().__init__()
        self.conv = sparse_backend.Conv3d(in_channels, out_channels, kernel_size=kernel_size, bias=bias)
        self.out_channels = out_channels

    def forward(self, x: SparseTensor) -> SparseTensor:
        result = self.conv(x.backend_data())
        return SparseTensor(
            data=result,
            shape=torch.Size((x.shape[0], self.out_channels)),
            scale=x.scale,
            spatial_cache=x._spatial_cache,
            _rows=x._rows,
        )


def _factor_tuple(factor: int | Sequence[int], dimensions: int) -> tuple[int, ...]:
    """One positive resampling factor per spatial axis."""
    per_axis = (factor,) * dimensions if not isinstance(factor, Sequence) else tuple(factor)
    if len(per_axis) != dimensions or min(per_axis, default=0) <= 0:
        raise ValueError("factor must provide one positive value per spatial dimension")
    return per_axis


def _cache_keys(factor: tuple[int, ...]) -> tuple[str, str, str]:
    return f"upsample_{factor}_coords", f"upsample_{factor}_layout", f"upsample_{factor}_idx"


class SparseDownsample(nn.Module):
    """Mean of the rows that share a coarse cell (any positive factor per axis, product at
    most 256); the fine rows' coordinates, layout and parents are kept for the paired
    upsample."""

    def __init__(self, factor: int | Sequence[int]):
        super().__init__()
        self.factor = tuple(factor) if isinstance(factor, Sequence) else factor

    def forward(self, input: SparseTensor) -> SparseTensor:
        factor = _factor_tuple(self.factor, input.coords.shape[-1] - 1)
        fine = input.coords
        extent = [hi + 1 for hi in _kmap.column_bounds(fine)[1][1:]]
        structure = _kmap.resample_structure(fine, extent, factor)
        feats = input.feats.contiguous()
        device = _lib.require_gpu(feats)
        n_coarse, slots = int(structure.down.shape[0]), int(structure.down.shape[1])
        pooled = torch.empty((n_coarse, feats.shape[1]), dtype=feats.dtype, device=device)
        _lib.call(
            "hi3d_gather_mean",
            _lib.ptr(feats), int(fine.shape[0]), int(feats.shape[1]), _lib.ptr(structure.down), slots, n_coarse, 1,
            _lib.DTYPES[feats.dtype], _lib.ptr(pooled), _lib.stream(device),
        )
        coarse = SparseTensor(
            pooled,
            structure.low,
            shape=input.shape,
            scale=tuple(s * f for s, f in zip(input.scale, factor)),
            spatial_cache=input._spatial_cache,
        )
        for key, value in zip(_cache_keys(factor), (fine, input.layout, structure.inverse.long())):
            coarse.register_spatial_cache(key, value)
        return coarse


class SparseUpsample(nn.Module):
    """Copy each coarse row back to the fine rows of its paired downsample."""

    def __init__(self, factor: int | Sequence[int]):
        super().__init__()
        self.factor = tuple(factor) if isinstance(factor, Sequence) else factor

    def forward(self, input: SparseTensor) -> SparseTensor:
        factor = _factor_tuple(self.factor, input.coords.shape[-1] - 1)
        if any(s % f for s, f in zip(input.scale, factor)):
            raise ValueError(
                f"cannot upsample by {factor} from scale {input.scale}; "
                "SparseUpsample must mirror its paired SparseDownsample"
            )
        coords, layout, parent = (input.get_spatial_cache(key) for key in _cache_keys(factor))
        if coords is None or layout is None or parent is None:
            raise ValueError("upsample cache not found; SparseUpsample must follow its paired SparseDownsample")
        return SparseTensor(
            input.feats[parent],
            coords,
            shape=input.shape,
            layout=layout,
            scale=tuple(s // f for s, f in zip(input.scale, factor)),
            spatial_cache=input._spatial_cache,
        )
