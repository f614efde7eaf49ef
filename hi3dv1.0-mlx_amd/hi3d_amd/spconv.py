"""The spconv 2.3.6 API subset the Hi3D refiner uses, on the gfx950 HIP kernels.

Same names, arguments, layouts and errors as the reference's pure-PyTorch stand-in
(src/hi3d_mac/torch_backend/sparse_conv.py): ``ConvAlgo`` :29-34, ``_PairTable`` :37-50,
``IndiceData`` :53-75, ``SparseConvTensor`` :78-106, ``subm_pairs`` :115-149,
``subm_conv`` :165-195, ``SubMConv3d`` :198-247, ``get_indice_pair_data`` :250-261,
``get_indice_pairs`` :264-283. :func:`install` registers the modules ``spconv``,
``spconv.pytorch``, ``spconv.pytorch.ops`` and ``spconv.pytorch.core`` the way
src/hi3d_mac/torch_backend/__init__.py:34-55 does, so unmodified callers
(``sparc3d.ops.sparse_backend``) resolve to this module.

Added for the strided pair (which the reference does not implement): spconv-named
``SparseConv3d(kernel_size=2, stride=2)`` and ``SparseInverseConv3d(kernel_size=2,
indice_key=...)``. The coarse set is the sorted unique ``coords // 2``
(downsample_structure, src/hi3d_mac/mlx_backend/sparse.py:217-233) and the output grid
is ``ceil(spatial_shape / 2)``; every fine voxel feeds its parent through kernel offset
``slot = (x&1)*4 + (y&1)*2 + (z&1)``.

Every computation runs on the GPU; CPU tensors raise ``ValueError``.
"""

from __future__ import annotations

import enum
import importlib.machinery
import sys
import types
from typing import Any, Sequence

import torch
from torch import nn

from . import conv as _conv
from . import kmap as _kmap


class ConvAlgo(enum.Enum):
    """Accepted for spconv compatibility; the value is ignored: every member runs the
    one output-stationary gather-MFMA kernel."""

    Native = 0
    MaskImplicitGemm = 1
    MaskSplitImplicitGemm = 2


class _PairTable:
    """Answers ``pairs[side, k, rows]`` from the GPU's compacted lists: side 0 = input
    rows, side 1 = output rows, offset k occupying ``[offsets[k], offsets[k+1])`` of one
    flat buffer per side (so no ``[2, K, N]`` padding is ever materialised)."""

    def __init__(self, src: torch.Tensor, dst: torch.Tensor, offsets: torch.Tensor):
        self._sides = (src, dst)
        self._offsets = [int(v) for v in offsets.tolist()]

    def __getitem__(self, index: tuple[int, int, slice]) -> torch.Tensor:
        side, offset, rows = index
        lo, hi = self._offsets[offset], self._offsets[offset + 1]
        return self._sides[side][lo:hi][rows].long()


class IndiceData:
    """Cached kernel map, mirroring ``spconv.pytorch.core.IndiceData``.

    Beside the reference's fields it carries the GPU kernel map (``kmap``) or the
    stride-2 structure (``stride2``) the convolutions run from. ``indice_pairs`` is
    built on first access (a GPU compaction of the dense table).
    """

    def __init__(
        self,
        out_indices: torch.Tensor,
        indices: torch.Tensor,
        indice_pairs: Any,
        indice_pair_num: torch.Tensor,
        spatial_shape: Sequence[int],
        out_spatial_shape: Sequence[int],
        is_subm: bool = True,
        algo: ConvAlgo = ConvAlgo.Native,
        kmap: _kmap.KernelMap | None = None,
        stride2: _kmap.Stride2Structure | None = None,
        **_: Any,
    ):
        self.out_indices = out_indices
        self.indices = indices
        self._indice_pairs = indice_pairs
        self.indice_pair_num = indice_pair_num
        self.spatial_shape = list(spatial_shape)
        self.out_spatial_shape = list(out_spatial_shape)
        self.is_subm = is_subm
        self.algo = algo
        self.kmap = kmap
        self.stride2 = stride2

    @property
    def indice_pairs(self) -> Any:
        if self._indice_pairs is None:
            if self.kmap is not None:
                self._indice_pairs = _PairTable(*self.kmap.pairs())
            elif self.stride2 is not None:
                self._indice_pairs = _PairTable(*_stride2_pairs(self.stride2))
        return self._indice_pairs

    @indice_pairs.setter
    def indice_pairs(self, value: Any) -> None:
        self._indice_pairs = value


class SparseConvTensor:
    """A feature matrix over its voxel coordinates (rows of ``(batch, x, y, z)``), the
    grid extent, and the ``indice_dict`` that every tensor derived from it shares, so a
    kernel map built for one layer is found by the next layer with the same key."""

    def __init__(
        self,
        features: torch.Tensor,
        indices: torch.Tensor,
        spatial_shape: Sequence[int],
        batch_size: int,
        indice_dict: dict[str, IndiceData] | None = None,
    ):
        self._features = features
        self.indices = indices
        self.spatial_shape = [int(v) for v in spatial_shape]
        self.batch_size = int(batch_size)
        self.indice_dict = {} if indice_dict is None else indice_dict

    @property
    def features(self) -> torch.Tensor:
        return self._features

    def replace_feature(self, feature: torch.Tensor) -> "SparseConvTensor":
        """New features on the same voxels; the coordinate rows and the cache are shared,
    not copied."""
        return SparseConvTensor(feature, self.indices, self.spatial_shape, self.batch_size, self.indice_dict)

    def find_indice_pair(self, key: str | None) -> IndiceData | None:
        return None if key is None else self.indice_dict.get(key)


def _voxel_keys(indices: torch.Tensor, spatial_shape: Sequence[int]) -> torch.Tensor:
    """Packed voxel keys ``((b*sx + x)*sy + y)*sz + z`` (int64), as the hash packs them."""
    batch, x, y, z = indices.long().unbind(1)
    sx, sy, sz = (int(v) for v in spatial_shape)
    return ((batch * sx + x) * sy + y) * sz + z


def subm_pairs(
    indices: torch.Tensor, spatial_shape: Sequence[int], kernel_size: int = 3
) -> tuple[list[torch.Tensor], list[torch.Tensor], torch.Tensor]:
    """The kernel map as lists: for each of the ``kernel_size**3`` offsets, the input
    rows and the output rows they feed (int64, ascending input row), and the list
    lengths. Built on the GPU (dense grid or hash, then a compaction of the table)."""
    km = _kmap.build_kernel_map(indices, spatial_shape, None, kernel_size)
    src, dst, offsets = km.pairs()
    off = offsets.tolist()
    sources = [src[off[k] : off[k + 1]].long() for k in range(km.kvol)]
    targets = [dst[off[k] : off[k + 1]].long() for k in range(km.kvol)]
    counts = torch.tensor([off[k + 1] - off[k] for k in range(km.kvol)], dtype=torch.int32)
    return sources, targets, counts


def _table_from_pairs(pairs: IndiceData, n: int, kvol: int) -> torch.Tensor:
    """Dense table from per-offset lists (for an ``IndiceData`` built elsewhere)."""
    device = pairs.indices.device
    table = torch.full((n, kvol), n, dtype=torch.int32, device=device)
    for k in range(kvol):
        count = int(pairs.indice_pair_num[k])
        if count:
            src = pairs.indice_pairs[0, k, :count].to(device)
            dst = pairs.indice_pairs[1, k, :count].to(device)
            table[src, kvol - 1 - k] = dst.int()
    return table


def subm_conv(
    features: torch.Tensor,
    pairs: IndiceData,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
) -> torch.Tensor:
    """Apply a submanifold convolution given cached pairs (one gather-MFMA pass)."""
    out_channels = weight.shape[0]
    kernel_volume = weight[0, ..., 0].numel()
    if features.dtype != weight.dtype:
        raise RuntimeError(f"features ({features.dtype}) and weight ({weight.dtype}) dtypes differ")
    if pairs.kmap is not None:
        plan = pairs.kmap.plan()
    else:
        n = int(features.shape[0])
        plan = _kmap.build_plan(_table_from_pairs(pairs, n, kernel_volume), n, pairs.indices)
    w = weight.reshape(out_channels, kernel_volume, weight.shape[-1])
    b = None if bias is None else bias.to(features.dtype)
    return _conv.conv(features, plan, w, b)


def get_indice_pair_data(input: SparseConvTensor, kernel_size: int = 3) -> IndiceData:
    km = _kmap.build_kernel_map(input.indices, input.spatial_shape, input.batch_size, kernel_size)
    return IndiceData(
        input.indices,
        input.indices,
        None,
        km.counts.cpu(),
        input.spatial_shape,
        input.spatial_shape,
        is_subm=True,
        algo=ConvAlgo.Native,
        kmap=km,
    )


def _stride2_data(input: SparseConvTensor) -> IndiceData:
    s = _kmap.stride2_structure(input.indices, input.spatial_shape, input.batch_size)
    counts = torch.bincount(s.slot.long(), minlength=8).to(torch.int32).cpu()
    return IndiceData(
        s.low, input.indices, None, counts, input.spatial_shape, s.out_spatial_shape, is_subm=False,
        algo=ConvAlgo.Native, stride2=s,
    )


def _stride2_pairs(s: _kmap.Stride2Structure):
    # list k: (fine i, parent(i)) for fine rows of slot k, ascending i
    return _kmap.pair_lists(s.up.flip(1).contiguous())


def _check_weight_dtype(features: torch.Tensor, weight: torch.Tensor) -> None:
    if features.dtype != weight.dtype:
        raise RuntimeError(f"features ({features.dtype}) and weight ({weight.dtype}) dtypes differ")


class SubMConv3d(nn.Module):
    """3x3x3 (any odd k) convolution evaluated only at the input's own voxels. Takes
    spconv's constructor arguments and keeps its weight as ``[Cout, k, k, k, Cin]``, so
    checkpoints load unchanged; the forward pass is one gather-MFMA launch over the
    kernel map cached under ``indice_key``."""

    def __init__(
        self,
        in_channels: int,
        out_channels: int,
        kernel_size: int | Sequence[int] = 3,
        stride: int | Sequence[int] = 1,
        padding: int | Sequence[int] = 0,
        dilation: int | Sequence[int] = 1,
        groups: int = 1,
        bias: bool = True,
        indice_key: str | None = None,
        algo: ConvAlgo | None = None,
        **_: Any,
    ):
        super().__init__()
        ks = (kernel_size,) * 3 if isinstance(kernel_size, int) else tuple(kernel_size)
        if len(set(ks)) != 1 or ks[0] % 2 == 0:
            raise ValueError(f"only cubic odd kernels are supported, got {ks}")
        if groups != 1:
            raise ValueError("grouped sparse convolution is not supported")
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = ks
        self.stride = (1, 1, 1)
        self.padding = tuple(k // 2 for k in ks)
        self.dilation = (1, 1, 1)
        self.output_padding = (0, 0, 0)
        self.indice_key = indice_key
        self.algo = algo or ConvAlgo.MaskImplicitGemm
        self.weight = nn.Parameter(torch.empty(out_channels, *ks, in_channels))
        self.bias = nn.Parameter(torch.empty(out_channels)) if bias else None
        nn.init.kaiming_uniform_(self.weight, a=5**0.5)
        if self.bias is not None:
            nn.init.zeros_(self.bias)

    def _pairs(self, input: SparseConvTensor) -> IndiceData:
        data = input.find_indice_pair(self.indice_key)
        if data is None:
            data = get_indice_pair_data(input, self.kernel_size[0])
            if self.indice_key is not None:
                input.indice_dict[self.indice_key] = data
        return data

    def forward(self, input: SparseConvTensor) -> SparseConvTensor:
        data = self._pairs(input)
        output = subm_conv(input.features, data, self.weight, self.bias)
        return input.replace_feature(output)


class SparseConv3d(nn.Module):
    """2x2x2 / stride-2 downsampling sparse convolution (spconv's name and layout)."""

    def __init__(
        self,
        in_channels: int,
        out_channels: int,
        kernel_size: int | Sequence[int] = 2,
        stride: int | Sequence[int] = 2,
        padding: int | Sequence[int] = 0,
        dilation: int | Sequence[int] = 1,
        groups: int = 1,
        bias: bool = True,
        indice_key: str | None = None,
        algo: ConvAlgo | None = None,
        **_: Any,
    ):
        super().__init__()
        triple = lambda v: (v,) * 3 if isinstance(v, int) else tuple(v)  # noqa: E731
        if triple(kernel_size) != (2, 2, 2) or triple(stride) != (2, 2, 2):
            raise NotImplementedError("only kernel_size 2 / stride 2 strided convolution is implemented")
        if triple(padding) != (0, 0, 0) or triple(dilation) != (1, 1, 1):
            raise NotImplementedError("only padding 0 / dilation 1 are implemented")
        if groups != 1:
            raise ValueError("grouped sparse convolution is not supported")
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = (2, 2, 2)
        self.stride = (2, 2, 2)
        self.padding = (0, 0, 0)
        self.dilation = (1, 1, 1)
        self.indice_key = indice_key
        self.algo = algo or ConvAlgo.MaskImplicitGemm
        self.weight = nn.Parameter(torch.empty(out_channels, 2, 2, 2, in_channels))
        self.bias = nn.Parameter(torch.empty(out_channels)) if bias else None
        nn.init.kaiming_uniform_(self.weight, a=5**0.5)
        if self.bias is not None:
            nn.init.zeros_(self.bias)

    def forward(self, input: SparseConvTensor) -> SparseConvTensor:
        data = input.find_indice_pair(self.indice_key)
        if data is None or data.stride2 is None or data.indices is not input.indices:
            data = _stride2_data(input)
            if self.indice_key is not None:
                input.indice_dict[self.indice_key] = data
        _check_weight_dtype(input.features, self.weight)
        s = data.stride2
        w = self.weight.reshape(self.out_channels, 8, self.in_channels)
        b = None if self.bias is None else self.bias.to(input.features.dtype)
        out = _conv.conv(input.features, s.down_plan(), w, b)
        return SparseConvTensor(out, s.low, s.out_spatial_shape, input.batch_size, input.indice_dict)


class SparseInverseConv3d(nn.Module):
    """Transpose of a :class:`SparseConv3d` back onto its input's coordinates, found in
    the shared pair cache under ``indice_key``: ``z[i] = b + W[:, slot(i), :] @ y[parent(i)]``."""

    def __init__(
        self,
        in_channels: int,
        out_channels: int,
        kernel_size: int | Sequence[int] = 2,
        indice_key: str | None = None,
        bias: bool = True,
        algo: ConvAlgo | None = None,
        **_: Any,
    ):
        super().__init__()
        ks = (kernel_size,) * 3 if isinstance(kernel_size, int) else tuple(kernel_size)
        if ks != (2, 2, 2):
            raise NotImplementedError("only kernel_size 2 inverse convolution is implemented")
        if indice_key is None:
            raise ValueError("SparseInverseConv3d needs the indice_key of its SparseConv3d")
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = ks
        self.indice_key = indice_key
        self.algo = algo or ConvAlgo.MaskImplicitGemm
        self.weight = nn.Parameter(torch.empty(out_channels, 2, 2, 2, in_channels))
        self.bias = nn.Parameter(torch.empty(out_channels)) if bias else None
        nn.init.kaiming_uniform_(self.weight, a=5**0.5)
        if self.bias is not None:
            nn.init.zeros_(self.bias)

    def forward(self, input: SparseConvTensor) -> SparseConvTensor:
        data = input.find_indice_pair(self.indice_key)
        if data is None or data.stride2 is None:
            raise ValueError(f"no strided convolution registered under indice_key {self.indice_key!r}")
        s = data.stride2
        if int(input.features.shape[0]) != s.n_coarse:
            raise ValueError("input rows do not match the coarse set of the paired SparseConv3d")
        _check_weight_dtype(input.features, self.weight)
        w = self.weight.reshape(self.out_channels, 8, self.in_channels)
        b = None if self.bias is None else self.bias.to(input.features.dtype)
        out = _conv.stride2_up(input.features, s, w, b)
        return SparseConvTensor(out, data.indices, data.spatial_shape, input.batch_size, input.indice_dict)


def get_indice_pairs(
    indices: torch.Tensor,
    batch_size: int,
    spatial_shape: Sequence[int],
    algo: ConvAlgo,
    ksize: Sequence[int],
    stride: Sequence[int],
    padding: Sequence[int],
    dilation: Sequence[int],
    out_padding: Sequence[int],
    subm: bool = False,
    transpose: bool = False,
):
    """``spconv.pytorch.ops.get_indice_pairs`` for the submanifold case and the 2x2x2
    stride-2 downsampling (pairs (fine, coarse) per slot)."""
    if transpose:
        raise NotImplementedError("transposed index pairs are not implemented")
    if tuple(dilation) != (1, 1, 1):
        raise NotImplementedError("only dilation 1 is implemented")
    if subm:
        if tuple(stride) != (1, 1, 1):
            raise NotImplementedError("only stride 1 / dilation 1 are implemented")
        km = _kmap.build_kernel_map(indices, spatial_shape, batch_size, int(ksize[0]))
        return indices, _PairTable(*km.pairs()), km.counts.cpu()
    if tuple(ksize) != (2, 2, 2) or tuple(stride) != (2, 2, 2) or tuple(padding) != (0, 0, 0):
        raise NotImplementedError("only submanifold and 2x2x2/s2 index pairs are implemented")
    s = _kmap.stride2_structure(indices, spatial_shape, batch_size)
    src, dst, offsets = _stride2_pairs(s)
    counts = (offsets[1:] - offsets[:-1]).to(torch.int32).cpu()
    return s.low, _PairTable(src, dst, offsets), counts


_INSTALLED_NAMES = ("spconv", "spconv.pytorch", "spconv.pytorch.ops", "spconv.pytorch.core")


def _module(name: str) -> types.ModuleType:
    module = types.ModuleType(name)
    module.__spec__ = importlib.machinery.ModuleSpec(name, loader=None)
    module.__hi3d_amd_shim__ = True
    return module


def install() -> None:
    """Register this module as ``spconv`` (refusing to shadow a real spconv)."""
    existing = sys.modules.get("spconv")
    if existing is not None:
        if getattr(existing, "__hi3d_amd_shim__", False):
            return
        raise RuntimeError("a real spconv is already imported; refusing to shadow it")
    pytorch = _module("spconv.pytorch")
    for name in ("SubMConv3d", "SparseConv3d", "SparseInverseConv3d", "SparseConvTensor", "ConvAlgo"):
        setattr(pytorch, name, globals()[name])
    ops = _module("spconv.pytorch.ops")
    ops.get_indice_pairs = get_indice_pairs
    core = _module("spconv.pytorch.core")
    core.IndiceData = IndiceData
    pytorch.ops = ops
    pytorch.core = core
    root = _module("spconv")
    root.pytorch = pytorch
    sys.modules.update({"spconv": root, "spconv.pytorch": pytorch, "spconv.pytorch.ops": ops, "spconv.pytorch.core": core})


def uninstall() -> None:
    """Remove the registered shim modules (only ours)."""
    for name in _INSTALLED_NAMES:
        mod = sys.modules.get(name)
        if mod is not None and getattr(mod, "__hi3d_amd_shim__", False):
            del sys.modules[name]
