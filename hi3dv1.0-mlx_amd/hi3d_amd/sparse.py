"""The MLX backend's sparse-structure helpers, on torch GPU tensors and the HIP kernels.

Same names and array layouts as src/hi3d_mac/mlx_backend/sparse.py: ``OFFSETS`` /
``CENTER`` :20-23, ``GATHER_ELEMENTS`` :25-26, ``neighbour_table`` :29-43,
``child_neighbour_table`` :64-95, ``Level`` :98-115, ``ASSEMBLE_IN_PLACE_BYTES`` and
``blocked`` :118-172, ``pad_rows`` / ``gather_neighbours`` :175-182, ``conv_weight``
:185-188, ``sparse_conv`` :191-214, ``downsample_structure`` :217-233. The reference builds tables with NumPy on the host
and gathers a dense ``[rows, 27*Cin]`` block per row block; here the table is hashed on
the GPU and the convolution runs only the offsets present per 128-row tile.
"""

from __future__ import annotations

import itertools

import numpy as np
import torch

from . import _lib
from . import conv as _conv
from . import kmap as _kmap

OFFSETS = np.array(list(itertools.product(range(3), repeat=3)), dtype=np.int64) - 1
"""``[27, 3]`` neighbour displacement ``r_k - 1`` for each flat kernel offset."""

CENTER = 13

GATHER_ELEMENTS = 1 << 27
"""Elements per gathered ``[rows, 27, C]`` block in :func:`blocked` callers (256 MB at
fp16). The convolutions here never materialise that block; the constant sizes the
callers' own row blocks."""

ASSEMBLE_IN_PLACE_BYTES = 1 << 30
"""Blocked results larger than this are written into one preallocated tensor instead
of concatenated (which would briefly hold the result twice)."""

neighbour_table = _kmap.neighbour_table
downsample_structure = _kmap.downsample_structure
child_neighbour_table = _kmap.child_neighbour_table


class Level:
    """One coordinate set and its convolution gather table (``N`` marks absent)."""

    def __init__(self, coords: torch.Tensor, table: torch.Tensor):
        self.coords = coords
        self.n = int(coords.shape[0])
        self.table = table
        self._plan: _kmap.ConvPlan | None = None

    @classmethod
    def from_coords(cls, coords: torch.Tensor) -> "Level":
        coords = torch.as_tensor(coords, dtype=torch.int32)
        return cls(coords, neighbour_table(coords))

    @property
    def plan(self) -> _kmap.ConvPlan:
        if self._plan is None:
            xyz = self.coords.to(self.table.device, torch.int32)
            indices = torch.cat([torch.zeros((self.n, 1), dtype=torch.int32, device=xyz.device), xyz], 1)
            self._plan = _kmap.build_plan(self.table, self.n, indices)
        return self._plan


def blocked(n: int, rows: int, block_fn, width: int, dtype: torch.dtype, accumulate: list | None = None,
            device: torch.device | str = "cuda") -> torch.Tensor:
    """``[n, width]`` result of ``block_fn(start, stop)`` over row blocks of ``rows``
    (sparse.py:132-172). With ``accumulate`` (a one-element list holding the only
    reference to an ``[n, width]`` tensor ``a``) returns ``a + blocks``, added block by
    block into ``a``'s own buffer; results above ``ASSEMBLE_IN_PLACE_BYTES`` are
    written into one preallocated tensor."""
    if accumulate is not None:
        out = accumulate.pop()
        for start in range(0, n, rows):
            stop = min(start + rows, n)
            out[start:stop] += block_fn(start, stop)
        return out
    if rows >= n:
        return block_fn(0, n)
    itemsize = torch.empty((), dtype=dtype).element_size()
    if n * width * itemsize > ASSEMBLE_IN_PLACE_BYTES:
        out = torch.empty((n, width), dtype=dtype, device=device)
        for start in range(0, n, rows):
            stop = min(start + rows, n)
            out[start:stop] = block_fn(start, stop)
        return out
    return torch.cat([block_fn(start, min(start + rows, n)) for start in range(0, n, rows)], 0)


def pad_rows(x: torch.Tensor) -> torch.Tensor:
    """``x`` with one zero row appended: the target of absent neighbours (index ``N``)."""
    return torch.cat([x, torch.zeros((1, x.shape[1]), dtype=x.dtype, device=x.device)], 0)


def gather_neighbours(padded: torch.Tensor, level: Level, start: int, stop: int) -> torch.Tensor:
    """``[stop - start, 27, C]`` neighbour features of :func:`pad_rows` output, gathered by
    the GPU row copy (``hi3d_gather_rows``; entries outside the padded rows read zeros)."""
    device = _lib.require_gpu(padded, level.table)
    c = int(padded.shape[1])
    idx = level.table[start:stop].reshape(-1).to(torch.int32).contiguous()
    rb = c * padded.element_size()
    if rb % 16:
        return padded[idx.long()].reshape(stop - start, 27, c)
    src = padded.contiguous()
    if src.data_ptr() % 16:
        src = src.clone()
    out = torch.empty((idx.shape[0], c), dtype=padded.dtype, device=device)
    _lib.call("hi3d_gather_rows", _lib.ptr(src), int(src.shape[0]), rb, _lib.ptr(idx), int(idx.shape[0]),
              _lib.ptr(out), _lib.stream(device))
    return out.reshape(stop - start, 27, c)


def conv_weight(weight: torch.Tensor) -> torch.Tensor:
    """spconv ``(out, 3, 3, 3, in)`` -> GEMM layout ``[27 * in, out]``."""
    out_channels = weight.shape[0]
    return weight.reshape(out_channels, -1).T


def sparse_conv(x: torch.Tensor, level: Level, weight_t: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    """Submanifold 3x3x3 convolution; ``weight_t [27 * Cin, Cout]`` from
    :func:`conv_weight`, computed in ``weight_t.dtype`` with fp32 accumulation."""
    cin = int(x.shape[1])
    cout = int(weight_t.shape[1])
    w = weight_t.T.reshape(cout, 27, cin)
    b = None if bias is None else bias.to(weight_t.dtype)
    return _conv.conv(x.to(weight_t.dtype), level.plan, w, b)
