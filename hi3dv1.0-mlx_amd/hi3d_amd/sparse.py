"""The MLX backend's sparse-structure helpers, on torch GPU tensors and the HIP kernels.

Same names and array layouts as src/hi3d_mac/mlx_backend/sparse.py: ``OFFSETS`` /
``CENTER`` :20-23, ``neighbour_table`` :29-43, ``child_neighbour_table`` :64-95,
``Level`` :98-115, ``conv_weight`` :185-188, ``sparse_conv`` :191-214,
``downsample_structure`` :217-233. The reference builds tables with NumPy on the host
and gathers a dense ``[rows, 27*Cin]`` block per row block; here the table is hashed on
the GPU and the convolution runs only the offsets present per 128-row tile.
"""

from __future__ import annotations

import itertools

import numpy as np
import torch

from . import conv as _conv
from . import kmap as _kmap

OFFSETS = np.array(list(itertools.product(range(3), repeat=3)), dtype=np.int64) - 1
"""``[27, 3]`` neighbour displacement ``r_k - 1`` for each flat kernel offset."""

CENTER = 13

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
