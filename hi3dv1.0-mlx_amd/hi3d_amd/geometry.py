"""The refiner transformer's index structures for one sampling pass: the full and the
2x2x2-coarse voxel sets, mean-pool down, parent-copy up, and the first convolution of
the up block evaluated over the coarse rows.

Mirrors ``Geometry`` (src/hi3d_mac/mlx_backend/transformer.py:234-266) and
``Sparc3DTransformerMLX._up_conv`` (:449-473) on torch GPU tensors and the HIP library.
The reference projects every coarse row through all 27 taps (``[N_low, 27 * Cout]``) and
gather-sums per fine voxel; here ``_up_conv``'s sum is the gather-MFMA convolution over
a composed map ``parent[full.table[o, k]]`` whose inputs are the coarse rows, so neither
the projection nor the upsampled features are materialised. That map has the full
map's presence pattern, so its plan equals the full level's and the result equals the
convolution of ``upsample(h_low)`` bit for bit.
"""

from __future__ import annotations

import torch

from . import _lib
from . import conv as _conv
from . import kmap as _kmap
from .sparse import Level


class Geometry:
    """Index structures of one sampling pass (coordinates never change within it)."""

    def __init__(self, coords: torch.Tensor):
        device = _lib.require_gpu(coords)
        coords = coords.to(torch.int32).contiguous()
        if coords.dim() != 2 or coords.shape[1] != 3:
            raise ValueError(f"expected coords [N, 3], got {tuple(coords.shape)}")
        self.coords = coords
        self.full = Level.from_coords(coords)
        n = self.full.n
        indices = torch.cat([torch.zeros((n, 1), dtype=torch.int32, device=device), coords], 1)
        extent = [v + 1 for v in _kmap.column_bounds(coords)[1]] if n else [1, 1, 1]
        s = _kmap.stride2_structure(indices, extent, 1)
        self._structure = s
        self.low = Level.from_coords(s.low[:, 1:].contiguous())
        self.inverse = s.inverse
        self.counts = s.counts
        # scatter_reduce(mean) onto a zero-initialised output divides by children + 1
        self.mean_divisor = (s.counts + 1).to(torch.float32)[:, None]
        self._up_plan: _kmap.ConvPlan | None = None

    @property
    def up_conv_table(self) -> torch.Tensor:
        """``[N, 27]`` map whose inputs are the coarse parents of the fine neighbours
        (``N_low`` where the neighbour is absent)."""
        return self.up_conv_plan.table

    @property
    def up_conv_plan(self) -> _kmap.ConvPlan:
        if self._up_plan is None:
            n, n_low = self.full.n, self.low.n
            device = self.full.table.device
            table = torch.empty((n, 27), dtype=torch.int32, device=device)
            _lib.call("hi3d_parent_table", _lib.ptr(self.full.table), n, 27, _lib.ptr(self.inverse), n_low,
                      _lib.ptr(table), _lib.stream(device))
            indices = torch.cat([torch.zeros((n, 1), dtype=torch.int32, device=device), self.coords], 1)
            self._up_plan = _kmap.build_plan(table, n_low, indices)
        return self._up_plan

    def downsample(self, x: torch.Tensor) -> torch.Tensor:
        """Mean of each coarse voxel's children, divided by children + 1 (the reference's
        zero-initialised ``scatter_reduce(mean)``), accumulated in fp32 and returned in
        ``x.dtype`` (transformer.py:261-263)."""
        device = _lib.require_gpu(x)
        if x.dim() != 2 or x.shape[0] != self.full.n:
            raise ValueError(f"expected x [{self.full.n}, C], got {tuple(x.shape)}")
        if x.dtype not in _lib.DTYPES:
            raise ValueError(f"unsupported dtype {x.dtype}")
        xc = x.contiguous()
        out = torch.empty((self.low.n, x.shape[1]), dtype=x.dtype, device=device)
        _lib.call("hi3d_gather_mean", _lib.ptr(xc), self.full.n, int(x.shape[1]), _lib.ptr(self._structure.down), 8,
                  self.low.n, 1, _lib.DTYPES[x.dtype], _lib.ptr(out), _lib.stream(device))
        return out

    def upsample(self, x: torch.Tensor) -> torch.Tensor:
        """Each fine voxel's parent row (transformer.py:265-266)."""
        device = _lib.require_gpu(x)
        if x.dim() != 2 or x.shape[0] != self.low.n:
            raise ValueError(f"expected x [{self.low.n}, C], got {tuple(x.shape)}")
        rb = int(x.shape[1]) * x.element_size()
        if rb % 16:
            return x[self.inverse.long()]
        xc = x.contiguous()
        if xc.data_ptr() % 16:
            xc = xc.clone()
        out = torch.empty((self.full.n, x.shape[1]), dtype=x.dtype, device=device)
        _lib.call("hi3d_gather_rows", _lib.ptr(xc), self.low.n, rb, _lib.ptr(self.inverse), self.full.n,
                  _lib.ptr(out), _lib.stream(device))
        return out

    def up_conv(self, h_low: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
                out: torch.dtype | None = None) -> torch.Tensor:
        """``_up_conv`` (transformer.py:449-473): the 3x3x3 convolution of
        ``upsample(h_low)`` over the full set, computed from the coarse rows. ``weight``
        in the reference's ``[Cout, 27 * Cin]`` (or spconv ``[Cout, 3, 3, 3, Cin]``)
        layout; fp32 accumulation, bias added in fp32, result in ``out`` (default: the
        weight dtype)."""
        _lib.require_gpu(h_low, weight)
        cout = int(weight.shape[0])
        cin = int(h_low.shape[1])
        w = weight.reshape(cout, 27, cin).contiguous()
        x = h_low.to(weight.dtype).contiguous()
        out = weight.dtype if out is None else out
        if bias is None or out != weight.dtype:
            y = _conv.conv(x, self.up_conv_plan, w, None)
            if bias is not None:
                y = (y.float() + bias.float()).to(out)
            return y.to(out)
        return _conv.conv(x, self.up_conv_plan, w, bias.to(weight.dtype))
