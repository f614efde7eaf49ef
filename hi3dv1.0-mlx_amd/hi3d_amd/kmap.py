"""Kernel maps on the GPU: the dense neighbour table, pair lists, stride-2 structure,
octree child tables and the tile plans the convolution consumes.

Reference functions replaced here:
  * ``_voxel_keys`` / ``subm_pairs`` (src/hi3d_mac/torch_backend/sparse_conv.py:109-149)
  * ``neighbour_table`` (src/hi3d_mac/mlx_backend/sparse.py:29-43)
  * ``_PairTable`` / ``get_indice_pairs`` (sparse_conv.py:37-50,264-283)
  * ``downsample_structure`` (src/hi3d_mac/mlx_backend/sparse.py:217-233)
  * ``child_neighbour_table`` (src/hi3d_mac/mlx_backend/sparse.py:46-95)
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Sequence

import torch

from . import _lib

PLAN_WINDOW_ROWS: int | None = None
"""Rows per mask-sorting window of a convolution plan (``0``: one window over all
rows); ``None`` picks by size (``PLAN_SMALL_WINDOW`` up to ``PLAN_GLOBAL_ROWS`` rows,
else ``PLAN_LARGE_WINDOW``). Smaller windows keep the gathers of neighbouring tiles in
L2; larger ones group more rows of equal offset masks, so tiles run fewer absent
(row, offset) pairs. Measured with the corner-major mask keys: on the 543k-voxel C128
shells one window 0.3775 ms against 0.3804 ms at 2^18; on the 1.1M-voxel shells one
window C64 0.243 / C128 0.554 ms against 0.257 / 0.575 ms at 2^18; on the 4.4M-voxel
C256 shells 2^19 is best (7.09 ms; 7.28 at 2^18, 7.22-7.25 at 2^20 .. one window)."""
KMAP_DENSE_MAX_CELLS: int = 1 << 28
"""Grids of at most this many cells (batch * sx * sy * sz) build their map through a
dense grid of rows (4 bytes per cell, kept between builds) instead of the brick hash;
``0`` always hashes. Up to 2^28 cells the dense grid is the faster map (543k voxels at
256^3: 0.13 against 0.17 ms hashed; 1.1M at 512^3: 0.18 against 0.25 ms). Above it the
two run at the same speed (4.4M voxels at 1024^3: 0.74 ms on the kept grid against
0.73 ms hashed) and the grid would hold 4 GiB per 2^30 cells, against the hash's
~110 bytes per voxel for the duration of the build, so the hash builds those maps."""

KMAP_DENSE_KEEP: bool = True
"""Keep one dense grid per (device, cell count) between calls (``hi3d_kmap_subm_dense_kept``:
the grid stays -1 outside a call, and a call touches only its rows' cells) instead of
clearing a per-call grid of 4 bytes per cell. The kept grid holds its memory until
:func:`release_dense_grids` (4 GiB for a 1024^3 grid)."""

KMAP_DENSE_ORDER_MIN_BYTES: int | None = 256 << 20
"""With a kept grid of more than this many bytes, visit the rows in cell order (a radix
sort of their cell keys) so that neighbouring rows store, read and restore neighbouring
cells whatever order the coordinates arrive in; ``None`` never sorts. Below it the grid
stays in the GPU's 256 MB last-level cache and the sort costs more than it saves (config
5, 4.4M randomly ordered voxels at 1024^3: 1.01 ms sorted against 1.19 ms; config 2,
543k voxels at 256^3: 0.22 against 0.14 ms)."""

KMAP_DENSE_KEEP_BYTES: int = 8 << 30
"""Kept dense grids beyond this many bytes in total are freed, least recently used
first (the grid of the current build always stays)."""

@dataclass
class _KeptGrid:
    """A dense grid kept between builds (every cell -1 outside a build) and the event
    recorded on the stream of its last build, after that build's restore."""

    grid: torch.Tensor
    done: torch.cuda.Event | None = None


_DENSE_GRIDS: dict[tuple[int, int], _KeptGrid] = {}


def release_dense_grids() -> None:
    """Free the dense grids kept between kernel-map builds."""
    _DENSE_GRIDS.clear()


def _kept_grid(device: torch.device, cells: int, nbytes: int) -> tuple[tuple[int, int], _KeptGrid]:
    key = (device.index if device.index is not None else torch.cuda.current_device(), cells)
    entry = _DENSE_GRIDS.pop(key, None)
    if entry is None:
        held = sum(e.grid.numel() * 4 for e in _DENSE_GRIDS.values())
        for k in list(_DENSE_GRIDS):
            if held + nbytes <= KMAP_DENSE_KEEP_BYTES:
                break
            held -= _DENSE_GRIDS.pop(k).grid.numel() * 4
        entry = _KeptGrid(torch.full((nbytes // 4,), -1, dtype=torch.int32, device=device))
    _DENSE_GRIDS[key] = entry  # most recently used last
    return key, entry


def _build_on_kept_grid(key: tuple[int, int], entry: _KeptGrid, device: torch.device, launch) -> None:
    """Run ``launch(grid)`` (one kept-grid build) on the current stream of ``device``.

    The build stores its rows in the grid's cells and puts them back, so two builds must
    not overlap on one grid: the current stream first waits for the previous build's
    event (a no-op on the same stream), and records its own after the launch. A launch
    that raises drops the grid, since its cells may no longer all be -1."""
    current = torch.cuda.current_stream(device)
    if entry.done is not None:
        current.wait_event(entry.done)
    entry.grid.record_stream(current)  # freeing the grid waits for this stream's work too
    try:
        launch(entry.grid)
    except BaseException:
        _DENSE_GRIDS.pop(key, None)
        raise
    done = torch.cuda.Event()
    done.record(current)
    entry.done = done

UP_ORDER_WINDOW_LOG2: int = 31
"""Windows (log2 rows) of the sorted up convolution's mask sort: 31 sorts every coarse
row by its children's slot mask at once (the tiles then share masks best; the rows it
gathers stay inside the coarse set, which the last-level cache holds)."""

PLAN_GLOBAL_ROWS = 1 << 21
PLAN_SMALL_WINDOW = 0
PLAN_LARGE_WINDOW = 1 << 19


def column_bounds(a: torch.Tensor) -> tuple[list[int], list[int]]:
    """Per-column minima and maxima of non-empty integer rows ``a [N, d]`` (d <= 8), from
    one GPU pass (``hi3d_row_bounds``) and one host read."""
    device = _lib.require_gpu(a)
    if a.dim() != 2 or a.shape[0] == 0 or a.dtype not in (torch.int32, torch.int64):
        raise ValueError("column_bounds needs non-empty int32 / int64 rows [N, d]")
    a = a.contiguous()
    d = int(a.shape[1])
    bounds = torch.empty((2, d), dtype=torch.int64, device=device)
    _lib.call("hi3d_row_bounds", _lib.ptr(a), _lib.I64 if a.dtype == torch.int64 else _lib.I32, int(a.shape[0]), d,
              _lib.ptr(bounds[0]), _lib.ptr(bounds[1]), _lib.stream(device))
    lo, hi = bounds.tolist()
    return lo, hi


def _as_coords(indices: torch.Tensor) -> torch.Tensor:
    if indices.ndim != 2 or indices.shape[1] != 4:
        raise ValueError(f"expected coords [N, 4], got {tuple(indices.shape)}")
    return indices.to(torch.int32).contiguous()


@dataclass
class HaloPlan:
    """Halo plan of a 27-offset submanifold table: tiles of 256 output rows in Morton
    order, each with the sorted unique input rows its offsets touch (the halo) and every
    (row, offset)'s position in it; the halo convolution gathers each tile's halo into
    LDS once per K step."""

    rows: torch.Tensor  # [ntiles * 256] output row per slot, -1 for padding
    halo: torch.Tensor  # [ntiles, 768] input rows, n_in where unused
    hcount: torch.Tensor  # [ntiles]
    loff: torch.Tensor  # [ntiles * 256, 32] int16 halo positions (offsets 0..26), -1 absent
    bmask: torch.Tensor  # [ntiles * 8] offsets present per 32-row block
    n_out: int
    n_in: int

    @property
    def ntiles(self) -> int:
        return int(self.hcount.shape[0])


def morton_bits(spatial_shape: Sequence[int], batch_size: int) -> tuple[int, int]:
    """``(coord_bits, batch_bits)`` of the Morton sort for coordinates inside
    ``spatial_shape`` and batch indices below ``batch_size``: the plan sorts on
    ``3 * coord_bits + batch_bits`` key bits instead of 64 (four radix passes instead of
    eight at 1024^3)."""
    coord_bits = max(1, (max(int(v) for v in spatial_shape) - 1).bit_length())
    batch_bits = (int(batch_size) - 1).bit_length()
    if coord_bits > 19 or batch_bits > 7:
        return (0, 0)
    return (coord_bits, batch_bits)


def build_halo_plan(
    table: torch.Tensor, n_in: int, coords: torch.Tensor | None = None, bits: tuple[int, int] | None = None
) -> HaloPlan | None:
    """Halo plan of ``table [n_out, 27]``, or None when a tile's halo exceeds the
    kernel's capacity (callers then use the tile plan). ``bits``: :func:`morton_bits` of
    the coordinates' grid (None: the full 64-bit Morton key)."""
    device = _lib.require_gpu(table, coords)
    table = table.to(torch.int32).contiguous()
    n_out, kvol = int(table.shape[0]), int(table.shape[1])
    if kvol != 27:
        raise ValueError(f"halo plans cover 27-offset maps, got {kvol} offsets")
    if coords is not None:
        coords = _as_coords(coords)
        if coords.shape[0] != n_out:
            raise ValueError("plan coordinates must have one row per output row")
    L = _lib.lib()
    t, cap = int(L.hi3d_halo_tile_rows()), int(L.hi3d_halo_capacity())
    ntiles = (n_out + t - 1) // t
    rows = torch.empty(ntiles * t, dtype=torch.int32, device=device)
    halo = torch.empty((ntiles, cap), dtype=torch.int32, device=device)
    hcount = torch.empty(ntiles, dtype=torch.int32, device=device)
    loff = torch.empty((ntiles * t, 32), dtype=torch.int16, device=device)
    bmask = torch.empty(ntiles * (t // 32), dtype=torch.int32, device=device)
    overflow = torch.empty(1, dtype=torch.int32, device=device)
    ws = _lib.workspace(_lib.query("hi3d_halo_plan_workspace", n_out), device)
    _lib.call(
        "hi3d_halo_plan",
        _lib.ptr(table), n_out, kvol, int(n_in), _lib.ptr(coords), *(bits or (0, 0)), _lib.ptr(ws), ws.numel(),
        _lib.ptr(rows),
        _lib.ptr(halo), _lib.ptr(hcount), _lib.ptr(loff), _lib.ptr(bmask), _lib.ptr(overflow), _lib.stream(device),
    )
    if int(overflow.item()) != 0:
        return None
    return HaloPlan(rows, halo, hcount, loff, bmask, n_out, int(n_in))


@dataclass
class ConvPlan:
    """Tile plan of one gather table: output row per tile slot, transposed gather
    indices per tile and offset, and the offsets present in each tile. For 27-offset
    submanifold tables it also builds (once, on request) the halo plan."""

    rows: torch.Tensor
    gidx: torch.Tensor
    tile_mask: torch.Tensor
    n_out: int
    n_in: int
    kvol: int
    table: torch.Tensor
    coords: torch.Tensor | None = None
    bits: tuple[int, int] | None = None
    _halo: list = field(default_factory=list, repr=False)

    @property
    def ntiles(self) -> int:
        return int(self.tile_mask.shape[0])

    def halo(self) -> HaloPlan | None:
        """The halo plan (None when the table is not a 27-offset map over its own rows
        or a tile's halo does not fit)."""
        if not self._halo:
            ok = self.kvol == 27 and self.n_out == self.n_in
            self._halo.append(build_halo_plan(self.table, self.n_in, self.coords, self.bits) if ok else None)
        return self._halo[0]


def build_plan(
    table: torch.Tensor,
    n_in: int,
    coords: torch.Tensor | None = None,
    window_rows: int | None = None,
    bits: tuple[int, int] | None = None,
) -> ConvPlan:
    """Plan a gather convolution over ``table [n_out, kvol]`` (entries >= n_in absent).
    ``bits``: :func:`morton_bits` of the coordinates' grid (None: the full 64-bit Morton
    key; coordinates beyond the bits still give a valid plan, in a coarser order)."""
    device = _lib.require_gpu(table, coords)
    table = table.to(torch.int32).contiguous()
    n_out, kvol = int(table.shape[0]), int(table.shape[1])
    if coords is not None:
        coords = _as_coords(coords)
        if coords.shape[0] != n_out:
            raise ValueError("plan coordinates must have one row per output row")
    if window_rows is None:
        window_rows = PLAN_WINDOW_ROWS
    if window_rows is None:
        window_rows = PLAN_SMALL_WINDOW if n_out <= PLAN_GLOBAL_ROWS else PLAN_LARGE_WINDOW
    t = int(_lib.lib().hi3d_conv_tile_rows())
    ntiles = (n_out + t - 1) // t
    rows = torch.empty(ntiles * t, dtype=torch.int32, device=device)
    gidx = torch.empty(ntiles * kvol * t, dtype=torch.int32, device=device)
    tile_mask = torch.empty(ntiles, dtype=torch.int32, device=device)
    ws = _lib.workspace(_lib.query("hi3d_conv_plan_workspace", n_out), device)
    _lib.call(
        "hi3d_conv_plan",
        _lib.ptr(table), n_out, kvol, int(n_in), _lib.ptr(coords), *(bits or (0, 0)), int(window_rows),
        _lib.ptr(ws), ws.numel(), _lib.ptr(rows), _lib.ptr(gidx), _lib.ptr(tile_mask), _lib.stream(device),
    )
    return ConvPlan(rows, gidx, tile_mask, n_out, int(n_in), kvol, table, coords, bits)


def identity_plan(n: int, device: torch.device) -> ConvPlan:
    """Plan of the one-offset identity table (output row i gathers input row i): the
    gather convolution over it is a row-wise linear layer ``out = x @ W[:, 0, :].T + b``
    with the convolutions' epilogues (bias, SiLU, residual). Rows stay in order, so the
    plan is built without sorting."""
    t = int(_lib.lib().hi3d_conv_tile_rows())
    ntiles = (int(n) + t - 1) // t
    slots = torch.arange(ntiles * t, dtype=torch.int32, device=device)
    past = slots >= n
    rows = slots.masked_fill(past, -1)
    gidx = slots.masked_fill(past, int(n))
    tile_mask = torch.ones(ntiles, dtype=torch.int32, device=device)
    table = slots[:n].reshape(-1, 1).clone()
    return ConvPlan(rows, gidx, tile_mask, int(n), int(n), 1, table)


@dataclass
class KernelMap:
    """Submanifold kernel map of one coordinate set (built once, reused by every
    convolution over the set, like the reference's ``indice_dict`` cache)."""

    indices: torch.Tensor
    spatial_shape: list[int]
    batch_size: int
    ksize: int
    table: torch.Tensor  # [N, ksize^3] int32, sentinel N
    counts: torch.Tensor  # [ksize^3] int32 (device)
    _pairs: tuple | None = field(default=None, repr=False)
    _plans: dict = field(default_factory=dict, repr=False)

    @property
    def n(self) -> int:
        return int(self.table.shape[0])

    @property
    def kvol(self) -> int:
        return int(self.table.shape[1])

    def pairs(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """``(src, dst, offsets)``: per-offset lists back to back (list k spans
        ``offsets[k]:offsets[k+1]``), in spconv's orientation."""
        if self._pairs is None:
            self._pairs = pair_lists(self.table)
        return self._pairs

    def identity_plan(self) -> ConvPlan:
        """The row-wise (one-offset identity) plan over this map's rows, cached."""
        if "identity" not in self._plans:
            self._plans["identity"] = identity_plan(self.n, self.table.device)
        return self._plans["identity"]

    def plan(self, window_rows: int | None = None) -> ConvPlan:
        key = window_rows
        if key not in self._plans:
            self._plans[key] = build_plan(
                self.table, self.n, self.indices, window_rows, morton_bits(self.spatial_shape, self.batch_size)
            )
        return self._plans[key]


def build_kernel_map(
    indices: torch.Tensor,
    spatial_shape: Sequence[int],
    batch_size: int | None = None,
    ksize: int = 3,
    capacity: int | None = None,
    check: bool = True,
) -> KernelMap:
    """Submanifold kernel map of ``indices [N, 4]`` ``(batch, x, y, z)``: through a dense
    grid of rows when the grid has at most ``KMAP_DENSE_MAX_CELLS`` cells and no hash
    ``capacity`` is asked for (kept between calls when ``KMAP_DENSE_KEEP``), else
    through the brick hash (same table either way). Builds on a kept grid are ordered
    across streams by an event recorded after each one.

    With ``check`` the device status word is read (one sync): duplicate or out-of-range
    coordinates raise ``ValueError``, a full hash table raises ``RuntimeError``.
    """
    coords = _as_coords(indices)
    device = _lib.require_gpu(coords)
    sx, sy, sz = (int(v) for v in spatial_shape)
    n = int(coords.shape[0])
    if batch_size is None:
        batch_size = int(coords[:, 0].max()) + 1 if n else 1
    if ksize % 2 == 0 or ksize < 1:
        raise ValueError(f"only odd kernel sizes have a submanifold map, got {ksize}")
    kvol = ksize**3
    cells = int(batch_size) * sx * sy * sz
    table = torch.empty((n, kvol), dtype=torch.int32, device=device)
    counts = torch.empty(kvol, dtype=torch.int32, device=device)
    status = torch.empty(1, dtype=torch.int32, device=device)
    if capacity is None and cells <= KMAP_DENSE_MAX_CELLS:
        nbytes = _lib.query("hi3d_kmap_dense_workspace", int(batch_size), sx, sy, sz)
        if KMAP_DENSE_KEEP:
            key, entry = _kept_grid(device, cells, nbytes)
            order, order_bytes = None, 0
            if KMAP_DENSE_ORDER_MIN_BYTES is not None and nbytes > KMAP_DENSE_ORDER_MIN_BYTES and n:
                order = _lib.workspace(_lib.query("hi3d_kmap_dense_order_workspace", n), device)
                order_bytes = order.numel()

            def launch(grid: torch.Tensor) -> None:
                _lib.call(
                    "hi3d_kmap_subm_dense_kept",
                    _lib.ptr(coords), n, sx, sy, sz, int(batch_size), int(ksize), _lib.ptr(grid), grid.numel() * 4,
                    _lib.ptr(order), order_bytes,
                    _lib.ptr(table), _lib.ptr(counts), _lib.ptr(status), _lib.stream(device),
                )

            _build_on_kept_grid(key, entry, device, launch)
        else:
            ws = _lib.workspace(nbytes, device)
            _lib.call(
                "hi3d_kmap_subm_dense",
                _lib.ptr(coords), n, sx, sy, sz, int(batch_size), int(ksize), _lib.ptr(ws), ws.numel(),
                _lib.ptr(table), _lib.ptr(counts), _lib.ptr(status), _lib.stream(device),
            )
    else:
        key64 = cells >= 0xFFFFFFFF
        cap = int(capacity or 0)
        ws = _lib.workspace(_lib.query("hi3d_kmap_workspace", n, cap, int(key64)), device)
        _lib.call(
            "hi3d_kmap_subm",
            _lib.ptr(coords), n, sx, sy, sz, int(batch_size), int(ksize), cap, _lib.ptr(ws), ws.numel(),
            _lib.ptr(table), _lib.ptr(counts), _lib.ptr(status), _lib.stream(device),
        )
    if check:
        flags = int(status.item())
        if flags & _lib.MAP_DUPLICATE:
            raise ValueError("duplicate coordinates: every active voxel must appear once")
        if flags & _lib.MAP_RANGE:
            raise ValueError(f"coordinates outside spatial_shape {[sx, sy, sz]} or batch {batch_size}")
        if flags & _lib.MAP_OVERFLOW:
            raise RuntimeError("voxel hash table overflow: capacity too small for the active set")
    return KernelMap(coords, [sx, sy, sz], int(batch_size), int(ksize), table, counts)


def pair_lists(table: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Per-offset ``(src, dst)`` lists from a neighbour table: list k holds
    ``(i, table[i, kvol-1-k])`` for every row i with that entry present, ascending i."""
    device = _lib.require_gpu(table)
    table = table.to(torch.int32).contiguous()
    n, kvol = int(table.shape[0]), int(table.shape[1])
    offsets = torch.empty(kvol + 1, dtype=torch.int64, device=device)
    ws = _lib.workspace(_lib.query("hi3d_kmap_pairs_workspace", n, kvol), device)
    total_cap = n * kvol
    src = torch.empty(max(total_cap, 1), dtype=torch.int32, device=device)
    dst = torch.empty(max(total_cap, 1), dtype=torch.int32, device=device)
    _lib.call(
        "hi3d_kmap_pairs",
        _lib.ptr(table), n, kvol, _lib.ptr(ws), ws.numel(), _lib.ptr(src), _lib.ptr(dst), _lib.ptr(offsets),
        _lib.stream(device),
    )
    total = int(offsets[-1].item())
    return src[:total], dst[:total], offsets


def neighbour_table(coords: torch.Tensor) -> torch.Tensor:
    """``[N, 27]`` row of each voxel's neighbours (``N`` where absent), for ``[N, 3]``
    coordinates ``(x, y, z)`` of one batch element (the reference's MLX-side helper)."""
    if coords.ndim != 2 or coords.shape[1] != 3:
        raise ValueError(f"expected coords [N, 3], got {tuple(coords.shape)}")
    _lib.require_gpu(coords)
    xyz = coords.to(torch.int32)
    n = int(xyz.shape[0])
    if n == 0:
        return torch.empty((0, 27), dtype=torch.int32, device=coords.device)
    lo, hi = column_bounds(xyz)
    if min(lo) < 0:
        raise ValueError("grid coordinates must be non-negative")
    extent = [v + 1 for v in hi]
    indices = torch.cat([torch.zeros((n, 1), dtype=torch.int32, device=coords.device), xyz], 1)
    return build_kernel_map(indices, extent, 1, 3).table


@dataclass
class Stride2Structure:
    """Coarse set of a 2x2x2/s2 downsampling and its gather tables."""

    low: torch.Tensor  # [Nc, 4] int32 (batch, x, y, z), lexicographic
    inverse: torch.Tensor  # [Nf] int32
    counts: torch.Tensor  # [Nc] int32
    slot: torch.Tensor  # [Nf] uint8
    down: torch.Tensor  # [Nc, 8] fine child per slot (sentinel Nf)
    up: torch.Tensor  # [Nf, 8] parent in column slot (sentinel Nc)
    fine_indices: torch.Tensor
    spatial_shape: list[int]
    out_spatial_shape: list[int]
    _plans: dict = field(default_factory=dict, repr=False)

    @property
    def n_fine(self) -> int:
        return int(self.inverse.shape[0])

    @property
    def n_coarse(self) -> int:
        return int(self.low.shape[0])

    def down_plan(self) -> ConvPlan:
        if "down" not in self._plans:
            bits = morton_bits(self.out_spatial_shape, 128)  # batch indices fit 7 bits
            self._plans["down"] = build_plan(self.down, self.n_fine, self.low, bits=bits)
        return self._plans["down"]

    def up_order(self, window_log2: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """``(order, down_sorted)`` of the sorted parent-major up convolution: coarse
        rows sorted by the slot mask of their children (within windows of
        ``2**window_log2`` rows; ``None``: ``UP_ORDER_WINDOW_LOG2``), padded to whole
        tiles (``hi3d_stride2_up_plan``)."""
        w = UP_ORDER_WINDOW_LOG2 if window_log2 is None else int(window_log2)
        key = ("up_order", w)
        if key not in self._plans:
            device = self.down.device
            n_c, n_f = self.n_coarse, self.n_fine
            t = int(_lib.lib().hi3d_stride2_up_tile_rows())
            npad = (n_c + t - 1) // t * t
            order = torch.empty(max(npad, 1), dtype=torch.int32, device=device)
            down_sorted = torch.empty((max(npad, 1), 8), dtype=torch.int32, device=device)
            ws = _lib.workspace(_lib.query("hi3d_stride2_up_plan_workspace", n_c), device)
            _lib.call("hi3d_stride2_up_plan", _lib.ptr(self.down), n_c, n_f, w, _lib.ptr(ws), ws.numel(),
                      _lib.ptr(order), _lib.ptr(down_sorted), _lib.stream(device))
            self._plans[key] = (order, down_sorted)
        return self._plans[key]

    def up_plan(self) -> ConvPlan:
        if "up" not in self._plans:
            bits = morton_bits(self.spatial_shape, 128)
            self._plans["up"] = build_plan(self.up, self.n_coarse, self.fine_indices, bits=bits)
        return self._plans["up"]


def stride2_structure(indices: torch.Tensor, spatial_shape: Sequence[int], batch_size: int | None = None) -> Stride2Structure:
    """Coarse set, parent/slot maps and gather tables of a 2x2x2 stride-2 convolution.
    Raises ``ValueError`` for coordinates outside ``spatial_shape`` / ``batch_size`` and
    for repeated coordinates (one host read of the device status word, taken with the
    coarse row count)."""
    coords = _as_coords(indices)
    device = _lib.require_gpu(coords)
    n = int(coords.shape[0])
    sx, sy, sz = (int(v) for v in spatial_shape)
    if batch_size is None:
        batch_size = int(coords[:, 0].max()) + 1 if n else 1
    low = torch.empty((max(n, 1), 4), dtype=torch.int32, device=device)
    inverse = torch.empty(n, dtype=torch.int32, device=device)
    counts = torch.empty(max(n, 1), dtype=torch.int32, device=device)
    slot = torch.empty(n, dtype=torch.uint8, device=device)
    n_low_t = torch.empty(2, dtype=torch.int64, device=device)  # coarse row count, then the status word
    ws = _lib.workspace(_lib.query("hi3d_downsample_workspace", n), device)
    stream = _lib.stream(device)
    _lib.call(
        "hi3d_downsample_structure",
        _lib.ptr(coords), n, sx, sy, sz, int(batch_size), _lib.ptr(ws), ws.numel(), _lib.ptr(low),
        _lib.ptr(inverse), _lib.ptr(counts), _lib.ptr(slot), _lib.ptr(n_low_t), _lib.ptr(n_low_t[1:]), stream,
    )
    n_low, flags = (int(v) for v in n_low_t.tolist())
    flags &= 0xFFFFFFFF
    if flags & _lib.MAP_RANGE:
        raise ValueError(f"coordinates outside spatial_shape {[sx, sy, sz]} or batch {batch_size}")
    if flags & _lib.MAP_DUPLICATE:
        raise ValueError("duplicate coordinates: every active voxel must appear once")
    low, counts = low[:n_low], counts[:n_low]
    down = torch.empty((n_low, 8), dtype=torch.int32, device=device)
    up = torch.empty((n, 8), dtype=torch.int32, device=device)
    _lib.call("hi3d_stride2_tables", _lib.ptr(inverse), _lib.ptr(slot), n, n_low, _lib.ptr(down), _lib.ptr(up), stream)
    out_shape = [(sx + 1) // 2, (sy + 1) // 2, (sz + 1) // 2]
    return Stride2Structure(low, inverse, counts, slot, down, up, coords, [sx, sy, sz], out_shape)


@dataclass
class ResampleStructure:
    """Coarse set of a downsampling by any per-axis factor and its mean-pool table."""

    low: torch.Tensor  # [Nc, 4] int32 (batch, x // fx, y // fy, z // fz), lexicographic
    inverse: torch.Tensor  # [Nf] int32
    counts: torch.Tensor  # [Nc] int32
    slot: torch.Tensor  # [Nf] uint8: ((x % fx) fy + y % fy) fz + z % fz
    down: torch.Tensor  # [Nc, fx fy fz] fine row per slot (sentinel Nf)
    factor: tuple[int, int, int]


def resample_structure(indices: torch.Tensor, spatial_shape: Sequence[int], factor: Sequence[int],
                       batch_size: int | None = None) -> ResampleStructure:
    """Coarse set of ``indices [N, 4]`` downsampled by ``factor`` (one positive value per
    axis, product at most 256): the coordinates divided by the factor, sorted unique in
    lexicographic ``(batch, x, y, z)`` order (src/sparc3d/nn/sparse/spatial.py:36-72),
    each fine row's parent and slot, and the ``[Nc, fx fy fz]`` table of the mean pool.
    Raises ``ValueError`` for coordinates outside ``spatial_shape`` / ``batch_size`` and
    for repeated coordinates."""
    coords = _as_coords(indices)
    device = _lib.require_gpu(coords)
    fx, fy, fz = (int(v) for v in factor)
    if min(fx, fy, fz) <= 0 or fx * fy * fz > 256:
        raise ValueError(f"factors must be positive with a product of at most 256, got {(fx, fy, fz)}")
    n = int(coords.shape[0])
    sx, sy, sz = (int(v) for v in spatial_shape)
    if batch_size is None:
        batch_size = int(coords[:, 0].max()) + 1 if n else 1
    low = torch.empty((max(n, 1), 4), dtype=torch.int32, device=device)
    inverse = torch.empty(n, dtype=torch.int32, device=device)
    counts = torch.empty(max(n, 1), dtype=torch.int32, device=device)
    slot = torch.empty(n, dtype=torch.uint8, device=device)
    n_low_t = torch.empty(2, dtype=torch.int64, device=device)  # coarse row count, then the status word
    ws = _lib.workspace(_lib.query("hi3d_downsample_workspace", n), device)
    stream = _lib.stream(device)
    _lib.call(
        "hi3d_resample_structure",
        _lib.ptr(coords), n, sx, sy, sz, int(batch_size), fx, fy, fz, _lib.ptr(ws), ws.numel(), _lib.ptr(low),
        _lib.ptr(inverse), _lib.ptr(counts), _lib.ptr(slot), _lib.ptr(n_low_t), _lib.ptr(n_low_t[1:]), stream,
    )
    n_low, flags = (int(v) for v in n_low_t.tolist())
    flags &= 0xFFFFFFFF
    if flags & _lib.MAP_RANGE:
        raise ValueError(f"coordinates outside spatial_shape {[sx, sy, sz]} or batch {batch_size}")
    if flags & _lib.MAP_DUPLICATE:
        raise ValueError("duplicate coordinates: every active voxel must appear once")
    slots = fx * fy * fz
    down = torch.empty((n_low, slots), dtype=torch.int32, device=device)
    _lib.call("hi3d_resample_down_table", _lib.ptr(inverse), _lib.ptr(slot), n, n_low, slots, _lib.ptr(down), stream)
    return ResampleStructure(low[:n_low], inverse, counts[:n_low], slot, down, (fx, fy, fz))


def downsample_structure(coords: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``(low [Nc, 3], inverse [N], counts [Nc])``: unique ``coords // 2`` in
    lexicographic ``(x, y, z)`` order, each row's parent, and children per parent."""
    if coords.ndim != 2 or coords.shape[1] != 3:
        raise ValueError(f"expected coords [N, 3], got {tuple(coords.shape)}")
    _lib.require_gpu(coords)
    xyz = coords.to(torch.int32)
    n = int(xyz.shape[0])
    extent = [v + 1 for v in column_bounds(xyz)[1]] if n else [1, 1, 1]
    indices = torch.cat([torch.zeros((n, 1), dtype=torch.int32, device=coords.device), xyz], 1)
    s = stride2_structure(indices, extent, 1)
    return s.low[:, 1:].contiguous(), s.inverse, s.counts


def child_neighbour_table(
    parent_table: torch.Tensor, child_mask: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Children's ``[C, 27]`` table (sentinel C), parent ``[C]`` and slot ``[C]`` from
    the parent table ``[P, 27]`` (sentinel P) and occupancy ``[P, 8]``, parent-major."""
    device = _lib.require_gpu(parent_table, child_mask)
    parent_table = parent_table.to(torch.int32).contiguous()
    mask = child_mask.to(torch.uint8).contiguous()
    p = int(parent_table.shape[0])
    if mask.shape != (p, 8) or parent_table.shape[1] != 27:
        raise ValueError("expected parent_table [P, 27] and child_mask [P, 8]")
    cap = max(p * 8, 1)
    table = torch.empty((cap, 27), dtype=torch.int32, device=device)
    parent = torch.empty(cap, dtype=torch.int32, device=device)
    slot = torch.empty(cap, dtype=torch.int32, device=device)
    n_children = torch.empty(1, dtype=torch.int64, device=device)
    ws = _lib.workspace(_lib.query("hi3d_child_table_workspace", p), device)
    _lib.call(
        "hi3d_child_neighbour_table",
        _lib.ptr(parent_table), _lib.ptr(mask), p, _lib.ptr(ws), ws.numel(), _lib.ptr(table), _lib.ptr(parent),
        _lib.ptr(slot), _lib.ptr(n_children), _lib.stream(device),
    )
    c = int(n_children.item())
    return table[:c], parent[:c], slot[:c]
