"""Kernel maps on the GPU against the oracle: bit-exact tables, counts and pair lists,
stride-2 structures and child tables; error paths (duplicates, range, overflow)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import kmap as okmap

pytestmark = pytest.mark.gpu


def _rand_indices(rng, n_side, density, batch=1):
    rows = []
    for b in range(batch):
        xyz = np.argwhere(rng.random((n_side,) * 3) < density)
        rows.append(np.concatenate([np.full((len(xyz), 1), b), xyz], 1))
    idx = np.concatenate(rows).astype(np.int32)
    return idx[rng.permutation(len(idx))]


def test_golden_8cube_table_counts_pairs(cuda):
    from hi3d_amd import kmap

    data = np.load(GOLDEN / "kmap_8cube.npz")
    km = kmap.build_kernel_map(torch.as_tensor(data["indices"]).to(cuda), [8, 8, 8])
    assert np.array_equal(km.table.cpu().numpy(), data["table"])
    assert np.array_equal(km.counts.cpu().numpy(), data["counts"])
    src, dst, off = km.pairs()
    assert np.array_equal(off.cpu().numpy(), data["offsets"])
    assert np.array_equal(src.cpu().numpy(), data["src"])
    assert np.array_equal(dst.cpu().numpy(), data["dst"])


@pytest.mark.parametrize("ksize,batch,n_side,density", [(3, 1, 12, 0.3), (3, 3, 10, 0.5), (1, 2, 6, 0.5), (5, 2, 9, 0.2)])
def test_random_sets_bit_exact(cuda, ksize, batch, n_side, density):
    from hi3d_amd import kmap

    rng = np.random.default_rng(100 + ksize + batch)
    idx = _rand_indices(rng, n_side, density, batch)
    shape = [n_side, n_side + 1, n_side + 2]
    km = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), shape, batch, ksize)
    ref = okmap.neighbour_table(idx, shape, ksize)
    assert np.array_equal(km.table.cpu().numpy(), ref)
    assert np.array_equal(km.counts.cpu().numpy(), (ref != len(idx)).sum(0).astype(np.int32))
    src, dst, off = km.pairs()
    rs, rd, ro = okmap.pairs_from_table(ref)
    assert np.array_equal(off.cpu().numpy(), ro)
    assert np.array_equal(src.cpu().numpy(), rs) and np.array_equal(dst.cpu().numpy(), rd)


def test_64bit_keys(cuda):
    """batch * sx * sy * sz >= 2^32 selects the 64-bit key hash."""
    from hi3d_amd import kmap

    rng = np.random.default_rng(7)
    n = 5000
    shape = [3000, 3000, 1000]
    base = rng.integers(0, [2999, 2999, 999], size=(n // 5, 3))
    pts = np.concatenate([base + d for d in ([0, 0, 0], [1, 0, 0], [0, 1, 0], [0, 0, 1], [1, 1, 1])])
    pts = np.unique(pts, axis=0)
    idx = np.concatenate([rng.integers(0, 2, size=(len(pts), 1)), pts], 1).astype(np.int32)
    idx = np.unique(idx, axis=0)
    idx = idx[rng.permutation(len(idx))]
    assert 2 * shape[0] * shape[1] * shape[2] >= 2**32
    km = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), shape, 2)
    assert np.array_equal(km.table.cpu().numpy(), okmap.neighbour_table(idx, shape))


def test_errors_duplicate_range_overflow(cuda):
    from hi3d_amd import kmap

    idx = np.array([[0, 1, 1, 1], [0, 2, 2, 2], [0, 1, 1, 1]], np.int32)
    for ksize in (1, 3, 5):
        with pytest.raises(ValueError, match="duplicate"):
            kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [4, 4, 4], ksize=ksize)
    rng = np.random.default_rng(2)
    many = _rand_indices(rng, 9, 0.4)
    many = np.concatenate([many, many[::50]])
    for ksize in (3, 5):
        with pytest.raises(ValueError, match="duplicate"):
            kmap.build_kernel_map(torch.as_tensor(many).to(cuda), [9, 9, 9], ksize=ksize)
    idx = np.array([[0, 1, 1, 1], [0, 4, 2, 2]], np.int32)
    with pytest.raises(ValueError, match="outside"):
        kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [4, 4, 4])
    rng = np.random.default_rng(1)
    idx = _rand_indices(rng, 8, 0.5)
    assert len(idx) > 64
    with pytest.raises(RuntimeError, match="overflow"):  # 16 buckets for the 8^3 grid's 64 bricks
        kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [8, 8, 8], capacity=16)


def test_stride2_structure_errors(cuda):
    """The stride-2 structure raises the submanifold map's errors: a coordinate outside
    spatial_shape (also negative, or a batch index past batch_size) and a repeated
    coordinate, including through get_indice_pairs with a caller's spatial_shape; a
    valid set after a failing call is unaffected (the status word is cleared)."""
    from hi3d_amd import kmap, spconv

    dup = np.array([[0, 1, 1, 1], [0, 2, 2, 2], [0, 1, 1, 1], [0, 3, 3, 3]], np.int32)
    with pytest.raises(ValueError, match="duplicate"):
        kmap.stride2_structure(torch.as_tensor(dup).to(cuda), [4, 4, 4])
    for bad in ([0, 4, 2, 2], [0, 1, -1, 2], [0, 1, 2, 5], [1, 1, 1, 1]):
        idx = np.array([[0, 1, 1, 1], bad], np.int32)
        with pytest.raises(ValueError, match="outside"):
            kmap.stride2_structure(torch.as_tensor(idx).to(cuda), [4, 4, 5], 1)
    idx = np.array([[0, 1, 1, 1], [0, 7, 2, 2]], np.int32)
    with pytest.raises(ValueError, match="outside"):
        spconv.get_indice_pairs(torch.as_tensor(idx).to(cuda), 1, [4, 4, 4], spconv.ConvAlgo.Native, (2, 2, 2),
                                (2, 2, 2), (0, 0, 0), (1, 1, 1), (0, 0, 0), False, False)
    ok = np.array([[0, 1, 1, 1], [0, 0, 1, 1], [0, 3, 2, 2]], np.int32)
    s = kmap.stride2_structure(torch.as_tensor(ok).to(cuda), [4, 4, 4])
    assert s.low.cpu().tolist() == [[0, 0, 0, 0], [0, 1, 1, 1]]
    assert s.inverse.cpu().tolist() == [0, 0, 1] and s.counts.cpu().tolist() == [2, 1]
    assert s.slot.cpu().tolist() == [7, 3, 4]


def test_empty_and_single(cuda):
    from hi3d_amd import kmap

    km = kmap.build_kernel_map(torch.zeros((0, 4), dtype=torch.int32, device=cuda), [4, 4, 4], 1)
    assert km.table.shape == (0, 27) and int(km.counts.sum()) == 0
    src, dst, off = km.pairs()
    assert src.numel() == 0 and off.cpu().tolist() == [0] * 28
    km = kmap.build_kernel_map(torch.tensor([[0, 0, 0, 0]], dtype=torch.int32, device=cuda), [1, 1, 1])
    t = km.table.cpu().numpy()
    assert t[0, 13] == 0 and (t == 1).sum() == 26


@pytest.mark.parametrize("name", ["subm3_c64_fp32", "subm3_c128_fp16"])
def test_workload_maps_bit_exact(cuda, name):
    from hi3d_amd import kmap, workloads

    idx = workloads.coords_for(name)
    grid = workloads.WORKLOADS[name].grid
    km = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [grid] * 3, 1)
    ref = okmap.neighbour_table(idx, [grid] * 3)
    got = km.table.cpu().numpy()
    assert np.array_equal(got, ref)
    if name == "subm3_c64_fp32":
        assert int((ref != len(idx)).sum()) == 474_776


def test_large_shell_map_properties(cuda):
    """The 1024^3 workload (~4.4M voxels): the whole table of the default map (the brick
    hash at this grid size) equals the oracle's (the sort + searchsorted lookup over
    key-ordered rows, every row and offset) and the kept dense grid's, and over all rows
    the size-independent properties hold: neighbour coordinates, symmetry, count
    symmetry."""
    from hi3d_amd import kmap, workloads

    idx = workloads.coords_for("resblock_c256_fp16", device=cuda)
    n = len(idx)
    coords = torch.as_tensor(idx).to(cuda)
    km = kmap.build_kernel_map(coords, [1024] * 3, 1)
    table = km.table
    print(f"comparing the full {n} x 27 table with the oracle", flush=True)
    assert np.array_equal(table.cpu().numpy(), okmap.neighbour_table_sorted(idx, [1024] * 3))
    old = kmap.KMAP_DENSE_MAX_CELLS
    try:
        kmap.KMAP_DENSE_MAX_CELLS = 1 << 31
        dense = kmap.build_kernel_map(coords, [1024] * 3, 1)
    finally:
        kmap.KMAP_DENSE_MAX_CELLS = old
    kmap.release_dense_grids()
    assert torch.equal(dense.table, table) and torch.equal(dense.counts, km.counts)
    offs = torch.as_tensor(okmap.kernel_offsets(3) - 1, device=cuda, dtype=torch.int32)
    present = table != n
    for k in range(27):
        p = present[:, k]
        nb = table[p, k].long()
        assert torch.equal(coords[nb, 1:], coords[p, 1:] + offs[k])
        assert torch.equal(table[nb, 26 - k], torch.nonzero(p).squeeze(1).int())
    counts = km.counts.cpu().numpy()
    assert np.array_equal(counts, counts[::-1]) and counts[13] == n


def test_stride2_structure(cuda):
    from hi3d_amd import kmap

    rng = np.random.default_rng(3)
    idx = _rand_indices(rng, 11, 0.3, batch=2)
    s = kmap.stride2_structure(torch.as_tensor(idx).to(cuda), [11, 11, 11], 2)
    low, inverse, counts, slot, down, up = okmap.stride2_structure(idx)
    assert np.array_equal(s.low.cpu().numpy(), low)
    assert np.array_equal(s.inverse.cpu().numpy(), inverse)
    assert np.array_equal(s.counts.cpu().numpy(), counts)
    assert np.array_equal(s.slot.cpu().numpy(), slot)
    assert np.array_equal(s.down.cpu().numpy(), down)
    assert np.array_equal(s.up.cpu().numpy(), up)
    assert s.out_spatial_shape == [6, 6, 6]


def test_stride2_golden_and_workload(cuda):
    from hi3d_amd import kmap, workloads

    data = np.load(GOLDEN / "stride2_12cube.npz")
    s = kmap.stride2_structure(torch.as_tensor(data["indices"]).to(cuda), [12, 12, 12])
    assert np.array_equal(s.low.cpu().numpy(), data["low"])
    assert np.array_equal(s.inverse.cpu().numpy(), data["inverse"])
    idx = workloads.coords_for("down2_up2_c64_c128_fp16")
    s = kmap.stride2_structure(torch.as_tensor(idx).to(cuda), [512] * 3, 1)
    low, inverse, counts, slot, down, up = okmap.stride2_structure(idx)
    assert np.array_equal(s.low.cpu().numpy(), low)
    assert np.array_equal(s.inverse.cpu().numpy(), inverse)
    assert np.array_equal(s.down.cpu().numpy(), down)


def test_mlx_shaped_helpers(cuda):
    from hi3d_amd import sparse

    data = np.load(GOLDEN / "child_10cube.npz")
    coords = torch.as_tensor(data["coords"]).to(cuda)
    table = sparse.neighbour_table(coords)
    assert np.array_equal(table.cpu().numpy(), okmap.neighbour_table_dense(data["coords"]))
    ct, parent, slot = sparse.child_neighbour_table(table, torch.as_tensor(data["mask"]).to(cuda))
    assert np.array_equal(ct.cpu().numpy(), data["table"])
    assert np.array_equal(parent.cpu().numpy(), data["parent"])
    assert np.array_equal(slot.cpu().numpy(), data["slot"])
    low, inv, cnt = sparse.downsample_structure(coords)
    rl, ri, rc = okmap.downsample_structure(data["coords"])
    assert np.array_equal(low.cpu().numpy(), rl) and np.array_equal(inv.cpu().numpy(), ri)
    assert np.array_equal(cnt.cpu().numpy(), rc)


def test_plan_covers_every_row_once(cuda):
    from hi3d_amd import kmap, workloads

    idx = workloads.coords_for("subm3_c128_fp16")
    km = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [256] * 3, 1)
    for window in (0, 1 << 15):
        plan = kmap.build_plan(km.table, km.n, km.indices, window)
        rows = plan.rows.cpu().numpy()
        valid = rows[rows >= 0]
        assert np.array_equal(np.sort(valid), np.arange(km.n))
        gidx = plan.gidx.view(plan.ntiles, 27, 128).cpu().numpy()
        table = km.table.cpu().numpy()
        t = np.where(rows.reshape(-1, 128)[:, None, :] >= 0,
                     table[np.maximum(rows, 0)].reshape(plan.ntiles, 128, 27).transpose(0, 2, 1), km.n)
        assert np.array_equal(gidx, t)
        masks = plan.tile_mask.cpu().numpy().astype(np.uint32)
        present = (gidx != km.n)
        exp = (present.any(axis=2).astype(np.uint64) << np.arange(27, dtype=np.uint64)).sum(1).astype(np.uint32)
        assert np.array_equal(masks, exp)


def test_plan_work_on_shell_set(cuda):
    """The default plan of the 543k-voxel shell set (one mask-sorting window) runs at
    most 1.052 (row, offset) products per present pair in 128-row tiles: rows sorted by
    their presence mask with the corner offsets as the most significant key bits give
    1.0453; sorting the plain mask value gives 1.0592."""
    from hi3d_amd import kmap, workloads

    idx = workloads.coords_for("subm3_c128_fp16")
    km = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [256] * 3, 1)
    plan = km.plan()
    masks = plan.tile_mask.cpu().numpy().astype(np.uint32)
    computed = sum(bin(int(m)).count("1") for m in masks) * 128
    present = int((km.table != km.n).sum())
    assert computed <= 1.052 * present, computed / present


def test_blocked_assembly_matches_single_block(cuda):
    """The reference's blocked-assembly test (tests/test_mlx_kernels.py:92-102): row
    blocks concatenated, and assembled in place past the size threshold, equal one block."""
    from hi3d_amd import sparse

    x = torch.randn((1000, 16), device=cuda)
    fn = lambda s, e: x[s:e] * 2 + 1
    whole = fn(0, 1000)
    assert torch.equal(sparse.blocked(1000, 64, fn, 16, torch.float32), whole)
    old = sparse.ASSEMBLE_IN_PLACE_BYTES
    try:
        sparse.ASSEMBLE_IN_PLACE_BYTES = 0  # force the in-place path
        assert torch.equal(sparse.blocked(1000, 64, fn, 16, torch.float32, device=cuda), whole)
    finally:
        sparse.ASSEMBLE_IN_PLACE_BYTES = old


def test_blocked_accumulate_adds_in_place(cuda):
    """tests/test_mlx_kernels.py:105-121: the accumulated result lives in the donated
    buffer and the peak stays within one block of the inputs."""
    from hi3d_amd import sparse

    n, c = 200_000, 128
    base = torch.randn((n, c), device=cuda)
    h = torch.randn((n, c), device=cuda)
    expected = base + h * 2
    ptr = base.data_ptr()
    fn = lambda s, e: h[s:e] * 2
    holder = [base]
    del base
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(cuda)
    before = torch.cuda.memory_allocated(cuda)
    out = sparse.blocked(n, 20_000, fn, c, torch.float32, accumulate=holder)
    torch.cuda.synchronize()
    assert out.data_ptr() == ptr and torch.equal(out, expected)
    assert torch.cuda.max_memory_allocated(cuda) - before < n * c * 4 // 2


@pytest.mark.parametrize("dtype,c", [(torch.float16, 64), (torch.float32, 3)])
def test_gather_neighbours_matches_take(cuda, dtype, c):
    """``gather_neighbours(pad_rows(x), level, s, e)`` equals taking the padded rows by
    the table (sparse.py:175-182), absent neighbours reading the zero row."""
    from hi3d_amd import sparse

    data = np.load(GOLDEN / "child_10cube.npz")
    level = sparse.Level.from_coords(torch.as_tensor(data["coords"]).to(cuda))
    x = torch.randn((level.n, c), device=cuda).to(dtype)
    padded = sparse.pad_rows(x)
    assert padded.shape == (level.n + 1, c) and not padded[-1].any()
    got = sparse.gather_neighbours(padded, level, 5, 77)
    assert torch.equal(got, padded[level.table[5:77].long()])


# (column, value for a grid of side n) of coordinates outside the grid: one cell past an
# edge, and z (whose cells the 3x3x3 lookup loads as runs) far outside on either side
_OUT_OF_RANGE = [(2, lambda n: n), (3, lambda n: 1 << 30), (3, lambda n: -(1 << 30)), (3, lambda n: n + 40),
                 (3, lambda n: -1)]


@pytest.mark.parametrize("ksize,batch,n_side,density", [(3, 1, 20, 0.2), (3, 3, 16, 0.5), (5, 2, 12, 0.3),
                                                        (3, 1, 64, 0.01)])
def test_dense_and_hash_maps_agree(cuda, ksize, batch, n_side, density):
    """The dense-grid map (rows in input order and in cell order) and the hash map give
    the same table and counts bit for bit, and equal the oracle; all flag duplicates and
    out-of-range coordinates. Hash capacities: 2^16 buckets (rows in input order), 2^20
    (a table above 16 MiB: rows in superblock order, coordinates decoded from the sorted
    keys) and 2^25 (buckets past 2^24: the probe's 64-bit bucket exchange)."""
    from hi3d_amd import kmap

    rng = np.random.default_rng(n_side * 10 + batch)
    idx = _rand_indices(rng, n_side, density, batch=batch)
    t = torch.as_tensor(idx).to(cuda)
    dense = kmap.build_kernel_map(t, [n_side] * 3, batch, ksize)
    for cap in (1 << 16, 1 << 20, 1 << 25):
        hashed = kmap.build_kernel_map(t, [n_side] * 3, batch, ksize, capacity=cap)
        assert torch.equal(dense.table, hashed.table) and torch.equal(dense.counts, hashed.counts), cap
    del hashed
    ref = okmap.neighbour_table(idx, [n_side] * 3, ksize)
    assert np.array_equal(dense.table.cpu().numpy(), ref)
    dup = torch.cat([t, t[3:4]])
    for cap in (None, 1 << 16, 1 << 20):
        with pytest.raises(ValueError, match="duplicate"):
            kmap.build_kernel_map(dup, [n_side] * 3, batch, ksize, capacity=cap)
        for col, value in _OUT_OF_RANGE:
            bad = t.clone()
            bad[5, col] = value(n_side)
            with pytest.raises(ValueError, match="outside"):
                kmap.build_kernel_map(bad, [n_side] * 3, batch, ksize, capacity=cap)
    old = kmap.KMAP_DENSE_MAX_CELLS
    try:
        kmap.KMAP_DENSE_MAX_CELLS = 0  # the hash without a capacity
        assert torch.equal(kmap.build_kernel_map(t, [n_side] * 3, batch, ksize).table, dense.table)
    finally:
        kmap.KMAP_DENSE_MAX_CELLS = old
    # the kept grid with the rows in cell order (forced on this small grid): same map and
    # the same errors, for this kernel size too
    old_order = kmap.KMAP_DENSE_ORDER_MIN_BYTES
    try:
        kmap.KMAP_DENSE_ORDER_MIN_BYTES = 0
        ordered = kmap.build_kernel_map(t, [n_side] * 3, batch, ksize)
        assert torch.equal(ordered.table, dense.table) and torch.equal(ordered.counts, dense.counts)
        with pytest.raises(ValueError, match="duplicate"):
            kmap.build_kernel_map(dup, [n_side] * 3, batch, ksize)
        for col, value in _OUT_OF_RANGE:
            bad = t.clone()
            bad[5, col] = value(n_side)
            with pytest.raises(ValueError, match="outside"):
                kmap.build_kernel_map(bad, [n_side] * 3, batch, ksize)
        assert torch.equal(kmap.build_kernel_map(t, [n_side] * 3, batch, ksize).table, dense.table)
    finally:
        kmap.KMAP_DENSE_ORDER_MIN_BYTES = old_order


@pytest.mark.parametrize("shape,batch,ksize,density", [((13, 20, 7), 2, 3, 0.3), ((1, 9, 33), 3, 3, 0.4),
                                                        ((17, 5, 11), 2, 5, 0.25), ((31, 2, 19), 1, 3, 0.6)])
def test_non_cubic_odd_grids(cuda, shape, batch, ksize, density):
    """Odd, non-cubic extents (bricks and superblocks cut by every face, a one-cell-thick
    axis, a two-cell one) and several batch elements: the hash map at small and large
    capacities (input order and superblock order) and the dense grid give the oracle's
    table and counts bit for bit, voxels on every face included."""
    from hi3d_amd import kmap

    rng = np.random.default_rng(sum(shape) * 7 + batch + ksize)
    rows = []
    for b in range(batch):
        xyz = np.argwhere(rng.random(shape) < density)
        rows.append(np.concatenate([np.full((len(xyz), 1), b), xyz], 1))
    idx = np.concatenate(rows).astype(np.int32)
    idx = idx[rng.permutation(len(idx))]
    t = torch.as_tensor(idx).to(cuda)
    ref = okmap.neighbour_table(idx, list(shape), ksize)
    ref_counts = (ref < len(idx)).sum(0)
    dense = kmap.build_kernel_map(t, list(shape), batch, ksize)
    assert np.array_equal(dense.table.cpu().numpy(), ref)
    assert np.array_equal(dense.counts.cpu().numpy(), ref_counts)
    for cap in (1 << 12, 1 << 20):
        hashed = kmap.build_kernel_map(t, list(shape), batch, ksize, capacity=cap)
        assert torch.equal(hashed.table, dense.table) and torch.equal(hashed.counts, dense.counts), cap
    bad = t.clone()
    bad[0, 1 + int(np.argmin(shape))] = min(shape)  # one cell past the thinnest axis
    with pytest.raises(ValueError, match="outside"):
        kmap.build_kernel_map(bad, list(shape), batch, ksize, capacity=1 << 12)


def test_hash_wide_grid_superblock_order(cuda):
    """A grid whose superblock-major cell keys pass 32 bits (65536 x 65536 x 256): the
    hash sorts the superblocks alone and carries the coordinates in sorted order. The
    543k-voxel C128 shells moved to x + 40000, y + 50000 there have the neighbour table
    of the same shells in their own 256^3 grid (the dense map), nothing crossing an edge."""
    from hi3d_amd import kmap, workloads

    idx = workloads.coords_for("subm3_c128_fp16", device=cuda)
    coords = torch.as_tensor(idx).to(cuda)
    ref = kmap.build_kernel_map(coords, [256] * 3, 1)
    moved = coords.clone()
    moved[:, 1] += 40000
    moved[:, 2] += 50000
    wide = kmap.build_kernel_map(moved, [65536, 65536, 256], 1)
    assert torch.equal(wide.table, ref.table) and torch.equal(wide.counts, ref.counts)
    dup = torch.cat([moved, moved[11:12]])
    with pytest.raises(ValueError, match="duplicate"):
        kmap.build_kernel_map(dup, [65536, 65536, 256], 1)
    bad = moved.clone()
    bad[7, 3] = 300
    with pytest.raises(ValueError, match="outside"):
        kmap.build_kernel_map(bad, [65536, 65536, 256], 1)


@pytest.mark.parametrize("ordered", [True, False])
def test_kept_dense_grid_stays_clear(cuda, ordered):
    """The dense map over a grid kept between calls, with the rows visited in cell order
    or in input order: each build of a shuffled set equals the oracle and the per-call
    grid's map, and leaves every cell of the kept grid at -1 again, also after a build
    that reports duplicate or out-of-range coordinates; two different sets in a row on the
    same grid both come out exact (no cell of the first survives into the second)."""
    from hi3d_amd import kmap

    rng = np.random.default_rng(42)
    side = 24
    kmap.release_dense_grids()
    sets = [_rand_indices(rng, side, 0.2, batch=2), _rand_indices(rng, side, 0.05, batch=2)]
    old_order = kmap.KMAP_DENSE_ORDER_MIN_BYTES
    kmap.KMAP_DENSE_ORDER_MIN_BYTES = 0 if ordered else None
    try:
        _kept_grid_sets(cuda, kmap, sets, side)
    finally:
        kmap.KMAP_DENSE_ORDER_MIN_BYTES = old_order
    kmap.release_dense_grids()
    assert not kmap._DENSE_GRIDS


def _kept_grid_sets(cuda, kmap, sets, side):
    for idx in sets:
        t = torch.as_tensor(idx).to(cuda)
        kept = kmap.build_kernel_map(t, [side] * 3, 2)
        assert np.array_equal(kept.table.cpu().numpy(), okmap.neighbour_table(idx, [side] * 3))
        old = kmap.KMAP_DENSE_KEEP
        try:
            kmap.KMAP_DENSE_KEEP = False
            fresh = kmap.build_kernel_map(t, [side] * 3, 2)
        finally:
            kmap.KMAP_DENSE_KEEP = old
        assert torch.equal(kept.table, fresh.table) and torch.equal(kept.counts, fresh.counts)
        (entry,) = kmap._DENSE_GRIDS.values()
        grid = entry.grid
        assert int(grid.numel()) >= 2 * side**3 and bool((grid == -1).all())
        dup = torch.cat([t, t[7:9]])
        with pytest.raises(ValueError, match="duplicate"):
            kmap.build_kernel_map(dup, [side] * 3, 2)
        for col, value in [(1, lambda n: n)] + _OUT_OF_RANGE:
            bad = t.clone()
            bad[3, col] = value(side)
            with pytest.raises(ValueError, match="outside"):
                kmap.build_kernel_map(bad, [side] * 3, 2)
        assert bool((grid == -1).all())


def test_kept_dense_grid_across_streams_and_errors(cuda, monkeypatch):
    """Builds on one kept grid from two streams in a row give the oracle's map each time
    (the second stream waits for the first build's restore), and a build whose call
    raises drops the kept grid, so the next build starts from a fresh one."""
    from hi3d_amd import _lib, kmap

    rng = np.random.default_rng(7)
    side = 32
    kmap.release_dense_grids()
    sets = [_rand_indices(rng, side, 0.15), _rand_indices(rng, side, 0.3)]
    streams = [torch.cuda.Stream(cuda), torch.cuda.Stream(cuda)]
    tables = []
    for idx, s in zip(sets, streams):
        t = torch.as_tensor(idx).to(cuda)
        torch.cuda.current_stream(cuda).synchronize()
        with torch.cuda.stream(s):
            tables.append(kmap.build_kernel_map(t, [side] * 3, 1, check=False).table)
    torch.cuda.synchronize(cuda)
    for idx, table in zip(sets, tables):
        assert np.array_equal(table.cpu().numpy(), okmap.neighbour_table(idx, [side] * 3))
    (entry,) = kmap._DENSE_GRIDS.values()
    assert bool((entry.grid == -1).all())

    real_call = _lib.call

    def failing(name, *args):
        if name == "hi3d_kmap_subm_dense_kept":
            raise _lib.Hi3dError("planted failure")
        return real_call(name, *args)

    monkeypatch.setattr(_lib, "call", failing)
    with pytest.raises(_lib.Hi3dError, match="planted"):
        kmap.build_kernel_map(torch.as_tensor(sets[0]).to(cuda), [side] * 3, 1)
    assert not kmap._DENSE_GRIDS
    monkeypatch.setattr(_lib, "call", real_call)
    again = kmap.build_kernel_map(torch.as_tensor(sets[1]).to(cuda), [side] * 3, 1)
    assert np.array_equal(again.table.cpu().numpy(), okmap.neighbour_table(sets[1], [side] * 3))
    kmap.release_dense_grids()
