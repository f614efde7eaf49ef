"""Kernel-map oracle (NumPy): voxel keys, submanifold pairs, neighbour tables, the
stride-2 coarse structure and the octree child table. Test infrastructure only."""

from __future__ import annotations

import itertools

import numpy as np


def voxel_keys(indices: np.ndarray, spatial_shape) -> np.ndarray:
    """``((b*sx + x)*sy + y)*sz + z`` as int64
    (src/hi3d_mac/torch_backend/sparse_conv.py:109-112)."""
    c = np.asarray(indices, dtype=np.int64)
    sx, sy, sz = (int(v) for v in spatial_shape)
    return ((c[:, 0] * sx + c[:, 1]) * sy + c[:, 2]) * sz + c[:, 3]


def kernel_offsets(ksize: int = 3) -> np.ndarray:
    """``[ksize^3, 3]`` positions ``r`` in flat order ``k = r0*ks^2 + r1*ks + r2``
    (itertools.product order, sparse_conv.py:131; sparse.py:20)."""
    return np.array(list(itertools.product(range(ksize), repeat=3)), dtype=np.int64)


def subm_pairs(indices: np.ndarray, spatial_shape, kernel_size: int = 3):
    """``(sources, targets, counts)`` restating ``subm_pairs``
    (src/hi3d_mac/torch_backend/sparse_conv.py:115-149): sort the keys once; for every
    offset ``r`` shift by ``center - r``, mask the grid bounds, ``searchsorted`` and keep
    exact matches. Sources are ascending rows; the centre offset is the identity."""
    coords = np.asarray(indices, dtype=np.int64)
    shape = [int(v) for v in spatial_shape]
    center = kernel_size // 2
    keys = voxel_keys(coords, shape)
    order = np.argsort(keys, kind="stable")
    sorted_keys = keys[order]
    n = coords.shape[0]
    arange = np.arange(n, dtype=np.int64)
    sources, targets = [], []
    for r in itertools.product(range(kernel_size), repeat=3):
        if r == (center, center, center):
            sources.append(arange.copy())
            targets.append(arange.copy())
            continue
        shift = np.array([0, center - r[0], center - r[1], center - r[2]], dtype=np.int64)
        neighbour = coords + shift
        inside = np.ones(n, dtype=bool)
        for axis in range(3):
            inside &= (neighbour[:, axis + 1] >= 0) & (neighbour[:, axis + 1] < shape[axis])
        query = voxel_keys(neighbour, shape)
        if n:
            position = np.minimum(np.searchsorted(sorted_keys, query), n - 1)
            found = inside & (sorted_keys[position] == query)
        else:
            position = np.zeros(0, dtype=np.int64)
            found = np.zeros(0, dtype=bool)
        sources.append(arange[found])
        targets.append(order[position[found]])
    counts = np.array([len(s) for s in sources], dtype=np.int32)
    return sources, targets, counts


def table_from_pairs(sources, targets, n: int) -> np.ndarray:
    """Dense table through the identity ``pairs[k] = {(i, table[i, K-1-k])}``."""
    kvol = len(sources)
    table = np.full((n, kvol), n, dtype=np.int32)
    for k in range(kvol):
        table[sources[k], kvol - 1 - k] = targets[k]
    return table


def pairs_from_table(table: np.ndarray):
    """``(src, dst, offsets)``: list k = ``(i, table[i, K-1-k])`` for present entries,
    ascending i, concatenated over k."""
    n, kvol = table.shape
    srcs, dsts, offsets = [], [], [0]
    for k in range(kvol):
        col = table[:, kvol - 1 - k]
        i = np.nonzero(col != n)[0]
        srcs.append(i.astype(np.int32))
        dsts.append(col[i].astype(np.int32))
        offsets.append(offsets[-1] + len(i))
    return np.concatenate(srcs), np.concatenate(dsts), np.array(offsets, dtype=np.int64)


def neighbour_table(indices: np.ndarray, spatial_shape, ksize: int = 3) -> np.ndarray:
    """``[N, ks^3]`` table (sentinel N) from the sort-based pairs (any grid size)."""
    sources, targets, _ = subm_pairs(indices, spatial_shape, ksize)
    return table_from_pairs(sources, targets, len(indices))


def neighbour_rows(indices: np.ndarray, spatial_shape, rows: np.ndarray, ksize: int = 3) -> np.ndarray:
    """Table rows ``rows`` only, by the same sorted-key ``searchsorted`` lookup as
    :func:`subm_pairs` (for spot checks of very large sets)."""
    coords = np.asarray(indices, dtype=np.int64)
    shape = [int(v) for v in spatial_shape]
    n = coords.shape[0]
    keys = voxel_keys(coords, shape)
    order = np.argsort(keys, kind="stable")
    sorted_keys = keys[order]
    half = ksize // 2
    sel = coords[np.asarray(rows)]
    table = np.full((len(sel), ksize**3), n, dtype=np.int32)
    for k, r in enumerate(itertools.product(range(ksize), repeat=3)):
        q = sel.copy()
        q[:, 1:] += np.array(r) - half
        inside = np.all((q[:, 1:] >= 0) & (q[:, 1:] < np.array(shape)), axis=1)
        qk = voxel_keys(q, shape)
        pos = np.minimum(np.searchsorted(sorted_keys, qk), max(n - 1, 0))
        found = inside & (sorted_keys[pos] == qk)
        table[found, k] = order[pos[found]]
    return table


def neighbour_table_sorted(indices: np.ndarray, spatial_shape, ksize: int = 3) -> np.ndarray:
    """``[N, ks^3]`` table (sentinel N) by the same sorted-key ``searchsorted`` lookup as
    :func:`subm_pairs` (src/hi3d_mac/torch_backend/sparse_conv.py:115-149), with the
    queries taken in key order: the packed key is linear in the coordinates, so the
    shifted keys of the key-sorted rows are the sorted keys plus one constant, and the
    search runs over sorted needles (minutes become seconds at millions of voxels).
    Writes the table directly instead of per-offset lists."""
    coords = np.asarray(indices, dtype=np.int64)
    shape = np.array([int(v) for v in spatial_shape], dtype=np.int64)
    n = coords.shape[0]
    kvol = ksize**3
    table = np.full((n, kvol), n, dtype=np.int32)
    if n == 0:
        return table
    keys = voxel_keys(coords, shape)
    order = np.argsort(keys, kind="stable")
    sorted_keys = keys[order]
    sorted_xyz = [coords[order, 1 + a] for a in range(3)]
    half = ksize // 2
    in_sorted = np.full((n, kvol), n, dtype=np.int32)  # rows in key order, then permuted once
    for k, r in enumerate(itertools.product(range(ksize), repeat=3)):
        d = [int(v) - half for v in r]
        delta = (d[0] * int(shape[1]) + d[1]) * int(shape[2]) + d[2]
        inside = np.ones(n, dtype=bool)
        for a in range(3):
            if d[a] < 0:
                inside &= sorted_xyz[a] >= -d[a]
            elif d[a] > 0:
                inside &= sorted_xyz[a] < shape[a] - d[a]
        query = sorted_keys + delta
        pos = np.minimum(np.searchsorted(sorted_keys, query), n - 1)
        found = inside & (sorted_keys[pos] == query)
        in_sorted[found, k] = order[pos[found]]
    table[order] = in_sorted
    return table


def neighbour_table_dense(coords: np.ndarray) -> np.ndarray:
    """Dense-grid ``neighbour_table`` (src/hi3d_mac/mlx_backend/sparse.py:29-43): a padded
    index grid of extent ``max + 3``, 27 fancy gathers. ``coords`` is ``[N, 3]``."""
    coords = np.asarray(coords, dtype=np.int64)
    n = coords.shape[0]
    offsets = kernel_offsets(3) - 1
    extent = coords.max(axis=0) + 3
    grid = np.full(tuple(extent), n, dtype=np.int32)
    grid[tuple((coords + 1).T)] = np.arange(n, dtype=np.int32)
    table = np.empty((n, 27), dtype=np.int32)
    for k, d in enumerate(offsets):
        table[:, k] = grid[tuple((coords + 1 + d).T)]
    return table


def brute_force_table(indices: np.ndarray, spatial_shape, ksize: int = 3) -> np.ndarray:
    """Definition by dictionary lookup (pure Python; tiny inputs only)."""
    coords = [tuple(int(v) for v in row) for row in np.asarray(indices)]
    where = {c: i for i, c in enumerate(coords)}
    n = len(coords)
    half = ksize // 2
    table = np.full((n, ksize**3), n, dtype=np.int32)
    for i, (b, x, y, z) in enumerate(coords):
        for k, r in enumerate(itertools.product(range(ksize), repeat=3)):
            q = (b, x + r[0] - half, y + r[1] - half, z + r[2] - half)
            if all(0 <= q[a + 1] < spatial_shape[a] for a in range(3)):
                table[i, k] = where.get(q, n)
    return table


def downsample_structure(coords: np.ndarray):
    """``(low, inverse, counts)`` of ``SparseDownsample(2)``
    (src/hi3d_mac/mlx_backend/sparse.py:217-233): unique ``coords // 2`` in lexicographic
    order by ``np.unique`` of packed codes."""
    half = np.asarray(coords, dtype=np.int64) // 2
    extent = half.max(axis=0) + 1
    codes = (half[:, 0] * extent[1] + half[:, 1]) * extent[2] + half[:, 2]
    unique, inverse, counts = np.unique(codes, return_inverse=True, return_counts=True)
    low = np.stack(
        [unique // (extent[1] * extent[2]), (unique // extent[2]) % extent[1], unique % extent[2]], axis=1
    ).astype(np.int32)
    return low, inverse.astype(np.int32).reshape(-1), counts.astype(np.int32)


def stride2_structure(indices: np.ndarray):
    """Batch-aware coarse structure + gather tables of the 2x2x2/s2 pair:
    ``(low [Nc,4], inverse [N], counts [Nc], slot [N], down [Nc,8], up [N,8])``."""
    c = np.asarray(indices, dtype=np.int64)
    n = c.shape[0]
    half = c.copy()
    half[:, 1:] //= 2
    extent = half.max(axis=0) + 1
    codes = ((half[:, 0] * extent[1] + half[:, 1]) * extent[2] + half[:, 2]) * extent[3] + half[:, 3]
    unique, inverse, counts = np.unique(codes, return_inverse=True, return_counts=True)
    inverse = inverse.reshape(-1)
    low = np.empty((unique.shape[0], 4), dtype=np.int64)
    rest = unique
    for axis in (3, 2, 1):
        low[:, axis] = rest % extent[axis]
        rest = rest // extent[axis]
    low[:, 0] = rest
    slot = ((c[:, 1] & 1) << 2) | ((c[:, 2] & 1) << 1) | (c[:, 3] & 1)
    nc = unique.shape[0]
    down = np.full((nc, 8), n, dtype=np.int32)
    down[inverse, slot] = np.arange(n, dtype=np.int32)
    up = np.full((n, 8), nc, dtype=np.int32)
    up[np.arange(n), slot] = inverse
    return low.astype(np.int32), inverse.astype(np.int32), counts.astype(np.int32), slot.astype(np.uint8), down, up


def child_offset_tables():
    """``(pk, ss)`` [8, 27]: parent-neighbourhood offset and child slot of each child's
    neighbour (src/hi3d_mac/mlx_backend/sparse.py:46-61)."""
    offsets = kernel_offsets(3) - 1
    pk = np.zeros((8, 27), np.int32)
    ss = np.zeros((8, 27), np.int32)
    for s in range(8):
        bits = np.array([(s >> 2) & 1, (s >> 1) & 1, s & 1])
        for k, d in enumerate(offsets):
            t = bits + d
            pd, cb = t >> 1, t & 1
            pk[s, k] = (pd[0] + 1) * 9 + (pd[1] + 1) * 3 + (pd[2] + 1)
            ss[s, k] = cb[0] * 4 + cb[1] * 2 + cb[2]
    return pk, ss


def child_neighbour_table(parent_table: np.ndarray, child_mask: np.ndarray):
    """``(table [C,27], parent [C], slot [C])`` of the octree children
    (src/hi3d_mac/mlx_backend/sparse.py:64-95), parent-major, slot-minor."""
    pk, ss = child_offset_tables()
    num_parents = child_mask.shape[0]
    ids = np.flatnonzero(child_mask.reshape(-1))
    c = int(ids.size)
    lookup = np.full(num_parents * 8 + 8, c, dtype=np.int32)
    lookup[ids] = np.arange(c, dtype=np.int32)
    parent, slot = ids // 8, ids % 8
    rows = parent_table[parent]
    neighbour_parent = np.take_along_axis(rows, pk[slot], axis=1)
    table = lookup[neighbour_parent.astype(np.int64) * 8 + ss[slot]]
    return table.astype(np.int32), parent.astype(np.int32), slot.astype(np.int32)
