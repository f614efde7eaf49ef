"""Pins the CPU oracle itself (no GPU): every oracle function is checked against
something that does not restate its own formula — the reference tests' dense
``F.conv3d`` check, brute force on tiny sets, independent constructions, closed forms,
library routines and the committed golden vectors.

Pinning map (oracle function -> checks here):
  kmap.subm_pairs / neighbour_table   -> brute_force_table, neighbour_table_dense, the
                                         layout invariants of tests/test_backends.py:53-67
  kmap.neighbour_table_dense          -> brute_force_table
  kmap.neighbour_rows / neighbour_table_sorted -> brute_force_table (corners, faces, batch
                                         2, ksize 5, keys above 2^62) and neighbour_table
  kmap.pairs_from_table/table_from_pairs -> round trip + subm_pairs lists
  kmap.stride2_structure / downsample_structure -> brute-force parents and slots
  kmap.child_neighbour_table          -> dense-grid table of the children
                                         (tests/test_mlx_kernels.py:79-89)
  conv.subm_conv_pairs / gather_conv_f64 -> dense F.conv3d (tests/test_backends.py:32-50)
  conv.dense_down2 / dense_up2        -> explicit per-voxel sums over parents/children
  conv.gather_mean                    -> scatter_reduce(mean) of PyTorch
  w8a8.rotate_h64                     -> float64 Hadamard matrix, closed forms (constant
                                         and one-hot rows), orthonormality
  w8a8.quantize_activation            -> zero row (s = 1e-8/127), hand-computed rows,
                                         codes within one step of v/s, |q| <= 127
  w8a8.int_gemm / epilogue            -> float64 matmul of small integers, the reference
                                         test's tolerance (tests/test_w8a8_inference.py:20)
  norm.layer_norm_modulate            -> float64 LayerNorm (torch.nn.functional)
  norm.adaln_projection              -> closed forms (zero weight, identity halves, SiLU
                                         from math.exp), torch linear + chunk(2)
  norm.residual_block_f64            -> explicit float64 composition
  norm.silu_f16                       -> float64 u / (1 + exp(-u)) within two roundings
  norm.res_block3d_f64                -> torch float64 modules (F.layer_norm, F.silu,
                                         F.linear, chunk) + dense F.conv3d per batch
  vae.group_stats_f64 / group_norm_swish / gather_group_norm_swish -> numpy per-group
                                         moments, u / (1 + exp(-u)), element-wise block
  vae.conv_gn_swish_f64 / resnet_f64 / occupancy_f64 -> per-group GroupNorm + dense
                                         F.conv3d(padding=1) over the scattered grid
  geometry.sparse_downsample          -> dictionary grouping by divided coordinates
  vae.children_f64 / child_coords / upsample_f64 -> s*I slot weights, per-child products,
                                         SerializedUnpooling's masked view, inv_grid_coord,
                                         brute-force child table
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import GOLDEN
from oracle import conv as oconv
from oracle import kmap as okmap
from oracle import norm as onorm
from oracle import w8a8 as ow8a8


def _rand_indices(rng, n_side, density, batch=1):
    rows = []
    for b in range(batch):
        xyz = np.argwhere(rng.random((n_side,) * 3) < density)
        rows.append(np.concatenate([np.full((len(xyz), 1), b), xyz], 1))
    idx = np.concatenate(rows).astype(np.int32)
    return idx


# ----------------------------------------------------------------------------- kmap


@pytest.mark.parametrize("ksize", [1, 3, 5])
def test_subm_pairs_matches_brute_force(ksize):
    rng = np.random.default_rng(0)
    idx = _rand_indices(rng, 7, 0.3, batch=2)
    idx = idx[rng.permutation(len(idx))]
    table = okmap.neighbour_table(idx, [7, 7, 7], ksize)
    assert np.array_equal(table, okmap.brute_force_table(idx, [7, 7, 7], ksize))


def test_dense_grid_table_matches_brute_force():
    rng = np.random.default_rng(1)
    idx = _rand_indices(rng, 9, 0.35)
    idx = idx[rng.permutation(len(idx))]
    dense = okmap.neighbour_table_dense(idx[:, 1:])
    assert np.array_equal(dense, okmap.brute_force_table(idx, [9, 9, 9], 3))
    # the extent-agnostic dense grid agrees with the bounded sort-based map
    assert np.array_equal(dense, okmap.neighbour_table(idx, [9, 9, 9], 3))


def _with_edges(idx, side, batch):
    """``idx`` plus every corner, one voxel on each face centre and the grid centre of
    every batch element (deduplicated)."""
    extra = []
    for b in range(batch):
        for x in (0, side - 1):
            for y in (0, side - 1):
                for z in (0, side - 1):
                    extra.append((b, x, y, z))
        m = side // 2
        for face in ((0, m, m), (side - 1, m, m), (m, 0, m), (m, side - 1, m), (m, m, 0), (m, m, side - 1),
                     (m, m, m)):
            extra.append((b, *face))
    allrows = np.concatenate([idx, np.array(extra, np.int32)])
    return np.unique(allrows, axis=0)


@pytest.mark.parametrize("ksize,batch", [(3, 1), (3, 2), (5, 2)])
def test_neighbour_rows_and_sorted_table_match_brute_force(ksize, batch):
    """``neighbour_rows`` (the sampled-row lookup) and ``neighbour_table_sorted`` (the
    full-size table) against the dictionary brute force and the pair-list table, on sets
    with voxels on every corner and face of the grid, two batch elements and ksize 5;
    sampled rows in any order and with repeats."""
    rng = np.random.default_rng(40 + ksize + batch)
    side = 8
    idx = _with_edges(_rand_indices(rng, side, 0.25, batch=batch), side, batch)
    idx = idx[rng.permutation(len(idx))]
    brute = okmap.brute_force_table(idx, [side] * 3, ksize)
    assert np.array_equal(okmap.neighbour_table(idx, [side] * 3, ksize), brute)
    assert np.array_equal(okmap.neighbour_table_sorted(idx, [side] * 3, ksize), brute)
    rows = np.concatenate([rng.permutation(len(idx)), rng.integers(0, len(idx), 17)])
    assert np.array_equal(okmap.neighbour_rows(idx, [side] * 3, rows, ksize), brute[rows])


def test_neighbour_rows_and_sorted_table_with_64bit_keys():
    """Grids whose packed keys exceed 2^62: clusters of voxels near the far corners of a
    [2e6, 2e6, 1e6] grid with two batch elements (keys below 2^63), so keys differ in
    their high bits; both lookups against the brute force, which packs no keys."""
    rng = np.random.default_rng(44)
    shape = [2_000_000, 2_000_000, 1_000_000]
    parts = []
    for corner in ((0, 0, 0), (shape[0] - 6, shape[1] - 6, shape[2] - 6), (shape[0] - 6, 0, shape[2] - 6),
                   (1 << 20, 1 << 19, 1 << 18)):
        xyz = np.argwhere(rng.random((6, 6, 6)) < 0.4) + np.array(corner)
        for b in range(2):
            parts.append(np.concatenate([np.full((len(xyz), 1), b), xyz], 1))
    idx = np.concatenate(parts).astype(np.int64)
    idx = idx[rng.permutation(len(idx))]
    keys = okmap.voxel_keys(idx, shape)
    assert int(keys.max()) > (1 << 62) and int(keys.min()) >= 0
    brute = okmap.brute_force_table(idx, shape, 3)
    assert np.array_equal(okmap.neighbour_table_sorted(idx, shape), brute)
    assert np.array_equal(okmap.neighbour_rows(idx, shape, np.arange(len(idx))), brute)
    assert np.array_equal(okmap.neighbour_table(idx, shape), brute)


def test_pair_layout_invariants():
    """tests/test_backends.py:53-67: coords[dst] == coords[src] + 1 - r and
    counts[k] == counts[26 - k]."""
    data = np.load(GOLDEN / "kmap_8cube.npz")
    idx = data["indices"]
    sources, targets, counts = okmap.subm_pairs(idx, [8, 8, 8])
    coords = idx[:, 1:].astype(np.int64)
    for k in range(27):
        r = np.array([k // 9, (k // 3) % 3, k % 3])
        assert np.array_equal(coords[targets[k]], coords[sources[k]] + 1 - r)
        assert counts[k] == counts[26 - k]
        assert np.all(np.diff(sources[k]) > 0)


def test_pairs_table_round_trip_and_golden():
    data = np.load(GOLDEN / "kmap_8cube.npz")
    idx = data["indices"]
    sources, targets, counts = okmap.subm_pairs(idx, [8, 8, 8])
    table = okmap.table_from_pairs(sources, targets, len(idx))
    assert np.array_equal(table, data["table"])
    src, dst, off = okmap.pairs_from_table(table)
    assert np.array_equal(src, data["src"]) and np.array_equal(dst, data["dst"])
    assert np.array_equal(off, data["offsets"])
    assert np.array_equal(np.concatenate(sources), src) and np.array_equal(np.concatenate(targets), dst)
    assert np.array_equal(counts, data["counts"])


def test_empty_and_single_voxel_maps():
    empty = np.zeros((0, 4), np.int32)
    s, t, c = okmap.subm_pairs(empty, [4, 4, 4])
    assert c.sum() == 0
    one = np.array([[0, 0, 0, 0]], np.int32)
    table = okmap.neighbour_table(one, [1, 1, 1])
    expected = np.full((1, 27), 1, np.int32)
    expected[0, 13] = 0
    assert np.array_equal(table, expected)


def test_stride2_structure_matches_brute_force():
    rng = np.random.default_rng(2)
    idx = _rand_indices(rng, 9, 0.3, batch=2)
    idx = idx[rng.permutation(len(idx))]
    low, inverse, counts, slot, down, up = okmap.stride2_structure(idx)
    parents = sorted({(int(b), int(x) // 2, int(y) // 2, int(z) // 2) for b, x, y, z in idx})
    assert [tuple(r) for r in low.tolist()] == parents
    pos = {p: i for i, p in enumerate(parents)}
    for i, (b, x, y, z) in enumerate(idx.tolist()):
        assert inverse[i] == pos[(b, x // 2, y // 2, z // 2)]
        assert slot[i] == (x & 1) * 4 + (y & 1) * 2 + (z & 1)
        assert down[inverse[i], slot[i]] == i
        assert up[i, slot[i]] == inverse[i] and (up[i] == len(low)).sum() == 7
    assert np.array_equal(counts, np.bincount(inverse, minlength=len(low)))
    # batch-free restatement of downsample_structure agrees on one batch element
    one = idx[idx[:, 0] == 0][:, 1:]
    low3, inv3, cnt3 = okmap.downsample_structure(one)
    exp = sorted({(x // 2, y // 2, z // 2) for x, y, z in one.tolist()})
    assert [tuple(r) for r in low3.tolist()] == exp
    assert np.array_equal(cnt3, np.bincount(inv3, minlength=len(exp)))


def test_child_table_matches_dense_grid_of_children():
    """tests/test_mlx_kernels.py:79-89: the hash-free child table equals the dense-grid
    table of the children's own coordinates."""
    data = np.load(GOLDEN / "child_10cube.npz")
    coords, mask = data["coords"], data["mask"]
    parent_table = okmap.neighbour_table_dense(coords)
    table, parent, slot = okmap.child_neighbour_table(parent_table, mask)
    bits = np.stack([(slot >> 2) & 1, (slot >> 1) & 1, slot & 1], 1)
    child_coords = coords[parent] * 2 + bits
    assert np.array_equal(table, okmap.neighbour_table_dense(child_coords))
    assert np.array_equal(table, data["table"])
    assert np.array_equal(parent, data["parent"]) and np.array_equal(slot, data["slot"])


# ----------------------------------------------------------------------------- conv


def test_subm_conv_matches_dense_conv3d_golden():
    """The reference's own oracle: dense F.conv3d(padding=1) in float64 on the
    14^3 / density 0.15 / C 5->7 recipe (tests/test_backends.py:32-50)."""
    data = np.load(GOLDEN / "subm_14cube.npz")
    idx, feats, w, b = data["indices"], data["feats"], data["weight"], data["bias"]
    dense = oconv.dense_subm_conv3d(idx, feats, w, b, [14, 14, 14])
    assert np.array_equal(dense, data["out"])
    sources, targets, counts = okmap.subm_pairs(idx, [14, 14, 14])
    pairs_out = oconv.subm_conv_pairs(torch.as_tensor(feats), sources, targets, counts, torch.as_tensor(w),
                                      torch.as_tensor(b)).numpy()
    assert np.allclose(pairs_out, dense, atol=1e-12, rtol=1e-12)
    table = okmap.neighbour_table(idx, [14, 14, 14])
    assert np.allclose(oconv.gather_conv_f64(feats, table, w, b), dense, atol=1e-12, rtol=1e-12)


def test_subm_conv_ksize5_matches_dense():
    rng = np.random.default_rng(3)
    idx = _rand_indices(rng, 8, 0.2)
    x = rng.standard_normal((len(idx), 3))
    w = rng.standard_normal((4, 5, 5, 5, 3))
    table = okmap.neighbour_table(idx, [8, 8, 8], 5)
    dense = oconv.dense_subm_conv3d(idx, x, w, None, [8, 8, 8])
    assert np.allclose(oconv.gather_conv_f64(x, table, w), dense, atol=1e-11)


def test_stride2_dense_equivalents():
    """down = F.conv3d(stride 2) at the coarse voxels equals the explicit sum over each
    parent's children; up = F.conv_transpose3d(stride 2) equals W[:, slot] @ y[parent]."""
    data = np.load(GOLDEN / "stride2_12cube.npz")
    idx, x, w, b = data["indices"], data["feats"], data["weight"], data["bias"]
    low, inverse, counts, slot, down, up = okmap.stride2_structure(idx)
    y = oconv.dense_down2(idx, x, w, b, [12, 12, 12], low)
    explicit = np.tile(b, (len(low), 1)).astype(np.float64)
    for i in range(len(idx)):
        s = slot[i]
        explicit[inverse[i]] += w[:, s >> 2, (s >> 1) & 1, s & 1, :] @ x[i]
    assert np.allclose(y, explicit, atol=1e-12)
    assert np.allclose(oconv.gather_conv_f64(x, down, w.reshape(10, 8, 6), b), y, atol=1e-12)
    assert np.array_equal(y, data["down_out"])
    wu, bu = data["up_weight"], data["up_bias"]
    z = oconv.dense_up2(low, y, wu, bu, [6, 6, 6], idx)
    explicit_up = np.stack([wu[:, s >> 2, (s >> 1) & 1, s & 1, :] @ y[inverse[i]] + bu for i, s in enumerate(slot)])
    assert np.allclose(z, explicit_up, atol=1e-11)
    assert np.allclose(oconv.gather_conv_f64(y, up, wu.reshape(6, 8, 10), bu), z, atol=1e-11)
    assert np.array_equal(z, data["up_out"])


def test_gather_mean_matches_scatter_reduce():
    rng = np.random.default_rng(4)
    idx = _rand_indices(rng, 8, 0.4)
    x = rng.standard_normal((len(idx), 5))
    low, inverse, counts, slot, down, up = okmap.stride2_structure(idx)
    ref = torch.zeros(len(low), 5, dtype=torch.float64).scatter_reduce(
        0, torch.as_tensor(inverse, dtype=torch.long)[:, None].expand(-1, 5), torch.as_tensor(x), reduce="mean"
    )
    assert np.allclose(oconv.gather_mean(x, down, extra=1), ref.numpy(), atol=1e-12)


def test_rel_err_statistic():
    ref = np.array([3.0, -4.0])
    assert oconv.rel_err(ref, ref) == 0
    assert abs(oconv.rel_err(ref + [0.0, 0.5], ref) - 0.5 / np.sqrt(12.5)) < 1e-15


# ----------------------------------------------------------------------------- W8A8


def test_signs_golden():
    data = np.load(GOLDEN / "signs.npz")
    for key in data.files:
        k = int(key[1:])
        s = ow8a8.signs(k)
        assert s.dtype == np.float32 and np.array_equal(s, data[key])
        assert set(np.unique(s)) <= {-1.0, 1.0}


def test_h64_matches_hadamard_matrix():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((9, 192)).astype(np.float16)
    sign = ow8a8.signs(192)
    got = ow8a8.rotate_h64(x)
    h = ow8a8.hadamard64()
    xs = x.astype(np.float64) * sign
    ref = np.concatenate([xs[:, 64 * j : 64 * j + 64] @ h.T for j in range(3)], 1)
    assert np.allclose(got, ref, atol=1e-5)
    # orthonormal: the rotation keeps each 64-block's norm
    assert np.allclose(np.linalg.norm(got.reshape(9, 3, 64), axis=2), np.linalg.norm(xs.reshape(9, 3, 64), axis=2), rtol=1e-5)


def test_h64_closed_forms():
    ones = np.ones((1, 64), np.float16)
    mult = np.ones(64, np.float32)
    got = ow8a8.rotate_h64(ones, mult)
    expected = np.zeros(64, np.float32)
    expected[0] = 8.0  # sum of 64 ones / 8
    assert np.array_equal(got[0], expected)
    for j in (0, 5, 33, 63):
        e = np.zeros((1, 64), np.float16)
        e[0, j] = 1
        got = ow8a8.rotate_h64(e, mult)[0]
        p = np.arange(64)
        want = np.array([(-1.0) ** bin(int(pp) & j).count("1") / 8 for pp in p], np.float32)
        assert np.array_equal(got, want)


def test_quantiser_special_rows():
    x = np.zeros((2, 64), np.float16)
    x[1, 3] = 2.0
    q, s = ow8a8.quantize_activation(x, rotation="none")
    assert s[0] == np.float32(1e-8) / np.float32(127) and not q[0].any()
    assert s[1] == np.float32(2.0) / np.float32(127) and q[1, 3] == 127 and (q[1] != 0).sum() == 1
    # half-way values round to even: 0.5 * 127/63.5 ...
    x2 = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, 0.0, 0.0]], np.float16)
    q2, s2 = ow8a8.quantize_activation(x2, rotation="none")
    assert s2[0] == np.float32(1.0)
    assert q2[0].tolist() == [127, 0, 2, 2, 0, -2, 0, 0]


def test_quantiser_codes_within_one_step():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((17, 256)) * 4).astype(np.float16)
    for rotation in ("h64", "none"):
        q, s = ow8a8.quantize_activation(x, rotation=rotation)
        v = ow8a8.rotate_h64(x) if rotation == "h64" else x.astype(np.float32)
        assert np.all(np.abs(q.astype(np.float64) - v / s[:, None].astype(np.float64)) <= 0.5 + 1e-6)
        assert np.abs(q).max() == 127 and q.min() >= -127
        assert np.allclose(s, np.abs(v).max(1) / 127, rtol=1e-7)


def test_integer_gemm_and_epilogue():
    x, w, sw, bias = _w8a8_inputs(65, 131, 2112)
    q, sa = ow8a8.quantize_activation(x)
    acc = ow8a8.int_gemm(q, w)
    assert np.array_equal(acc, (q.astype(np.float64) @ w.astype(np.float64).T).astype(np.int64))
    out = ow8a8.epilogue(acc.astype(np.int32), sa, sw, bias)
    expected = acc.astype(np.float32) * sa[:, None] * sw[None, :] + bias.astype(np.float32)
    np.testing.assert_allclose(out.astype(np.float32), expected, rtol=5e-4, atol=2e-6 + 1e-3 * np.abs(expected).max())


def _w8a8_inputs(rows, cols, width):
    rng = np.random.default_rng(7)
    x = rng.normal(size=(rows, width)).astype(np.float16)
    w = rng.integers(-127, 128, size=(cols, width), dtype=np.int8)
    sw = rng.uniform(0.0001, 0.001, cols).astype(np.float32)
    bias = rng.normal(0, 0.01, cols).astype(np.float16)
    return x, w, sw, bias


def test_w8a8_golden_digests():
    import hashlib

    data = np.load(GOLDEN / "w8a8.npz")
    for rows, cols, width in ((3, 17, 64), (65, 131, 2112), (7, 33, 8448)):
        x, w, sw, bias = _w8a8_inputs(rows, cols, width)
        q, sa = ow8a8.quantize_activation(x)
        tag = f"{rows}_{cols}_{width}"
        assert hashlib.sha256(q.tobytes()).hexdigest() == str(data[f"q_{tag}"])
        assert hashlib.sha256(sa.tobytes()).hexdigest() == str(data[f"s_{tag}"])


# ----------------------------------------------------------------------------- norm / block


def test_layer_norm_matches_float64():
    rng = np.random.default_rng(8)
    x = (rng.standard_normal((40, 2112)) * 3 + 0.5).astype(np.float16)
    got = onorm.layer_norm_modulate(x, 1e-6).astype(np.float64)
    ref = F.layer_norm(torch.as_tensor(x.astype(np.float64)), (2112,), eps=1e-6).numpy()
    assert np.abs(got - ref).max() <= 2e-3  # one fp16 ulp at |y| ~ 4
    scale = (1 + 0.1 * rng.standard_normal(2112)).astype(np.float16)
    shift = (0.1 * rng.standard_normal(2112)).astype(np.float16)
    got = onorm.layer_norm_modulate(x, 1e-6, scale=scale, shift=shift).astype(np.float64)
    want = ref * scale.astype(np.float64) + shift.astype(np.float64)
    assert np.abs(got - want).max() <= 1e-2


def test_layer_norm_golden():
    import hashlib

    data = np.load(GOLDEN / "layer_norm.npz")
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((100, 2112)) * 3 + 0.5).astype(np.float16)
    scale = (1 + 0.1 * rng.standard_normal(2112)).astype(np.float16)
    shift = (0.1 * rng.standard_normal(2112)).astype(np.float16)
    got = onorm.layer_norm_modulate(x, 1e-6, scale=scale, shift=shift)
    assert hashlib.sha256(got.tobytes()).hexdigest() == str(data["mod"])


def test_adaln_projection_closed_forms():
    """adaln_projection pinned by closed forms that a swapped (scale, shift) split, a
    dropped ``1 +`` or a missing bias would fail (chunk order (scale, shift):
    src/hi3d_mac/mlx_backend/transformer.py:413-416, sparc3d_transformer.py:134):
      * W = 0, b = [s; t]        -> (fp16(1 + fp16(s)), fp16(t));
      * W = [I; 0], b = 0         -> (fp16(1 + fp16(cond)), 0);
      * W = [0; I], b = 0         -> (1, fp16(cond));
      * W = [I; 0] with SiLU      -> (fp16(1 + fp16(c / (1 + e^-c))), 0), per element from
        math.exp, with silu(0) = 0;
      * a dense W against torch's linear + chunk(2) in float64."""
    import math

    c, d = 6, 6
    s = np.array([0.5, -0.25, 0.0, 2.0, -1.0, 0.125])
    t = np.array([0.75, -3.0, 0.0625, 1.0, -0.5, 4.0])
    scale1p, shift = onorm.adaln_projection(np.zeros((2 * c, d)), np.concatenate([s, t]), np.ones(d))
    assert scale1p.dtype == np.float16 and shift.dtype == np.float16
    assert np.array_equal(scale1p, (1.0 + s).astype(np.float16))
    assert np.array_equal(shift, t.astype(np.float16))
    cond = np.array([0.1, -0.2, 0.3, 0.0, 5.0, -7.0])
    eye, zero = np.eye(c), np.zeros((c, d))
    scale1p, shift = onorm.adaln_projection(np.vstack([eye, zero]), None, cond)
    want = (np.float32(1.0) + cond.astype(np.float16).astype(np.float32)).astype(np.float16)
    assert np.array_equal(scale1p, want) and np.array_equal(shift, np.zeros(c, np.float16))
    scale1p, shift = onorm.adaln_projection(np.vstack([zero, eye]), np.zeros(2 * c), cond)
    assert np.array_equal(scale1p, np.ones(c, np.float16)) and np.array_equal(shift, cond.astype(np.float16))
    scale1p, shift = onorm.adaln_projection(np.vstack([eye, zero]), None, cond, apply_silu=True)
    silu = np.array([v / (1.0 + math.exp(-v)) for v in cond])
    assert silu[3] == 0.0
    want = (np.float32(1.0) + silu.astype(np.float16).astype(np.float32)).astype(np.float16)
    assert np.array_equal(scale1p, want) and np.array_equal(shift, np.zeros(c, np.float16))
    rng = np.random.default_rng(13)
    w, b, x = rng.standard_normal((2 * c, d)), rng.standard_normal(2 * c), rng.standard_normal(d)
    y = F.linear(torch.as_tensor(x)[None], torch.as_tensor(w), torch.as_tensor(b))
    scale, sh = (v[0].numpy() for v in y.chunk(2, dim=1))
    scale1p, shift = onorm.adaln_projection(w, b, x)
    assert np.array_equal(scale1p, (1.0 + scale.astype(np.float16).astype(np.float32)).astype(np.float16))
    assert np.array_equal(shift, sh.astype(np.float16))


def test_residual_block_composition():
    rng = np.random.default_rng(9)
    idx = _rand_indices(rng, 8, 0.3)
    n, c, d = len(idx), 8, 12
    x = rng.standard_normal((n, c)).astype(np.float16)
    cond = rng.standard_normal(d)
    pw, pb = rng.standard_normal((2 * c, d)) * 0.1, rng.standard_normal(2 * c) * 0.1
    w1, w2 = rng.standard_normal((c, 3, 3, 3, c)) * 0.1, rng.standard_normal((c, 3, 3, 3, c)) * 0.1
    b1, b2 = rng.standard_normal(c) * 0.1, rng.standard_normal(c) * 0.1
    table = okmap.neighbour_table(idx, [8, 8, 8])
    full = onorm.residual_block_f64(x, table, cond, pw, pb, w1, b1, w2, b2)
    rows = np.array([0, 3, n - 1])
    part = onorm.residual_block_f64(x, table, cond, pw, pb, w1, b1, w2, b2, rows=rows)
    assert np.allclose(full[rows], part, atol=1e-12)
    # explicit composition through dense conv3d
    s1p, sh = onorm.adaln_projection(pw, pb, cond)
    xt = torch.as_tensor(x.astype(np.float64))
    h = F.layer_norm(xt, (c,), eps=1e-6).numpy() * s1p.astype(np.float64) + sh.astype(np.float64)
    h1 = oconv.dense_subm_conv3d(idx, h, w1, b1, [8, 8, 8])
    h1 = h1 / (1 + np.exp(-h1))
    ref = oconv.dense_subm_conv3d(idx, h1, w2, b2, [8, 8, 8]) + x.astype(np.float64)
    assert np.allclose(full, ref, atol=1e-10)


def test_silu_f16_against_float64():
    """fp16 SiLU within two fp16 roundings of ``u / (1 + exp(-u))`` (relative half-ulps
    of the product and the sigmoid, plus the sigmoid's absolute subnormal half-ulp
    2^-25 times |u|); exact at 0."""
    u = np.linspace(-12, 12, 4001).astype(np.float16)
    got = onorm.silu_f16(u).astype(np.float64)
    u64 = u.astype(np.float64)
    want = u64 / (1 + np.exp(-u64))
    assert np.all(np.abs(got - want) <= 2 * 2.0**-11 * np.abs(want) + np.abs(u64) * 2.0**-25 + 2.0**-25)
    assert onorm.silu_f16(np.array([0.0]))[0] == 0


@pytest.mark.parametrize("cin,cout,batches", [(16, None, 1), (8, 16, 2)])
def test_res_block3d_oracle_against_torch_modules(cin, cout, batches):
    """res_block3d_f64 against the block written with torch's own float64 operators: a
    dense ``F.conv3d(padding=1)`` per batch element for the submanifold convolutions
    (the reference's conv oracle, tests/test_backends.py:32-50), ``F.layer_norm``,
    ``F.silu``, ``F.linear`` and ``chunk(2)`` of the embedding projection
    (sparc3d_transformer.py:132-144)."""
    rng = np.random.default_rng(70 + cin)
    side = 8
    idx = _rand_indices(rng, side, 0.3, batch=batches)
    spans, start = [], 0
    for b in range(batches):
        count = int((idx[:, 0] == b).sum())
        spans.append(slice(start, start + count))
        start += count
    n = len(idx)
    cout = cout or cin
    hidden = cout // 2
    p = {
        "norm1.weight": rng.uniform(0.5, 1.5, cin), "norm1.bias": rng.normal(0, 0.2, cin),
        "conv1.conv.weight": rng.normal(0, 0.1, (hidden, 3, 3, 3, cin)), "conv1.conv.bias": rng.normal(0, 0.1, hidden),
        "conv2.conv.weight": rng.normal(0, 0.1, (hidden, 3, 3, 3, hidden)),
        "conv2.conv.bias": rng.normal(0, 0.1, hidden),
        "linear.weight": rng.normal(0, 0.3, (cout, hidden)), "linear.bias": rng.normal(0, 0.1, cout),
        "emb_layers.1.weight": rng.normal(0, 0.3, (2 * hidden, 12)), "emb_layers.1.bias": rng.normal(0, 0.1, 2 * hidden),
    }
    if cout != cin:
        p["skip_connection.weight"] = rng.normal(0, 0.3, (cout, cin))
        p["skip_connection.bias"] = rng.normal(0, 0.1, cout)
    x = rng.normal(0.3, 1.2, (n, cin))
    emb = rng.normal(size=(batches, 12))
    table = okmap.neighbour_table(idx, [side] * 3)
    got = onorm.res_block3d_f64(x, table, emb, p, spans)

    t = {k: torch.as_tensor(v) for k, v in p.items()}

    def conv(v, w, b):
        return torch.as_tensor(oconv.dense_subm_conv3d(idx, v.numpy(), w.numpy(), b.numpy(), [side] * 3))

    xt = torch.as_tensor(x)
    y = F.linear(F.silu(torch.as_tensor(emb)), t["emb_layers.1.weight"], t["emb_layers.1.bias"])
    scale, shift = y.chunk(2, dim=1)
    h = F.silu(F.layer_norm(xt, (cin,), t["norm1.weight"], t["norm1.bias"], eps=1e-6))
    h = conv(h, t["conv1.conv.weight"], t["conv1.conv.bias"])
    h = F.layer_norm(h, (hidden,), eps=1e-6)
    batch = torch.as_tensor(idx[:, 0]).long()
    h = F.silu(h * (1 + scale[batch]) + shift[batch])
    h = F.silu(conv(h, t["conv2.conv.weight"], t["conv2.conv.bias"]))
    skip = F.linear(xt, t["skip_connection.weight"], t["skip_connection.bias"]) if cout != cin else xt
    want = (F.linear(h, t["linear.weight"], t["linear.bias"]) + skip).numpy()
    assert np.allclose(got, want, rtol=1e-10, atol=1e-10)


def test_cpu_baseline_runs_on_a_sample():
    """The timed CPU baseline (reference CPU fallback) runs and its conv equals the
    float64 gather sum over the same pairs."""
    from oracle import baseline

    rng = np.random.default_rng(4)
    idx = _rand_indices(rng, 10, 0.3)
    r = baseline.time_subm_conv(idx, [10] * 3, 8, 6, repeats=1, max_rows=200, threads=1)
    assert r["rows"] == 200 and r["conv_s"] > 0 and r["torch_threads"] >= 1
    feats = rng.standard_normal((len(idx), 8)).astype(np.float32)
    weight = (rng.standard_normal((6, 3, 3, 3, 8)) / 10).astype(np.float32)
    pairs = baseline.kernel_map(torch.as_tensor(idx), [10] * 3)
    got = baseline.subm_conv(torch.as_tensor(feats), *pairs, torch.as_tensor(weight), None).numpy()
    table = okmap.neighbour_table(idx, [10] * 3)
    ref = oconv.gather_conv_f64(feats, table, weight.reshape(6, 27, 8))
    assert oconv.rel_err(got, ref) <= 1e-5
    # the sampled-row form: the sample's part of the full map, queried from the output
    # side, gives the same pair sets, and the conv of those rows equals the full conv's
    n = len(idx)
    sample = torch.as_tensor(rng.permutation(n)[:150])
    full = baseline.restrict_to_rows(pairs[0], pairs[1], n, sample)
    part = baseline.kernel_map_rows(torch.as_tensor(idx), [10] * 3, sample)
    for k in range(27):
        assert sorted(zip(full[0][k].tolist(), full[1][k].tolist())) == sorted(
            zip(part[0][k].tolist(), part[1][k].tolist()))
    rows = baseline.subm_conv_rows(torch.as_tensor(feats), *part, torch.as_tensor(weight), None, sample).numpy()
    assert oconv.rel_err(rows, ref[sample.numpy()]) <= 1e-5
    r = baseline.time_resblock(idx, [10] * 3, 8, 12, sample_rows=100, repeats=1, threads=1)
    assert r["sample_rows"] == 100 and r["rows"] == n and r["block_s"] > 0


def test_vae_group_stats_oracle_against_numpy_moments():
    """group_stats_f64 against per-group numpy mean / variance of the consecutive-channel
    groups (the divisor n w + eps differs from n w by 1e-6 / (n w)); group counts of
    PointGroupNorm (vae.py:152)."""
    from oracle import vae as ovae

    assert [ovae.groups_for(c) for c in (32, 64, 96, 128, 256, 512)] == [8, 16, 24, 32, 32, 32]
    rng = np.random.default_rng(21)
    for c in (64, 256):
        x = rng.normal(0.7, 2.0, (1500, c))
        mean, inv = ovae.group_stats_f64(x)
        g = ovae.groups_for(c)
        w = c // g
        for k in range(g):
            blk = x[:, k * w:(k + 1) * w]
            assert np.allclose(mean[k * w:(k + 1) * w], blk.mean(), rtol=1e-9, atol=0)
            assert np.allclose(inv[k * w:(k + 1) * w], 1 / np.sqrt(blk.var() + 1e-6), rtol=1e-8, atol=0)


def test_vae_swish_form_and_gathered_block():
    """The reference's sigmoid form equals the textbook u / (1 + exp(-u)); swish(0) = 0,
    swish(u) -> u for large u and -> 0 for very negative u; the gathered block puts the
    activation of row table[o, k] at columns k C .. k C + C - 1 and zeros for absent."""
    from oracle import vae as ovae

    u = np.linspace(-60.0, 60.0, 2401)
    assert np.allclose(ovae.swish_reference_form(u), u / (1.0 + np.exp(-u)), rtol=1e-12, atol=1e-300)
    assert ovae.swish_reference_form(np.array([0.0]))[0] == 0.0
    assert abs(ovae.swish_reference_form(np.array([40.0]))[0] - 40.0) < 1e-12
    assert abs(ovae.swish_reference_form(np.array([-40.0]))[0]) < 1e-15
    rng = np.random.default_rng(22)
    n, c = 11, 8
    x = rng.normal(size=(n, c))
    mean, inv, w, b = rng.normal(size=c), rng.uniform(0.5, 2, c), rng.normal(size=c), rng.normal(size=c)
    table = rng.integers(0, n + 1, (5, 3))
    blk = ovae.gather_group_norm_swish(x, table, mean, inv, w, b)
    for o in range(5):
        for k in range(3):
            r = table[o, k]
            want = np.zeros(c) if r == n else ovae.swish_reference_form(((x[r] - mean) * inv) * w + b)
            assert np.array_equal(blk[o, k * c:(k + 1) * c], want)


def test_vae_children_oracle_slot_layout():
    """The child projection oracle against three independent forms: a weight stacking
    ``s * I`` per slot gives ``slot * x[parent]`` (a transposed or reordered block layout
    fails this), a per-child product with that slot's ``[C, C]`` block, and
    SerializedUnpooling's own masking of the full projection ``feat.view(8P, C)[mask]``
    (src/sparc3d/models/autoencoders/blocks.py:535-543) with the mask flattened
    parent-major."""
    from oracle import vae as ovae

    rng = np.random.default_rng(31)
    p, c = 9, 6
    x = rng.integers(-4, 5, size=(p, c)).astype(np.float64)
    mask = rng.random((p, 8)) < 0.5
    table = rng.integers(0, p + 1, (p, 27)).astype(np.int32)
    _, parent, slot = okmap.child_neighbour_table(table, mask)
    eye = np.concatenate([s * np.eye(c) for s in range(8)])
    got = ovae.children_f64(x, parent, slot, eye)
    assert np.array_equal(got, slot[:, None] * x[parent])
    w = rng.normal(size=(8 * c, c))
    got = ovae.children_f64(x, parent, slot, w)
    for i in range(parent.size):
        s = slot[i]
        assert np.allclose(got[i], w[s * c:(s + 1) * c] @ x[parent[i]], rtol=1e-13, atol=1e-13)
    feat = x @ w.T
    assert np.array_equal(feat.reshape(p * 8, c)[mask.reshape(-1)], got)


def _vae_params(rng, name, cin, cout, res_conv=False, head=False):
    """Random decoder parameters under the reference's key names (vae.py:166-218,
    270-271): GroupNorm ``weights``/``bias`` and conv ``weight [27 Cin, Cout]``/``bias``."""
    p = {}
    pairs = [("cls_head.fc.0", "cls_head.fc.2", cin, cout)] if head else \
        [("block.0", "block.2", cin, cout), ("block.3", "block.5", cout, cout)]
    for norm, conv, ci, co in pairs:
        p[f"{name}.{norm}.weights"] = rng.uniform(0.5, 1.5, ci)
        p[f"{name}.{norm}.bias"] = rng.normal(0, 0.3, ci)
        p[f"{name}.{conv}.weight"] = rng.normal(0, 1 / np.sqrt(27 * ci), (27 * ci, co))
        p[f"{name}.{conv}.bias"] = rng.normal(0, 0.1, co)
    if res_conv:
        p[f"{name}.res_conv.weight"] = rng.normal(0, 1 / np.sqrt(cin), (cout, cin))
        p[f"{name}.res_conv.bias"] = rng.normal(0, 0.1, cout)
    return p


def _independent_gn_swish(x, weight, bias, eps=1e-6):
    """GroupNorm + swish written out per group: per-group sums with the reference's
    divisor ``n * width + eps`` (vae.py:153-164), then ``u / (1 + exp(-u))``."""
    from oracle import vae as ovae

    n, c = x.shape
    g = ovae.groups_for(c)
    w = c // g
    u = np.empty_like(x)
    for k in range(g):
        blk = x[:, k * w:(k + 1) * w]
        cnt = n * w + eps
        mean = blk.sum() / cnt
        var = (blk * blk).sum() / cnt - mean * mean
        u[:, k * w:(k + 1) * w] = (blk - mean) / np.sqrt(var + eps)
    u = u * weight + bias
    return u / (1.0 + np.exp(-u))


def _dense_conv_wt(a, xyz, weight_t, bias, side):
    """3x3x3 convolution of the rows ``a`` at ``xyz`` by ``F.conv3d(padding=1)`` over the
    scattered dense grid, with ``W_t`` row ``k Cin + ci`` (k = 9 kx + 3 ky + kz) as tap
    ``(kx, ky, kz)`` of input channel ci (sparse.py:185-189)."""
    cin = a.shape[1]
    cout = weight_t.shape[1]
    vol = torch.zeros((1, cin, side, side, side), dtype=torch.float64)
    x, y, z = (torch.as_tensor(xyz[:, i]).long() for i in range(3))
    vol[0, :, x, y, z] = torch.as_tensor(a).T
    w = torch.as_tensor(weight_t).reshape(3, 3, 3, cin, cout).permute(4, 3, 0, 1, 2)
    out = F.conv3d(vol, w, padding=1)[0][:, x, y, z].T.numpy()
    return out + bias


def test_vae_compositions_against_dense_conv3d():
    """conv_gn_swish_f64, resnet_f64 (identity and projected shortcuts) and occupancy_f64
    against an independent composition: per-group GroupNorm with the reference's
    divisor, ``u / (1 + exp(-u))`` and a dense ``F.conv3d(padding=1)`` over the scattered
    grid (src/hi3d_mac/mlx_backend/vae.py:141-218, 270-271;
    tests/test_mlx_kernels.py:63-76,124-150)."""
    from oracle import vae as ovae

    rng = np.random.default_rng(60)
    side = 9
    idx = _rand_indices(rng, side, 0.3)
    idx = idx[rng.permutation(len(idx))]
    xyz = idx[:, 1:]
    table = okmap.neighbour_table(idx, [side] * 3)
    n = len(idx)
    for cin, cout, res in ((16, 16, False), (16, 32, True)):
        p = _vae_params(rng, "blk", cin, cout, res_conv=res)
        x = rng.normal(0.4, 1.7, (n, cin))
        f = lambda k: p[f"blk.{k}"]
        a = _independent_gn_swish(x, f("block.0.weights"), f("block.0.bias"))
        h = _dense_conv_wt(a, xyz, f("block.2.weight"), f("block.2.bias"), side)
        got = ovae.conv_gn_swish_f64(x, table, f("block.0.weights"), f("block.0.bias"), f("block.2.weight"),
                                     f("block.2.bias"))
        assert np.allclose(got, h, rtol=1e-10, atol=1e-10)
        shortcut = x @ f("res_conv.weight").T + f("res_conv.bias") if res else x
        want = shortcut + _dense_conv_wt(_independent_gn_swish(h, f("block.3.weights"), f("block.3.bias")), xyz,
                                         f("block.5.weight"), f("block.5.bias"), side)
        assert np.allclose(ovae.resnet_f64(x, table, p, "blk"), want, rtol=1e-10, atol=1e-10)
    head = _vae_params(rng, "up", 16, 8, head=True)
    x = rng.normal(size=(n, 16))
    want = _dense_conv_wt(_independent_gn_swish(x, head["up.cls_head.fc.0.weights"], head["up.cls_head.fc.0.bias"]),
                          xyz, head["up.cls_head.fc.2.weight"], head["up.cls_head.fc.2.bias"], side)
    assert np.allclose(ovae.occupancy_f64(x, table, head, "up"), want, rtol=1e-10, atol=1e-10)


def test_vae_upsample_oracle_against_brute_force_children():
    """upsample_f64 against an independent construction: the mask ``logits > 0`` of the
    dense-conv occupancy, the kept children enumerated parent-major and slot-minor, each
    child's features as its slot's ``[C, C]`` block times its parent's row, coordinates
    ``2 p + (s>>2&1, s>>1&1, s&1)``, and the children's table by dictionary brute force
    over their own coordinates (vae.py:220-244,316-327; blocks.py:526-543)."""
    from oracle import vae as ovae

    rng = np.random.default_rng(61)
    side, c = 7, 8
    idx = _rand_indices(rng, side, 0.3)
    idx = idx[rng.permutation(len(idx))]
    xyz = idx[:, 1:]
    table = okmap.neighbour_table(idx, [side] * 3)
    n = len(idx)
    p = _vae_params(rng, "up", c, 8, head=True)
    p["up.proj.weight"] = rng.normal(0, 1 / np.sqrt(c), (8 * c, c))
    x = rng.normal(size=(n, c))
    logits = _dense_conv_wt(_independent_gn_swish(x, p["up.cls_head.fc.0.weights"], p["up.cls_head.fc.0.bias"]),
                            xyz, p["up.cls_head.fc.2.weight"], p["up.cls_head.fc.2.bias"], side)
    feats, ccoords, ctable, parent, slot, mask = ovae.upsample_f64(x, xyz, table, p, "up")
    assert np.array_equal(mask, logits > 0) and 0 < mask.sum() < mask.size
    kept = [(i, s) for i in range(n) for s in range(8) if logits[i, s] > 0]
    assert parent.tolist() == [i for i, _ in kept] and slot.tolist() == [s for _, s in kept]
    w = p["up.proj.weight"]
    for j, (i, s) in enumerate(kept):
        assert np.allclose(feats[j], w[s * c:(s + 1) * c] @ x[i], rtol=1e-12, atol=1e-12)
        bits = np.array([(s >> 2) & 1, (s >> 1) & 1, s & 1])
        assert np.array_equal(ccoords[j], 2 * xyz[i] + bits)
    cidx = np.concatenate([np.zeros((len(kept), 1), np.int64), ccoords], 1)
    assert np.array_equal(ctable, okmap.brute_force_table(cidx, [2 * side] * 3, 3))
    # a given mask is used as is
    given = rng.random((n, 8)) < 0.3
    out = ovae.upsample_f64(x, xyz, table, p, "up", mask=given)
    assert np.array_equal(out[5], given) and len(out[3]) == int(given.sum())


def test_vae_child_coords_match_unpooling_grid():
    """Child coordinates against SerializedUnpooling's ``inv_grid_coord`` table
    (src/sparc3d/models/autoencoders/blocks.py:526-533): ``coords * 2 + inv_grid[slot]``."""
    from oracle import vae as ovae

    inv_grid = np.array([[0, 0, 0], [0, 0, 1], [0, 1, 0], [0, 1, 1], [1, 0, 0], [1, 0, 1], [1, 1, 0], [1, 1, 1]])
    rng = np.random.default_rng(32)
    coords = rng.integers(0, 50, (20, 3)).astype(np.int32)
    parent = rng.integers(0, 20, 40)
    slot = rng.integers(0, 8, 40)
    assert np.array_equal(ovae.child_coords(coords, parent, slot), coords[parent] * 2 + inv_grid[slot])


@pytest.mark.parametrize("factor", [(2, 2, 2), (3, 3, 3), (2, 3, 4), (1, 1, 1), (5, 1, 2)])
def test_sparse_downsample_oracle_against_grouping(factor):
    """sparse_downsample against a dictionary grouping of the rows by
    ``(b, x // fx, y // fy, z // fz)``: coarse rows in sorted order, each one's mean over
    its rows and one extra zero, every fine row's parent; two batch elements."""
    from oracle import geometry as ogeo

    rng = np.random.default_rng(sum(factor))
    idx = _rand_indices(rng, 9, 0.2, batch=2)
    idx = idx[rng.permutation(len(idx))]
    x = rng.normal(size=(len(idx), 5))
    low, pooled, inverse = ogeo.sparse_downsample(idx, x, factor)
    groups = {}
    for i, (b, px, py, pz) in enumerate(idx.tolist()):
        groups.setdefault((b, px // factor[0], py // factor[1], pz // factor[2]), []).append(i)
    keys = sorted(groups)
    assert low.tolist() == [list(k) for k in keys]
    for c, k in enumerate(keys):
        rows = groups[k]
        assert np.allclose(pooled[c], x[rows].sum(0) / (len(rows) + 1), rtol=1e-13, atol=1e-13)
        assert all(inverse[r] == c for r in rows)


def test_unique_oracle_against_numpy_and_torch():
    """The unique oracle against ``np.unique`` (keys: negatives, duplicates, the int64
    extremes, empty) and against ``torch.unique(dim=0)`` on the reference test's rows
    (tests/test_backends.py:182-190: 20000 x 3 in [-5, 40), generator seed 0)."""
    from oracle import unique as ounique

    rng = np.random.default_rng(41)
    keys = np.concatenate([rng.integers(-1000, 1000, 5000), [np.iinfo(np.int64).min, np.iinfo(np.int64).max, 0]])
    for counts in (False, True):
        got = ounique.unique_keys(keys, return_counts=counts)
        ref = np.unique(keys, return_inverse=True, return_counts=counts)
        assert np.array_equal(got[0], ref[0]) and np.array_equal(got[1], ref[1])
        if counts:
            assert np.array_equal(got[2], ref[2])
        empty = ounique.unique_keys(np.empty(0, np.int64), return_counts=counts)
        ref = np.unique(np.empty(0, np.int64), return_inverse=True, return_counts=counts)
        assert np.array_equal(empty[0], ref[0]) and np.array_equal(empty[1], ref[1])
        assert (empty[2] is None) == (not counts)
    g = torch.Generator().manual_seed(0)
    rows = torch.randint(-5, 40, (20000, 3), generator=g)
    ref = torch.unique(rows, dim=0, return_inverse=True, return_counts=True)
    got = ounique.unique_rows(rows.numpy(), return_inverse=True, return_counts=True)
    for a, b in zip(ref, got):
        assert np.array_equal(a.numpy(), b)
    assert ounique.packed_keys(np.array([[0, 0], [2**40, 2**30]])) is None


def test_geometry_oracle_up_conv_is_conv_of_upsampled():
    """The reference's projection form of the up block's first convolution equals a
    dense ``F.conv3d(padding=1)`` of the upsampled volume (float64, 12^3 grid), and the
    mean pool equals ``scatter_reduce(mean, include_self)`` onto zeros."""
    from oracle import geometry as ogeo

    rng = np.random.default_rng(51)
    side = 12
    idx = np.argwhere(rng.random((side,) * 3) < 0.3).astype(np.int32)
    n = len(idx)
    table = okmap.neighbour_table_dense(idx)
    low, inverse = np.unique(idx // 2, axis=0, return_inverse=True)
    inverse = inverse.reshape(-1)
    n_low = len(low)
    cin, cout = 5, 3
    h = rng.normal(size=(n_low, cin))
    w = rng.normal(size=(cout, 27 * cin))
    b = rng.normal(size=cout)
    got = ogeo.up_conv_f64(h, table, inverse, w, b)
    up = ogeo.upsample(h, inverse)
    dense = torch.zeros((1, cin, side, side, side), dtype=torch.float64)
    dense[0, :, idx[:, 0], idx[:, 1], idx[:, 2]] = torch.as_tensor(up.T)
    wt = torch.as_tensor(w.reshape(cout, 3, 3, 3, cin)).permute(0, 4, 1, 2, 3)
    ref = F.conv3d(dense, wt, torch.as_tensor(b), padding=1)[0][:, idx[:, 0], idx[:, 1], idx[:, 2]].T.numpy()
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
    x = rng.normal(size=(n, 4))
    pooled = torch.zeros((n_low, 4), dtype=torch.float64).scatter_reduce(
        0, torch.as_tensor(inverse)[:, None].expand(-1, 4), torch.as_tensor(x), reduce="mean", include_self=True)
    assert np.allclose(ogeo.downsample_f64(x, inverse, n_low), pooled.numpy(), rtol=1e-12, atol=1e-12)
