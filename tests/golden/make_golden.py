"""Write the committed golden fixtures of the test suite (run from the repo root:
``python tests/golden/make_golden.py``).

Inputs follow the seeded recipes of the reference's own tests where they exist
(tests/test_backends.py:21-29 ``_random_sparse``; tests/test_mlx_kernels.py:79-89;
tests/test_w8a8_inference.py:8-20); expected outputs come from the oracle, whose
functions are pinned independently in tests/test_oracle.py (dense ``F.conv3d``, brute
force, closed forms). Larger arrays are stored as SHA-256 digests.
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from oracle import conv as oconv  # noqa: E402
from oracle import kmap as okmap  # noqa: E402
from oracle import norm as onorm  # noqa: E402
from oracle import w8a8 as ow8a8  # noqa: E402

SIGN_WIDTHS = (64, 128, 1024, 2112, 4096, 8448)
W8A8_SHAPES = ((3, 17, 64), (65, 131, 2112), (7, 33, 8448))


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def random_sparse(n_side=14, density=0.15, channels=5, seed=0):
    """The reference test's input recipe (tests/test_backends.py:21-29)."""
    g = torch.Generator().manual_seed(seed)
    occ = torch.rand(n_side, n_side, n_side, generator=g) < density
    xyz = occ.nonzero().int()
    perm = torch.randperm(xyz.shape[0], generator=g)
    xyz = xyz[perm]
    feats = torch.randn(xyz.shape[0], channels, generator=g, dtype=torch.float64)
    indices = torch.cat([torch.zeros(xyz.shape[0], 1, dtype=torch.int32), xyz], 1)
    return indices.numpy(), feats.numpy()


def w8a8_inputs(rows, columns, width):
    """The reference test's input recipe (tests/test_w8a8_inference.py:10-14)."""
    rng = np.random.default_rng(7)
    x = rng.normal(size=(rows, width)).astype(np.float16)
    w = rng.integers(-127, 128, size=(columns, width), dtype=np.int8)
    sw = rng.uniform(0.0001, 0.001, columns).astype(np.float32)
    bias = rng.normal(0, 0.01, columns).astype(np.float16)
    return x, w, sw, bias


def ln_inputs(seed=5, rows=100, c=2112):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, c)) * 3 + 0.5).astype(np.float16)
    scale = (1 + 0.1 * rng.standard_normal(c)).astype(np.float16)
    shift = (0.1 * rng.standard_normal(c)).astype(np.float16)
    w = rng.standard_normal(c).astype(np.float32)
    b = rng.standard_normal(c).astype(np.float32)
    return x, scale, shift, w, b


def child_inputs():
    """The reference test's recipe (tests/test_mlx_kernels.py:80-84)."""
    rng = np.random.default_rng(1)
    occ = rng.random((10, 10, 10)) < 0.35
    coords = np.argwhere(occ).astype(np.int32)
    mask = rng.random((len(coords), 8)) < 0.5
    return coords, mask


def stride2_inputs(seed=3, n_side=12, density=0.3, cin=6, cout=10):
    rng = np.random.default_rng(seed)
    occ = rng.random((n_side,) * 3) < density
    xyz = np.argwhere(occ)
    xyz = xyz[rng.permutation(len(xyz))]
    idx = np.concatenate([np.zeros((len(xyz), 1), np.int64), xyz], 1).astype(np.int32)
    x = rng.standard_normal((len(idx), cin))
    w = rng.standard_normal((cout, 2, 2, 2, cin))
    b = rng.standard_normal(cout)
    return idx, x, w, b


def main() -> None:
    np.savez_compressed(HERE / "signs.npz", **{f"k{k}": ow8a8.signs(k) for k in SIGN_WIDTHS})

    idx8, _ = random_sparse(n_side=8, density=0.4)
    table8 = okmap.brute_force_table(idx8, [8, 8, 8])
    src, dst, off = okmap.pairs_from_table(table8)
    np.savez_compressed(HERE / "kmap_8cube.npz", indices=idx8, table=table8, src=src, dst=dst, offsets=off,
                        counts=np.diff(off).astype(np.int32))

    idx14, feats14 = random_sparse()
    rng = np.random.default_rng(11)
    w14 = rng.standard_normal((7, 3, 3, 3, 5))
    b14 = rng.standard_normal(7)
    out14 = oconv.dense_subm_conv3d(idx14, feats14, w14, b14, [14, 14, 14])
    np.savez_compressed(HERE / "subm_14cube.npz", indices=idx14, feats=feats14, weight=w14, bias=b14, out=out14)

    w8 = {}
    for rows, cols, width in W8A8_SHAPES:
        x, w, sw, bias = w8a8_inputs(rows, cols, width)
        q, sa = ow8a8.quantize_activation(x)
        acc = ow8a8.int_gemm(q, w).astype(np.int32)
        out = ow8a8.epilogue(acc, sa, sw, bias)
        tag = f"{rows}_{cols}_{width}"
        w8[f"q_{tag}"] = digest(q)
        w8[f"s_{tag}"] = digest(sa)
        w8[f"acc_{tag}"] = digest(acc)
        w8[f"out_{tag}"] = digest(out)
        if rows * width <= 4096:
            w8[f"qarr_{tag}"] = q
            w8[f"sarr_{tag}"] = sa
            w8[f"outarr_{tag}"] = out
    np.savez_compressed(HERE / "w8a8.npz", **w8)

    x, scale, shift, w, b = ln_inputs()
    ln = {
        "mod": digest(onorm.layer_norm_modulate(x, 1e-6, scale=scale, shift=shift)),
        "affine": digest(onorm.layer_norm_modulate(x, 1e-6, weight=w, bias=b)),
        "plain": digest(onorm.layer_norm_modulate(x, 1e-6)),
        "mod_head": onorm.layer_norm_modulate(x[:2], 1e-6, scale=scale, shift=shift),
    }
    np.savez_compressed(HERE / "layer_norm.npz", **ln)

    coords, mask = child_inputs()
    parent_table = okmap.neighbour_table_dense(coords)
    table, parent, slot = okmap.child_neighbour_table(parent_table, mask)
    np.savez_compressed(HERE / "child_10cube.npz", coords=coords, mask=mask, table=table, parent=parent, slot=slot)

    idx, x, w, b = stride2_inputs()
    low, inverse, counts, slot, down, up = okmap.stride2_structure(idx)
    y = oconv.dense_down2(idx, x, w, b, [12, 12, 12], low)
    wu = np.random.default_rng(4).standard_normal((6, 2, 2, 2, 10))
    bu = np.random.default_rng(5).standard_normal(6)
    z = oconv.dense_up2(low, y, wu, bu, [6, 6, 6], idx)
    np.savez_compressed(HERE / "stride2_12cube.npz", indices=idx, feats=x, weight=w, bias=b, low=low,
                        inverse=inverse, counts=counts, slot=slot, down_out=y, up_weight=wu, up_bias=bu, up_out=z)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
