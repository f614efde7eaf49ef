"""Seeded synthetic inputs of the five benchmark workloads of the sparse hot path.

The active sets are voxel shells:

* ``sphere_shell``: every voxel of an ``n^3`` grid whose centre ``idx + 0.5`` lies at
  distance ``r`` from the grid centre ``n/2`` with ``|r - radius| < 0.5``
  (the shell generator of the reference's ``tests/test_backends.py:145-147`` uses the
  same voxel-centre convention).
* ``ellipsoid_shells``: the union of the surface shells of 8 seeded axis-aligned
  ellipsoids (semi-axes U(20, 100), centres U(0, 256)^3, both multiplied by ``scale``),
  on a ``(256*scale)^3`` grid. A voxel centre ``p`` belongs to the shell of thickness
  ``t`` when its first-order distance to the surface is below ``t/2``:
  ``|r_e(p) - 1| / |grad r_e(p)| < t/2`` with ``r_e(p) = |(p - c) / a|``.

Both return ``int32 [N, 4]`` ``(batch=0, x, y, z)`` coordinates, deduplicated and in a
seeded random row order, as real sparse tensors arrive.

The evaluation only visits 8^3 blocks that can hold shell voxels. ``r_e`` is
Lipschitz with constant ``1 / a_min`` and ``|grad r_e| <= 1 / a_min``, so a block whose
centre ``q`` satisfies ``|r_e(q) - 1| > (t/2 + h) / a_min`` (``h`` the block's
half-diagonal) holds none; the pruning is exact, not a heuristic.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

_BLOCK = 8


def sphere_shell(n: int = 128, radius: float = 60.0, seed: int = 1) -> np.ndarray:
    """Workload 1's active set: 1-voxel spherical shell (``N = 45,128`` for the defaults)."""
    idx = np.stack(np.meshgrid(*[np.arange(n)] * 3, indexing="ij"), -1).reshape(-1, 3)
    r = np.linalg.norm(idx + 0.5 - n / 2, axis=1)
    xyz = idx[np.abs(r - radius) < 0.5]
    return _finish(xyz, n, seed)


def ellipsoid_params(seed: int, count: int = 8, scale: int = 1) -> tuple[np.ndarray, np.ndarray]:
    """``(axes [count, 3], centres [count, 3])`` of the seeded ellipsoids, scaled."""
    rng = np.random.default_rng(seed)
    axes = rng.uniform(20.0, 100.0, size=(count, 3))
    centres = rng.uniform(0.0, 256.0, size=(count, 3))
    return axes * scale, centres * scale


def _shell_of(axes, centre, n, thickness, device, chunk_blocks=8192):
    a = torch.tensor(axes, dtype=torch.float64, device=device)
    c = torch.tensor(centre, dtype=torch.float64, device=device)
    lo = np.maximum(np.floor(centre - axes - thickness - 1).astype(np.int64), 0)
    hi = np.minimum(np.ceil(centre + axes + thickness + 1).astype(np.int64), n)
    if np.any(hi <= lo):
        return torch.empty((0, 3), dtype=torch.int64, device=device)
    blo = lo // _BLOCK
    bhi = (hi + _BLOCK - 1) // _BLOCK
    axes_b = [torch.arange(int(blo[i]), int(bhi[i]), device=device, dtype=torch.int64) for i in range(3)]
    bx, by, bz = torch.meshgrid(*axes_b, indexing="ij")
    blocks = torch.stack([bx.reshape(-1), by.reshape(-1), bz.reshape(-1)], 1)
    q = blocks.double() * _BLOCK + _BLOCK / 2.0  # centre of the block's voxel centres
    re = torch.linalg.norm((q - c) / a, dim=1)
    half_diag = (_BLOCK - 1) * math.sqrt(3.0) / 2.0
    a_min = float(np.min(axes))
    keep = (re - 1.0).abs() <= (thickness / 2.0 + half_diag) / a_min + 1e-9
    blocks = blocks[keep]
    inner = torch.stack(
        torch.meshgrid(*[torch.arange(_BLOCK, device=device, dtype=torch.int64)] * 3, indexing="ij"), -1
    ).reshape(-1, 3)
    out = []
    for s in range(0, blocks.shape[0], chunk_blocks):
        idx = (blocks[s : s + chunk_blocks, None, :] * _BLOCK + inner[None]).reshape(-1, 3)
        idx = idx[((idx >= 0) & (idx < n)).all(1)]
        p = idx.double() + 0.5
        d = (p - c) / a
        re = torch.linalg.norm(d, dim=1)
        g = torch.linalg.norm(d / a, dim=1)  # |grad r_e| * r_e
        # |r_e - 1| / |grad r_e| = |r_e - 1| * r_e / |d / a|
        dist = (re - 1.0).abs() * re / g.clamp_min(1e-300)
        out.append(idx[dist < thickness / 2.0])
    return torch.cat(out) if out else torch.empty((0, 3), dtype=torch.int64, device=device)


def ellipsoid_shells(
    seed: int = 0, scale: int = 1, thickness: float = 2.0, count: int = 8, device: str | torch.device = "cpu"
) -> np.ndarray:
    """Union of ``count`` seeded ellipsoid shells on a ``(256*scale)^3`` grid."""
    n = 256 * scale
    axes, centres = ellipsoid_params(seed, count, scale)
    parts = [_shell_of(axes[i], centres[i], n, thickness, device) for i in range(count)]
    xyz = torch.cat(parts)
    keys = torch.unique((xyz[:, 0] * n + xyz[:, 1]) * n + xyz[:, 2]).cpu().numpy()
    xyz = np.stack([keys // (n * n), (keys // n) % n, keys % n], 1)
    return _finish(xyz, n, seed)


def _finish(xyz: np.ndarray, n: int, seed: int) -> np.ndarray:
    order = np.random.default_rng(seed + 1000).permutation(xyz.shape[0])
    xyz = np.asarray(xyz, dtype=np.int32)[order]
    coords = np.zeros((xyz.shape[0], 4), dtype=np.int32)
    coords[:, 1:] = xyz
    return coords


@dataclass(frozen=True)
class Workload:
    """Sizes and generator of one benchmark workload."""

    name: str
    grid: int
    description: str


WORKLOADS = {
    "subm3_c64_fp32": Workload("subm3_c64_fp32", 128, "submanifold 3x3x3, C 64->64, fp32, 128^3 sphere shell R=60"),
    "subm3_c128_fp16": Workload(
        "subm3_c128_fp16", 256, "submanifold 3x3x3, C 128->128, fp16, 256^3 union of 8 ellipsoid 2-voxel shells"
    ),
    "down2_up2_c64_c128_fp16": Workload(
        "down2_up2_c64_c128_fp16", 512, "2x2x2/s2 conv 64->128 then transpose 128->64, fp16, 512^3 1-voxel shells"
    ),
    "w8a8_linear": Workload("w8a8_linear", 0, "W8A8 [65536,1024]x[4096,1024]^T and [65536,4096]x[1024,4096]^T"),
    "resblock_c256_fp16": Workload(
        "resblock_c256_fp16", 1024, "LN+adaLN -> subm conv+SiLU -> subm conv + residual, C=256 fp16, 1024^3 shells"
    ),
}


def coords_for(name: str, device: str | torch.device = "cpu", seed: int = 0) -> np.ndarray:
    """Active set of a named workload (seed 0 for the ellipsoid generator)."""
    if name == "subm3_c64_fp32":
        return sphere_shell()
    if name == "subm3_c128_fp16":
        return ellipsoid_shells(seed=seed, scale=1, thickness=2.0, device=device)
    if name == "down2_up2_c64_c128_fp16":
        return ellipsoid_shells(seed=seed, scale=2, thickness=1.0, device=device)
    if name == "resblock_c256_fp16":
        return ellipsoid_shells(seed=seed, scale=4, thickness=1.0, device=device)
    raise KeyError(name)


def normal(shape, std: float, seed: int, dtype=np.float32) -> np.ndarray:
    """Seeded ``N(0, std^2)`` array (generated in float32, then cast)."""
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(size=shape, dtype=np.float32) * np.float32(std)).astype(dtype)
