"""The allocation-free kernel map (``hi3d_kmap_subm_noalloc``, hash table in a device
array of the library) against ``hi3d_kmap_subm`` (caller workspace), through the C ABI:
equal tables, counts and status on two calls in a row, the second smaller (the array
keeps the first call's contents, so a missing clear would show), on 32-bit and 64-bit
keys and with duplicate / out-of-range coordinates; sets past the array's capacity are
refused before any launch."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _noalloc(coords: torch.Tensor, shape, batch: int, n: int | None = None):
    from hi3d_amd import _lib

    dev = coords.device
    n = int(coords.shape[0]) if n is None else n
    table = torch.empty((int(coords.shape[0]), 27), dtype=torch.int32, device=dev)
    counts = torch.empty(27, dtype=torch.int32, device=dev)
    status = torch.empty(1, dtype=torch.int32, device=dev)
    _lib.call("hi3d_kmap_subm_noalloc", _lib.ptr(coords), n, *shape, batch, 3, _lib.ptr(table), _lib.ptr(counts),
              _lib.ptr(status), _lib.stream(dev))
    return table, counts, status


def _hashed(coords: torch.Tensor, shape, batch: int):
    from hi3d_amd import _lib

    dev = coords.device
    n = int(coords.shape[0])
    key64 = int(batch * shape[0] * shape[1] * shape[2] >= 0xFFFFFFFF)
    ws = _lib.workspace(_lib.query("hi3d_kmap_workspace", n, 0, key64), dev)
    table = torch.empty((n, 27), dtype=torch.int32, device=dev)
    counts = torch.empty(27, dtype=torch.int32, device=dev)
    status = torch.empty(1, dtype=torch.int32, device=dev)
    _lib.call("hi3d_kmap_subm", _lib.ptr(coords), n, *shape, batch, 3, 0, _lib.ptr(ws), ws.numel(), _lib.ptr(table),
              _lib.ptr(counts), _lib.ptr(status), _lib.stream(dev))
    return table, counts, status


def _same(coords, shape, batch, table=True):
    """Both maps of ``coords``; with ``table`` False only counts and status are compared
    (with repeated coordinates, which repeat wins a hash slot is a race, so the rows
    recorded for them may differ between any two builds)."""
    got = _noalloc(coords, shape, batch)
    want = _hashed(coords, shape, batch)
    for g, w in list(zip(got, want))[(0 if table else 1):]:
        assert torch.equal(g, w)
    return got


def test_noalloc_map_equals_workspace_map(cuda):
    from hi3d_amd import workloads

    big = torch.as_tensor(workloads.coords_for("subm3_c128_fp16", device=cuda)).to(cuda)
    table, counts, status = _same(big, [256, 256, 256], 1)
    assert int(status.item()) == 0 and int(counts.sum()) == 9_711_641
    rng = np.random.default_rng(3)
    xyz = np.argwhere(rng.random((12, 12, 12)) < 0.3)
    small = np.concatenate([rng.integers(0, 2, (len(xyz), 1)), xyz], 1).astype(np.int32)
    small = small[np.lexsort((small[:, 3], small[:, 2], small[:, 1], small[:, 0]))]
    table, counts, status = _same(torch.as_tensor(small).to(cuda), [12, 12, 12], 2)
    assert int(status.item()) == 0 and table.shape == (len(small), 27)
    # 64-bit keys (2 * 2048 * 2048 * 1024 cells), then duplicate and out-of-range rows
    wide = torch.as_tensor(small * np.array([1, 170, 170, 85], np.int32)).to(cuda)
    _same(wide, [2048, 2048, 1024], 2)
    dup = torch.as_tensor(np.concatenate([small, small[:3]])).to(cuda)
    assert int(_same(dup, [12, 12, 12], 2, table=False)[2].item()) & 1
    out = torch.as_tensor(np.concatenate([small, [[0, 12, 0, 0]]]).astype(np.int32)).to(cuda)
    assert int(_same(out, [12, 12, 12], 2)[2].item()) & 4


def test_noalloc_map_capacity_limits(cuda):
    """2^22 + 1 voxels exceed the 64-bit-key limit (refused, nothing launched past the
    argument checks) and fit the 32-bit-key one (here all one coordinate: every insert
    after the first is a duplicate, as the workspace map reports too)."""
    coords = torch.zeros(((1 << 22) + 1, 4), dtype=torch.int32, device=cuda)
    with pytest.raises(ValueError, match="allocation-free map holds at most"):
        _noalloc(coords, [2048, 2048, 1024], 2)
    table, counts, status = _same(coords, [64, 64, 64], 1)
    assert int(status.item()) == 1 and int(counts.sum()) == (1 << 22) + 1
