"""The library's device radix sort and scan against NumPy: stable order by a key bit
range (unsigned), values carried along, for 32- and 64-bit keys, sizes around the
4096-element tile and heavy duplicates; prefix sums against ``np.cumsum``."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SIZES = [1, 63, 4095, 4096, 4097, 100_003, 1_000_000]


def _ref(keys_u: np.ndarray, begin: int, end: int):
    """Stable order of the unsigned keys by bits [begin, end)."""
    width = end - begin
    field = keys_u >> np.uint64(begin)
    if width < 64:
        field = field & np.uint64((1 << width) - 1)
    return np.argsort(field, kind="stable")


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("dtype,bits", [(torch.int32, (0, 32)), (torch.int32, (5, 29)), (torch.int32, (0, 7)),
                                        (torch.int64, (0, 64)), (torch.int64, (3, 47))])
def test_sort_pairs_matches_numpy_stable(cuda, n, dtype, bits):
    from hi3d_amd import sort

    rng = np.random.default_rng(n + bits[0] * 7 + bits[1])
    if dtype == torch.int32:
        raw = rng.integers(0, 2**32, size=n, dtype=np.uint64)
        keys = torch.as_tensor(raw.astype(np.uint32).view(np.int32))
    else:
        raw = rng.integers(0, 2**64, size=n, dtype=np.uint64)
        keys = torch.as_tensor(raw.view(np.int64))
    vals = torch.arange(n, dtype=torch.int32)
    sk, sv = sort.sort_pairs(keys.to(cuda), vals.to(cuda), *bits)
    order = _ref(raw, *bits)
    assert np.array_equal(sv.cpu().numpy(), order)
    assert torch.equal(sk.cpu(), keys[torch.as_tensor(order)])


@pytest.mark.parametrize("n", [4097, 300_001])
def test_sort_pairs_stable_on_duplicates(cuda, n):
    """Seven distinct keys: equal keys keep their input order (values ascend inside each
    run), over one digit pass and over four."""
    from hi3d_amd import sort

    rng = np.random.default_rng(5)
    raw = rng.integers(0, 7, size=n).astype(np.uint64) * np.uint64(0x01010101)
    keys = torch.as_tensor(raw.astype(np.uint32).view(np.int32))
    vals = torch.as_tensor(rng.permutation(n).astype(np.int32))
    for bits in ((0, 8), (0, 32)):
        sk, sv = sort.sort_pairs(keys.to(cuda), vals.to(cuda), *bits)
        order = _ref(raw, *bits)
        assert np.array_equal(sv.cpu().numpy(), vals.numpy()[order])
        assert torch.equal(sk.cpu(), keys[torch.as_tensor(order)])


def test_sort_pairs_empty_and_empty_range(cuda):
    from hi3d_amd import sort

    k = torch.tensor([5, 3, 9], dtype=torch.int32, device=cuda)
    v = torch.tensor([0, 1, 2], dtype=torch.int32, device=cuda)
    sk, sv = sort.sort_pairs(k, v, 4, 4)
    assert sk.cpu().tolist() == [5, 3, 9] and sv.cpu().tolist() == [0, 1, 2]
    sk, sv = sort.sort_pairs(k[:0], v[:0])
    assert sk.numel() == 0 and sv.numel() == 0


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("inclusive", [False, True])
def test_scan_matches_cumsum(cuda, n, inclusive):
    from hi3d_amd import sort

    rng = np.random.default_rng(n)
    x = rng.integers(-50, 100, size=n).astype(np.int32)
    got = sort.scan(torch.as_tensor(x).to(cuda), inclusive).cpu().numpy()
    c = np.cumsum(x, dtype=np.int64).astype(np.int32)
    ref = c if inclusive else np.concatenate([[0], c[:-1]]).astype(np.int32)
    assert np.array_equal(got, ref)
