"""GPU unique of int64 keys and integer rows against the oracle, ``np.unique`` and
``torch.unique(dim=0)``: bit-exact values, inverse maps and counts, dtypes included
(the reference's tests: tests/test_backends.py:182-190, tests/test_empty_geometry.py:8-18)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import unique as ounique

pytestmark = pytest.mark.gpu


def test_reference_rows_match_torch_unique(cuda):
    """The reference test's recipe: 20000 x 3 rows in [-5, 40), generator seed 0."""
    from hi3d_amd import fast_unique

    g = torch.Generator().manual_seed(0)
    rows = torch.randint(-5, 40, (20000, 3), generator=g)
    ref = torch.unique(rows, dim=0, return_inverse=True, return_counts=True)
    new = fast_unique.unique_rows(rows.to(cuda), return_inverse=True, return_counts=True)
    for a, b in zip(ref, new):
        assert a.dtype == b.dtype and torch.equal(a, b.cpu())
    only = fast_unique.unique_rows(rows.to(cuda))
    assert torch.equal(only.cpu(), ref[0])


@pytest.mark.parametrize("counts", [False, True])
def test_empty_keys_match_numpy(cuda, counts):
    from hi3d_amd import fast_unique

    values, inverse, observed = fast_unique.unique_keys(torch.empty(0, dtype=torch.int64, device=cuda),
                                                        return_counts=counts)
    ref = np.unique(np.empty(0, np.int64), return_inverse=True, return_counts=counts)
    assert np.array_equal(values.cpu().numpy(), ref[0]) and np.array_equal(inverse.cpu().numpy(), ref[1])
    if counts:
        assert np.array_equal(observed.cpu().numpy(), ref[2])
    else:
        assert observed is None


@pytest.mark.parametrize("n,lo,hi", [(1, 0, 1), (5000, -1000, 1000), (300000, -(2**62), 2**62),
                                     (2_000_000, 0, 50_000)])
def test_keys_match_numpy(cuda, n, lo, hi):
    """Random keys with many duplicates, negative and huge values, the int64 extremes and
    a single key; all 64 bits sorted (sign flipped) and, for non-negative keys, only the
    bits that can differ."""
    from hi3d_amd import fast_unique

    rng = np.random.default_rng(n)
    keys = rng.integers(lo, hi, n, dtype=np.int64)
    if n > 10:
        keys[:3] = [np.iinfo(np.int64).min, np.iinfo(np.int64).max, 0] if lo < 0 else [lo, hi - 1, lo]
    ref = np.unique(keys, return_inverse=True, return_counts=True)
    kt = torch.as_tensor(keys).to(cuda)
    for bits in ([0, (hi - 1).bit_length()] if lo >= 0 else [0]):
        values, inverse, counts = fast_unique.unique_keys(kt, return_counts=True, key_bits=bits)
        assert np.array_equal(values.cpu().numpy(), ref[0])
        assert np.array_equal(inverse.cpu().numpy(), ref[1])
        assert np.array_equal(counts.cpu().numpy(), ref[2])


@pytest.mark.parametrize("dtype,d,lo,hi", [(torch.int32, 3, -5, 40), (torch.int64, 4, -(2**14), 2**14),
                                           (torch.int16, 2, -300, 300), (torch.uint8, 1, 0, 256),
                                           (torch.int64, 8, 0, 6), (torch.int32, 3, 0, 1024)])
def test_rows_match_torch_unique(cuda, dtype, d, lo, hi):
    """Row widths 1..8, the four integer dtypes the reference packs, tight and wide value
    ranges (the last: 1024^3 cube corners as in mesh extraction)."""
    from hi3d_amd import fast_unique

    g = torch.Generator().manual_seed(d * 100 + hi)
    rows = torch.randint(lo, hi, (50000, d), generator=g, dtype=torch.int64).to(dtype)
    rows = torch.cat([rows, rows[::7]])  # guaranteed repeats
    ref = torch.unique(rows, dim=0, return_inverse=True, return_counts=True)
    new = fast_unique.unique_rows(rows.to(cuda), return_inverse=True, return_counts=True)
    for a, b in zip(ref, new):
        assert a.dtype == b.dtype and torch.equal(a, b.cpu())
    orows, oinv, ocnt = ounique.unique_rows(rows.to(torch.int64).numpy(), return_inverse=True, return_counts=True)
    assert np.array_equal(new[0].cpu().numpy().astype(np.int64), orows)
    assert np.array_equal(new[1].cpu().numpy(), oinv) and np.array_equal(new[2].cpu().numpy(), ocnt)


def test_wide_rows_and_dispatch(cuda):
    """Rows whose ranges multiply past 2^62 go to torch.unique (as in the reference);
    the ``unique`` dispatcher sends 2-D integer rows with dim=0 to the GPU path and
    everything else to torch.unique."""
    from hi3d_amd import fast_unique

    rows = torch.tensor([[0, 0, 0], [2**40, 5, 2**30], [0, 0, 0]], dtype=torch.int64, device=cuda)
    ref = torch.unique(rows.cpu(), dim=0, return_inverse=True, return_counts=True)
    new = fast_unique.unique_rows(rows, return_inverse=True, return_counts=True)
    for a, b in zip(ref, new):
        assert torch.equal(a, b.cpu())
    x = torch.randint(0, 9, (1000, 3), device=cuda, dtype=torch.int32)
    for a, b in zip(torch.unique(x.cpu(), dim=0, return_inverse=True),
                    fast_unique.unique(x, dim=0, return_inverse=True)):
        assert torch.equal(a, b.cpu())
    f = torch.rand(100, device=cuda)
    assert torch.equal(fast_unique.unique(f), torch.unique(f))
