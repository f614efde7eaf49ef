"""The refiner transformer's geometry on the GPU against the float64 oracle
(src/hi3d_mac/mlx_backend/transformer.py:234-266,449-473): coarse set, inverse and
counts exact; mean pool within fp32 / fp16 rounding; parent copy exact; the up block's
first convolution within the conv gates and bit-equal to the convolution of the
upsampled features."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import conv as oconv
from oracle import geometry as ogeo
from oracle import kmap as okmap

pytestmark = pytest.mark.gpu

GATE = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 3e-2}


def _geometry(cuda, side=20, density=0.3, seed=5):
    from hi3d_amd.geometry import Geometry

    rng = np.random.default_rng(seed)
    coords = np.argwhere(rng.random((side,) * 3) < density).astype(np.int32)
    return rng, coords, Geometry(torch.as_tensor(coords).to(cuda))


def test_structure_matches_oracle(cuda):
    rng, coords, geo = _geometry(cuda)
    assert np.array_equal(geo.full.table.cpu().numpy(), okmap.neighbour_table_dense(coords))
    low, inverse, counts = np.unique(coords // 2, axis=0, return_inverse=True, return_counts=True)
    assert np.array_equal(geo.low.coords.cpu().numpy(), low)
    assert np.array_equal(geo.inverse.cpu().numpy(), inverse.reshape(-1))
    assert np.array_equal(geo.counts.cpu().numpy(), counts)
    assert np.array_equal(geo.low.table.cpu().numpy(), okmap.neighbour_table_dense(low.astype(np.int32)))
    flat = ogeo.up_conv_index(geo.full.table.cpu().numpy(), inverse.reshape(-1), len(low))
    parent = np.where(flat == len(low) * 27, len(low), flat // 27)
    assert np.array_equal(geo.up_conv_table.cpu().numpy(), parent)


@pytest.mark.parametrize("dtype,gate", [(torch.float32, 1e-6), (torch.float16, 4e-3), (torch.bfloat16, 3e-2)])
def test_downsample_and_upsample(cuda, dtype, gate):
    """Mean pool: max-abs error / RMS within fp32 summation rounding, or one rounding to
    fp16 / bf16 (up to half an ulp of the largest means, about 4x the RMS); parent copy
    exact, for 16-byte rows (HIP row gather) and 12-byte rows."""
    rng, coords, geo = _geometry(cuda, seed=6)
    x = torch.as_tensor(rng.normal(0, 1, (len(coords), 96)).astype(np.float32)).to(cuda).to(dtype)
    got = geo.downsample(x)
    ref = ogeo.downsample_f64(x.float().cpu().numpy(), geo.inverse.cpu().numpy(), geo.low.n)
    assert got.dtype == dtype
    assert oconv.rel_err(got.float().cpu().numpy(), ref) <= gate
    h = torch.as_tensor(rng.normal(0, 1, (geo.low.n, 96)).astype(np.float32)).to(cuda).to(dtype)
    assert torch.equal(geo.upsample(h), h[geo.inverse.long()])
    h3 = torch.as_tensor(rng.normal(0, 1, (geo.low.n, 3)).astype(np.float32)).to(cuda)  # 12-byte rows
    assert torch.equal(geo.upsample(h3), h3[geo.inverse.long()])


@pytest.mark.parametrize("dtype,cin,cout,with_bias", [(torch.float16, 128, 128, True), (torch.float16, 256, 256, True),
                                                      (torch.float32, 64, 64, True), (torch.bfloat16, 128, 64, False),
                                                      (torch.float16, 64, 8, True)])
def test_up_conv_matches_float64_and_conv_of_upsampled(cuda, dtype, cin, cout, with_bias):
    from hi3d_amd import conv

    rng, coords, geo = _geometry(cuda, seed=cin + cout)
    h = torch.as_tensor(rng.normal(0, 1, (geo.low.n, cin)).astype(np.float32)).to(cuda).to(dtype)
    w = torch.as_tensor(rng.normal(0, (27 * cin) ** -0.5, (cout, 27 * cin)).astype(np.float32)).to(cuda).to(dtype)
    b = torch.as_tensor(rng.normal(0, 0.1, cout).astype(np.float32)).to(cuda).to(dtype) if with_bias else None
    y = geo.up_conv(h, w, b)
    ref = ogeo.up_conv_f64(h.float().cpu().numpy(), geo.full.table.cpu().numpy(), geo.inverse.cpu().numpy(),
                           w.float().cpu().numpy(), None if b is None else b.float().cpu().numpy())
    assert y.dtype == dtype and y.shape == (geo.full.n, cout)
    assert oconv.rel_err(y.float().cpu().numpy(), ref) <= GATE[dtype]
    direct = conv.conv(geo.upsample(h), geo.full.plan, w.reshape(cout, 27, cin).contiguous(), b)
    assert torch.equal(y, direct)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.bfloat16])
def test_mean_pool_vector_and_element_paths_agree(cuda, dtype):
    """The 16-byte-per-thread mean pool (aligned rows) and the one-element-per-thread
    kernel (a misaligned view) sum the present children in the same order: equal bits."""
    rng, coords, geo = _geometry(cuda, seed=9)
    c = 64
    buf = torch.as_tensor(rng.normal(0, 1, geo.full.n * c + 1).astype(np.float32)).to(cuda).to(dtype)
    aligned = buf[: geo.full.n * c].view(geo.full.n, c).clone()
    shifted = buf[1:].view(geo.full.n, c)
    shifted.copy_(aligned)
    assert shifted.data_ptr() % 16 != 0
    assert torch.equal(geo.downsample(aligned), geo.downsample(shifted))
