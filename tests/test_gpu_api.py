"""The reference's operator surfaces, run on the GPU and checked against the oracle:

* spconv's ``ops.get_indice_pairs`` with the reference's own layout test
  (tests/test_backends.py:53-67) and the golden pair lists;
* the upstream ``sparse_backend.Conv3d`` dtype policy: autocast off, features cast to
  the weight dtype, output cast back (src/sparc3d/ops/sparse_backend.py:130-148);
* ``sparc3d.nn.sparse.SparseConv3d.forward`` (src/sparc3d/nn/sparse/conv.py:79-88);
* the MLX-shaped ``sparse_conv(x, level, conv_weight(W), bias)``
  (src/hi3d_mac/mlx_backend/sparse.py:185-214).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import conv as oconv
from oracle import kmap as okmap

pytestmark = pytest.mark.gpu


def _random_sparse(n_side=14, density=0.15, channels=5, seed=0):
    """The reference test's recipe (torch generator, permuted rows, batch 0)."""
    g = torch.Generator().manual_seed(seed)
    occ = torch.rand(n_side, n_side, n_side, generator=g) < density
    xyz = occ.nonzero().int()
    xyz = xyz[torch.randperm(xyz.shape[0], generator=g)]
    feats = torch.randn(xyz.shape[0], channels, generator=g, dtype=torch.float64)
    return torch.cat([torch.zeros(xyz.shape[0], 1, dtype=torch.int32), xyz], 1), feats


def test_get_indice_pairs_reference_layout(cuda):
    """``pairs[side, k, :count]`` of the GPU map: the reference test's invariants (an
    input at p feeds the output at p + centre - r; counts symmetric under k -> 26 - k),
    and the lists equal the golden ones bit for bit."""
    from hi3d_amd import spconv

    golden = np.load(GOLDEN / "kmap_8cube.npz")
    indices, _ = _random_sparse(n_side=8, density=0.4)
    assert np.array_equal(indices.numpy(), golden["indices"])
    out_inds, pairs, counts = spconv.get_indice_pairs(
        indices.to(cuda), 1, [8, 8, 8], spconv.ConvAlgo.Native, (3, 3, 3), (1, 1, 1), (1, 1, 1), (1, 1, 1),
        (0, 0, 0), True, False,
    )
    assert torch.equal(out_inds.cpu(), indices)
    assert np.array_equal(counts.numpy(), golden["counts"])
    coords = indices[:, 1:].long()
    offsets = golden["offsets"]
    for k in range(27):
        r = torch.tensor([k // 9, (k // 3) % 3, k % 3])
        n = int(counts[k])
        src, dst = pairs[0, k, :n].cpu(), pairs[1, k, :n].cpu()
        assert torch.equal(coords[dst], coords[src] + 1 - r)
        assert n == int(counts[26 - k])
        assert np.array_equal(src.numpy(), golden["src"][offsets[k]:offsets[k + 1]])
        assert np.array_equal(dst.numpy(), golden["dst"][offsets[k]:offsets[k + 1]])


def _dense_reference(indices, feats64, weight64, bias64, n_side):
    idx = indices.numpy()
    w = weight64.reshape(weight64.shape[0], 27, weight64.shape[-1])
    table = okmap.neighbour_table(idx, [n_side] * 3)
    return oconv.gather_conv_f64(feats64, table, w, bias64)


@pytest.mark.parametrize("cin,cout", [(5, 7), (64, 128)])
@pytest.mark.parametrize("feat_dtype,weight_dtype", [(torch.float16, torch.float32), (torch.float32, torch.float16),
                                                     (torch.bfloat16, torch.float32)])
def test_sparse_backend_conv3d_dtype_policy(cuda, cin, cout, feat_dtype, weight_dtype):
    """Under fp16 autocast the upstream factory's convolution runs in the weight dtype
    (features cast to it), returns the features' dtype, keeps coordinates and row
    order, and matches float64 over the same rounded operands. Gate: max error / RMS
    <= 1e-2, or 3e-2 for bf16 outputs (the output rounding is the largest term, and
    bf16 keeps 8 significant bits against fp16's 11)."""
    from hi3d_amd import sparse_backend

    indices, feats = _random_sparse(n_side=14, density=0.15, channels=cin)
    torch.manual_seed(3)
    conv = sparse_backend.Conv3d(cin, cout, 3).to(cuda, weight_dtype)
    torch.nn.init.normal_(conv.bias, std=0.1)
    assert sparse_backend.is_sparse_conv(conv)
    x = sparse_backend.sparse_tensor(feats.to(cuda, feat_dtype), indices.to(cuda), (14, 14, 14))
    with torch.autocast("cuda", dtype=torch.float16):
        y = conv(x)
    out = sparse_backend.get_feats(y)
    assert out.dtype == feat_dtype and out.shape == (len(indices), cout)
    assert torch.equal(y.indices.cpu(), indices)
    f64 = feats.to(feat_dtype).to(weight_dtype).double().numpy()
    w64 = conv.weight.detach().double().cpu().numpy()
    b64 = conv.bias.detach().double().cpu().numpy()
    ref = _dense_reference(indices, f64, w64, b64, 14)
    gate = 3e-2 if feat_dtype == torch.bfloat16 else 1e-2
    assert oconv.rel_err(out.double().cpu().numpy(), ref) <= gate
    # the map is cached under the factory's key and reused by the next call
    key = "subm3"
    assert key in y.indice_dict
    data = y.indice_dict[key]
    y2 = conv(sparse_backend.replace_feats(y, torch.zeros_like(sparse_backend.get_feats(x))))
    assert y2.indice_dict[key] is data


def test_nn_sparse_conv3d_forward(cuda):
    """``SparseConv3d.forward`` on a SparseTensor: output over the same coordinates and
    layout with ``out_channels`` features, spatial cache and scale carried over, values
    within the fp16 gate of float64; a second tensor over the same rows reuses the map."""
    from hi3d_amd import nn as snn

    indices, feats = _random_sparse(n_side=16, density=0.2, channels=64)
    torch.manual_seed(4)
    layer = snn.SparseConv3d(64, 64, 3).to(cuda, torch.float16)
    x = snn.SparseTensor(feats.half().to(cuda), indices.to(cuda), scale=(2, 2, 2))
    x.register_spatial_cache("probe", 7)
    y = layer(x)
    assert isinstance(y, snn.SparseTensor)
    assert y.shape == (1, 64) and torch.equal(y.coords, x.coords) and y.layout == x.layout
    assert y.scale == (2, 2, 2) and y.get_spatial_cache("probe") == 7
    w64 = layer.conv.weight.detach().double().cpu().numpy()
    b64 = layer.conv.bias.detach().double().cpu().numpy()
    ref = _dense_reference(indices, feats.half().double().numpy(), w64, b64, 16)
    assert oconv.rel_err(y.feats.double().cpu().numpy(), ref) <= 1e-2
    maps = x.backend_data().indice_dict
    assert "subm3" in maps
    z = layer(x.replace(torch.randn_like(x.feats)))
    assert z.backend_data().indice_dict["subm3"] is maps["subm3"]


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_mlx_shaped_sparse_conv(cuda, dtype):
    """``sparse_conv(x, level, conv_weight(W), bias)`` with the reference's
    ``W_t [27 Cin, Cout]`` layout (row k Cin + ci) against float64 (fp16 gate 1e-2,
    fp32 1e-5), with and without bias; ``Level.from_coords`` builds the table."""
    from hi3d_amd import sparse

    indices, feats = _random_sparse(n_side=18, density=0.2, channels=64)
    coords = indices[:, 1:].to(cuda)
    level = sparse.Level.from_coords(coords)
    rng = np.random.default_rng(8)
    w = rng.standard_normal((128, 3, 3, 3, 64)) / np.sqrt(27 * 64)
    b = rng.standard_normal(128) * 0.1
    wt = sparse.conv_weight(torch.as_tensor(w).to(cuda, dtype))
    assert tuple(wt.shape) == (27 * 64, 128)
    assert torch.equal(wt[5 * 64 + 3], torch.as_tensor(w[:, 0, 1, 2, 3]).to(cuda, dtype))
    x = feats.to(cuda, dtype)
    gate = 1e-2 if dtype == torch.float16 else 1e-5
    f64 = feats.to(dtype).double().numpy()
    w64 = torch.as_tensor(w).to(dtype).double().numpy()
    for bias in (None, torch.as_tensor(b).to(cuda, dtype)):
        y = sparse.sparse_conv(x, level, wt, bias)
        assert y.dtype == dtype and y.shape == (len(indices), 128)
        b64 = None if bias is None else bias.double().cpu().numpy()
        ref = _dense_reference(indices, f64, w64, b64, 18)
        assert oconv.rel_err(y.double().cpu().numpy(), ref) <= gate


@pytest.mark.parametrize("factor", [2, (3, 3, 3), (2, 3, 4), (1, 1, 1), (4, 1, 2)])
def test_nn_sparse_downsample_any_factor(cuda, factor):
    """``SparseDownsample(factor)`` for any per-axis factor against the oracle's
    restatement of the reference (src/sparc3d/nn/sparse/spatial.py:34-79): coarse
    coordinates in the reference's order, the mean over each cell's rows and one zero,
    the scale, and the paired ``SparseUpsample`` restoring the fine rows and copying each
    parent's row to its children; two batch elements, fp16 and fp32 features."""
    from oracle import geometry as ogeo
    from hi3d_amd.nn import SparseDownsample, SparseTensor, SparseUpsample

    f3 = (factor,) * 3 if isinstance(factor, int) else factor
    rng = np.random.default_rng(sum(f3) + 11)
    parts = []
    for b in range(2):
        xyz = np.argwhere(rng.random((13, 11, 12)) < 0.15)
        parts.append(np.concatenate([np.full((len(xyz), 1), b), xyz[rng.permutation(len(xyz))]], 1))
    idx = np.concatenate(parts).astype(np.int32)
    for dtype, tol in ((torch.float32, 1e-6), (torch.float16, 2e-3)):
        x = rng.standard_normal((len(idx), 24)).astype(np.float32)
        st = SparseTensor(torch.as_tensor(x).to(dtype).to(cuda), torch.as_tensor(idx).to(cuda))
        coarse = SparseDownsample(factor)(st)
        low, pooled, inverse = ogeo.sparse_downsample(idx, torch.as_tensor(x).to(dtype).double().numpy(), f3)
        assert np.array_equal(coarse.coords.cpu().numpy(), low)
        np.testing.assert_allclose(coarse.feats.double().cpu().numpy(), pooled, rtol=tol, atol=tol)
        assert coarse.scale == f3
        fine = SparseUpsample(factor)(coarse)
        assert torch.equal(fine.coords, st.coords) and fine.scale == (1, 1, 1)
        assert torch.equal(fine.feats, coarse.feats[torch.as_tensor(inverse, device=cuda)])
    with pytest.raises(ValueError, match="factor"):
        SparseDownsample((2, 2))(st)
