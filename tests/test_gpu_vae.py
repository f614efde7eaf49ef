"""VAE decoder pieces on the GPU: GroupNorm statistics, GroupNorm + swish (per row and
gathered), the conv_gn_swish / resnet compositions, and octree upsampling (occupancy
logits, child map, child projection) against the float64 oracle
(src/hi3d_mac/mlx_backend/vae.py:141-244,316-327, kernels.py:240-296). Gates:
statistics to fp32 rounding (rel 1e-5); activations 1e-5 (fp32) / 2e-3 (fp16), the
reference test's tolerances (tests/test_mlx_kernels.py:63-76); convolutions and
projections max-abs / RMS <= 1e-5 (fp32), 1e-2 (fp16), 3e-2 (bf16); the residual block
<= 1e-4 (fp32, two chained GroupNorms); child tables, parents, slots and coordinates
exact."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import conv as oconv
from oracle import vae as ovae

pytestmark = pytest.mark.gpu


def _level(cuda, side=16, density=0.5, seed=3):
    from hi3d_amd import sparse

    rng = np.random.default_rng(seed)
    idx = np.stack(np.meshgrid(*[np.arange(side)] * 3, indexing="ij"), -1).reshape(-1, 3)
    coords = idx[rng.random(idx.shape[0]) < density].astype(np.int32)
    return coords, sparse.Level.from_coords(torch.as_tensor(coords).to(cuda))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("c", [64, 128, 256])
def test_group_stats_matches_float64(cuda, dtype, c):
    from hi3d_amd import vae

    rng = np.random.default_rng(c)
    x = torch.as_tensor(rng.normal(0.5, 2.0, (20011, c)).astype(np.float32)).to(dtype)
    mean, inv = vae.group_stats(x.to(cuda))
    rm, ri = ovae.group_stats_f64(x.float().numpy())
    std = 1 / ri
    assert np.max(np.abs(mean.cpu().numpy() - rm) / std) <= 1e-5
    assert np.max(np.abs(inv.cpu().numpy() - ri) / ri) <= 1e-5


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.float16, 2e-3)])
def test_gather_group_norm_swish_matches_composed(cuda, dtype, tol):
    """The reference test's case: n = 300, C = 64, a [120, 27] table with n for absent."""
    from hi3d_amd import kernels

    rng = np.random.default_rng(10)
    n, c = 300, 64
    x = rng.normal(size=(n, c)).astype(np.float32)
    mean = rng.normal(size=c).astype(np.float32)
    inv = rng.uniform(0.5, 2.0, c).astype(np.float32)
    w, b = rng.normal(size=(1, c)).astype(np.float32), rng.normal(size=(1, c)).astype(np.float32)
    table = rng.integers(0, n + 1, (120, 27)).astype(np.int32)
    t = lambda a: torch.as_tensor(a).to(cuda)
    got = kernels.gather_group_norm_swish(t(x), t(table), t(mean), t(inv), t(w), t(b), dtype).float().cpu().numpy()
    ref = ovae.gather_group_norm_swish(x, table, mean, inv, w, b, np.float32).astype(np.float32)
    ref = torch.as_tensor(ref).to(dtype).float().numpy()
    assert got.shape == (120, 27 * c)
    assert np.allclose(got, ref, atol=tol, rtol=tol)
    assert np.all(got[np.repeat(table == n, c, axis=1)] == 0)


@pytest.mark.parametrize("din,dout", [(torch.float16, torch.float16), (torch.float32, torch.float32),
                                      (torch.bfloat16, torch.float32), (torch.float32, torch.float16)])
def test_group_norm_swish_rows(cuda, din, dout):
    from hi3d_amd import kernels, vae

    rng = np.random.default_rng(4)
    x = torch.as_tensor(rng.normal(0.2, 1.5, (3001, 128)).astype(np.float32)).to(din)
    w = rng.uniform(0.5, 1.5, (1, 128)).astype(np.float32)
    b = rng.normal(0, 0.1, (1, 128)).astype(np.float32)
    mean, inv = vae.group_stats(x.to(cuda))
    got = kernels.group_norm_swish(x.to(cuda), mean, inv, torch.as_tensor(w).to(cuda), torch.as_tensor(b).to(cuda),
                                   dout).float().cpu().numpy()
    ref = ovae.group_norm_swish(x.float().numpy(), mean.cpu().numpy(), inv.cpu().numpy(), w, b, np.float64)
    tol = 1e-5 if dout == torch.float32 else 2e-3
    assert np.allclose(got, ref, atol=tol, rtol=tol)


@pytest.mark.parametrize("dtype,gate", [(torch.float32, 1e-5), (torch.float16, 1e-2)])
def test_conv_gn_swish_matches_float64(cuda, dtype, gate):
    from hi3d_amd import vae

    coords, level = _level(cuda)
    table = level.table.cpu().numpy()
    rng = np.random.default_rng(5)
    c = 32
    x = rng.normal(0, 1, (len(coords), c)).astype(np.float32)
    gw, gb = rng.uniform(0.5, 1.5, (1, c)).astype(np.float32), rng.normal(0, 0.1, (1, c)).astype(np.float32)
    wt = rng.normal(0, 0.05, (27 * c, c)).astype(np.float32)
    bias = rng.normal(0, 0.1, c).astype(np.float32)
    res = rng.normal(0, 1, (len(coords), c)).astype(np.float32)
    t = lambda a, d=torch.float32: torch.as_tensor(a).to(cuda).to(d)
    got = vae.conv_gn_swish(t(x, dtype), level, t(gw), t(gb), t(wt, dtype), t(bias, dtype), residual=t(res, dtype))
    xr = t(x, dtype).float().cpu().numpy()
    ref = ovae.conv_gn_swish_f64(xr, table, gw, gb, t(wt, dtype).float().cpu().numpy(),
                                 t(bias, dtype).float().cpu().numpy(), residual=t(res, dtype).float().cpu().numpy())
    assert got.dtype == dtype
    assert oconv.rel_err(got.float().cpu().numpy(), ref) <= gate


@pytest.mark.parametrize("with_res_conv", [False, True])
def test_resnet_matches_float64(cuda, with_res_conv):
    """The reference's residual-block test geometry (16^3 cube at density 0.5, C = 32,
    tests/test_mlx_kernels.py:125-150) in fp32 against the float64 composition."""
    from hi3d_amd import vae

    coords, level = _level(cuda)
    table = level.table.cpu().numpy()
    rng = np.random.default_rng(3)
    c = 32
    p = {}
    for name in ("r.block.0", "r.block.3"):
        p[f"{name}.weights"] = rng.uniform(0.5, 1.5, (1, c)).astype(np.float32)
        p[f"{name}.bias"] = rng.normal(0, 0.1, (1, c)).astype(np.float32)
    for name in ("r.block.2", "r.block.5"):
        p[f"{name}.weight"] = rng.normal(0, 0.05, (27 * c, c)).astype(np.float32)
        p[f"{name}.bias"] = rng.normal(0, 0.1, (c,)).astype(np.float32)
    if with_res_conv:
        p["r.res_conv.weight"] = rng.normal(0, 0.2, (c, c)).astype(np.float32)
        p["r.res_conv.bias"] = rng.normal(0, 0.1, (c,)).astype(np.float32)
    x = rng.normal(0, 1, (len(coords), c)).astype(np.float32)
    gp = {k: torch.as_tensor(v).to(cuda) for k, v in p.items()}
    got = vae.resnet(torch.as_tensor(x).to(cuda), level, gp, "r").cpu().numpy()
    ref = ovae.resnet_f64(x, table, p, "r")
    assert oconv.rel_err(got, ref) <= 1e-4
    # above skip_points rows the block returns its input itself (upstream's skip), also
    # from a holder, which it empties
    xt = torch.as_tensor(x).to(cuda)
    assert vae.resnet(xt, level, gp, "r", skip_points=len(coords) - 1) is xt
    holder = [xt]
    assert vae.resnet(holder, level, gp, "r", skip_points=len(coords) - 1) is xt and holder == []
    assert vae.SKIP_POINTS == 12_000_000


GATE = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 3e-2}


def _children_case(cuda, p, c, density, seed):
    """Parents with random occupancy and the child map of a random parent table."""
    from hi3d_amd import sparse

    rng = np.random.default_rng(seed)
    mask = rng.random((p, 8)) < density
    table = rng.integers(0, p + 1, (p, 27)).astype(np.int32)
    _, parent, slot = sparse.child_neighbour_table(torch.as_tensor(table).to(cuda), torch.as_tensor(mask).to(cuda))
    return rng, mask, parent, slot


@pytest.mark.parametrize("dtype,c", [(torch.float16, 64), (torch.float16, 256), (torch.float16, 512),
                                     (torch.bfloat16, 128), (torch.float32, 512)])
def test_children_slot_layout_exact(cuda, dtype, c):
    """A weight stacking ``s * I`` per slot makes child ``(p, s)`` equal ``s * x[p]``
    exactly (small integers): every child's row, slot block and order, bit for bit."""
    from hi3d_amd import vae

    rng, _, parent, slot = _children_case(cuda, 700, c, 0.5, c)
    x = torch.as_tensor(rng.integers(-8, 9, (700, c)).astype(np.float32)).to(cuda).to(dtype)
    w = torch.cat([s * torch.eye(c, device=cuda) for s in range(8)]).to(dtype)
    got = vae.children(x, parent, slot, w)
    want = slot.to(dtype)[:, None] * x[parent.long()]
    assert got.dtype == dtype and torch.equal(got, want)


@pytest.mark.parametrize("dtype,c,p,density", [(torch.float16, 128, 3000, 0.5), (torch.float16, 256, 2500, 0.3),
                                               (torch.float16, 512, 1500, 0.6), (torch.bfloat16, 256, 2000, 0.5),
                                               (torch.float32, 64, 3000, 0.5), (torch.float32, 256, 1200, 0.4),
                                               (torch.float32, 512, 900, 0.5)])
def test_children_matches_float64(cuda, dtype, c, p, density):
    """Kept children's projected features against the reference's full projection and
    take (vae.py:220-244), at the decoder's projection widths (512, 512, 256) and
    narrower ones; output in the weight dtype and converted to fp32 on request."""
    from hi3d_amd import vae

    rng, mask, parent, slot = _children_case(cuda, p, c, density, p + c)
    x = torch.as_tensor(rng.normal(0, 1, (p, c)).astype(np.float32)).to(cuda).to(dtype)
    w = torch.as_tensor(rng.normal(0, c ** -0.5, (8 * c, c)).astype(np.float32)).to(cuda).to(dtype)
    got = vae.children(x, parent, slot, w)
    ref = ovae.children_f64(x.float().cpu().numpy(), parent.cpu().numpy(), slot.cpu().numpy(), w.float().cpu().numpy())
    assert got.shape == (int(mask.sum()), c) and got.dtype == dtype
    assert oconv.rel_err(got.float().cpu().numpy(), ref) <= GATE[dtype]
    as_f32 = vae.children(x, parent, slot, w, out=torch.float32)
    assert as_f32.dtype == torch.float32 and torch.equal(as_f32, got.float())


def _upsample_params(rng, c, wdt):
    p = {
        "u.cls_head.fc.0.weights": rng.uniform(0.5, 1.5, (1, c)).astype(np.float32),
        "u.cls_head.fc.0.bias": rng.normal(0, 0.1, (1, c)).astype(np.float32),
        "u.cls_head.fc.2.weight": rng.normal(0, (27 * c) ** -0.5, (27 * c, 8)).astype(np.float32),
        "u.cls_head.fc.2.bias": rng.normal(0, 0.3, (8,)).astype(np.float32),
        "u.proj.weight": rng.normal(0, c ** -0.5, (8 * c, c)).astype(np.float32),
    }
    gemm = ("u.cls_head.fc.2.weight", "u.cls_head.fc.2.bias", "u.proj.weight")
    gp = {k: torch.as_tensor(v).to(wdt if k in gemm else torch.float32) for k, v in p.items()}
    return {k: v.float().numpy() for k, v in gp.items()}, gp


@pytest.mark.parametrize("dtype,c", [(torch.float32, 64), (torch.float16, 128), (torch.float32, 256)])
def test_upsample_matches_float64(cuda, dtype, c):
    """One decoder upsampling (vae.py:316-327) on a 16^3 cube at density 0.5: occupancy
    logits against float64 (the decision ``> 0`` agrees wherever the float64 logit is
    clear of zero by the gate), then, on the GPU's own mask, child table, parents,
    slots and coordinates exact and projected features within the gate."""
    from hi3d_amd import vae

    coords, level = _level(cuda)
    table = level.table.cpu().numpy()
    rng = np.random.default_rng(c)
    p, gp = _upsample_params(rng, c, dtype)
    gp = {k: v.to(cuda) for k, v in gp.items()}
    x = torch.as_tensor(rng.normal(0, 1, (len(coords), c)).astype(np.float32)).to(cuda).to(dtype)
    xr = x.float().cpu().numpy()
    logits = vae.occupancy(x, level, gp, "u")
    ref_logits = ovae.occupancy_f64(xr, table, p, "u")
    assert oconv.rel_err(logits.float().cpu().numpy(), ref_logits) <= GATE[dtype]
    y, child, mask = vae.upsample(x, level, gp, "u")
    m = mask.cpu().numpy()
    clear = np.abs(ref_logits) > 4 * GATE[dtype] * np.sqrt(np.mean(ref_logits ** 2))
    assert np.array_equal(m[clear], ref_logits[clear] > 0)
    assert 0.2 < m.mean() < 0.8
    feats, ccoords, ctable, parent, slot, _ = ovae.upsample_f64(xr, coords, table, p, "u", mask=m)
    assert np.array_equal(child.table.cpu().numpy(), ctable)
    assert np.array_equal(child.coords.cpu().numpy(), ccoords)
    assert y.dtype == dtype and oconv.rel_err(y.float().cpu().numpy(), feats) <= GATE[dtype]
    # the children's own map is what a fresh hash of their coordinates gives
    from hi3d_amd import sparse

    assert torch.equal(sparse.neighbour_table(child.coords), child.table)


def test_upsample_with_given_and_empty_masks(cuda):
    """A caller's mask replaces the occupancy decision (the reference's force_masks,
    vae.py:318-320); an all-empty mask yields no children."""
    from hi3d_amd import vae

    coords, level = _level(cuda, side=8)
    rng = np.random.default_rng(9)
    c = 64
    p, gp = _upsample_params(rng, c, torch.float16)
    gp = {k: v.to(cuda) for k, v in gp.items()}
    x = torch.as_tensor(rng.normal(0, 1, (len(coords), c)).astype(np.float16)).to(cuda)
    m = rng.random((len(coords), 8)) < 0.25
    y, child, mask = vae.upsample(x, level, gp, "u", mask=torch.as_tensor(m).to(cuda))
    feats, ccoords, ctable, _, _, _ = ovae.upsample_f64(x.float().cpu().numpy(), coords, level.table.cpu().numpy(),
                                                       p, "u", mask=m)
    assert np.array_equal(child.coords.cpu().numpy(), ccoords) and np.array_equal(child.table.cpu().numpy(), ctable)
    assert oconv.rel_err(y.float().cpu().numpy(), feats) <= 1e-2
    y, child, _ = vae.upsample(x, level, gp, "u", mask=torch.zeros((len(coords), 8), dtype=torch.bool, device=cuda))
    assert y.shape == (0, c) and child.n == 0 and child.table.shape == (0, 27)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_resnet_in_place_matches_composed(cuda, dtype):
    """The reference's in-place residual test (tests/test_mlx_kernels.py:124-150): the
    block on a donated input (a one-element holder) accumulates its second convolution
    into the input's buffer and equals the composed block bit for bit."""
    from hi3d_amd import vae

    coords, level = _level(cuda)
    rng = np.random.default_rng(3)
    c = 32 if dtype == torch.float32 else 64
    p = {}
    for name in ("r.block.0", "r.block.3"):
        p[f"{name}.weights"] = torch.as_tensor(rng.uniform(0.5, 1.5, (1, c)).astype(np.float32)).to(cuda)
        p[f"{name}.bias"] = torch.as_tensor(rng.normal(0, 0.1, (1, c)).astype(np.float32)).to(cuda)
    for name in ("r.block.2", "r.block.5"):
        p[f"{name}.weight"] = torch.as_tensor(rng.normal(0, 0.05, (27 * c, c)).astype(np.float32)).to(cuda).to(dtype)
        p[f"{name}.bias"] = torch.as_tensor(rng.normal(0, 0.1, (c,)).astype(np.float32)).to(cuda).to(dtype)
    x = torch.as_tensor(rng.normal(0, 1, (len(coords), c)).astype(np.float32)).to(cuda).to(dtype)
    composed = vae.resnet(x.clone(), level, p, "r")
    donated = x.clone()
    ptr = donated.data_ptr()
    holder = [donated]
    del donated
    in_place = vae.resnet(holder, level, p, "r")
    assert not holder and in_place.data_ptr() == ptr
    assert torch.equal(composed, in_place)


def test_conv_gn_swish_residual_holder(cuda):
    """``residual`` as a holder: the result lives in the residual's buffer and equals
    the out-of-place sum; the narrow kernel (8 outputs) accumulates in place too."""
    from hi3d_amd import vae

    coords, level = _level(cuda, seed=4)
    rng = np.random.default_rng(8)
    for c, cout in ((64, 64), (64, 8)):
        t = lambda a: torch.as_tensor(a).to(cuda)
        x = t(rng.normal(0, 1, (len(coords), c)).astype(np.float16))
        gw, gb = t(rng.uniform(0.5, 1.5, (1, c)).astype(np.float32)), t(rng.normal(0, 0.1, (1, c)).astype(np.float32))
        wt = t(rng.normal(0, 0.05, (27 * c, cout)).astype(np.float16))
        bias = t(rng.normal(0, 0.1, cout).astype(np.float16))
        r = t(rng.normal(0, 1, (len(coords), cout)).astype(np.float16))
        ref = vae.conv_gn_swish(x, level, gw, gb, wt, bias, residual=r)
        donated = r.clone()
        ptr = donated.data_ptr()
        got = vae.conv_gn_swish(x, level, gw, gb, wt, bias, residual=[donated])
        assert got.data_ptr() == ptr and torch.equal(got, ref)
