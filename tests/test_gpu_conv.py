"""Gather convolutions on the GPU against the oracle.

Gates (max|y - y_ref| / rms(y_ref)): fp32 <= 1e-5, fp16 <= 1e-2 (bf16 <= 3e-2, one
bf16 ulp being 8x an fp16 ulp); float64 (the reference test's C 5->7 case) <= 1e-12
absolute. Large workloads are checked on sampled output rows against float64 sums.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import conv as oconv
from oracle import kmap as okmap

pytestmark = pytest.mark.gpu

GATE = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 3e-2}


def _rand_indices(rng, n_side, density, batch=1):
    rows = []
    for b in range(batch):
        xyz = np.argwhere(rng.random((n_side,) * 3) < density)
        rows.append(np.concatenate([np.full((len(xyz), 1), b), xyz], 1))
    idx = np.concatenate(rows).astype(np.int32)
    return idx[rng.permutation(len(idx))]


def _case(rng, n, cin, cout, dtype, kvol=27):
    x = torch.as_tensor(rng.standard_normal((n, cin), dtype=np.float32)).to(dtype)
    w = torch.as_tensor(rng.standard_normal((cout, kvol, cin), dtype=np.float32) / np.sqrt(kvol * cin)).to(dtype)
    b = torch.as_tensor(rng.standard_normal(cout, dtype=np.float32) * 0.1).to(dtype)
    return x, w, b


def test_reference_case_float64_golden(cuda):
    """tests/test_backends.py:32-50 recipe through the spconv API in float64."""
    from hi3d_amd import spconv

    data = np.load(GOLDEN / "subm_14cube.npz")
    conv = spconv.SubMConv3d(5, 7, 3, bias=True, indice_key="subm3").double().to(cuda)
    with torch.no_grad():
        conv.weight.copy_(torch.as_tensor(data["weight"]))
        conv.bias.copy_(torch.as_tensor(data["bias"]))
    x = spconv.SparseConvTensor(torch.as_tensor(data["feats"]).to(cuda), torch.as_tensor(data["indices"]).to(cuda),
                                [14] * 3, 1)
    out = conv(x).features.cpu().numpy()
    assert np.allclose(out, data["out"], atol=1e-12, rtol=1e-12)
    assert "subm3" in x.indice_dict


@pytest.mark.parametrize("dtype,cin,cout", [
    (torch.float32, 64, 64), (torch.float32, 32, 96), (torch.float16, 128, 128), (torch.float16, 64, 64),
    (torch.float16, 256, 256), (torch.float16, 64, 320), (torch.float16, 200, 40), (torch.bfloat16, 128, 64),
])
def test_mfma_conv_matches_float64(cuda, dtype, cin, cout):
    from hi3d_amd import conv, kmap

    rng = np.random.default_rng(cin * 1000 + cout)
    idx = _rand_indices(rng, 24, 0.15, batch=2)
    km = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [24] * 3, 2)
    x, w, b = _case(rng, len(idx), cin, cout, dtype)
    y = conv.gather_conv(x.to(cuda), km.plan(), w.to(cuda), b.to(cuda))
    ref = oconv.gather_conv_f64(x.float().numpy(), km.table.cpu().numpy(), w.float().numpy(), b.float().numpy())
    assert y.dtype == dtype and y.shape == (len(idx), cout)
    assert oconv.rel_err(y.float().cpu().numpy(), ref) <= GATE[dtype]


@pytest.mark.parametrize("dtype,cin,cout,kvol,density,act,res", [
    (torch.float16, 256, 8, 27, 0.15, None, False), (torch.float32, 512, 8, 27, 0.1, None, False),
    (torch.bfloat16, 128, 16, 27, 0.2, "silu", True), (torch.float16, 32, 1, 27, 0.3, None, True),
    (torch.float32, 48, 5, 27, 0.004, "silu", False), (torch.float16, 96, 12, 8, 0.2, None, False),
    (torch.float16, 512, 8, 27, 0.05, None, False), (torch.bfloat16, 64, 8, 8, 0.2, "silu", True),
    (torch.float16, 128, 3, 27, 0.02, None, True),
])
def test_narrow_conv_matches_float64(cuda, dtype, cin, cout, kvol, density, act, res):
    """The narrow-output kernels (cout <= 16, 16x16 MFMAs; 16-bit rows of 128-byte
    multiples staged through LDS, the others loaded to registers) against float64 and
    against the tile kernels on the same inputs: occupancy-head shapes (C 256 / 512 -> 8),
    odd output counts, K steps of one, two and four 64-byte blocks, sparse sets where
    most offsets of a 64-row tile are absent, and a few-offset table."""
    from hi3d_amd import conv, kmap

    rng = np.random.default_rng(cin * 31 + cout + kvol)
    idx = _rand_indices(rng, 24, density, batch=2)
    n = len(idx)
    if kvol == 27:
        table = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [24] * 3, 2).table
    else:
        t = rng.integers(0, n + 1, (n - 7, kvol)).astype(np.int32)
        t[rng.random(t.shape) < 0.6] = n
        table = torch.as_tensor(t).to(cuda)
    x, w, b = _case(rng, n, cin, cout, dtype, kvol)
    r = torch.as_tensor(rng.standard_normal((int(table.shape[0]), cout), dtype=np.float32)).to(dtype) if res else None
    xd, wd, bd = x.to(cuda), w.to(cuda), b.to(cuda)
    rd = None if r is None else r.to(cuda)
    assert conv.narrow_supported(dtype, cin, cout, kvol)
    plan = kmap.build_plan(table, n)
    y = conv.gather_conv_narrow(xd, plan, wd, bd, act=act, residual=rd)
    ref = oconv.gather_conv_f64(x.float().numpy(), table.cpu().numpy(), w.float().numpy(), b.float().numpy(),
                                act=act, residual=None if r is None else r.float().numpy())
    assert y.dtype == dtype and y.shape == (int(table.shape[0]), cout)
    assert oconv.rel_err(y.float().cpu().numpy(), ref) <= GATE[dtype]
    assert torch.equal(conv.conv(xd, plan, wd, bd, act=act, residual=rd), y)  # conv() takes this kernel
    if conv.mfma_supported(dtype, cin, cout):
        tile = conv.gather_conv(xd, plan, wd, bd, act=act, residual=rd)
        assert oconv.rel_err(tile.float().cpu().numpy(), ref) <= GATE[dtype]


def test_epilogue_silu_and_residual(cuda):
    from hi3d_amd import conv, kmap

    rng = np.random.default_rng(5)
    idx = _rand_indices(rng, 16, 0.25)
    km = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [16] * 3, 1)
    x, w, b = _case(rng, len(idx), 64, 64, torch.float16)
    r = torch.as_tensor(rng.standard_normal((len(idx), 64), dtype=np.float32)).half()
    t = km.table.cpu().numpy()
    xf, wf, bf = x.float().numpy(), w.float().numpy(), b.float().numpy()
    y = conv.gather_conv(x.to(cuda), km.plan(), w.to(cuda), b.to(cuda), act="silu")
    assert oconv.rel_err(y.float().cpu().numpy(), oconv.gather_conv_f64(xf, t, wf, bf, act="silu")) <= 1e-2
    y = conv.gather_conv(x.to(cuda), km.plan(), w.to(cuda), b.to(cuda), residual=r.to(cuda))
    ref = oconv.gather_conv_f64(xf, t, wf, bf, residual=r.float().numpy())
    assert oconv.rel_err(y.float().cpu().numpy(), ref) <= 1e-2


@pytest.mark.parametrize("dtype,cin,cout,density,act,res", [
    (torch.bfloat16, 128, 256, 0.15, None, False), (torch.float16, 160, 128, 0.15, "silu", True),
    (torch.float16, 256, 128, 0.3, "silu", False), (torch.float16, 128, 128, 0.004, None, True),
    (torch.float16, 256, 256, 0.2, "silu", True), (torch.bfloat16, 192, 512, 0.1, None, True),
    (torch.float16, 256, 256, 0.004, None, False),
    (torch.float32, 64, 128, 0.15, "silu", True), (torch.float32, 128, 64, 0.1, None, True),
    (torch.float16, 512, 512, 0.1, "silu", True), (torch.bfloat16, 512, 256, 0.15, None, False),
    (torch.float16, 448, 128, 0.1, None, True), (torch.float16, 512, 128, 0.05, "silu", False),
    (torch.float16, 64, 64, 0.15, "silu", True), (torch.bfloat16, 64, 128, 0.1, None, False),
    (torch.float16, 128, 64, 0.004, None, True),
    (torch.float32, 256, 256, 0.1, "silu", True), (torch.float32, 512, 128, 0.1, None, False),
    (torch.float32, 64, 256, 0.15, None, True), (torch.float32, 80, 128, 0.1, "silu", False),
    (torch.bfloat16, 256, 128, 0.15, "silu", True), (torch.float16, 128, 384, 0.1, None, True),
])
def test_ring_kernel_variants(cuda, dtype, cin, cout, density, act, res):
    """The ring kernels (fp16/bf16, Cout a multiple of 128, 256..1024-byte rows): 256 x 256
    tiles of 64-byte K steps (Cout a multiple of 256), 256 x 128 tiles of 128-byte K steps
    (rows a multiple of 128 bytes) and 384 x 128 tiles of 64-byte steps (320-byte rows);
    fp16/bf16 64- and 128-channel rows into 64 or 128 outputs, and fp32 (Cout 64 or a
    multiple of 128, rows up to 2 KB), on 128-row tiles (fp32: four 32x32x2 MFMAs per
    fragment);
    several output-column tiles, two to sixteen K steps per offset, SiLU and residual in
    the epilogue, and isolated voxels (tiles whose only offset is the centre)."""
    from hi3d_amd import conv, kmap

    rng = np.random.default_rng(cin * 7 + cout + int(density * 1000))
    idx = _rand_indices(rng, 24, density, batch=2)
    km = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [24] * 3, 2)
    x, w, b = _case(rng, len(idx), cin, cout, dtype)
    r = torch.as_tensor(rng.standard_normal((len(idx), cout), dtype=np.float32)).to(dtype) if res else None
    y = conv.gather_conv(x.to(cuda), km.plan(), w.to(cuda), b.to(cuda), act=act,
                         residual=None if r is None else r.to(cuda))
    ref = oconv.gather_conv_f64(x.float().numpy(), km.table.cpu().numpy(), w.float().numpy(), b.float().numpy(),
                                act=act, residual=None if r is None else r.float().numpy())
    # fp32 sums of up to 27 * Cin products: above 256 input channels the rounding of the
    # accumulation alone reaches 1.2-1.5e-5 of the RMS (the pipelined kernel's as well)
    gate = 2e-5 if dtype == torch.float32 and cin > 256 else GATE[dtype]
    assert oconv.rel_err(y.float().cpu().numpy(), ref) <= gate


def test_halo_plan_resolves_the_table(cuda):
    """Halo plan kernel, exact: every (row, offset) of every tile resolves through its
    halo position to the table's input row (absent stays absent), each halo is sorted
    and unique with the unused tail (and always the last slot) absent, each output row
    appears once, and the 32-row block masks are the OR of the rows' presence."""
    from hi3d_amd import kmap

    rng = np.random.default_rng(17)
    idx = _rand_indices(rng, 28, 0.12, batch=2)
    km = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [28] * 3, 2)
    hp = km.plan().halo()
    assert hp is not None
    n = km.n
    table = km.table.cpu().numpy()
    rows = hp.rows.cpu().numpy().reshape(hp.ntiles, 256)
    halo = hp.halo.cpu().numpy()
    hcount = hp.hcount.cpu().numpy()
    loff = hp.loff.cpu().numpy().view(np.uint16).reshape(hp.ntiles, 256, 32)
    bmask = hp.bmask.cpu().numpy().view(np.uint32).reshape(hp.ntiles, 8)
    assert np.array_equal(np.sort(rows[rows >= 0]), np.arange(n))
    for t in range(hp.ntiles):
        h = halo[t]
        c = int(hcount[t])
        assert np.all(np.diff(h[:c]) > 0) and np.all(h[c:] == n) and h[-1] == n
        for r in range(256):
            o = rows[t, r]
            want = table[o] if o >= 0 else np.full(27, n)
            got = np.where(loff[t, r, :27] == 0xFFFF, n, h[np.minimum(loff[t, r, :27], 767)])
            assert np.array_equal(got, np.where(want < n, want, n)), (t, r)
            assert np.all(loff[t, r, 27:] == 0xFFFF)
        for b in range(8):
            sub = [rows[t, r] for r in range(32 * b, 32 * b + 32) if rows[t, r] >= 0]
            m = 0
            for o in sub:
                for k in range(27):
                    if table[o, k] < n:
                        m |= 1 << k
            assert bmask[t, b] == m


@pytest.mark.parametrize("dtype,cin,cout,density,act,res", [
    (torch.float16, 128, 128, 0.15, None, False), (torch.bfloat16, 256, 256, 0.2, "silu", True),
    (torch.float16, 192, 384, 0.05, None, True), (torch.float16, 128, 128, 0.004, "silu", False),
])
def test_halo_conv_matches_float64_and_tile_plan(cuda, dtype, cin, cout, density, act, res):
    """The halo convolution (fp16/bf16, Cout % 128 == 0, 256..512-byte rows) against
    the float64 oracle, and against the tile-plan kernels on the same inputs."""
    from hi3d_amd import conv, kmap

    rng = np.random.default_rng(cin + cout * 3 + int(density * 1000))
    idx = _rand_indices(rng, 24, density, batch=2)
    km = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [24] * 3, 2)
    plan = km.plan()
    assert plan.halo() is not None
    x, w, b = _case(rng, len(idx), cin, cout, dtype)
    r = torch.as_tensor(rng.standard_normal((len(idx), cout), dtype=np.float32)).to(dtype) if res else None
    args = (x.to(cuda), plan, w.to(cuda), b.to(cuda), act, None if r is None else r.to(cuda))
    conv.HALO = True
    try:
        y = conv.gather_conv(*args)
    finally:
        conv.HALO = False
    ref = oconv.gather_conv_f64(x.float().numpy(), km.table.cpu().numpy(), w.float().numpy(), b.float().numpy(),
                                act=act, residual=None if r is None else r.float().numpy())
    assert oconv.rel_err(y.float().cpu().numpy(), ref) <= GATE[dtype]
    y2 = conv.gather_conv(*args)
    assert oconv.rel_err(y.float().cpu().numpy(), y2.float().cpu().numpy().astype(np.float64)) <= GATE[dtype]


@pytest.mark.parametrize("side,density,batch,kvol,act,res", [
    (24, 0.15, 2, 27, "silu", True), (24, 0.004, 2, 27, None, False), (20, 0.5, 1, 27, None, True),
    (24, 0.2, 2, 8, "silu", False), (30, 0.05, 3, 27, None, False),
])
def test_fp32_block_kernel(cuda, side, density, batch, kvol, act, res):
    """The fp32 64 -> 64 kernel of 16-row blocks (each wave runs only the offsets present
    in its rows, the workgroup walks their union): against float64 with SiLU and the
    residual, isolated voxels (blocks whose only offset is the centre), a dense set
    (every offset present), a few-offset table, and set sizes that end in a partial
    workgroup; and bitwise independent of the plan's tile order (each row sums its
    offsets in increasing order whatever block it lands in)."""
    from hi3d_amd import conv, kmap

    rng = np.random.default_rng(side * 100 + kvol + int(density * 1000))
    idx = _rand_indices(rng, side, density, batch=batch)
    n = len(idx)
    if kvol == 27:
        table = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [side] * 3, batch).table
    else:
        t = rng.integers(0, n + 1, (n - 5, kvol)).astype(np.int32)
        t[rng.random(t.shape) < 0.6] = n
        table = torch.as_tensor(t).to(cuda)
    x, w, b = _case(rng, n, 64, 64, torch.float32, kvol)
    r = torch.as_tensor(rng.standard_normal((int(table.shape[0]), 64), dtype=np.float32)) if res else None
    xd, wd, bd = x.to(cuda), w.to(cuda), b.to(cuda)
    rd = None if r is None else r.to(cuda)
    y = conv.gather_conv(xd, kmap.build_plan(table, n), wd, bd, act=act, residual=rd)
    ref = oconv.gather_conv_f64(x.numpy(), table.cpu().numpy(), w.numpy(), b.numpy(), act=act,
                                residual=None if r is None else r.numpy())
    assert y.dtype == torch.float32 and y.shape == (int(table.shape[0]), 64)
    assert oconv.rel_err(y.cpu().numpy(), ref) <= GATE[torch.float32]
    y2 = conv.gather_conv(xd, kmap.build_plan(table, n, window_rows=64), wd, bd, act=act, residual=rd)
    assert torch.equal(y, y2)


@pytest.mark.parametrize("dtype,mode", [
    (torch.float16, "one"), (torch.float16, "mixed"), (torch.bfloat16, "mixed"), (torch.float16, "blocks"),
])
def test_wide_kernel_128_byte_rows(cuda, dtype, mode):
    """Few-offset tables of 128-byte rows into 128 outputs (the stride-2
    down-convolution's shape) run the 128-byte-step wide kernel, where a tile with one
    offset has a single K stage: every tile one offset ("one"), random tables ("mixed"),
    and tiles of one offset, of two and of none in one launch ("blocks"), with partial
    tiles at the end; against float64."""
    from hi3d_amd import conv, kmap

    rng = np.random.default_rng({"one": 1, "mixed": 2, "blocks": 3}[mode] + (10 if dtype == torch.bfloat16 else 0))
    n_in, n_out = 3001, 1300
    t = np.full((n_out, 8), n_in, np.int32)
    if mode == "one":
        t[:, 5] = rng.integers(0, n_in, n_out)
    elif mode == "mixed":
        t = rng.integers(0, n_in + 1, (n_out, 8)).astype(np.int32)
        t[rng.random(t.shape) < 0.6] = n_in
    else:
        t[:512, 3] = rng.integers(0, n_in, 512)
        t[512:1024, 1] = rng.integers(0, n_in, 512)
        t[512:1024, 6] = rng.integers(0, n_in, 512)
    x = torch.as_tensor(rng.standard_normal((n_in, 64), dtype=np.float32)).to(dtype)
    w = torch.as_tensor(rng.standard_normal((128, 8, 64), dtype=np.float32) / np.sqrt(8 * 64)).to(dtype)
    b = torch.as_tensor(rng.standard_normal(128, dtype=np.float32) * 0.1).to(dtype)
    table = torch.as_tensor(t).to(cuda)
    y = conv.gather_conv(x.to(cuda), kmap.build_plan(table, n_in), w.to(cuda), b.to(cuda))
    ref = oconv.gather_conv_f64(x.float().numpy(), t, w.float().numpy(), b.float().numpy())
    assert y.dtype == dtype and y.shape == (n_out, 128)
    assert oconv.rel_err(y.float().cpu().numpy(), ref) <= GATE[dtype]


def test_plan_choice_does_not_change_results(cuda):
    """Within a kernel family the output is bitwise independent of the plan: the tile-plan
    kernels accumulate each row's present (offset, K-block) products in the same order
    under any tiling or window, and the halo kernel accumulates (K step, offset) in the
    same order in every halo tile. The two families sum in different orders and agree
    to the fp16 gate."""
    from hi3d_amd import conv, kmap

    rng = np.random.default_rng(6)
    idx = _rand_indices(rng, 32, 0.1)
    km = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [32] * 3, 1)
    x, w, b = _case(rng, len(idx), 128, 128, torch.float16)
    x, w, b = x.to(cuda), w.to(cuda), b.to(cuda)
    plans = [kmap.build_plan(km.table, km.n, coords, win)
             for coords, win in ((km.indices, 0), (km.indices, 512), (None, 0), (None, 4096))]
    outs = [conv.gather_conv(x, p, w, b) for p in plans]
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    conv.HALO = True
    try:
        halo_outs = [conv.gather_conv(x, p, w, b) for p in plans if p.halo() is not None]
    finally:
        conv.HALO = False
    assert halo_outs, "the Morton-ordered plan has a halo plan"
    for o in halo_outs[1:]:
        assert torch.equal(o, halo_outs[0])
    assert oconv.rel_err(halo_outs[0].float().cpu().numpy(), outs[0].float().cpu().numpy().astype(np.float64)) <= 1e-2


@pytest.mark.parametrize("dtype,act,res", [(torch.float16, None, False), (torch.float16, "silu", True),
                                           (torch.bfloat16, "silu", False)])
def test_wide2_offset_skips_are_exact(cuda, dtype, act, res):
    """The 256 x 256 kernel's waves skip the MFMAs of offsets that none of their 64 rows
    has. On a sphere shell (structured masks, so many 64-row blocks lack offsets of their
    256-row tile) the output is bitwise the same under plans that skip different
    (block, offset) pairs, and within the fp16 gate of float64."""
    from hi3d_amd import conv, kmap, workloads

    rng = np.random.default_rng(31)
    idx = workloads.sphere_shell(64, 27.0, seed=3)
    km = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [64] * 3, 1)
    x, w, b = _case(rng, len(idx), 256, 256, dtype)
    r = torch.as_tensor(rng.standard_normal((len(idx), 256), dtype=np.float32)).to(dtype) if res else None
    xd, wd, bd = x.to(cuda), w.to(cuda), b.to(cuda)
    rd = r.to(cuda) if res else None
    plans = [kmap.build_plan(km.table, km.n, coords, win)
             for coords, win in ((km.indices, 0), (km.indices, 256), (km.indices, None), (None, 0))]
    skipped = []
    for p in plans:  # (64-row block, offset) pairs a wave skips under this plan
        g = (p.gidx.reshape(p.ntiles, p.kvol, 128) < p.n_in).cpu().numpy()
        blk = g.reshape(p.ntiles, p.kvol, 2, 64).any(3)  # [plan tile, offset, half]
        tm = p.tile_mask.cpu().numpy().astype(np.int64)
        pairs = np.arange(p.ntiles) // 2
        union = np.zeros(pairs[-1] + 1, np.int64)
        np.bitwise_or.at(union, pairs, tm)
        bits = (union[pairs][:, None] >> np.arange(p.kvol)) & 1
        skipped.append(int((bits[:, :, None].astype(bool) & ~blk).sum()))
    assert min(skipped) > 0 and len(set(skipped)) > 1, skipped
    outs = [conv.gather_conv(xd, p, wd, bd, act=act, residual=rd) for p in plans]
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    ref = oconv.gather_conv_f64(x.float().numpy(), km.table.cpu().numpy(), w.float().numpy(), b.float().numpy())
    if act == "silu":
        ref = ref / (1.0 + np.exp(-ref))
    if res:
        ref = ref + r.float().numpy()
    assert outs[0].dtype == dtype
    assert oconv.rel_err(outs[0].float().cpu().numpy(), ref) <= GATE[dtype]


def test_unaligned_channels_use_simple_kernel(cuda):
    from hi3d_amd import conv, kmap

    rng = np.random.default_rng(7)
    idx = _rand_indices(rng, 12, 0.3)
    km = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [12] * 3, 1)
    for dtype, cin, cout in ((torch.float16, 12, 20), (torch.float32, 3, 5), (torch.float64, 7, 9)):
        x, w, b = _case(rng, len(idx), cin, cout, dtype)
        y = conv.conv(x.to(cuda), km.plan(), w.to(cuda), b.to(cuda))
        ref = oconv.gather_conv_f64(x.double().numpy(), km.table.cpu().numpy(), w.double().numpy(), b.double().numpy())
        tol = {torch.float16: 1e-2, torch.float32: 1e-5, torch.float64: 1e-12}[dtype]
        assert oconv.rel_err(y.double().cpu().numpy(), ref) <= tol


def test_workload1_fp32_full(cuda):
    """128^3 sphere shell, C 64->64 fp32: every output row within 1e-5 of float64."""
    from hi3d_amd import conv, kmap, workloads

    idx = workloads.coords_for("subm3_c64_fp32")
    km = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [128] * 3, 1)
    x = workloads.normal((len(idx), 64), 1.0, seed=11)
    w = workloads.normal((64, 27, 64), 1.0 / np.sqrt(27 * 64), seed=12)
    y = conv.gather_conv(torch.as_tensor(x).to(cuda), km.plan(), torch.as_tensor(w).to(cuda))
    ref = oconv.gather_conv_f64(x, km.table.cpu().numpy(), w)
    assert oconv.rel_err(y.cpu().numpy(), ref) <= 1e-5


def test_workload2_fp16_sampled(cuda):
    from hi3d_amd import conv, kmap, workloads

    idx = workloads.coords_for("subm3_c128_fp16")
    km = kmap.build_kernel_map(torch.as_tensor(idx).to(cuda), [256] * 3, 1)
    x = workloads.normal((len(idx), 128), 1.0, seed=21, dtype=np.float16)
    w = workloads.normal((128, 27, 128), 1.0 / np.sqrt(27 * 128), seed=22, dtype=np.float16)
    y = conv.gather_conv(torch.as_tensor(x).to(cuda), km.plan(), torch.as_tensor(w).to(cuda))
    rows = np.random.default_rng(0).choice(len(idx), 4096, replace=False)
    ref = oconv.gather_conv_f64(x, km.table.cpu().numpy(), w, rows=rows)
    assert oconv.rel_err(y.float().cpu().numpy()[rows], ref) <= 1e-2
    assert torch.isfinite(y).all()


def test_stride2_golden_float64(cuda):
    from hi3d_amd import spconv

    data = np.load(GOLDEN / "stride2_12cube.npz")
    idx = torch.as_tensor(data["indices"]).to(cuda)
    x = spconv.SparseConvTensor(torch.as_tensor(data["feats"]).to(cuda), idx, [12] * 3, 1)
    down = spconv.SparseConv3d(6, 10, 2, stride=2, indice_key="s2").double().to(cuda)
    up = spconv.SparseInverseConv3d(10, 6, 2, indice_key="s2").double().to(cuda)
    with torch.no_grad():
        down.weight.copy_(torch.as_tensor(data["weight"]))
        down.bias.copy_(torch.as_tensor(data["bias"]))
        up.weight.copy_(torch.as_tensor(data["up_weight"]))
        up.bias.copy_(torch.as_tensor(data["up_bias"]))
    y = down(x)
    assert np.array_equal(y.indices.cpu().numpy(), data["low"]) and y.spatial_shape == [6, 6, 6]
    assert np.allclose(y.features.cpu().numpy(), data["down_out"], atol=1e-12)
    z = up(y)
    assert z.indices is idx and z.spatial_shape == [12, 12, 12]
    assert np.allclose(z.features.cpu().numpy(), data["up_out"], atol=1e-11)


def test_stride2_workload_fp16(cuda):
    """512^3 shell, fp16: down 64->128 then up 128->64 against float64 gather sums."""
    from hi3d_amd import conv, kmap, workloads

    idx = workloads.coords_for("down2_up2_c64_c128_fp16")
    s = kmap.stride2_structure(torch.as_tensor(idx).to(cuda), [512] * 3, 1)
    x = workloads.normal((len(idx), 64), 1.0, seed=31, dtype=np.float16)
    wd = workloads.normal((128, 8, 64), 1.0 / np.sqrt(8 * 64), seed=32, dtype=np.float16)
    wu = workloads.normal((64, 8, 128), 1.0 / np.sqrt(8 * 128), seed=33, dtype=np.float16)
    y = conv.gather_conv(torch.as_tensor(x).to(cuda), s.down_plan(), torch.as_tensor(wd).to(cuda))
    z = conv.gather_conv(y, s.up_plan(), torch.as_tensor(wu).to(cuda))
    down_t, up_t = s.down.cpu().numpy(), s.up.cpu().numpy()
    rows_c = np.random.default_rng(1).choice(s.n_coarse, 4096, replace=False)
    ref_y = oconv.gather_conv_f64(x, down_t, wd, rows=rows_c)
    assert oconv.rel_err(y.float().cpu().numpy()[rows_c], ref_y) <= 1e-2
    rows_f = np.random.default_rng(2).choice(s.n_fine, 4096, replace=False)
    ref_z = oconv.gather_conv_f64(y.float().cpu().numpy(), up_t, wu, rows=rows_f)
    assert oconv.rel_err(z.float().cpu().numpy()[rows_f], ref_z) <= 1e-2


def test_gather_mean_pooling(cuda):
    from hi3d_amd import nn as snn

    rng = np.random.default_rng(8)
    idx = _rand_indices(rng, 10, 0.4)
    idx = idx[np.argsort(idx[:, 0], kind="stable")]
    x = rng.standard_normal((len(idx), 16)).astype(np.float32)
    t = snn.SparseTensor(torch.as_tensor(x).to(cuda), torch.as_tensor(idx).to(cuda))
    pooled = snn.SparseDownsample(2)(t)
    low, inverse, counts, slot, down, up = okmap.stride2_structure(idx)
    assert np.array_equal(pooled.coords.cpu().numpy(), low)
    assert np.allclose(pooled.feats.cpu().numpy(), oconv.gather_mean(x, down, 1), atol=1e-6)
    back = snn.SparseUpsample(2)(pooled)
    assert torch.equal(back.coords, t.coords)
    assert np.allclose(back.feats.cpu().numpy(), pooled.feats.cpu().numpy()[inverse])


@pytest.mark.parametrize("dtype,cin,n_side,density,with_bias", [
    (torch.float16, 128, 20, 0.3, True), (torch.bfloat16, 128, 16, 0.5, False), (torch.float16, 64, 24, 0.2, True),
    (torch.bfloat16, 64, 9, 0.9, True),
])
def test_stride2_up_parent_major(cuda, dtype, cin, n_side, density, with_bias):
    """The parent-major transposed kernel against float64 and bit for bit against the
    gather convolution over the up table (both sum each output's 8-slot products in the
    same K order and add the bias in fp32 once); coarse sets that are not a multiple of
    the 32-row tile, parents with one to eight children."""
    from hi3d_amd import conv, kmap

    rng = np.random.default_rng(cin + n_side)
    idx = _rand_indices(rng, n_side, density)
    s = kmap.stride2_structure(torch.as_tensor(idx).to(cuda), [n_side] * 3, 1)
    y = torch.as_tensor(rng.standard_normal((s.n_coarse, cin), dtype=np.float32)).to(dtype).to(cuda)
    w = torch.as_tensor(rng.standard_normal((64, 2, 2, 2, cin), dtype=np.float32) / np.sqrt(8 * cin)).to(dtype).to(cuda)
    b = torch.as_tensor(rng.standard_normal(64, dtype=np.float32) * 0.1).to(dtype).to(cuda) if with_bias else None
    assert conv.stride2_up_supported(dtype, cin, 64)
    z = conv.stride2_up(y, s, w, b)
    assert z.shape == (s.n_fine, 64) and z.dtype == dtype
    gathered = conv.gather_conv(y, s.up_plan(), w.reshape(64, 8, cin), b)
    assert torch.equal(z, gathered)
    ref = oconv.gather_conv_f64(y.float().cpu().numpy(), s.up.cpu().numpy(), w.reshape(64, 8, cin).float().cpu().numpy(),
                                None if b is None else b.float().cpu().numpy())
    assert oconv.rel_err(z.float().cpu().numpy(), ref) <= GATE[dtype]
    out = torch.full_like(z, float("nan"))
    assert conv.stride2_up(y, s, w, b, out=out) is out and torch.equal(out, z)
    # rows in the mask-sorted order (the default) and in row order: the same bits
    assert torch.equal(conv.stride2_up(y, s, w, b, sorted_rows=False), z)
    assert torch.equal(conv.stride2_up(y, s, w, b, sorted_rows=True), z)


def test_stride2_up_workload_fp16(cuda):
    """512^3 shells, C128 -> 64 fp16: every fine row written, bit-equal to the gather
    convolution, and within the fp16 gate of float64 on sampled rows."""
    from hi3d_amd import conv, kmap, workloads

    idx = workloads.coords_for("down2_up2_c64_c128_fp16")
    s = kmap.stride2_structure(torch.as_tensor(idx).to(cuda), [512] * 3, 1)
    y = torch.as_tensor(workloads.normal((s.n_coarse, 128), 1.0, 41, np.float16)).to(cuda)
    w = torch.as_tensor(workloads.normal((64, 8, 128), 1.0 / np.sqrt(8 * 128), 42, np.float16)).to(cuda)
    z = conv.stride2_up(y, s, w, None, out=torch.full((s.n_fine, 64), float("nan"), dtype=torch.float16, device=cuda))
    assert bool(torch.isfinite(z).all())
    assert torch.equal(z, conv.gather_conv(y, s.up_plan(), w))
    for sorted_rows in (False, True):
        again = torch.full((s.n_fine, 64), float("nan"), dtype=torch.float16, device=cuda)
        assert torch.equal(conv.stride2_up(y, s, w, None, out=again, sorted_rows=sorted_rows), z)
    rows = np.random.default_rng(3).choice(s.n_fine, 4096, replace=False)
    ref = oconv.gather_conv_f64(y.float().cpu().numpy(), s.up.cpu().numpy(), w.float().cpu().numpy(), rows=rows)
    assert oconv.rel_err(z.float().cpu().numpy()[rows], ref) <= 1e-2


@pytest.mark.parametrize("window_log2", [31, 4, 0])
def test_stride2_up_order_plan(cuda, window_log2):
    """The sorted up convolution's plan: ``order`` is a permutation of the coarse rows
    (padded with row n_c - 1 to whole 32-row tiles), stable-sorted by (row window, slot
    mask of the row's children); ``down_sorted`` is ``down[order]`` with absent padding;
    the convolution over it equals the row-order kernel bit for bit."""
    from hi3d_amd import conv, kmap

    rng = np.random.default_rng(90 + window_log2)
    idx = _rand_indices(rng, 21, 0.25, batch=2)
    s = kmap.stride2_structure(torch.as_tensor(idx).to(cuda), [21] * 3, 2)
    order, down_sorted = s.up_order(window_log2)
    n_c, n_f = s.n_coarse, s.n_fine
    down = s.down.cpu().numpy()
    mask = ((down < n_f) * (1 << np.arange(8))).sum(1)
    key = ((np.arange(n_c) >> window_log2) << 8) | mask
    want = np.argsort(key, kind="stable")
    npad = (n_c + 31) // 32 * 32
    o = order.cpu().numpy()
    assert o.shape == (npad,) and np.array_equal(o[:n_c], want) and np.all(o[n_c:] == n_c - 1)
    ds = down_sorted.cpu().numpy()
    assert np.array_equal(ds[:n_c], down[want]) and np.all(ds[n_c:] == n_f)
    y = torch.as_tensor(rng.standard_normal((n_c, 128), dtype=np.float32)).half().to(cuda)
    w = torch.as_tensor(rng.standard_normal((64, 8, 128), dtype=np.float32) / 32).half().to(cuda)
    old = kmap.UP_ORDER_WINDOW_LOG2
    try:
        kmap.UP_ORDER_WINDOW_LOG2 = window_log2
        assert torch.equal(conv.stride2_up(y, s, w, sorted_rows=True), conv.stride2_up(y, s, w, sorted_rows=False))
    finally:
        kmap.UP_ORDER_WINDOW_LOG2 = old
