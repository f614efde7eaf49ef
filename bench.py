"""Benchmark of the Hi3D sparse hot path on one MI355X.

Headline (``value``): voxels/s of the sparse residual block, C256 fp16 with fp32
accumulation, on the 1024^3 union of 8 seeded ellipsoid 1-voxel shells (~4.43M voxels,
kernel map cached as in the reference's usage). One step = one pass of the block over
the whole active set with inputs resident in HBM: adaLN projection of the conditioning
vector, LayerNorm + modulate, submanifold 3x3x3 conv + SiLU, conv + residual add.

``roofline`` is measured live for the block's convolution kernel (HIP events around
each convolution inside the timed steps, on the stream they run on): achieved =
2 * P * Cin * Cout / average launch time against the fp16 dense MFMA peak.
``cpu_baseline`` times the reference's CPU fallback of the block (oracle port: sort +
searchsorted map, per-offset gather / matmul / index_add_, LayerNorm) on the host cores
for a sample of output rows. ``extra`` reports the other workloads: the fp32 sphere
shell and the C128 shells (with kernel-map builds through the dense grid and the
hash), the strided pair, W8A8 int8 TOPS (GEMM alone and quantise + GEMM), the VAE
blocks, octree upsampling, transformer I/O resampling, unique cube corners and the
kernel-map builds of the 1024^3 and 256^3 shells (dense grid and brick hash), with
CPU baselines of the fp32 shell (in full) and of W8A8 (sampled tokens).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only a,b] [--quick] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "hi3dv1.0-mlx_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_FP16_TFLOPS = 2500.0
PEAK_FP32_TFLOPS = 157.3
PEAK_INT8_TOPS = 5000.0
PEAK_HBM_GBS = 8000.0

# Headline kernel (the block's C256 convolution: 256 x 256 ring tiles) and the counter
# summary that holds its measured HBM traffic per launch: FETCH_SIZE and WRITE_SIZE per dispatch from
# two rocprofv3 --pmc runs of this script, each scaled by the factor the same counter
# reads for a plain device copy of known size (`--copy-probe`).
HEADLINE_KERNEL = "conv_wide2_kernel<_Float16>"
TRAFFIC_SUMMARY = ROOT / "profiles" / "conv_wide2_resblock_c256_fp16_traffic.txt"


def measured_traffic():
    """HBM bytes per headline-kernel launch from the committed counter summary, or None."""
    try:
        for line in TRAFFIC_SUMMARY.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch"):
                return float(line.split("=", 1)[1])
    except (OSError, ValueError):
        pass
    return None


_COORDS: dict = {}


def coords_of(name: str, device=None):
    """Seeded voxel coordinates of a workload, generated once per run (on the GPU when a
    device is given) and shared by its GPU and host measurements."""
    if name not in _COORDS:
        from hi3d_amd import workloads

        _COORDS[name] = workloads.coords_for(name, device=device) if device is not None else workloads.coords_for(name)
    return _COORDS[name]


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


SETTLE_EACH_S = 0.3
"""Seconds of untimed calls before each timed measurement (after its warm-up): the shader
clock ramps under sustained load, and a few warm-up calls of a sub-millisecond kernel do
not reach it (the C128 layer: 0.44 ms per call after 5 warm-up calls, 0.39 ms after
2 s of calls on the same box)."""


def settle(fn, seconds: float) -> None:
    """Call fn repeatedly for about `seconds`, synchronising at least every 10 calls (so
    the host never queues far ahead of the GPU) and stopping at the first call that ends
    past the deadline (so an expensive call is not repeated ten times)."""
    import torch

    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(10):
            fn()
            if time.perf_counter() >= t_end:
                break
        torch.cuda.synchronize()


def timed(fn, steps: int, warmup: int, settle_s: float | None = None):
    """(ms per call from host clock around `steps` calls, mean per-call ms from events).
    settle_s: seconds of untimed calls after the warm-up (default SETTLE_EACH_S; 0 for a
    call that consumes its input)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    settle(fn, SETTLE_EACH_S if settle_s is None else settle_s)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    ev = sum(s.elapsed_time(e) for s, e in zip(starts, ends)) / steps
    return wall, ev


def timed_batch(fn, steps: int, warmup: int) -> float:
    """Mean ms per call over `steps` back-to-back calls between two events: the GPU stays
    busy while the host queues the next launch, so a short kernel is timed without the
    host's per-call overhead (events around each call would include it)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    settle(fn, SETTLE_EACH_S)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def dense_path(fn, keep: bool = True):
    """Run a kernel-map build through the dense grid whatever the grid size (kept between
    builds, or cleared inside the call)."""
    from hi3d_amd import kmap

    def run():
        old = kmap.KMAP_DENSE_KEEP, kmap.KMAP_DENSE_MAX_CELLS
        kmap.KMAP_DENSE_KEEP, kmap.KMAP_DENSE_MAX_CELLS = keep, 1 << 31
        try:
            return fn()
        finally:
            kmap.KMAP_DENSE_KEEP, kmap.KMAP_DENSE_MAX_CELLS = old

    return run


def dense_fresh(fn):
    """Run a kernel-map build with a dense grid cleared inside the call (not kept)."""
    return dense_path(fn, keep=False)


def bench_subm(name: str, grid: int, cin: int, cout: int, dtype, steps: int, warmup: int, seed: int = 0):
    import numpy as np
    import torch

    from hi3d_amd import conv, kmap, workloads

    dev = torch.device("cuda:0")
    idx = coords_of(name, dev)
    n = len(idx)
    coords = torch.as_tensor(idx).to(dev)
    np_dtype = np.float16 if dtype == torch.float16 else np.float32
    x = torch.as_tensor(workloads.normal((n, cin), 1.0, seed + 1, np_dtype)).to(dev)
    w = torch.as_tensor(workloads.normal((cout, 27, cin), 1.0 / np.sqrt(27 * cin), seed + 2, np_dtype)).to(dev)
    # kernel map build (hash insert + probe) and plan, timed separately
    map_wall, _ = timed(lambda: kmap.build_kernel_map(coords, [grid] * 3, 1, check=False), 5, 2)
    _, map_ev = timed(dense_path(lambda: kmap.build_kernel_map(coords, [grid] * 3, 1, check=False)), 5, 2)
    hash_wall, hash_ev = timed(lambda: kmap.build_kernel_map(coords, [grid] * 3, 1, capacity=0, check=False), 5, 2)
    _, fresh_ev = timed(dense_fresh(lambda: kmap.build_kernel_map(coords, [grid] * 3, 1, check=False)), 5, 2)
    km = kmap.build_kernel_map(coords, [grid] * 3, 1)
    bits = kmap.morton_bits(km.spatial_shape, km.batch_size)  # as KernelMap.plan() builds it
    plan_wall, plan_ev = timed(lambda: kmap.build_plan(km.table, km.n, km.indices, None, bits), 3, 1)
    plan = km.plan()
    pairs = int(km.counts.sum())
    out = torch.empty((n, cout), dtype=dtype, device=dev)
    wall, ev = timed(lambda: conv.gather_conv(x, plan, w, None, out=out), steps, warmup)
    flops = 2.0 * pairs * cin * cout
    es = 2 if dtype == torch.float16 else 4
    conv_bytes = es * (n * cin + n * cout + 27 * cin * cout) + 4 * 27 * n
    map_bytes = n * (16 + 8) + n * (16 + 26 * 8 + 108)
    return {
        "workload": name,
        "voxels": n,
        "pairs": pairs,
        "cin": cin,
        "cout": cout,
        "dtype": "fp16" if dtype == torch.float16 else "fp32",
        "conv_ms": wall,
        "conv_kernel_ms": ev,
        "voxels_per_s": n / (wall * 1e-3),
        "eff_tflops": flops / (ev * 1e-3) / 1e12,
        # dense MFMA peak of the compute type (fp32 157.3, fp16 2500 TFLOP/s)
        "mfma_frac": flops / (ev * 1e-3) / 1e12 / (2500.0 if dtype == torch.float16 else 157.3),
        "conv_alg_bytes": conv_bytes,
        "map_ms": map_wall,
        "map_dense_ms": map_ev,
        "map_dense_fresh_ms": fresh_ev,
        "map_hash_ms": hash_ev,
        "map_alg_gbs_hash": map_bytes / (hash_ev * 1e-3) / 1e9,
        "plan_ms": plan_wall,
        "flops": flops,
        "tile_rows": int(plan.rows.shape[0]) // max(plan.ntiles, 1),
    }


def bench_stride2(steps: int, warmup: int):
    import numpy as np
    import torch

    from hi3d_amd import conv, kmap, workloads

    dev = torch.device("cuda:0")
    idx = coords_of("down2_up2_c64_c128_fp16", dev)
    coords = torch.as_tensor(idx).to(dev)
    map_wall, _ = timed(lambda: kmap.stride2_structure(coords, [512] * 3, 1), 3, 1)
    s = kmap.stride2_structure(coords, [512] * 3, 1)
    dp, up = s.down_plan(), s.up_plan()
    nf, nc = s.n_fine, s.n_coarse
    x = torch.as_tensor(workloads.normal((nf, 64), 1.0, 31, np.float16)).to(dev)
    wd = torch.as_tensor(workloads.normal((128, 8, 64), 1.0 / np.sqrt(8 * 64), 32, np.float16)).to(dev)
    wu = torch.as_tensor(workloads.normal((64, 8, 128), 1.0 / np.sqrt(8 * 128), 33, np.float16)).to(dev)
    y = torch.empty((nc, 128), dtype=torch.float16, device=dev)
    z = torch.empty((nf, 64), dtype=torch.float16, device=dev)
    s.up_order()  # the sorted up convolution's plan, built with the structure's other plans
    d_wall, d_ev = timed(lambda: conv.gather_conv(x, dp, wd, None, out=y), steps, warmup)
    u_wall, u_ev = timed(lambda: conv.stride2_up(y, s, wu, None, out=z), steps, warmup)
    ug_wall, ug_ev = timed(lambda: conv.gather_conv(y, up, wu, None, out=z), steps, warmup)
    # kernel time: back-to-back launches between two events
    d_k = timed_batch(lambda: conv.gather_conv(x, dp, wd, None, out=y), 4 * steps, warmup)
    u_k = timed_batch(lambda: conv.stride2_up(y, s, wu, None, out=z), 4 * steps, warmup)
    u_k_rows = timed_batch(lambda: conv.stride2_up(y, s, wu, None, out=z, sorted_rows=False), 4 * steps, warmup)
    flops = 2.0 * nf * 64 * 128
    bytes_conv = 2 * (nf * 64 + nc * 128 + 8 * 64 * 128) + 5 * nf
    return {
        "workload": "down2_up2_c64_c128_fp16",
        "fine_voxels": nf,
        "coarse_voxels": nc,
        "structure_ms": map_wall,
        "down_ms": d_wall,
        "up_ms": u_wall,
        "up_gather_ms": ug_wall,
        "down_kernel_ms": d_k,
        "up_kernel_ms": u_k,
        "up_kernel_row_order_ms": u_k_rows,
        "down_call_gbs_alg": bytes_conv / (d_ev * 1e-3) / 1e9,
        "up_call_gbs_alg": bytes_conv / (u_ev * 1e-3) / 1e9,
        "down_tflops": flops / (d_k * 1e-3) / 1e12,
        "up_tflops": flops / (u_k * 1e-3) / 1e12,
        "down_gbs_alg": bytes_conv / (d_k * 1e-3) / 1e9,
        "up_gbs_alg": bytes_conv / (u_k * 1e-3) / 1e9,
        "down_hbm_frac": bytes_conv / (d_k * 1e-3) / 1e9 / PEAK_HBM_GBS,
        "up_hbm_frac": bytes_conv / (u_k * 1e-3) / 1e9 / PEAK_HBM_GBS,
        "voxels_per_s": nf / ((d_wall + u_wall) * 1e-3),
    }


def bench_w8a8(steps: int, warmup: int):
    import numpy as np
    import torch

    from hi3d_amd import w8a8

    dev = torch.device("cuda:0")
    res = {}
    for tag, (m, k, n) in {"A": (65536, 1024, 4096), "B": (65536, 4096, 1024)}.items():
        g = torch.Generator(device=dev).manual_seed(k)
        x = torch.randn((m, k), device=dev, generator=g, dtype=torch.float32)
        mask = torch.rand((m, k), device=dev, generator=g) < 0.01
        x = torch.where(mask, x * 20, x).half()
        wf = (torch.randn((n, k), device=dev, generator=g) / 32).half()
        bias = (torch.randn(n, device=dev, generator=g) * 0.02).half()
        for rotation in ("h64", "none"):
            wq, sw = w8a8.quantize_weight(wf, rotation)
            q, sa = w8a8.quantize_activation(x, rotation=rotation)
            out = w8a8.gemm(q, sa, wq, sw, bias)
            g_wall, g_ev = timed(lambda: w8a8.gemm(q, sa, wq, sw, bias), steps, warmup)
            q_wall, q_ev = timed(lambda: w8a8.quantize_activation(x, rotation=rotation), steps, warmup)
            e_wall, _ = timed(lambda: w8a8.linear(x, wq, sw, bias, rotation=rotation), steps, warmup)
            ops = 2.0 * m * n * k
            del out
            res[f"{tag}_{rotation}"] = {
                "m": m, "k": k, "n": n,
                "gemm_ms": g_ev, "gemm_tops": ops / (g_ev * 1e-3) / 1e12,
                "gemm_frac": ops / (g_ev * 1e-3) / 1e12 / PEAK_INT8_TOPS,
                "quant_ms": q_ev, "quant_gbs": (2 * m * k + m * k + 4 * m) / (q_ev * 1e-3) / 1e9,
                "e2e_ms": e_wall, "e2e_tops": ops / (e_wall * 1e-3) / 1e12,
            }
        if tag == "A":
            # shape A as the transformer block feeds it (mlp.0 after the modulated norm):
            # norm, quantiser and GEMM in sequence against the norm fused with the
            # quantiser, then the GEMM
            from hi3d_amd import kernels

            scale = (1 + 0.2 * torch.randn(k, device=dev, generator=g)).half()
            shift = (0.2 * torch.randn(k, device=dev, generator=g)).half()
            wq, sw = w8a8.quantize_weight(wf)
            _, ln_ev = timed(lambda: kernels.layer_norm_modulate(x, 1e-6, scale=scale, shift=shift), steps, warmup)
            _, nq_ev = timed(lambda: w8a8.norm_quantize(x, 1e-6, scale=scale, shift=shift), steps, warmup)
            seq_wall, _ = timed(lambda: w8a8.linear(kernels.layer_norm_modulate(x, 1e-6, scale=scale, shift=shift),
                                                    wq, sw, bias), steps, warmup)
            fused_wall, _ = timed(lambda: w8a8.norm_linear(x, 1e-6, wq, sw, bias, scale=scale, shift=shift), steps,
                                  warmup)
            ops = 2.0 * m * n * k
            res["A_norm_h64"] = {
                "m": m, "k": k, "n": n,
                "norm_ms": ln_ev,
                "norm_quant_ms": nq_ev, "norm_quant_gbs": (2 * m * k + m * k + 4 * m) / (nq_ev * 1e-3) / 1e9,
                "norm_then_linear_ms": seq_wall, "norm_linear_fused_ms": fused_wall,
                "fused_e2e_tops": ops / (fused_wall * 1e-3) / 1e12,
            }
    return res


def bench_block(steps: int, warmup: int, settle_s: float = 0.0):
    """The residual block on the 1024^3 shells, C256 fp16: one step = adaLN projection,
    LayerNorm + modulate, conv + SiLU, conv + residual over every voxel. HIP events
    around each convolution inside the timed steps give the convolution kernel's average
    launch time (both run on the current stream)."""
    import numpy as np
    import torch

    from hi3d_amd import block, kernels, kmap, workloads
    from hi3d_amd.block import ResBlockWeights

    dev = torch.device("cuda:0")
    idx = coords_of("resblock_c256_fp16", dev)
    n = len(idx)
    c, d = 256, 1024
    coords = torch.as_tensor(idx).to(dev)
    map_wall, _ = timed(lambda: kmap.build_kernel_map(coords, [1024] * 3, 1, check=False), 3, 1)
    _, map_ev = timed(dense_path(lambda: kmap.build_kernel_map(coords, [1024] * 3, 1, check=False)), 3, 1)
    hash_wall, hash_ev = timed(lambda: kmap.build_kernel_map(coords, [1024] * 3, 1, capacity=0, check=False), 3, 1)
    _, fresh_ev = timed(dense_fresh(lambda: kmap.build_kernel_map(coords, [1024] * 3, 1, check=False)), 3, 1)
    km = kmap.build_kernel_map(coords, [1024] * 3, 1)
    bits = kmap.morton_bits(km.spatial_shape, km.batch_size)  # as KernelMap.plan() builds it
    plan_wall, plan_ev = timed(lambda: kmap.build_plan(km.table, km.n, km.indices, None, bits), 3, 1)
    plan = km.plan()
    pairs = int(km.counts.sum())
    x = torch.as_tensor(workloads.normal((n, c), 1.0, 52, np.float16)).to(dev)
    cond = torch.as_tensor(workloads.normal((d,), 1.0, 53)).to(dev)
    weights = ResBlockWeights(
        torch.as_tensor(workloads.normal((2 * c, d), 1.0 / np.sqrt(d), 54)).to(dev),
        torch.as_tensor(workloads.normal((2 * c,), 0.02, 55)).to(dev),
        torch.as_tensor(workloads.normal((c, 27, c), 1.0 / np.sqrt(27 * c), 56, np.float16)).to(dev), None,
        torch.as_tensor(workloads.normal((c, 27, c), 1.0 / np.sqrt(27 * c), 57, np.float16)).to(dev), None,
    )
    # clocks settle on untimed passes first (the shader clock ramps under sustained load)
    t_end = time.perf_counter() + settle_s
    while time.perf_counter() < t_end:
        block.residual_block(x, plan, cond, weights)
        torch.cuda.synchronize()
    for _ in range(warmup):
        block.residual_block(x, plan, cond, weights)
    torch.cuda.synchronize()
    conv_ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        block.residual_block(x, plan, cond, weights, conv_events=conv_ev[i])
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    conv_ms = [e[0].elapsed_time(e[1]) for e in conv_ev] + [e[1].elapsed_time(e[2]) for e in conv_ev]
    conv_avg = sum(conv_ms) / len(conv_ms)
    s1p, sh = kernels.adaln_projection(weights.proj_weight, weights.proj_bias, cond)
    ln_wall, ln_ev = timed(lambda: kernels.layer_norm_modulate(x, 1e-6, scale=s1p, shift=sh), steps, warmup)
    conv_flops = 2.0 * pairs * c * c
    conv_bytes = 2 * (n * c + n * c + 27 * c * c) + 4 * 27 * n
    return {
        "workload": "resblock_c256_fp16",
        "voxels": n,
        "pairs": pairs,
        "channels": c,
        "block_ms": wall,
        "voxels_per_s": n / (wall * 1e-3),
        "block_eff_tflops": 2 * conv_flops / (wall * 1e-3) / 1e12,
        "conv_kernel_ms": conv_avg,
        "conv_kernel_ms_min": min(conv_ms),
        "conv_flops": conv_flops,
        "conv_alg_bytes": conv_bytes,
        "conv_eff_tflops": conv_flops / (conv_avg * 1e-3) / 1e12,
        "ln_ms": ln_ev,
        "ln_gbs": 4.0 * n * c / (ln_ev * 1e-3) / 1e9,
        "map_ms": map_wall,
        "map_dense_ms": map_ev,
        "map_dense_fresh_ms": fresh_ev,
        "map_hash_ms": hash_ev,
        "map_alg_gbs_hash": n * 356 / (hash_ev * 1e-3) / 1e9,
        "plan_ms": plan_ev,
    }


def bench_resblock3d(steps: int, warmup: int):
    """The transformer's own residual block (``SparseResBlock3d(256, 2112)``: norm1 +
    SiLU, conv 256 -> 128, norm2 + modulate + SiLU, conv 128 -> 128 + SiLU, linear
    128 -> 256 + the input) on the 1024^3 shells, fp16, one batch element; the kernel
    map and plans are built before the timed passes (cached on the rows, as the
    reference's ``indice_dict``)."""
    import numpy as np
    import torch

    from hi3d_amd import workloads
    from hi3d_amd.nn import SparseTensor
    from hi3d_amd.resblock import SparseResBlock3d

    dev = torch.device("cuda:0")
    idx = coords_of("resblock_c256_fp16", dev)
    n = len(idx)
    c, d = 256, 2112
    torch.manual_seed(61)
    m = SparseResBlock3d(c, d)
    with torch.no_grad():  # the released init zeroes the linear; give it weights to move
        m.linear.weight.normal_(0, 1 / np.sqrt(m.hidden_channels))
    m = m.half().to(dev)
    x = SparseTensor(torch.as_tensor(workloads.normal((n, c), 1.0, 62, np.float16)).to(dev),
                     torch.as_tensor(idx).to(dev))
    emb = torch.as_tensor(workloads.normal((1, d), 1.0, 63, np.float16)).to(dev)
    with torch.no_grad():
        m(x, emb)  # kernel map + plans
        torch.cuda.synchronize()
        wall, ev = timed(lambda: m(x, emb), steps, warmup)
    km = x.backend_data().find_indice_pair("subm3").kmap
    pairs = int(km.counts.sum())
    h = m.hidden_channels
    flops = 2.0 * pairs * (c * h + h * h) + 2.0 * n * h * c
    return {
        "workload": "sparse_resblock3d_c256_fp16",
        "voxels": n,
        "pairs": pairs,
        "channels": c,
        "hidden": h,
        "block_ms": ev,
        "block_wall_ms": wall,
        "voxels_per_s": n / (ev * 1e-3),
        "eff_tflops": flops / (ev * 1e-3) / 1e12,
    }


def bench_vae(steps: int, warmup: int):
    """VAE decoder residual block (GroupNorm + swish -> conv, twice, + shortcut) at the
    finest decoder stage's width, C128 fp16, on the 512^3 fine shells, with its kernels
    timed apart; the block on a donated input (in-place accumulate) beside it."""
    import numpy as np
    import torch

    from hi3d_amd import kernels, sparse, vae, workloads

    dev = torch.device("cuda:0")
    idx = coords_of("down2_up2_c64_c128_fp16", dev)
    level = sparse.Level.from_coords(torch.as_tensor(idx[:, 1:]).to(dev))
    n, c = level.n, 128
    x = torch.as_tensor(workloads.normal((n, c), 1.0, 61, np.float16)).to(dev)
    p = {}
    for i, name in enumerate(("v.block.0", "v.block.3")):
        p[f"{name}.weights"] = torch.as_tensor(1.0 + workloads.normal((1, c), 0.1, 62 + i)).to(dev)
        p[f"{name}.bias"] = torch.as_tensor(workloads.normal((1, c), 0.1, 64 + i)).to(dev)
    for i, name in enumerate(("v.block.2", "v.block.5")):
        p[f"{name}.weight"] = torch.as_tensor(workloads.normal((27 * c, c), 1.0 / np.sqrt(27 * c), 66 + i, np.float16)).to(dev)
        p[f"{name}.bias"] = torch.as_tensor(workloads.normal((c,), 0.02, 68 + i, np.float16)).to(dev)
    _, st = timed(lambda: vae.group_stats(x), steps, warmup)
    mean, inv = vae.group_stats(x)
    _, sw = timed(lambda: kernels.group_norm_swish(x, mean, inv, p["v.block.0.weights"], p["v.block.0.bias"],
                                                   torch.float16), steps, warmup)
    b_wall, b_ev = timed(lambda: vae.resnet(x, level, p, "v"), max(3, steps // 5), max(1, warmup // 2))
    pool = [x.clone() for _ in range(6)]  # each in-place call consumes its input
    ip_wall, _ = timed(lambda: vae.resnet([pool.pop()], level, p, "v"), 5, 1, settle_s=0.0)
    pairs = int((level.table < n).sum())
    return {
        "workload": "vae_resnet_c128_fp16",
        "voxels": n,
        "block_ms": b_wall,
        "block_in_place_ms": ip_wall,
        "block_conv_tflops": 2 * 2.0 * pairs * c * c / (b_wall * 1e-3) / 1e12,
        "group_stats_ms": st,
        "group_stats_gbs": n * c * 2 / (st * 1e-3) / 1e9,
        "gn_swish_ms": sw,
        "gn_swish_gbs": 2 * n * c * 2 / (sw * 1e-3) / 1e9,
        "voxels_per_s": n / (b_wall * 1e-3),
    }


def bench_upsample(steps: int, warmup: int):
    """One decoder octree upsampling at C256 fp16: the 512^3 fine shells' parents (their
    2x2x2 coarse set) with the fine shells' own occupancy as the child mask, so the kept
    children are exactly the fine set. Occupancy logits, child map and child projection
    timed apart."""
    import numpy as np
    import torch

    from hi3d_amd import kmap as _kmap
    from hi3d_amd import sparse, vae, workloads

    dev = torch.device("cuda:0")
    idx = torch.as_tensor(coords_of("down2_up2_c64_c128_fp16", dev)).to(dev)
    s2 = _kmap.stride2_structure(idx, [int(v) + 1 for v in idx[:, 1:].max(0).values.tolist()], 1)
    level = sparse.Level.from_coords(s2.low[:, 1:].contiguous())
    p_n, c = level.n, 256
    mask = torch.zeros((p_n, 8), dtype=torch.bool, device=dev)
    mask[s2.inverse.long(), s2.slot.long()] = True
    x = torch.as_tensor(workloads.normal((p_n, c), 1.0, 71, np.float16)).to(dev)
    params = {
        "u.cls_head.fc.0.weights": torch.as_tensor(1.0 + workloads.normal((1, c), 0.1, 72)).to(dev),
        "u.cls_head.fc.0.bias": torch.as_tensor(workloads.normal((1, c), 0.1, 73)).to(dev),
        "u.cls_head.fc.2.weight": torch.as_tensor(workloads.normal((27 * c, 8), 1.0 / np.sqrt(27 * c), 74, np.float16)).to(dev),
        "u.cls_head.fc.2.bias": torch.as_tensor(workloads.normal((8,), 0.02, 75, np.float16)).to(dev),
        "u.proj.weight": torch.as_tensor(workloads.normal((8 * c, c), 1.0 / np.sqrt(c), 76, np.float16)).to(dev),
    }
    _, occ = timed(lambda: vae.occupancy(x, level, params, "u"), steps, warmup)
    _, cmap = timed(lambda: sparse.child_neighbour_table(level.table, mask), steps, warmup)
    _, parent, slot = sparse.child_neighbour_table(level.table, mask)
    n_child = int(parent.shape[0])
    w = params["u.proj.weight"]
    _, plan_ms = timed(lambda: vae.child_plan(parent, slot, p_n), steps, warmup)
    plan = vae.child_plan(parent, slot, p_n)
    _, proj = timed(lambda: vae.children(x, parent, slot, w, plan=plan), steps, warmup)
    up_wall, _ = timed(lambda: vae.upsample(x, level, params, "u", mask=mask), max(3, steps // 5), max(1, warmup // 2))
    flops = 2.0 * n_child * c * c
    return {
        "workload": "vae_upsample_c256_fp16",
        "parents": p_n,
        "children": n_child,
        "occupancy_ms": occ,
        "child_map_ms": cmap,
        "child_plan_ms": plan_ms,
        "projection_ms": proj,
        "projection_tflops": flops / (proj * 1e-3) / 1e12,
        "projection_gbs": (n_child + p_n) * c * 2 / (proj * 1e-3) / 1e9,
        "upsample_given_mask_ms": up_wall,
        "children_per_s": n_child / (up_wall * 1e-3),
    }


def bench_geometry(steps: int, warmup: int):
    """Refiner transformer I/O resampling on the 1024^3 residual-block shells at C256
    fp16: mean pool down, parent copy up, and the up block's first convolution from the
    coarse rows (against the same convolution of materialised upsampled features)."""
    import numpy as np
    import torch

    from hi3d_amd import conv, workloads
    from hi3d_amd.geometry import Geometry

    dev = torch.device("cuda:0")
    idx = torch.as_tensor(coords_of("resblock_c256_fp16", dev)).to(dev)
    coords = idx[:, 1:].contiguous()
    build_wall, _ = timed(lambda: Geometry(coords), 2, 1)
    geo = Geometry(coords)
    c = 256
    x = torch.as_tensor(workloads.normal((geo.full.n, c), 1.0, 81, np.float16)).to(dev)
    h = torch.as_tensor(workloads.normal((geo.low.n, c), 1.0, 82, np.float16)).to(dev)
    w = torch.as_tensor(workloads.normal((c, 27 * c), 1.0 / np.sqrt(27 * c), 83, np.float16)).to(dev)
    b = torch.as_tensor(workloads.normal((c,), 0.02, 84, np.float16)).to(dev)
    geo.up_conv_plan  # built once per pass, like the reference's up_conv_index
    geo.full.plan
    _, down = timed(lambda: geo.downsample(x), steps, warmup)
    _, up = timed(lambda: geo.upsample(h), steps, warmup)
    _, upc = timed(lambda: geo.up_conv(h, w, b), max(3, steps // 5), max(1, warmup // 2))
    w3 = w.reshape(c, 27, c).contiguous()
    _, composed = timed(lambda: conv.conv(geo.upsample(h), geo.full.plan, w3, b), max(3, steps // 5),
                        max(1, warmup // 2))
    pairs = int((geo.full.table < geo.full.n).sum())
    return {
        "workload": "transformer_io_c256_fp16",
        "voxels": geo.full.n,
        "coarse_voxels": geo.low.n,
        "geometry_build_ms": build_wall,
        "downsample_ms": down,
        "downsample_gbs": (geo.full.n + geo.low.n) * c * 2 / (down * 1e-3) / 1e9,
        "upsample_ms": up,
        "upsample_gbs": (geo.full.n + geo.low.n) * c * 2 / (up * 1e-3) / 1e9,
        "up_conv_ms": upc,
        "up_conv_tflops": 2.0 * pairs * c * c / (upc * 1e-3) / 1e12,
        "upsample_then_conv_ms": composed,
    }


def bench_unique(steps: int, warmup: int):
    """Unique cube corners of the 1024^3 residual-block shells (mesh extraction's
    ``torch.unique(dim=0)``): 8 corner rows of 3 int32 per voxel, with inverse and
    counts; torch's own GPU ``unique(dim=0)`` timed on the same rows."""
    import torch

    from hi3d_amd import fast_unique, workloads

    dev = torch.device("cuda:0")
    idx = torch.as_tensor(coords_of("resblock_c256_fp16", dev)).to(dev)
    xyz = idx[:, 1:].to(torch.int32)
    off = torch.tensor([[i >> 2 & 1, i >> 1 & 1, i & 1] for i in range(8)], dtype=torch.int32, device=dev)
    corners = (xyz[:, None, :] + off[None]).reshape(-1, 3).contiguous()
    n = int(corners.shape[0])
    _, ours = timed(lambda: fast_unique.unique_rows(corners, return_inverse=True, return_counts=True),
                    steps, warmup)
    u = int(fast_unique.unique_rows(corners).shape[0])
    _, theirs = timed(lambda: torch.unique(corners, dim=0, return_inverse=True, return_counts=True),
                      max(2, steps // 5), 1)
    return {
        "workload": "unique_corners_1024",
        "rows": n,
        "unique_rows": u,
        "unique_ms": ours,
        "rows_per_s": n / (ours * 1e-3),
        "torch_unique_dim0_ms": theirs,
    }


def bench_kmap(steps: int, warmup: int):
    """Submanifold 3x3x3 kernel-map builds on the 1024^3 residual-block shells and the
    256^3 C128 shells: the dense grid (kept between builds; and cleared inside each
    build) and the brick hash (the default above 2^28 cells), each checked equal to the
    dense table."""
    import torch

    from hi3d_amd import kmap

    dev = torch.device("cuda:0")
    out = {}
    for name, grid in (("resblock_c256_fp16", 1024), ("subm3_c128_fp16", 256)):
        coords = torch.as_tensor(coords_of(name, dev)).to(dev)
        build = lambda: kmap.build_kernel_map(coords, [grid] * 3, 1, check=False)
        dense, fresh = dense_path(build), dense_fresh(build)
        ref = dense().table
        brick = lambda: kmap.build_kernel_map(coords, [grid] * 3, 1, capacity=0, check=False)
        _, dense_ms = timed(dense, steps, warmup)
        _, fresh_ms = timed(fresh, steps, warmup)
        _, hash_ms = timed(brick, steps, warmup)
        n = int(coords.shape[0])
        out[name] = {
            "grid": grid,
            "voxels": n,
            "dense_ms": dense_ms,
            "dense_fresh_ms": fresh_ms,
            "brick_hash_ms": hash_ms,
            "brick_hash_voxels_per_s": n / (hash_ms * 1e-3),
            "hash_equal": bool(torch.equal(brick().table, ref)),
            "dense_fresh_equal": bool(torch.equal(fresh().table, ref)),
        }
    return out


def cpu_threads() -> int:
    """Host threads for the CPU baselines: the process's CPU share (``OMP_NUM_THREADS``
    when the launcher sets it, as GPU hosts that split their cores per GPU do), else
    every core ``os.cpu_count()`` reports."""
    try:
        share = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        share = 0
    return share if share > 0 else (os.cpu_count() or 1)


def cpu_baseline_block(sample_rows: int):
    """The residual block on the host (reference CPU fallback per stage, oracle port),
    on a random sample of output rows over the full map of the 1024^3 shells."""
    from hi3d_amd import workloads
    from oracle import baseline

    idx = coords_of("resblock_c256_fp16")
    threads = cpu_threads()
    r = baseline.time_resblock(idx, [1024] * 3, 256, 1024, sample_rows=sample_rows, threads=threads)
    return r


def cpu_baseline_conv(name: str, grid: int, cin: int, cout: int):
    """One submanifold convolution on the host over the whole set (map cached)."""
    from hi3d_amd import workloads
    from oracle import baseline

    idx = coords_of(name)
    return baseline.time_subm_conv(idx, [grid] * 3, cin, cout, repeats=3, threads=cpu_threads())


def cpu_baseline_w8a8(rows: int):
    """Host quantiser + integer GEMM of both W8A8 shapes on ``rows`` sampled tokens."""
    import torch

    from oracle import baseline

    torch.set_num_threads(cpu_threads())
    out = {}
    for tag, (m, k, n) in {"A": (65536, 1024, 4096), "B": (65536, 4096, 1024)}.items():
        r = baseline.time_w8a8(rows, k, n)
        ops = 2.0 * rows * n * k
        out[tag] = {**r, "full_m": m, "tops_gemm": ops / r["gemm_s"] / 1e12,
                    "tops_quant_gemm": ops / (r["quant_s"] + r["gemm_s"]) / 1e12}
    return out


WORKLOADS = ("resblock", "subm3_c128_fp16", "subm3_c64_fp32", "stride2", "w8a8", "vae_resnet", "vae_upsample",
             "transformer_io", "resblock3d", "unique", "kmap")


def main() -> int:
    global SETTLE_EACH_S
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--settle", type=float, default=2.0,
                    help="seconds of untimed headline passes before its warm-up (clock ramp)")
    ap.add_argument("--settle-each", type=float, default=SETTLE_EACH_S,
                    help="seconds of untimed calls before each other timed measurement")
    ap.add_argument("--only", default="", help=f"comma-separated workloads to run, of {', '.join(WORKLOADS)}")
    ap.add_argument("--quick", action="store_true", help="headline workload only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--cpu-rows", type=int, default=400_000, help="output-row sample of the block's CPU baseline")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (calibrates HBM byte counters) and exit")
    args = ap.parse_args()
    SETTLE_EACH_S = max(0.0, args.settle_each)
    if args.copy_probe:
        import torch

        src = torch.ones(args.copy_probe * (1 << 20) // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": src.numel() * 4, "launches": 5}), flush=True)
        return 0
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the sparse hot path runs on a single MI355X here "
              "(multi-GPU sharding is a design note, not a measured path). Use --gpus 1.", file=sys.stderr)
        return 2
    only = [w for w in args.only.split(",") if w]
    unknown = sorted(set(only) - set(WORKLOADS))
    if unknown:
        print(f"unknown workloads {unknown}; choose from {WORKLOADS}", file=sys.stderr)
        return 2
    selected = only or (["resblock"] if args.quick else list(WORKLOADS))

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    from hi3d_amd import _lib

    _lib.lib()
    torch.backends.cuda.matmul.allow_tf32 = False

    head = None
    extra = {}
    half_steps, half_warm = max(10, args.steps // 2), max(2, args.warmup // 2)
    for name in selected:
        if name == "resblock":
            log("headline: residual block C256 fp16 on the 1024^3 ellipsoid shells")
            head = bench_block(args.steps, args.warmup, args.settle)
            log(f"  {head['voxels']} voxels, {head['block_ms']:.3f} ms/step, conv {head['conv_kernel_ms']:.3f} ms "
                f"({head['conv_eff_tflops']:.1f} TFLOP/s)")
        elif name == "subm3_c128_fp16":
            log("subm3 C128 fp16 on the 256^3 ellipsoid shells")
            extra[name] = bench_subm(name, 256, 128, 128, torch.float16, args.steps, args.warmup)
        elif name == "subm3_c64_fp32":
            log("subm3 C64 fp32, 128^3 sphere shell")
            extra[name] = bench_subm(name, 128, 64, 64, torch.float32, args.steps, args.warmup)
        elif name == "stride2":
            log("stride-2 down/up fp16, 512^3 shells")
            extra["down2_up2_c64_c128_fp16"] = bench_stride2(args.steps, args.warmup)
        elif name == "w8a8":
            log("W8A8 int8 linear")
            extra["w8a8_linear"] = bench_w8a8(half_steps, max(3, half_warm))
        elif name == "vae_resnet":
            log("VAE decoder residual block C128 fp16, 512^3 fine shells")
            extra["vae_resnet_c128_fp16"] = bench_vae(half_steps, half_warm)
        elif name == "vae_upsample":
            log("VAE decoder octree upsampling C256 fp16, 512^3 fine shells' parents")
            extra["vae_upsample_c256_fp16"] = bench_upsample(half_steps, half_warm)
        elif name == "transformer_io":
            log("transformer I/O resampling C256 fp16, 1024^3 shells")
            extra["transformer_io_c256_fp16"] = bench_geometry(half_steps, half_warm)
        elif name == "resblock3d":
            log("transformer SparseResBlock3d C256 (hidden 128, emb 2112) fp16, 1024^3 shells")
            extra["sparse_resblock3d_c256_fp16"] = bench_resblock3d(half_steps, half_warm)
        elif name == "unique":
            log("unique cube corners of the 1024^3 shells")
            extra["unique_corners_1024"] = bench_unique(max(5, args.steps // 10), 2)
        elif name == "kmap":
            log("submanifold kernel-map builds (dense grid, brick hash), 1024^3 and 256^3 shells")
            extra["kmap_subm3"] = bench_kmap(max(10, args.steps // 2), 3)
    if head is None:  # a partial run (profiling): the workloads' own figures only
        print(json.dumps({"partial": selected, "extra": extra}), flush=True)
        return 0

    cpu = None
    if not args.no_cpu:
        log(f"CPU baseline: residual block on {args.cpu_rows} sampled voxels (reference CPU fallback, oracle port)")
        r = cpu_baseline_block(args.cpu_rows)
        cpu = {
            "value": r["sample_rows"] / r["block_s"],
            "unit": "voxels/s",
            "cores": r["torch_threads"],
            "kind": "port",
            "sample": (f"C256 residual block (adaLN projection, LayerNorm + modulate, conv + SiLU, conv + residual; "
                       f"fp32 on host) for {r['sample_rows']} randomly sampled output voxels of the {r['rows']}-voxel "
                       f"1024^3 shells over the full kernel map (built once on host in {r['map_s']:.2f} s, cached); "
                       f"median of 2 after 1 warm-up; {r['torch_threads']} threads of the {r['cpu_count']} "
                       f"cores os.cpu_count() reports; {r['model']}"),
            "host_cpu_count": r["cpu_count"],
        }
        if "subm3_c64_fp32" in extra:
            log("CPU baseline: subm3 C64 fp32 sphere shell in full")
            c1 = cpu_baseline_conv("subm3_c64_fp32", 128, 64, 64)
            extra["subm3_c64_fp32"]["cpu_baseline"] = {
                "voxels_per_s": c1["rows"] / c1["conv_s"], "conv_s": c1["conv_s"], "map_s": c1["map_s"],
                "rows": c1["rows"], "threads": c1["torch_threads"], "sample": "all voxels, map cached"}
        if "w8a8_linear" in extra:
            log("CPU baseline: W8A8 quantiser + integer GEMM on 4096 sampled tokens")
            extra["w8a8_linear"]["cpu_baseline"] = cpu_baseline_w8a8(4096)
    conv_tflops = head["conv_eff_tflops"]
    line = {
        "metric": "sparse-conv voxels/s + eff. TFLOP/s; W8A8 GEMM int8 TOPS (1 MI355X)",
        "value": head["voxels_per_s"],
        "unit": "voxels/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["block_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": "resblock_c256_fp16",
            "grid": 1024,
            "voxels": head["voxels"],
            "pairs": head["pairs"],
            "channels": 256,
            "step": "adaLN projection + LayerNorm/modulate + 3x3x3 submanifold conv + SiLU + conv + residual, "
                    "kernel map cached",
            "clock_settle_s": args.settle,
        },
        "eff_tflops": head["block_eff_tflops"],
        "roofline": {
            "bound": "mfma",
            "achieved": conv_tflops,
            "peak": PEAK_FP16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": conv_tflops / PEAK_FP16_TFLOPS,
            "traffic": measured_traffic(),
            "traffic_source": TRAFFIC_SUMMARY.name,
            "alg_flops": head["conv_flops"],
            "alg_bytes": head["conv_alg_bytes"],
            "kernel": HEADLINE_KERNEL,
            "kernel_ms": head["conv_kernel_ms"],
        },
        "cpu_baseline": cpu,
        "headline_detail": head,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
