"""The reference's CPU fallback of the hot path, in PyTorch on host cores — the CPU
baseline timed beside the GPU run. Test / benchmark infrastructure only.

Restates src/hi3d_mac/torch_backend/sparse_conv.py:109-195: int64 voxel keys, one
``torch.sort``, 26 shifted ``searchsorted`` matches (the kernel map), then the centre
GEMM and per-offset gather -> matmul -> ``index_add_`` passes in 256 MiB chunks with the
bias last. fp16 workloads run in fp32 on the host (PyTorch's CPU fp16 matmul is not a
fair baseline), from fp16-rounded inputs.
"""

from __future__ import annotations

import itertools
import os
import time

import numpy as np
import torch

from .w8a8 import quantize_activation

GATHER_BYTES = 256 * 1024 * 1024


def kernel_map(indices: torch.Tensor, spatial_shape, kernel_size: int = 3):
    """``(sources, targets, counts)`` per offset (sparse_conv.py:115-149)."""
    center = kernel_size // 2
    coords = indices.long()
    sx, sy, sz = (int(v) for v in spatial_shape)

    def keys_of(c):
        return ((c[:, 0] * sx + c[:, 1]) * sy + c[:, 2]) * sz + c[:, 3]

    keys = keys_of(coords)
    sorted_keys, order = torch.sort(keys)
    arange = torch.arange(coords.shape[0])
    sources, targets = [], []
    shape = (sx, sy, sz)
    for r in itertools.product(range(kernel_size), repeat=3):
        if r == (center, center, center):
            sources.append(arange)
            targets.append(arange)
            continue
        shift = torch.tensor([0, center - r[0], center - r[1], center - r[2]])
        neighbour = coords + shift
        inside = torch.ones_like(neighbour[:, 0], dtype=torch.bool)
        for axis in range(3):
            inside &= (neighbour[:, axis + 1] >= 0) & (neighbour[:, axis + 1] < shape[axis])
        query = keys_of(neighbour)
        position = torch.searchsorted(sorted_keys, query).clamp_(max=keys.shape[0] - 1)
        found = inside & (sorted_keys[position] == query)
        sources.append(arange[found])
        targets.append(order[position[found]])
    counts = torch.tensor([len(s) for s in sources], dtype=torch.int32)
    return sources, targets, counts


def subm_conv(features: torch.Tensor, sources, targets, counts, weight: torch.Tensor, bias):
    """Centre GEMM, then offsets k and K-1-k, chunked gather/matmul/index_add_, bias last
    (sparse_conv.py:152-195)."""
    out_channels = weight.shape[0]
    kernel_volume = weight[0, ..., 0].numel()
    weights = weight.reshape(out_channels, kernel_volume, weight.shape[-1])
    center = kernel_volume // 2
    output = features @ weights[:, center, :].T
    rows = max(1, GATHER_BYTES // max(1, features.shape[1] * features.element_size()))
    for offset in range(center):
        for k in (offset, kernel_volume - 1 - offset):
            count = int(counts[k])
            for start in range(0, count, rows):
                stop = start + rows
                output.index_add_(0, targets[k][start:stop], features[sources[k][start:stop]] @ weights[:, k, :].T)
    if bias is not None:
        output = output + bias
    return output


def host_info() -> dict:
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(), "model": model}


def time_subm_conv(indices: np.ndarray, spatial_shape, cin: int, cout: int, seed: int = 0, repeats: int = 3,
                   max_rows: int | None = None, threads: int | None = None) -> dict:
    """Median seconds of the CPU map build and of one conv (map cached) on ``indices``
    (the first ``max_rows`` rows when given, a stated sample)."""
    if threads:
        torch.set_num_threads(threads)
    idx = torch.as_tensor(np.asarray(indices)[:max_rows] if max_rows else np.asarray(indices))
    n = int(idx.shape[0])
    rng = np.random.default_rng(seed)
    feats = torch.as_tensor(rng.standard_normal((n, cin), dtype=np.float32))
    weight = torch.as_tensor((rng.standard_normal((cout, 3, 3, 3, cin)) / np.sqrt(27 * cin)).astype(np.float32))
    t0 = time.perf_counter()
    pairs = kernel_map(idx, spatial_shape)
    t_map = time.perf_counter() - t0
    subm_conv(feats, *pairs, weight, None)  # warm-up
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        subm_conv(feats, *pairs, weight, None)
        times.append(time.perf_counter() - t0)
    return {"rows": n, "map_s": t_map, "conv_s": float(np.median(times)), **host_info()}


def time_w8a8(m: int, k: int, n: int, seed: int = 0, rotation: str = "h64") -> dict:
    """Seconds of the host quantiser and integer GEMM + epilogue on an ``[m, k] x [n, k]``
    sample (``torch._int_mm`` when the CPU build has it, else exact float64)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k), dtype=np.float32).astype(np.float16)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    t0 = time.perf_counter()
    q, s = quantize_activation(x, rotation=rotation)
    t_q = time.perf_counter() - t0
    t0 = time.perf_counter()
    try:
        acc = torch._int_mm(torch.as_tensor(q), torch.as_tensor(w).T.contiguous())
    except (RuntimeError, AttributeError):
        acc = torch.as_tensor(q.astype(np.float64)) @ torch.as_tensor(w.astype(np.float64)).T
    t_g = time.perf_counter() - t0
    del acc
    return {"m": m, "k": k, "n": n, "quant_s": t_q, "gemm_s": t_g, **host_info()}
