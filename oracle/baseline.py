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


def kernel_map_rows(indices: torch.Tensor, spatial_shape, sample: torch.Tensor, kernel_size: int = 3):
    """The pairs of :func:`kernel_map` whose output row lies in ``sample``, found the same
    way (one sort of every voxel key, then shifted ``searchsorted`` matches) but queried
    from the output side, only for the sampled rows: ``(sources, positions in sample,
    counts)`` per offset. An output row j takes input row i under offset r exactly when
    coords[i] = coords[j] + r - centre, the reference's pair (i, j) (sparse_conv.py:115-149)."""
    center = kernel_size // 2
    coords = indices.long()
    sx, sy, sz = (int(v) for v in spatial_shape)

    def keys_of(c):
        return ((c[:, 0] * sx + c[:, 1]) * sy + c[:, 2]) * sz + c[:, 3]

    keys = keys_of(coords)
    sorted_keys, order = torch.sort(keys)
    own = coords[sample]
    positions = torch.arange(sample.shape[0])
    sources, targets = [], []
    shape = (sx, sy, sz)
    for r in itertools.product(range(kernel_size), repeat=3):
        if r == (center, center, center):
            sources.append(sample.clone())
            targets.append(positions)
            continue
        shift = torch.tensor([0, r[0] - center, r[1] - center, r[2] - center])
        neighbour = own + shift
        inside = torch.ones_like(neighbour[:, 0], dtype=torch.bool)
        for axis in range(3):
            inside &= (neighbour[:, axis + 1] >= 0) & (neighbour[:, axis + 1] < shape[axis])
        query = keys_of(neighbour)
        position = torch.searchsorted(sorted_keys, query).clamp_(max=keys.shape[0] - 1)
        found = inside & (sorted_keys[position] == query)
        sources.append(order[position[found]])
        targets.append(positions[found])
    counts = torch.tensor([len(s) for s in sources], dtype=torch.int32)
    return sources, targets, counts


def restrict_to_rows(sources, targets, n: int, sample: torch.Tensor):
    """The pairs whose output row (``targets``) lies in ``sample``, output rows renumbered
    to positions in ``sample``: the same per-offset lists the conv of those rows uses."""
    position = torch.full((n,), -1, dtype=torch.long)
    position[sample] = torch.arange(sample.shape[0])
    kept_s, kept_t = [], []
    for src, dst in zip(sources, targets):
        p = position[dst]
        keep = p >= 0
        kept_s.append(src[keep])
        kept_t.append(p[keep])
    counts = torch.tensor([len(s) for s in kept_s], dtype=torch.int32)
    return kept_s, kept_t, counts


def subm_conv_rows(features: torch.Tensor, sources, targets, counts, weight: torch.Tensor, bias, sample):
    """``subm_conv`` evaluated for the output rows ``sample`` only, over pairs from
    :func:`restrict_to_rows`: the centre GEMM of those rows, then the per-offset chunked
    gather / matmul / ``index_add_`` passes, bias last (sparse_conv.py:152-195)."""
    out_channels = weight.shape[0]
    kernel_volume = weight[0, ..., 0].numel()
    weights = weight.reshape(out_channels, kernel_volume, weight.shape[-1])
    center = kernel_volume // 2
    output = features[sample] @ weights[:, center, :].T
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


def time_resblock(indices: np.ndarray, spatial_shape, channels: int = 256, cond_dim: int = 1024,
                  sample_rows: int | None = None, seed: int = 0, repeats: int = 2,
                  threads: int | None = None) -> dict:
    """Seconds of the residual block ``x + conv2(silu(conv1(LN(x) * (1 + scale) + shift)))``
    on the host (fp32), the reference's CPU fallback for each stage: the kernel map of the
    whole set (sort + ``searchsorted``, timed once, cached as in the reference's usage),
    the adaLN projection, LayerNorm + modulate, and both convolutions, each evaluated for
    the output rows of a random sample of ``sample_rows`` voxels (all when None) over the
    full map. Every stage costs the same per output row wherever the row lies, so the
    sample's time per voxel is the block's. The map is the sampled rows' part of the
    reference's (:func:`kernel_map_rows`; ``map_s`` is its time). Median of ``repeats``
    after one warm-up."""
    if threads:
        torch.set_num_threads(threads)
    idx = torch.as_tensor(np.asarray(indices))
    n = int(idx.shape[0])
    gen = torch.Generator().manual_seed(seed)
    sample = torch.arange(n) if sample_rows is None or sample_rows >= n else torch.randperm(n, generator=gen)[:sample_rows]
    s = int(sample.shape[0])
    # features: a 65,536-row N(0, 1) block tiled over the rows (the values do not change
    # the time; drawing 10^9 normals would take longer than the baseline itself)
    base = torch.randn((min(n, 65536), channels), generator=gen)
    reps = -(-n // base.shape[0])
    x = base.repeat(reps, 1)[:n].contiguous()
    h1 = torch.roll(base, 1, 0).repeat(reps, 1)[:n].contiguous()  # stands in for conv1's output
    cond = torch.randn(cond_dim, generator=gen)
    proj_w = torch.randn((2 * channels, cond_dim), generator=gen) / np.sqrt(cond_dim)
    proj_b = torch.zeros(2 * channels)
    w1 = torch.randn((channels, 3, 3, 3, channels), generator=gen) / np.sqrt(27 * channels)
    w2 = torch.randn((channels, 3, 3, 3, channels), generator=gen) / np.sqrt(27 * channels)
    t0 = time.perf_counter()
    restricted = kernel_map_rows(idx, spatial_shape, sample)
    t_map = time.perf_counter() - t0

    def block() -> None:
        scale, shift = (proj_w @ cond + proj_b).chunk(2)
        h = torch.nn.functional.layer_norm(x[sample], (channels,), eps=1e-6) * (1 + scale) + shift
        del h  # conv1 gathers its input at every row (x stands in for it)
        a = torch.nn.functional.silu(subm_conv_rows(x, *restricted, w1, None, sample))
        del a
        y = subm_conv_rows(h1, *restricted, w2, None, sample) + x[sample]
        del y

    block()  # warm-up
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        block()
        times.append(time.perf_counter() - t0)
    return {"rows": n, "sample_rows": s, "map_s": t_map, "block_s": float(np.median(times)), **host_info()}


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
