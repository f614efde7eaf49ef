"""Convolution oracle: the reference's pair-list convolution order, float64 gather sums
and dense PyTorch-CPU equivalents. Test infrastructure only."""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

GATHER_BYTES = 256 * 1024 * 1024
"""Chunk bound of one gathered block (src/hi3d_mac/torch_backend/sparse_conv.py:25)."""


def subm_conv_pairs(features: torch.Tensor, sources, targets, counts, weight: torch.Tensor, bias):
    """Restates ``subm_conv`` / ``_accumulate`` (sparse_conv.py:152-195): the centre tap as
    one GEMM, then offsets ``k`` and ``K-1-k`` for ``k < K/2`` as chunked
    gather -> matmul -> ``index_add_`` passes, bias last. PyTorch CPU, any float dtype."""
    out_channels = weight.shape[0]
    kernel_volume = weight[0, ..., 0].numel()
    weights = weight.reshape(out_channels, kernel_volume, weight.shape[-1])
    center = kernel_volume // 2
    output = features @ weights[:, center, :].T
    rows = max(1, GATHER_BYTES // max(1, features.shape[1] * features.element_size()))
    for offset in range(center):
        for k in (offset, kernel_volume - 1 - offset):
            count = int(counts[k])
            if not count:
                continue
            src = torch.as_tensor(np.asarray(sources[k][:count]), dtype=torch.long)
            dst = torch.as_tensor(np.asarray(targets[k][:count]), dtype=torch.long)
            for start in range(0, count, rows):
                stop = start + rows
                output.index_add_(0, dst[start:stop], features[src[start:stop]] @ weights[:, k, :].T)
    if bias is not None:
        output = output + bias
    return output


def gather_conv_f64(features, table, weight, bias=None, rows=None, act=None, residual=None) -> np.ndarray:
    """``out[o] = act(bias + sum_k x[table[o,k]] @ W[:, k, :].T) (+ residual[o])`` in
    float64 for the output rows ``rows`` (all if None); entries >= N_in are absent."""
    x = np.asarray(features, dtype=np.float64)
    t = np.asarray(table)
    if rows is not None:
        t = t[rows]
    cout = weight.shape[0]
    kvol = t.shape[1]
    w = np.asarray(weight, dtype=np.float64).reshape(cout, kvol, -1)
    padded = np.concatenate([x, np.zeros((1, x.shape[1]))], 0)
    idx = np.where((t >= 0) & (t < x.shape[0]), t, x.shape[0])
    out = np.zeros((t.shape[0], cout))
    for k in range(kvol):
        out += padded[idx[:, k]] @ w[:, k, :].T
    if bias is not None:
        out += np.asarray(bias, dtype=np.float64)
    if act == "silu":
        out = out / (1.0 + np.exp(-out))
    if residual is not None:
        r = np.asarray(residual, dtype=np.float64)
        out += r if rows is None else r[rows]
    return out


def dense_subm_conv3d(indices, features, weight, bias, spatial_shape) -> np.ndarray:
    """The reference's dense check (tests/test_backends.py:32-50): scatter to a dense
    grid, ``F.conv3d(padding=ks//2)`` in float64, read back at the active voxels."""
    idx = torch.as_tensor(np.asarray(indices), dtype=torch.long)
    feats = torch.as_tensor(np.asarray(features), dtype=torch.float64)
    w = torch.as_tensor(np.asarray(weight), dtype=torch.float64)  # [Cout, k, k, k, Cin]
    cin = feats.shape[1]
    ks = w.shape[1]
    b, i, j, k = idx.unbind(1)
    nb = int(b.max()) + 1 if len(b) else 1
    dense = torch.zeros(nb, cin, *[int(s) for s in spatial_shape], dtype=torch.float64)
    dense[b, :, i, j, k] = feats
    bias_t = None if bias is None else torch.as_tensor(np.asarray(bias), dtype=torch.float64)
    out = F.conv3d(dense, w.permute(0, 4, 1, 2, 3), bias_t, padding=ks // 2)
    return out[b, :, i, j, k].numpy()


def dense_down2(fine_indices, features, weight, bias, spatial_shape, coarse_indices) -> np.ndarray:
    """``F.conv3d(stride=2)`` (kernel 2) in float64, read at the coarse voxels."""
    idx = torch.as_tensor(np.asarray(fine_indices), dtype=torch.long)
    feats = torch.as_tensor(np.asarray(features), dtype=torch.float64)
    w = torch.as_tensor(np.asarray(weight), dtype=torch.float64)  # [Cout, 2, 2, 2, Cin]
    shape = [int(s) + (int(s) & 1) for s in spatial_shape]
    b, i, j, k = idx.unbind(1)
    nb = int(b.max()) + 1
    dense = torch.zeros(nb, feats.shape[1], *shape, dtype=torch.float64)
    dense[b, :, i, j, k] = feats
    bias_t = None if bias is None else torch.as_tensor(np.asarray(bias), dtype=torch.float64)
    out = F.conv3d(dense, w.permute(0, 4, 1, 2, 3), bias_t, stride=2)
    ci = torch.as_tensor(np.asarray(coarse_indices), dtype=torch.long)
    return out[ci[:, 0], :, ci[:, 1], ci[:, 2], ci[:, 3]].numpy()


def dense_up2(coarse_indices, features, weight, bias, coarse_shape, fine_indices) -> np.ndarray:
    """``F.conv_transpose3d(stride=2)`` (kernel 2) in float64 with PyTorch weight
    ``W_pt[Cin, Cout, s] = W[:, s, :].T``, read at the fine voxels."""
    ci = torch.as_tensor(np.asarray(coarse_indices), dtype=torch.long)
    feats = torch.as_tensor(np.asarray(features), dtype=torch.float64)
    w = torch.as_tensor(np.asarray(weight), dtype=torch.float64)  # [Cout, 2, 2, 2, Cin]
    b, i, j, k = ci.unbind(1)
    nb = int(b.max()) + 1
    dense = torch.zeros(nb, feats.shape[1], *[int(s) for s in coarse_shape], dtype=torch.float64)
    dense[b, :, i, j, k] = feats
    bias_t = None if bias is None else torch.as_tensor(np.asarray(bias), dtype=torch.float64)
    out = F.conv_transpose3d(dense, w.permute(4, 0, 1, 2, 3), bias_t, stride=2)
    fi = torch.as_tensor(np.asarray(fine_indices), dtype=torch.long)
    return out[fi[:, 0], :, fi[:, 1], fi[:, 2], fi[:, 3]].numpy()


def gather_mean(features, table, extra: int = 1) -> np.ndarray:
    """``sum_k x[table[o,k]] / (present + extra)`` in float64 (``extra = 1`` is
    ``scatter_reduce(reduce="mean")`` onto zeros, src/sparc3d/nn/sparse/spatial.py:53-62)."""
    x = np.asarray(features, dtype=np.float64)
    t = np.asarray(table)
    present = (t >= 0) & (t < x.shape[0])
    padded = np.concatenate([x, np.zeros((1, x.shape[1]))], 0)
    idx = np.where(present, t, x.shape[0])
    total = padded[idx].sum(axis=1)
    return total / (present.sum(axis=1, keepdims=True) + extra)


def rel_err(got, ref) -> float:
    """``max|got - ref| / rms(ref)`` — the conv correctness gate's statistic."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rms = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    err = float(np.max(np.abs(got - ref))) if ref.size else 0.0
    return err / rms if rms > 0 else err
