"""W8A8 oracle (NumPy float32 / int64). Test infrastructure only.

Restates src/hi3d_mac/mlx_backend/w8a8.py: ``signs`` :16-18, the ``_QUANT`` kernel :25-58
and the ``_GEMM`` epilogue :77, plus the integer check of tests/test_w8a8_inference.py:
15-20. Every float operation is a single IEEE float32 operation in the reference's
order, so codes and scales are exact by construction.
"""

from __future__ import annotations

import numpy as np


def signs(width: int) -> np.ndarray:
    """``default_rng(314159 + width).choice([-1., 1.], width)`` as float32."""
    return np.random.default_rng(314159 + width).choice([-1.0, 1.0], width).astype(np.float32)


def rotate_h64(x: np.ndarray, multiplier: np.ndarray | None = None) -> np.ndarray:
    """Signed H64 of each 64-column block, float32: ``u = x * sign``; butterflies over the
    column bits 0..4 (the reference's xor shuffles ``d = 1..16``: pair (L, H) -> (L + H,
    L - H)), then bit 5 as ``lo = (u + v) * 0.125``, ``hi = (u - v) * 0.125``."""
    x = np.asarray(x)
    m, k = x.shape
    if k % 64:
        raise ValueError("signed H64 requires width divisible by 64")
    s = signs(k) if multiplier is None else np.asarray(multiplier, dtype=np.float32)
    v = (x.astype(np.float32) * s[None, :]).reshape(m, k // 64, 2, 32)
    u, w = v[:, :, 0, :].copy(), v[:, :, 1, :].copy()
    for d in (1, 2, 4, 8, 16):
        for arr in (u, w):
            lanes = arr.reshape(m, k // 64, 32 // (2 * d), 2, d)
            low = lanes[:, :, :, 0, :].copy()
            high = lanes[:, :, :, 1, :].copy()
            lanes[:, :, :, 0, :] = low + high
            lanes[:, :, :, 1, :] = low - high
    lo = (u + w) * np.float32(0.125)
    hi = (u - w) * np.float32(0.125)
    return np.concatenate([lo, hi], axis=2).reshape(m, k).astype(np.float32)


def quantize_activation(x: np.ndarray, multiplier: np.ndarray | None = None, rotation: str = "h64"):
    """``(q int8 [M, K], s float32 [M])``: ``s = max(max|v|, 1e-8) / 127``,
    ``q = clamp(rint(v / s), -127, 127)`` over the rotated (or plain) float32 rows."""
    x = np.asarray(x).reshape(-1, np.asarray(x).shape[-1])
    v = rotate_h64(x, multiplier) if rotation == "h64" else x.astype(np.float32)
    maximum = np.abs(v).max(axis=1) if v.shape[1] else np.zeros(v.shape[0], np.float32)
    s = (np.maximum(maximum, np.float32(1e-8)) / np.float32(127.0)).astype(np.float32)
    q = np.clip(np.rint(v / s[:, None]), -127, 127).astype(np.int8)
    return q, s


def int_gemm(q: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Exact integer product ``q @ w.T`` (int64, fits int32 for K <= 2^17)."""
    return np.asarray(q, np.int64) @ np.asarray(w, np.int64).T


def epilogue(acc: np.ndarray, sa: np.ndarray, sw: np.ndarray, bias: np.ndarray | None) -> np.ndarray:
    """``half(((float)acc * sa[row]) * sw[col] + (float)bias[col])``, unfused float32."""
    y = (acc.astype(np.float32) * np.asarray(sa, np.float32)[:, None]) * np.asarray(sw, np.float32)[None, :]
    if bias is not None:
        y = y + np.asarray(bias).astype(np.float32)[None, :]
    return y.astype(np.float16)


def linear(x, w, sw, bias, multiplier=None, rotation: str = "h64"):
    """Quantise, integer GEMM, epilogue: the whole W8A8 linear (``[M, N]`` fp16)."""
    q, sa = quantize_activation(x, multiplier, rotation)
    return epilogue(int_gemm(q, w), sa, sw, bias)


def hadamard64() -> np.ndarray:
    """Orthonormal Sylvester Hadamard ``H[p, j] = (-1)^popcount(p & j) / 8`` (float64)."""
    p = np.arange(64)
    bits = np.bitwise_and(p[:, None], p[None, :])
    parity = np.array([bin(int(b)).count("1") & 1 for b in bits.reshape(-1)]).reshape(64, 64)
    return (1.0 - 2.0 * parity) / 8.0
