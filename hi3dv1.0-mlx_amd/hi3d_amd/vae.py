"""VAE decoder convolution prologue: GroupNorm statistics, GroupNorm + swish, and the
residual block built from them.

Mirrors ``SparconvVAEDecoderMLX.group_stats`` / ``conv_gn_swish`` / ``resnet``
(src/hi3d_mac/mlx_backend/vae.py:141-218) as functions of explicit tensors: ``level`` is
a :class:`hi3d_amd.sparse.Level`, convolution weights use the MLX GEMM layout
``[27 * Cin, Cout]`` (``sparse.conv_weight``), GroupNorm affines are ``[1, C]``.

The reference activates each gathered neighbour row while building the GEMM input
block. Here the activation runs once per row (``swish(GN(x))`` ``[n, C]``) and the
gather-MFMA convolution gathers the activated rows; absent neighbours read zeros, the
padding applied to activated features as in the reference.
"""

from __future__ import annotations

import torch

from . import _lib
from . import conv as _conv
from .kernels import gather_group_norm_swish, group_norm_swish
from .sparse import Level

__all__ = ["groups_for", "group_stats", "group_norm_swish", "gather_group_norm_swish", "conv_gn_swish", "resnet"]


def groups_for(c: int) -> int:
    """``PointGroupNorm``'s group count: 32, or ``C / 4`` below 128 channels (vae.py:152)."""
    return 32 if 4 * 32 <= c else c // 4


def group_stats(x: torch.Tensor, eps: float = 1e-6) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-channel ``(mean, 1 / sqrt(var + eps))`` in fp32 of ``x [n, C]`` over
    ``groups_for(C)`` groups (vae.py:141-164). Column sums are fp32 per block and fp64
    across blocks; the reference sums in fp32, so the statistics agree to fp32
    rounding, not bit for bit."""
    device = _lib.require_gpu(x)
    if x.dim() != 2 or x.shape[0] == 0:
        raise ValueError("x must be a non-empty [n, C]")
    n, c = int(x.shape[0]), int(x.shape[1])
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"unsupported dtype {x.dtype}")
    if c % 8 or c > 2048:
        raise ValueError("channels must be a multiple of 8, at most 2048")
    xc = x.contiguous()
    if xc.data_ptr() % 16:
        xc = xc.clone()
    ws = _lib.workspace(_lib.query("hi3d_group_stats_workspace", n, c), device)
    mean = torch.empty(c, dtype=torch.float32, device=device)
    inv = torch.empty(c, dtype=torch.float32, device=device)
    _lib.call("hi3d_group_stats", _lib.ptr(xc), _lib.DTYPES[xc.dtype], n, c, groups_for(c), float(eps),
              _lib.ptr(ws), ws.numel(), _lib.ptr(mean), _lib.ptr(inv), _lib.stream(device))
    return mean, inv


def conv_gn_swish(x: torch.Tensor, level: Level, norm_weight: torch.Tensor, norm_bias: torch.Tensor,
                  weight_t: torch.Tensor, bias: torch.Tensor | None, out: torch.dtype | None = None,
                  residual: torch.Tensor | None = None, eps: float = 1e-6) -> torch.Tensor:
    """``conv(swish(GroupNorm(x))) + bias`` (+ ``residual``) over ``level``'s map
    (vae.py:166-192). ``weight_t [27 * Cin, Cout]``; the activation is rounded to the
    weight dtype, the convolution accumulates in fp32 and adds ``bias`` in fp32; the
    result is in ``out`` (default: fp32 for fp32 weights, else the weight dtype)."""
    mean, inv = group_stats(x, eps)
    wdt = weight_t.dtype
    a = group_norm_swish(x, mean, inv, norm_weight, norm_bias, wdt)
    cin, cout = int(x.shape[1]), int(weight_t.shape[1])
    w = weight_t.T.reshape(cout, 27, cin).contiguous()
    if out is None:
        out = torch.float32 if wdt == torch.float32 else wdt
    if out != wdt:
        y = _conv.conv(a, level.plan, w, None)
        y = y.float() + (0 if bias is None else bias.float())
        y = y.to(out)
        return y if residual is None else (residual.float() + y.float()).to(residual.dtype)
    b = None if bias is None else bias.to(wdt)
    r = None if residual is None else residual.to(wdt)
    return _conv.conv(a, level.plan, w, b, residual=r)


def resnet(x: torch.Tensor, level: Level, params: dict, name: str, eps: float = 1e-6) -> torch.Tensor:
    """``shortcut + conv(swish(GN(conv(swish(GN(x))))))`` (vae.py:200-218) with the
    reference's parameter names: ``{name}.block.0`` / ``.block.3`` GroupNorm
    (``.weights``, ``.bias``), ``.block.2`` / ``.block.5`` convolutions (``.weight``
    ``[27 Cin, Cout]``, ``.bias``) and an optional ``{name}.res_conv`` linear."""
    p = params
    h = conv_gn_swish(x, level, p[f"{name}.block.0.weights"], p[f"{name}.block.0.bias"],
                      p[f"{name}.block.2.weight"], p[f"{name}.block.2.bias"], eps=eps)
    if f"{name}.res_conv.weight" in p:
        w = p[f"{name}.res_conv.weight"]
        shortcut = (x.to(w.dtype) @ w.T + p[f"{name}.res_conv.bias"]).to(h.dtype)
    else:
        shortcut = x.to(h.dtype)
    return conv_gn_swish(h, level, p[f"{name}.block.3.weights"], p[f"{name}.block.3.bias"],
                         p[f"{name}.block.5.weight"], p[f"{name}.block.5.bias"], out=h.dtype,
                         residual=shortcut, eps=eps)
