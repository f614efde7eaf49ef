"""Fused row kernels: LayerNorm (+ adaLN modulation) and the adaLN projection.

Mirrors ``layer_norm_modulate`` (src/hi3d_mac/mlx_backend/kernels.py:162-237): fp16 rows,
fp32 two-pass statistics, optional fp32 affine, optional fp16 ``h * scale + shift``
with two fp16 roundings.
"""

from __future__ import annotations

import torch

from . import _lib


def layer_norm_modulate(
    x: torch.Tensor,
    eps: float,
    weight: torch.Tensor | None = None,
    bias: torch.Tensor | None = None,
    scale: torch.Tensor | None = None,
    shift: torch.Tensor | None = None,
) -> torch.Tensor:
    """``LayerNorm32`` of fp16 rows, then optionally ``fp16(fp16(h * scale) + shift)``."""
    if x.dtype != torch.float16:
        raise ValueError("layer_norm_modulate takes fp16 rows")
    device = _lib.require_gpu(x, weight, bias, scale, shift)
    c = int(x.shape[-1])
    rows = x.numel() // c if c else 0
    xc = x.contiguous()
    w = None if weight is None else weight.to(torch.float32).reshape(-1).contiguous()
    b = None if bias is None else bias.to(torch.float32).reshape(-1).contiguous()
    if (w is None) != (b is None):
        raise ValueError("weight and bias must be given together")
    sc = None if scale is None else scale.to(torch.float16).reshape(-1).contiguous()
    sh = None if shift is None else shift.to(torch.float16).reshape(-1).contiguous()
    if (sc is None) != (sh is None):
        raise ValueError("scale and shift must be given together")
    for t in (w, b, sc, sh):
        if t is not None and t.numel() != c:
            raise ValueError(f"per-channel parameters must have {c} entries")
    out = torch.empty_like(xc)
    _lib.call(
        "hi3d_layer_norm_modulate",
        _lib.ptr(xc), rows, c, float(eps), _lib.ptr(w), _lib.ptr(b), _lib.ptr(sc), _lib.ptr(sh), _lib.ptr(out),
        _lib.stream(device),
    )
    return out


def adaln_projection(
    weight: torch.Tensor, bias: torch.Tensor | None, cond: torch.Tensor, apply_silu: bool = False
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(fp16(1 + scale), shift)`` from ``y = weight @ cond' + bias`` (fp32, chunk order
    (scale, shift) as ``_emb_scale_shift``, src/hi3d_mac/mlx_backend/transformer.py:413-416;
    ``cond' = silu(cond)`` when ``apply_silu``, as the reference's ``emb_layers``)."""
    device = _lib.require_gpu(weight, bias, cond)
    w = weight.to(torch.float32).contiguous()
    n_out, n_in = int(w.shape[0]), int(w.shape[1])
    if n_out % 2:
        raise ValueError("the projection must produce an even number of features")
    c = cond.to(torch.float32).reshape(-1).contiguous()
    if c.numel() != n_in:
        raise ValueError(f"cond must have {n_in} entries")
    b = None if bias is None else bias.to(torch.float32).reshape(-1).contiguous()
    scale1p = torch.empty(n_out // 2, dtype=torch.float16, device=device)
    shift = torch.empty(n_out // 2, dtype=torch.float16, device=device)
    _lib.call(
        "hi3d_adaln_projection",
        _lib.ptr(w), _lib.ptr(b), _lib.ptr(c), n_out, n_in, int(bool(apply_silu)), _lib.ptr(scale1p), _lib.ptr(shift),
        _lib.stream(device),
    )
    return scale1p, shift
