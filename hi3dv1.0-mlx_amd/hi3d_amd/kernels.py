"""Fused row kernels: LayerNorm (+ adaLN modulation), the adaLN projection, and the
VAE convolution prologue's GroupNorm + swish.

Mirrors ``layer_norm_modulate`` (src/hi3d_mac/mlx_backend/kernels.py:162-237): fp16 rows,
fp32 two-pass statistics, optional fp32 affine, optional fp16 ``h * scale + shift``
with two fp16 roundings; and ``gather_group_norm_swish`` (kernels.py:240-296).
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
    act: str | None = None,
) -> torch.Tensor:
    """``LayerNorm32`` of fp16 rows, then optionally ``fp16(fp16(h * scale) + shift)``,
    then optionally (``act="silu"``) the fp16 SiLU ``h * sigmoid(h)`` of the reference's
    res blocks (src/hi3d_mac/mlx_backend/transformer.py:172-173, 418-433)."""
    if act not in (None, "none", "silu"):
        raise ValueError(f"unknown activation {act!r}")
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
        "hi3d_layer_norm_act",
        _lib.ptr(xc), rows, c, float(eps), _lib.ptr(w), _lib.ptr(b), _lib.ptr(sc), _lib.ptr(sh),
        _lib.ACT_SILU if act == "silu" else _lib.ACT_NONE, _lib.ptr(out), _lib.stream(device),
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


def _vec(v: torch.Tensor, c: int, device: torch.device, what: str) -> torch.Tensor:
    out = v.to(device=device, dtype=torch.float32).reshape(-1).contiguous()
    if out.numel() != c:
        raise ValueError(f"{what} must hold {c} values")
    return out.clone() if out.data_ptr() % 16 else out


def _rows(x: torch.Tensor) -> torch.Tensor:
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"unsupported dtype {x.dtype}")
    if x.dim() != 2:
        raise ValueError("x must be [n, C]")
    if x.shape[1] % 8 or x.shape[1] > 2048:
        raise ValueError("channels must be a multiple of 8, at most 2048")
    xc = x.contiguous()
    return xc.clone() if xc.data_ptr() % 16 else xc


def group_norm_swish(x: torch.Tensor, mean: torch.Tensor, inv: torch.Tensor, weight: torch.Tensor,
                     bias: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """``u * sigmoid(u)`` with ``u = (x - mean) * inv * weight + bias`` in float32, per
    channel, for every row of ``x [n, C]``, returned in ``dtype``: the activation the
    reference applies while gathering (kernels.py:240-258), once per row."""
    device = _lib.require_gpu(x)
    xc = _rows(x)
    n, c = int(xc.shape[0]), int(xc.shape[1])
    vecs = [_vec(v, c, device, k) for v, k in ((mean, "mean"), (inv, "inv"), (weight, "weight"), (bias, "bias"))]
    out = torch.empty((n, c), dtype=dtype, device=device)
    _lib.call("hi3d_gn_swish", _lib.ptr(xc), _lib.DTYPES[xc.dtype], n, c, *[_lib.ptr(v) for v in vecs],
              _lib.ptr(out), _lib.DTYPES[dtype], _lib.stream(device))
    return out


def gather_group_norm_swish(x: torch.Tensor, table: torch.Tensor, mean: torch.Tensor, inv: torch.Tensor,
                            weight: torch.Tensor, bias: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Convolution input block ``swish(GN(x))[table]`` ``[rows, kvol * C]`` in ``dtype``,
    zeros where ``table`` holds ``n`` (absent), as ``gather_group_norm_swish``
    (src/hi3d_mac/mlx_backend/kernels.py:261-296)."""
    device = _lib.require_gpu(x, table)
    xc = _rows(x)
    n, c = int(xc.shape[0]), int(xc.shape[1])
    t = table.to(torch.int32).contiguous()
    rows = int(t.shape[0])
    kvol = int(t.shape[1]) if t.dim() == 2 else 1
    vecs = [_vec(v, c, device, k) for v, k in ((mean, "mean"), (inv, "inv"), (weight, "weight"), (bias, "bias"))]
    out = torch.empty((rows, kvol * c), dtype=dtype, device=device)
    _lib.call("hi3d_gather_gn_swish", _lib.ptr(xc), _lib.DTYPES[xc.dtype], n, c, _lib.ptr(t), rows * kvol,
              *[_lib.ptr(v) for v in vecs], _lib.ptr(out), _lib.DTYPES[dtype], _lib.stream(device))
    return out
