"""VAE decoder convolution prologue (GroupNorm statistics, GroupNorm + swish, the
residual block built from them) and octree upsampling (occupancy logits, child map,
child projection).

Mirrors ``SparconvVAEDecoderMLX.group_stats`` / ``conv_gn_swish`` / ``resnet`` /
``children`` / ``occupancy`` and the upsampling step of ``__call__``
(src/hi3d_mac/mlx_backend/vae.py:141-244,270-271,316-327) as functions of explicit
tensors: ``level`` is a :class:`hi3d_amd.sparse.Level`, convolution weights use the MLX
GEMM layout ``[27 * Cin, Cout]`` (``sparse.conv_weight``), GroupNorm affines are
``[1, C]``, parameter dictionaries use the reference's names.

The reference activates each gathered neighbour row while building the GEMM input
block. Here the activation runs once per row (``swish(GN(x))`` ``[n, C]``) and the
gather-MFMA convolution gathers the activated rows; absent neighbours read zeros, the
padding applied to activated features as in the reference.
"""

from __future__ import annotations

import torch

from . import _lib
from . import conv as _conv
from . import kmap as _kmap
from .kernels import gather_group_norm_swish, group_norm_swish
from .sparse import Level, child_neighbour_table

SKIP_POINTS = 12_000_000
"""Residual blocks over more rows than this return their input unchanged: upstream's
``_RESNET_SKIP_POINTS``, kept by the reference (vae.py:29-30,209-210)."""

__all__ = ["groups_for", "group_stats", "group_norm_swish", "gather_group_norm_swish", "conv_gn_swish", "resnet",
           "child_plan", "children", "occupancy", "upsample"]


def groups_for(c: int) -> int:
    """``PointGroupNorm``'s group count: 32, or ``C / 4`` below 128 channels (vae.py:152)."""
    return 32 if 4 * 32 <= c else c // 4


def group_stats(x: torch.Tensor, eps: float = 1e-6) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-channel ``(mean, 1 / sqrt(var + eps))`` in fp32 of ``x [n, C]`` over
    ``groups_for(C)`` groups (vae.py:141-164). Column sums are fp32 per block and fp64
    across blocks; the reference sums in fp32, so the statistics agree to fp32
    rounding, not bit for bit. With no rows the divisor ``n * width + eps`` gives mean 0
    and ``1 / sqrt(eps)``, as in the reference."""
    device = _lib.require_gpu(x)
    if x.dim() != 2:
        raise ValueError("x must be [n, C]")
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
                  residual: torch.Tensor | list | None = None, eps: float = 1e-6) -> torch.Tensor:
    """``conv(swish(GroupNorm(x))) + bias`` (+ ``residual``) over ``level``'s map
    (vae.py:166-192). ``weight_t [27 * Cin, Cout]``; the activation is rounded to the
    weight dtype and the convolution accumulates in fp32; the result is in ``out``
    (default: fp32 for fp32 weights, else the weight dtype).

    Bias rounding: when ``out`` differs from the weight dtype the accumulator is rounded
    to the weight dtype, the fp32 bias added in fp32 and the sum rounded to ``out``, as
    the reference computes ``((g @ w).astype(F32) + bias).astype(out)``. When ``out`` is
    the weight dtype the epilogue adds the bias (rounded to that dtype) to the fp32
    accumulator and rounds once, which skips the reference's intermediate rounding: the
    two differ by at most about one unit in the last place of ``out``, inside the
    1e-2-of-RMS gate the parity tests apply.

    ``residual`` as a one-element list holding ``r`` (the reference's donation idiom)
    returns ``r + conv(...)`` written into ``r``'s own buffer: the convolution's rounded
    output is added in ``r``'s dtype by the epilogue, which reads and writes each
    element once, so no second ``[n, Cout]`` tensor exists."""
    mean, inv = group_stats(x, eps)
    wdt = weight_t.dtype
    a = group_norm_swish(x, mean, inv, norm_weight, norm_bias, wdt)
    cin, cout = int(x.shape[1]), int(weight_t.shape[1])
    w = weight_t.T.reshape(cout, 27, cin).contiguous()
    if out is None:
        out = torch.float32 if wdt == torch.float32 else wdt
    donated = None
    if isinstance(residual, list):
        if len(residual) != 1:
            raise ValueError("residual holder must hold exactly one tensor")
        donated = residual.pop()
        residual = donated
    if out != wdt:
        y = _conv.conv(a, level.plan, w, None)
        y = y.float() + (0 if bias is None else bias.float())
        y = y.to(out)
        if residual is None:
            return y
        if donated is not None:
            return donated.add_(y.to(donated.dtype))
        return (residual.float() + y.float()).to(residual.dtype)
    b = None if bias is None else bias.to(wdt)
    if donated is not None and donated.dtype == wdt and donated.is_contiguous() and donated.data_ptr() != a.data_ptr():
        return _conv.conv(a, level.plan, w, b, residual=donated, out=donated)
    r = None if residual is None else residual.to(wdt)
    y = _conv.conv(a, level.plan, w, b, residual=r)
    return y if donated is None else donated.copy_(y)


def resnet(x: torch.Tensor | list, level: Level, params: dict, name: str, eps: float = 1e-6,
           skip_points: int = SKIP_POINTS) -> torch.Tensor:
    """``shortcut + conv(swish(GN(conv(swish(GN(x))))))`` (vae.py:200-218) with the
    reference's parameter names: ``{name}.block.0`` / ``.block.3`` GroupNorm
    (``.weights``, ``.bias``), ``.block.2`` / ``.block.5`` convolutions (``.weight``
    ``[27 Cin, Cout]``, ``.bias``) and an optional ``{name}.res_conv`` linear. Levels of
    more than ``skip_points`` rows return the input unchanged, as upstream does.

    ``x`` may be a one-element list holding the input (the reference's holder): with an
    identity shortcut the second convolution then accumulates into the input's buffer,
    so two full-size activations are alive instead of three."""
    p = params
    holder = x if isinstance(x, list) else None
    if holder is not None:
        if len(holder) != 1:
            raise ValueError("input holder must hold exactly one tensor")
        x = holder.pop()
    if int(x.shape[0]) > skip_points:
        return x
    h = conv_gn_swish(x, level, p[f"{name}.block.0.weights"], p[f"{name}.block.0.bias"],
                      p[f"{name}.block.2.weight"], p[f"{name}.block.2.bias"], eps=eps)
    if f"{name}.res_conv.weight" in p:
        w = p[f"{name}.res_conv.weight"]
        shortcut = (x.to(w.dtype) @ w.T + p[f"{name}.res_conv.bias"]).to(h.dtype)
    elif holder is not None and x.dtype == h.dtype:
        shortcut = [x]
        del x
    else:
        shortcut = x.to(h.dtype)
    return conv_gn_swish(h, level, p[f"{name}.block.3.weights"], p[f"{name}.block.3.bias"],
                         p[f"{name}.block.5.weight"], p[f"{name}.block.5.bias"], out=h.dtype,
                         residual=shortcut, eps=eps)


def child_plan(parent: torch.Tensor, slot: torch.Tensor, n_parents: int) -> _kmap.ConvPlan:
    """Gather plan of the child projection over ``n_parents`` parent rows: table
    ``[C, 8]`` holding child ``i``'s parent in column ``slot[i]`` (absent elsewhere), rows
    grouped by slot in child order, so every 128-row tile but the (at most seven) tiles
    that straddle two slots multiplies by one slot's matrix only."""
    device = _lib.require_gpu(parent, slot)
    n = int(parent.shape[0])
    if slot.shape[0] != n:
        raise ValueError("parent and slot must have one entry per child")
    par = parent.to(torch.int32).contiguous()
    sl = slot.to(torch.uint8).contiguous()
    up = torch.empty((n, 8), dtype=torch.int32, device=device)
    if n:
        _lib.call("hi3d_stride2_tables", _lib.ptr(par), _lib.ptr(sl), n, int(n_parents), None, _lib.ptr(up),
                  _lib.stream(device))
    return _kmap.build_plan(up, int(n_parents), None, window_rows=0)


def children(x: torch.Tensor, parent: torch.Tensor, slot: torch.Tensor, weight: torch.Tensor,
             out: torch.dtype | None = None, plan: _kmap.ConvPlan | None = None) -> torch.Tensor:
    """``SerializedUnpooling`` features of the kept children (vae.py:220-244): child
    ``(p, s)`` is ``x[p] @ weight[s*C:(s+1)*C].T``, row ``p * 8 + s`` of the full
    projection ``(x @ weight.T).reshape(-1, C)`` for ``weight [8C, C]``, in child order.
    Only the kept children are computed (one slot matrix per child, fp32 accumulation,
    result rounded to ``weight.dtype`` and then to ``out``)."""
    _lib.require_gpu(x, parent, slot, weight)
    if x.dim() != 2:
        raise ValueError("x must be [P, C]")
    p, c = int(x.shape[0]), int(x.shape[1])
    if tuple(weight.shape) != (8 * c, c):
        raise ValueError(f"weight must be [8C, C] = [{8 * c}, {c}], got {tuple(weight.shape)}")
    out = weight.dtype if out is None else out
    n = int(parent.shape[0])
    if n == 0:
        return torch.empty((0, c), dtype=out, device=x.device)
    if plan is None:
        plan = child_plan(parent, slot, p)
    w = weight.reshape(8, c, c).permute(1, 0, 2).contiguous()  # [C_out, slot, C_in]
    y = _conv.conv(x.to(weight.dtype).contiguous(), plan, w, None)
    return y if y.dtype == out else y.to(out)


def occupancy(x: torch.Tensor, level: Level, params: dict, name: str, eps: float = 1e-6) -> torch.Tensor:
    """Child occupancy logits ``[P, 8]`` of ``SparseClsHead`` (vae.py:270-271): GroupNorm
    ``{name}.cls_head.fc.0``, swish and the 3x3x3 convolution ``{name}.cls_head.fc.2``."""
    p = params
    return conv_gn_swish(x, level, p[f"{name}.cls_head.fc.0.weights"], p[f"{name}.cls_head.fc.0.bias"],
                         p[f"{name}.cls_head.fc.2.weight"], p[f"{name}.cls_head.fc.2.bias"], eps=eps)


def upsample(x: torch.Tensor, level: Level, params: dict, name: str, out: torch.dtype | None = None,
             mask: torch.Tensor | None = None, eps: float = 1e-6) -> tuple[torch.Tensor, Level, torch.Tensor]:
    """One octree upsampling of the decoder (vae.py:316-327): occupancy logits, children
    where a logit is positive (or the given ``[P, 8]`` ``mask``), their neighbour table
    from the parent table, their projected features and coordinates
    ``coords[parent] * 2 + (s >> 2 & 1, s >> 1 & 1, s & 1)``.
    Returns ``(features [C, ch], Level of the children, mask [P, 8])``."""
    if mask is None:
        mask = occupancy(x, level, params, name, eps) > 0
    table, parent, slot = child_neighbour_table(level.table, mask)
    w = params[f"{name}.proj.weight"]
    y = children(x, parent, slot, w, out=out if out is not None else x.dtype)
    coords = level.coords.to(table.device, torch.int32)
    sl = slot.to(torch.int32)
    bits = torch.stack([(sl >> 2) & 1, (sl >> 1) & 1, sl & 1], 1)
    child_coords = coords[parent.long()] * 2 + bits
    return y, Level(child_coords, table), mask
