"""Gather convolutions on the GPU (submanifold, 2x2x2/s2 and its transpose).

``gather_conv`` runs the MFMA kernel over a :class:`~hi3d_amd.kmap.ConvPlan`;
``gather_conv_simple`` runs the one-thread-per-output kernel straight from a table for
channel counts and dtypes (float64) the MFMA kernel does not take. Both compute

    out[o] = act(bias + sum_k in[table[o, k]] @ W[:, k, :].T) (+ residual[o])

with ``W`` in spconv's ``[Cout, K, Cin]`` layout (reference:
src/hi3d_mac/torch_backend/sparse_conv.py:152-195; src/hi3d_mac/mlx_backend/sparse.py:191-214).
``stride2_up`` runs the transpose of the 2x2x2 / stride-2 convolution parent-major, each
coarse row read once, for the shapes its kernel takes.
"""

from __future__ import annotations

import functools

import torch

from . import _lib
from .kmap import ConvPlan

ACTIVATIONS = {None: _lib.ACT_NONE, "none": _lib.ACT_NONE, "silu": _lib.ACT_SILU}

HALO = False
"""Use the halo convolution (3x3x3 submanifold maps, fp16/bf16, Cout % 128 == 0,
256..512-byte input rows) whenever the plan has a halo plan. Off by default: on the
ellipsoid-shell workloads it matches the tile-plan kernel at 128 channels and trails it
at 256 (a Morton tile computes every offset for every row, 33-47 % of them on absent
neighbours, and its halo reads conflict in LDS banks)."""


def _output(out: torch.Tensor | None, n: int, c: int, dtype: torch.dtype, device) -> torch.Tensor:
    """The output buffer: a new ``[n, c]`` tensor, or the caller's (which may be the
    residual itself: each output element is read and written by one thread)."""
    if out is None:
        return torch.empty((n, c), dtype=dtype, device=device)
    if tuple(out.shape) != (n, c) or out.dtype != dtype or not out.is_contiguous() or out.device != device:
        raise ValueError(f"out must be a contiguous [{n}, {c}] {dtype} tensor on {device}")
    return out


def halo_supported(dtype: torch.dtype, cin: int, cout: int, kvol: int) -> bool:
    """Whether the halo kernel takes this convolution."""
    if dtype not in (torch.float16, torch.bfloat16) or kvol != 27:
        return False
    rb = cin * 2
    return cout % 128 == 0 and rb % 64 == 0 and 256 <= rb <= 512


def _flat_weight(weight: torch.Tensor, kvol: int) -> torch.Tensor:
    cout, cin = int(weight.shape[0]), int(weight.shape[-1])
    w = weight.reshape(cout, -1, cin)
    if w.shape[1] != kvol:
        raise ValueError(f"weight has {w.shape[1]} kernel offsets, the map has {kvol}")
    return w.contiguous()


def mfma_supported(dtype: torch.dtype, cin: int, cout: int) -> bool:
    """Whether the MFMA kernel takes this dtype and channel count (16-byte rows)."""
    if dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return False
    es = torch.empty((), dtype=dtype).element_size()
    return (cin * es) % 16 == 0 and (cout * es) % 16 == 0


def gather_conv(
    features: torch.Tensor,
    plan: ConvPlan,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    act: str | None = None,
    residual: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """MFMA gather convolution; features, weight, bias, residual share one dtype."""
    device = _lib.require_gpu(features, weight, bias, residual, plan.gidx)
    dtype = features.dtype
    if weight.dtype != dtype or (bias is not None and bias.dtype != dtype) or (
        residual is not None and residual.dtype != dtype
    ):
        raise ValueError("features, weight, bias and residual must share one dtype")
    if features.ndim != 2 or features.shape[0] != plan.n_in:
        raise ValueError(f"expected features [{plan.n_in}, Cin], got {tuple(features.shape)}")
    x = features.contiguous()
    w = _flat_weight(weight, plan.kvol)
    cin, cout = int(x.shape[1]), int(w.shape[0])
    if int(w.shape[2]) != cin:
        raise ValueError(f"weight expects {int(w.shape[2])} input channels, features have {cin}")
    if not mfma_supported(dtype, cin, cout):
        raise ValueError(f"MFMA path needs fp16/bf16/fp32 and 16-byte channel rows (dtype {dtype}, {cin}->{cout})")
    b = None if bias is None else bias.contiguous()
    r = None if residual is None else residual.contiguous()
    if r is not None and tuple(r.shape) != (plan.n_out, cout):
        raise ValueError("residual must have the output's shape")
    out = _output(out, plan.n_out, cout, dtype, device)
    hp = plan.halo() if HALO and halo_supported(dtype, cin, cout, plan.kvol) else None
    if hp is not None:
        _lib.call(
            "hi3d_halo_conv",
            _lib.ptr(x), plan.n_in, cin, _lib.ptr(w), _lib.ptr(b), cout, _lib.ptr(hp.rows), _lib.ptr(hp.halo),
            _lib.ptr(hp.loff), hp.ntiles, _lib.ptr(r), ACTIVATIONS[act], _lib.DTYPES[dtype], _lib.ptr(out),
            _lib.stream(device),
        )
        return out
    _lib.call(
        "hi3d_gather_conv",
        _lib.ptr(x), plan.n_in, cin, _lib.ptr(w), _lib.ptr(b), cout, plan.kvol, _lib.ptr(plan.rows),
        _lib.ptr(plan.gidx), _lib.ptr(plan.tile_mask), plan.n_out, _lib.ptr(r), ACTIVATIONS[act],
        _lib.DTYPES[dtype], _lib.ptr(out), _lib.stream(device),
    )
    return out


def conv_ln_silu_supported(dtype: torch.dtype, cin: int, cout: int, kvol: int) -> bool:
    """Whether the convolution with the res block's second norm fused into its epilogue
    takes this shape (fp16, 128..512 input channels in steps of 64, 128 outputs)."""
    return dtype == torch.float16 and cout == 128 and cin % 64 == 0 and 128 <= cin <= 512 and 0 < kvol <= 27


def conv_ln_silu(
    features: torch.Tensor,
    plan: ConvPlan,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    coords: torch.Tensor,
    scale1p: torch.Tensor,
    shift: torch.Tensor,
    eps: float,
) -> torch.Tensor:
    """``silu(layer_norm(conv(x)) * scale1p[b] + shift[b])`` per output row, ``b`` the row's
    batch (``coords[:, 0]``): the res block's ``conv1`` then ``norm2`` with its modulation
    and SiLU in one launch (``hi3d_gather_conv_ln_silu``), bitwise :func:`gather_conv`
    followed by ``kernels.layer_norm_modulate(..., act="silu")`` on each batch's rows.
    ``scale1p`` and ``shift`` are fp16 ``[B, 128]``."""
    device = _lib.require_gpu(features, weight, bias, coords, scale1p, shift, plan.gidx)
    if features.ndim != 2 or features.shape[0] != plan.n_in:
        raise ValueError(f"expected features [{plan.n_in}, Cin], got {tuple(features.shape)}")
    x = features.contiguous()
    w = _flat_weight(weight, plan.kvol)
    cin, cout = int(x.shape[1]), int(w.shape[0])
    if int(w.shape[2]) != cin:
        raise ValueError(f"weight expects {int(w.shape[2])} input channels, features have {cin}")
    if x.dtype != torch.float16 or w.dtype != torch.float16 or not conv_ln_silu_supported(x.dtype, cin, cout, plan.kvol):
        raise ValueError(f"conv_ln_silu takes fp16 rows of 128..512 channels into 128 (got {x.dtype} {cin} -> {cout})")
    c = coords.to(torch.int32).contiguous()
    if tuple(c.shape) != (plan.n_out, 4):
        raise ValueError(f"coords must be [{plan.n_out}, 4]")
    sc = scale1p.to(torch.float16).reshape(-1, cout).contiguous()
    sh = shift.to(torch.float16).reshape(-1, cout).contiguous()
    if sc.shape != sh.shape or sc.shape[0] < 1:
        raise ValueError("scale1p and shift must both be [B, 128] with B >= 1")
    b = None if bias is None else bias.to(torch.float16).contiguous()
    out = torch.empty((plan.n_out, cout), dtype=torch.float16, device=device)
    _lib.call(
        "hi3d_gather_conv_ln_silu",
        _lib.ptr(x), plan.n_in, cin, _lib.ptr(w), _lib.ptr(b), cout, plan.kvol, _lib.ptr(plan.rows),
        _lib.ptr(plan.gidx), _lib.ptr(plan.tile_mask), plan.n_out, _lib.ptr(c), int(sc.shape[0]), _lib.ptr(sc),
        _lib.ptr(sh), float(eps), _lib.ptr(out), _lib.stream(device),
    )
    return out


def narrow_supported(dtype: torch.dtype, cin: int, cout: int, kvol: int) -> bool:
    """Whether the narrow-output kernel takes this convolution (at most 16 outputs)."""
    if dtype not in (torch.float16, torch.bfloat16, torch.float32) or not 1 <= cout <= 16 or not 1 <= kvol <= 32:
        return False
    es = torch.empty((), dtype=dtype).element_size()
    return (cin * es) % 64 == 0


def gather_conv_narrow(
    features: torch.Tensor,
    plan: ConvPlan,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    act: str | None = None,
    residual: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """The convolution for at most 16 output channels over a plan (16x16 MFMAs over
    64-row halves of its tiles); fp16 / bf16 / fp32, 64-byte input rows."""
    device = _lib.require_gpu(features, weight, bias, residual, plan.gidx)
    dtype = features.dtype
    if weight.dtype != dtype or (bias is not None and bias.dtype != dtype) or (
        residual is not None and residual.dtype != dtype
    ):
        raise ValueError("features, weight, bias and residual must share one dtype")
    if features.ndim != 2 or features.shape[0] != plan.n_in:
        raise ValueError(f"expected features [{plan.n_in}, Cin], got {tuple(features.shape)}")
    x = features.contiguous()
    w = _flat_weight(weight, plan.kvol)
    cin, cout = int(x.shape[1]), int(w.shape[0])
    if int(w.shape[2]) != cin:
        raise ValueError(f"weight expects {int(w.shape[2])} input channels, features have {cin}")
    if not narrow_supported(dtype, cin, cout, plan.kvol):
        raise ValueError(f"narrow path needs fp16/bf16/fp32, 1..16 outputs and 64-byte rows ({dtype}, {cin}->{cout})")
    if x.data_ptr() % 16:
        x = x.clone()
    b = None if bias is None else bias.contiguous()
    r = None if residual is None else residual.contiguous()
    if r is not None and tuple(r.shape) != (plan.n_out, cout):
        raise ValueError("residual must have the output's shape")
    out = _output(out, plan.n_out, cout, dtype, device)
    _lib.call(
        "hi3d_gather_conv_narrow",
        _lib.ptr(x), plan.n_in, cin, _lib.ptr(w), _lib.ptr(b), cout, plan.kvol, _lib.ptr(plan.rows),
        _lib.ptr(plan.gidx), _lib.ptr(plan.tile_mask), plan.n_out, _lib.ptr(r), ACTIVATIONS[act],
        _lib.DTYPES[dtype], _lib.ptr(out), _lib.stream(device),
    )
    return out


def gather_conv_simple(
    features: torch.Tensor,
    table: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    act: str | None = None,
    residual: torch.Tensor | None = None,
    n_in: int | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """The same convolution from a plain table, any channel count, float64 too."""
    device = _lib.require_gpu(features, table, weight, bias, residual)
    dtype = features.dtype
    if dtype not in _lib.DTYPES:
        raise ValueError(f"unsupported dtype {dtype}")
    if weight.dtype != dtype or (bias is not None and bias.dtype != dtype):
        raise ValueError("features, weight and bias must share one dtype")
    x = features.contiguous()
    t = table.to(torch.int32).contiguous()
    kvol = int(t.shape[1])
    w = _flat_weight(weight, kvol)
    cin, cout = int(x.shape[1]), int(w.shape[0])
    n_out = int(t.shape[0])
    n_in = int(x.shape[0]) if n_in is None else int(n_in)
    out = _output(out, n_out, cout, dtype, device)
    b = None if bias is None else bias.contiguous()
    r = None if residual is None else residual.to(dtype).contiguous()
    _lib.call(
        "hi3d_gather_conv_simple",
        _lib.ptr(x), n_in, cin, _lib.ptr(w), _lib.ptr(b), cout, kvol, _lib.ptr(t), n_out, _lib.ptr(r),
        ACTIVATIONS[act], _lib.DTYPES[dtype], _lib.ptr(out), _lib.stream(device),
    )
    return out


def conv(
    features: torch.Tensor,
    plan: ConvPlan,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    act: str | None = None,
    residual: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Dispatch to the narrow kernel for at most 16 outputs, to the MFMA tile kernels
    when they take the shape, else to the simple kernel. ``out`` may be ``residual``
    (the sum is then accumulated in place)."""
    cin, cout = int(features.shape[1]), int(weight.shape[0])
    if out is not None and features.numel() and out.data_ptr() == features.data_ptr():
        raise ValueError("out must not alias the gathered features")
    if narrow_supported(features.dtype, cin, cout, plan.kvol):
        return gather_conv_narrow(features, plan, weight, bias, act, residual, out)
    if mfma_supported(features.dtype, cin, cout):
        return gather_conv(features, plan, weight, bias, act, residual, out)
    return gather_conv_simple(features, plan.table, weight, bias, act, residual, n_in=plan.n_in, out=out)


def dense_linear_supported(dtype: torch.dtype, cin: int, cout: int) -> bool:
    """Whether the row-wise linear kernel takes this shape (fp16, Cin a multiple of 16 up
    to 128, Cout 64, 128, 192 or 256)."""
    return dtype == torch.float16 and 0 < cin <= 128 and cin % 16 == 0 and 0 < cout <= 256 and cout % 64 == 0


def dense_linear(
    features: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    residual: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``fp16(x W^T + bias)`` over fp16 rows ``x [N, Cin]`` with ``W [Cout, Cin]``, then
    with ``residual`` ``fp16(that + residual)``: the res block's ``linear(h) +
    skip_connection(x)`` in one pass over the rows (``hi3d_dense_linear``), with the
    bits of :func:`conv` over the one-offset identity plan. ``out`` may be ``residual``."""
    n, cin = int(features.shape[0]), int(features.shape[1])
    w = weight.reshape(int(weight.shape[0]), -1)
    cout = int(w.shape[0])
    if int(w.shape[1]) != cin:
        raise ValueError(f"weight takes {int(w.shape[1])} input channels, the rows hold {cin}")
    if not dense_linear_supported(features.dtype, cin, cout):
        raise ValueError(f"dense_linear takes fp16 rows, Cin % 16 == 0 up to 128 and Cout % 64 == 0 up to 256, "
                         f"got {features.dtype} {cin} -> {cout}")
    device = _lib.require_gpu(features, weight, bias, residual, out)
    x = features.contiguous()
    wc = w.to(torch.float16).contiguous()
    b = None if bias is None else bias.to(torch.float16).reshape(-1).contiguous()
    if b is not None and b.numel() != cout:
        raise ValueError(f"bias must have {cout} entries")
    r = None
    if residual is not None:
        if tuple(residual.shape) != (n, cout) or residual.dtype != torch.float16:
            raise ValueError(f"residual must be a [{n}, {cout}] float16 tensor")
        r = residual.contiguous()
    o = _output(out, n, cout, torch.float16, device)
    if o.numel() and o.data_ptr() == x.data_ptr():
        raise ValueError("out must not alias the input rows")
    _lib.call("hi3d_dense_linear", _lib.ptr(x), n, cin, _lib.ptr(wc), _lib.ptr(b), cout, _lib.ptr(r), _lib.ptr(o),
              _lib.stream(device))
    return o


@functools.lru_cache(maxsize=None)
def stride2_up_supported(dtype: torch.dtype, cin: int, cout: int) -> bool:
    """Whether the parent-major transposed kernel takes this shape."""
    if dtype not in (torch.float16, torch.bfloat16):
        return False
    return bool(_lib.lib().hi3d_stride2_up_supported(int(cin), int(cout), _lib.DTYPES[dtype]))


UP_SORTED = True
"""Run the transposed stride-2 convolution over the coarse rows sorted by their
children's slot mask (``hi3d_stride2_up_conv_sorted``, which skips the products of
slots a tile lacks) instead of in row order; the outputs are the same bits."""


def stride2_up(features: torch.Tensor, structure, weight: torch.Tensor, bias: torch.Tensor | None = None,
               out: torch.Tensor | None = None, sorted_rows: bool | None = None) -> torch.Tensor:
    """Transpose of the 2x2x2 / stride-2 convolution onto the fine set of ``structure``
    (a :class:`~hi3d_amd.kmap.Stride2Structure`): ``out[i] = b + W[:, slot(i), :] @
    features[parent(i)]`` with ``W [Cout, 8, Cin]`` (or spconv's ``[Cout, 2, 2, 2, Cin]``).
    ``sorted_rows`` (default ``UP_SORTED``): walk the coarse rows in the structure's
    mask order (``Stride2Structure.up_order``).
    Shapes the parent-major kernel takes (fp16 / bf16, Cin 64 or 128, Cout 64) read each
    coarse row once and write each fine row once; the others run the gather convolution
    over the structure's up table."""
    device = _lib.require_gpu(features, weight, bias, out)
    n_c, n_f = structure.n_coarse, structure.n_fine
    cin, cout = int(features.shape[1]), int(weight.shape[0])
    if features.dim() != 2 or int(features.shape[0]) != n_c:
        raise ValueError(f"expected features [{n_c}, C], got {tuple(features.shape)}")
    w = _flat_weight(weight, 8)
    if int(w.shape[2]) != cin:
        raise ValueError(f"weight takes {int(w.shape[2])} input channels, features have {cin}")
    if not stride2_up_supported(features.dtype, cin, cout):
        return conv(features, structure.up_plan(), w, bias, out=out)
    if w.dtype != features.dtype:
        raise ValueError(f"weight dtype {w.dtype} differs from the features' {features.dtype}")
    x = features.contiguous()
    if x.data_ptr() % 16:
        x = x.clone()
    b = None if bias is None else bias.to(features.dtype).contiguous()
    y = _output(out, n_f, cout, features.dtype, device)
    if UP_SORTED if sorted_rows is None else sorted_rows:
        order, down_sorted = structure.up_order()
        _lib.call("hi3d_stride2_up_conv_sorted", _lib.ptr(x), n_c, cin, _lib.ptr(w), _lib.ptr(b), cout,
                  _lib.ptr(order), _lib.ptr(down_sorted), n_f, _lib.DTYPES[features.dtype], _lib.ptr(y),
                  _lib.stream(device))
        return y
    _lib.call("hi3d_stride2_up_conv", _lib.ptr(x), n_c, cin, _lib.ptr(w), _lib.ptr(b), cout,
              _lib.ptr(structure.down), n_f, _lib.DTYPES[features.dtype], _lib.ptr(y), _lib.stream(device))
    return y
