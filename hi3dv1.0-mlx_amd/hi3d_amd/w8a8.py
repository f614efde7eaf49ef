"""W8A8 int8 linear on the GPU: per-token quantisation (signed-H64 rotation or none),
int8 MFMA GEMM with int32 accumulation and the dequant + bias epilogue fused.

Mirrors src/hi3d_mac/mlx_backend/w8a8.py: ``signs`` :16-18, ``quantize_activation``
:95-102, ``linear`` :105-119 (same names, argument meaning and ValueErrors). The extra
``rotation`` argument selects ``"h64"`` (the reference's signed block-Hadamard, default)
or ``"none"`` (plain per-token symmetric quantisation).
"""

from __future__ import annotations

from functools import lru_cache

import numpy as np
import torch

from . import _lib

ROTATIONS = ("h64", "none")

FORMAT = "hi3d-w8a8-h64"
"""safetensors metadata ``format`` of released W8A8 checkpoints (models/w8a8/manifest.json:11)."""
REQUIRED_SCALE = "blocks.0.self_attn.to_qkv.w8_scale"
"""The scale whose absence makes the reference refuse a file in W8A8 mode (transformer.py:299-300)."""


@lru_cache(None)
def _signs_np(width: int) -> np.ndarray:
    return np.random.default_rng(314159 + width).choice([-1.0, 1.0], width).astype(np.float32)


def signs(width: int, device: torch.device | str = "cuda") -> torch.Tensor:
    """``default_rng(314159 + width).choice([-1., 1.], width)`` as float32."""
    return _signs_cached(int(width), str(torch.device(device)))


@lru_cache(None)
def _signs_cached(width: int, device: str) -> torch.Tensor:
    return torch.from_numpy(_signs_np(width)).to(device)


def _multiplier(k: int, device, rotation: str, multiplier):
    if rotation not in ROTATIONS:
        raise ValueError(f"rotation must be one of {ROTATIONS}, got {rotation!r}")
    if rotation == "none":
        return None
    if multiplier is None:
        return signs(k, device)
    m = multiplier.to(device=device, dtype=torch.float32).contiguous()
    if m.shape != (k,):
        raise ValueError(f"multiplier must be [{k}]")
    if m.data_ptr() % 16:  # the kernel reads multipliers as 16-byte vectors
        m = m.clone()
    return m


def quantize_activation(x: torch.Tensor, multiplier: torch.Tensor | None = None, rotation: str = "h64"):
    """``(q int8 [M, K], s float32 [M])`` of fp16 rows ``x [..., K]``."""
    k = int(x.shape[-1])
    if rotation == "h64" and k % 64:
        raise ValueError("signed H64 requires width divisible by 64")
    if k % 8:
        raise ValueError("width must be a multiple of 8")
    device = _lib.require_gpu(x)
    x2 = x.reshape(-1, k).to(torch.float16).contiguous()
    m = int(x2.shape[0])
    mult = _multiplier(k, device, rotation, multiplier)
    q = torch.empty((m, k), dtype=torch.int8, device=device)
    s = torch.empty(m, dtype=torch.float32, device=device)
    _lib.call("hi3d_w8a8_quantize", _lib.ptr(x2), m, k, _lib.ptr(mult), _lib.ptr(q), _lib.ptr(s), _lib.stream(device))
    return q, s


def gemm(
    q: torch.Tensor,
    sa: torch.Tensor,
    w: torch.Tensor,
    sw: torch.Tensor,
    bias: torch.Tensor | None,
    return_acc: bool = False,
):
    """Int8 GEMM with fused dequant: ``fp16(((float)acc * sa) * sw + bias)``; with
    ``return_acc`` also the int32 accumulators. ``q [M, K]`` and ``w [N, K]`` int8,
    ``sa [M]`` and ``sw [N]`` float32, ``bias [N]`` (cast to fp16) or None."""
    device = _lib.require_gpu(q, sa, w, sw, bias)
    if q.dtype != torch.int8 or w.dtype != torch.int8 or q.ndim != 2 or w.ndim != 2 or int(w.shape[1]) != int(q.shape[1]):
        raise ValueError("q [M, K] and w [N, K] must be int8 with matching K")
    m, k = int(q.shape[0]), int(q.shape[1])
    n = int(w.shape[0])
    if sa.dtype != torch.float32 or sw.dtype != torch.float32:
        raise ValueError("W8A8 requires float32 scales")
    if tuple(sa.shape) != (m,) or tuple(sw.shape) != (n,):
        raise ValueError(f"scales must be sa [{m}] and sw [{n}], got {tuple(sa.shape)} and {tuple(sw.shape)}")
    if bias is not None and tuple(bias.shape) != (n,):
        raise ValueError(f"bias must be [{n}], got {tuple(bias.shape)}")
    # contiguous operands bound to locals, so every buffer outlives the launch
    qc, sac, wc, swc = q.contiguous(), sa.contiguous(), w.contiguous(), sw.contiguous()
    b = None if bias is None else bias.to(torch.float16).contiguous()
    out = torch.empty((m, n), dtype=torch.float16, device=device)
    acc = torch.empty((m, n), dtype=torch.int32, device=device) if return_acc else None
    _lib.call(
        "hi3d_w8a8_gemm",
        _lib.ptr(qc), _lib.ptr(sac), _lib.ptr(wc), _lib.ptr(swc), _lib.ptr(b), m, n, k, _lib.ptr(out), _lib.ptr(acc),
        _lib.stream(device),
    )
    return (out, acc) if return_acc else out


def linear(x, w, sw, bias, tile=(64, 128), multiplier=None, rotation: str = "h64"):
    """``x [..., K]`` fp16 through the int8 projection ``w [N, K]`` (int8, rows already
    rotated like the activations) with per-row scales ``sw [N]`` and fp16 ``bias [N]``.
    ``tile`` is accepted for signature parity; the GPU kernel picks its own tiles."""
    if w.dtype != torch.int8 or sw.dtype != torch.float32:
        raise ValueError("W8A8 requires int8 weights and float32 scales")
    if w.ndim != 2 or x.shape[-1] != w.shape[1] or tuple(sw.shape) != (w.shape[0],) or tuple(bias.shape) != (w.shape[0],):
        raise ValueError("incompatible W8A8 projection shapes")
    shape = tuple(x.shape[:-1])
    n = int(w.shape[0])
    a, sa = quantize_activation(x, multiplier, rotation)
    y = gemm(a, sa, w, sw, bias)
    return y.reshape(*shape, n)


def _norm_vec(v: torch.Tensor | None, c: int, dtype: torch.dtype, what: str) -> torch.Tensor | None:
    if v is None:
        return None
    t = v.to(dtype).reshape(-1).contiguous()
    if t.numel() != c:
        raise ValueError(f"{what} must have {c} entries")
    if t.data_ptr() % 16:  # the kernel reads per-channel vectors as 16-byte vectors
        t = t.clone()
    return t


def norm_quantize(
    x: torch.Tensor,
    eps: float,
    weight: torch.Tensor | None = None,
    bias: torch.Tensor | None = None,
    scale: torch.Tensor | None = None,
    shift: torch.Tensor | None = None,
    multiplier: torch.Tensor | None = None,
    rotation: str = "h64",
):
    """``quantize_activation(layer_norm_modulate(x, eps, weight, bias, scale, shift))`` in
    one pass, bitwise equal to the two in sequence: ``(q int8 [M, K], s float32 [M])``
    of fp16 rows ``x [..., K]``. The transformer block quantises a norm's output for
    ``to_qkv``, ``cross_attn.to_q`` and ``mlp.0``
    (src/hi3d_mac/mlx_backend/transformer.py:548-549, 570-571, 575-577); here the norm's
    fp16 rows never reach memory. Rows wider than 4096 run the two kernels in sequence."""
    if x.dtype != torch.float16:
        raise ValueError("norm_quantize takes fp16 rows")
    k = int(x.shape[-1])
    if rotation == "h64" and k % 64:
        raise ValueError("signed H64 requires width divisible by 64")
    if k % 8:
        raise ValueError("width must be a multiple of 8")
    if (weight is None) != (bias is None):
        raise ValueError("weight and bias must be given together")
    if (scale is None) != (shift is None):
        raise ValueError("scale and shift must be given together")
    device = _lib.require_gpu(x, weight, bias, scale, shift)
    if k > 4096:
        from . import kernels

        return quantize_activation(kernels.layer_norm_modulate(x, eps, weight, bias, scale, shift), multiplier, rotation)
    x2 = x.reshape(-1, k).contiguous()
    if x2.data_ptr() % 16:
        x2 = x2.clone()
    m = int(x2.shape[0])
    w = _norm_vec(weight, k, torch.float32, "weight")
    b = _norm_vec(bias, k, torch.float32, "bias")
    sc = _norm_vec(scale, k, torch.float16, "scale")
    sh = _norm_vec(shift, k, torch.float16, "shift")
    mult = _multiplier(k, device, rotation, multiplier)
    q = torch.empty((m, k), dtype=torch.int8, device=device)
    s = torch.empty(m, dtype=torch.float32, device=device)
    _lib.call("hi3d_layer_norm_quantize", _lib.ptr(x2), m, k, float(eps), _lib.ptr(w), _lib.ptr(b), _lib.ptr(sc),
              _lib.ptr(sh), _lib.ptr(mult), _lib.ptr(q), _lib.ptr(s), _lib.stream(device))
    return q, s


def norm_linear(x, eps, w, sw, bias, weight=None, norm_bias=None, scale=None, shift=None, multiplier=None,
                rotation: str = "h64"):
    """``linear(layer_norm_modulate(x, eps, weight, norm_bias, scale, shift), w, sw, bias)``
    with the norm and the activation quantiser fused (``norm_quantize``); the same
    output bits as the composition."""
    if w.dtype != torch.int8 or sw.dtype != torch.float32:
        raise ValueError("W8A8 requires int8 weights and float32 scales")
    if w.ndim != 2 or x.shape[-1] != w.shape[1] or tuple(sw.shape) != (w.shape[0],) or tuple(bias.shape) != (w.shape[0],):
        raise ValueError("incompatible W8A8 projection shapes")
    shape = tuple(x.shape[:-1])
    n = int(w.shape[0])
    a, sa = norm_quantize(x, eps, weight, norm_bias, scale, shift, multiplier, rotation)
    return gemm(a, sa, w, sw, bias).reshape(*shape, n)


def quantize_weight(weight: torch.Tensor, rotation: str = "h64", multiplier: torch.Tensor | None = None):
    """Offline weight conversion: ``(w int8 [N, K], sw float32 [N])``, symmetric per output
    row (``maxabs / 127``, round half to even), rows rotated by the same signed H64 as
    the activations when ``rotation == "h64"`` (format ``hi3d-w8a8-h64``,
    models/w8a8/manifest.json:10-17). Uses the activation quantiser on the rows."""
    return quantize_activation(weight.to(torch.float16), multiplier, rotation)


def load_checkpoint(path, device: torch.device | str = "cuda", require_blocks: bool = True) -> dict[str, torch.Tensor]:
    """Tensors of a released ``hi3d-w8a8-h64`` safetensors file on ``device``:
    ``<name>.weight`` int8 ``[N, K]`` (rows rotated like the activations),
    ``<name>.w8_scale`` float32 ``[N]`` and every other tensor as stored
    (transformer.py:289-301; models/w8a8/manifest.json:10-17). Read with the safetensors
    loader, which executes nothing from the file. Raises the reference's ValueError when
    the metadata format is not ``hi3d-w8a8-h64`` or (``require_blocks``) the first block's
    QKV scale is missing, and a ValueError for a scale whose weight is not a matching
    int8 matrix."""
    from safetensors import safe_open

    with safe_open(str(path), framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT:
            raise ValueError("W8A8 requires the released Hi3Dv1.0-mlx-w8a8 checkpoints")
        tensors = {k: f.get_tensor(k) for k in f.keys()}
    if require_blocks and REQUIRED_SCALE not in tensors:
        raise ValueError("W8A8 requires the released Hi3Dv1.0-mlx-w8a8 checkpoints")
    for key, scale in tensors.items():
        if not key.endswith(".w8_scale"):
            continue
        w = tensors.get(key[: -len(".w8_scale")] + ".weight")
        if w is None or w.dtype != torch.int8 or w.ndim != 2 or scale.dtype != torch.float32 or tuple(scale.shape) != (w.shape[0],):
            raise ValueError(f"{key}: expected an int8 [N, K] weight and a float32 [N] scale")
    return {k: v.to(device) for k, v in tensors.items()}


def quantize_checkpoint(tensors: dict[str, torch.Tensor], names, rotation: str = "h64") -> dict[str, torch.Tensor]:
    """``{name}.weight`` of every projection in ``names`` converted to the released layout
    (int8 rows + float32 ``{name}.w8_scale``, :func:`quantize_weight`); other tensors kept."""
    out = dict(tensors)
    for name in names:
        w, sw = quantize_weight(tensors[f"{name}.weight"], rotation)
        out[f"{name}.weight"] = w
        out[f"{name}.w8_scale"] = sw
    return out


def save_checkpoint(path, tensors: dict[str, torch.Tensor]) -> None:
    """Write ``tensors`` as a ``hi3d-w8a8-h64`` safetensors file (host copies)."""
    from safetensors.torch import save_file

    save_file({k: v.detach().cpu().contiguous() for k, v in tensors.items()}, str(path), metadata={"format": FORMAT})


def linear_named(x: torch.Tensor, tensors: dict[str, torch.Tensor], name: str) -> torch.Tensor:
    """``linear`` with ``{name}.weight`` / ``.w8_scale`` / ``.bias`` from a loaded
    checkpoint, as the reference's block linears call it (transformer.py:503-507)."""
    return linear(x, tensors[f"{name}.weight"], tensors[f"{name}.w8_scale"], tensors[f"{name}.bias"])
