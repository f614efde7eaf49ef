"""Sparse residual block on the GPU: LayerNorm + adaLN modulate, submanifold conv +
SiLU, submanifold conv + residual.

Semantic template: ``SparseResBlock3d.forward``
(src/sparc3d/models/transformers/sparc3d_transformer.py:132-144) and its MLX form
``_resblock`` / ``_resblock_tail`` (src/hi3d_mac/mlx_backend/transformer.py:413-437):
``scale, shift`` come from a linear projection of the conditioning vector (chunk order
(scale, shift)), the modulation is ``LN(x) * (1 + scale) + shift`` in fp16, and the
residual is added in the feature dtype.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import conv as _conv
from .kernels import adaln_projection, layer_norm_modulate
from .kmap import ConvPlan


@dataclass
class ResBlockWeights:
    proj_weight: torch.Tensor  # [2C, D] fp32
    proj_bias: torch.Tensor | None  # [2C] fp32
    conv1_weight: torch.Tensor  # [C, 3, 3, 3, C] fp16
    conv1_bias: torch.Tensor | None
    conv2_weight: torch.Tensor
    conv2_bias: torch.Tensor | None


def residual_block(
    x: torch.Tensor,
    plan: ConvPlan,
    cond: torch.Tensor,
    w: ResBlockWeights,
    eps: float = 1e-6,
    apply_silu_to_cond: bool = False,
    conv_events=None,
) -> torch.Tensor:
    """``x + conv2(silu(conv1(LN(x) * (1 + scale) + shift)))`` over one kernel map.

    ``conv_events``: optional three ``torch.cuda.Event``s recorded on the current stream
    before the first convolution, between the two and after the second (the convolutions
    run on that stream), for timing them inside a pass of the block."""
    scale1p, shift = adaln_projection(w.proj_weight, w.proj_bias, cond, apply_silu_to_cond)
    h = layer_norm_modulate(x, eps, scale=scale1p, shift=shift)
    if conv_events is not None:
        conv_events[0].record()
    h = _conv.conv(h, plan, w.conv1_weight, w.conv1_bias, act="silu")
    if conv_events is not None:
        conv_events[1].record()
    out = _conv.conv(h, plan, w.conv2_weight, w.conv2_bias, residual=x)
    if conv_events is not None:
        conv_events[2].record()
    return out
