"""The transformer's sparse residual block on the gfx950 kernels.

``SparseResBlock3d`` keeps the reference module's constructor, parameter names (so its
state dict loads unchanged) and forward signature
(src/sparc3d/models/transformers/sparc3d_transformer.py:78-144; the MLX form
``_resblock`` / ``_resblock_tail``, src/hi3d_mac/mlx_backend/transformer.py:413-437):

    scale, shift = emb_layers(embedding).chunk(2)         # SiLU -> Linear
    x = updown(x)                                         # optional resampling
    h = silu(norm1(x))                                    # LayerNorm32, affine
    h = conv1(h)                                          # submanifold 3x3x3
    h = silu(norm2(h) * (1 + scale) + shift)              # LayerNorm32, no affine
    h = silu(conv2(h))
    return linear(h) + skip_connection(x)

Each line after the projection is one kernel: the LayerNorm kernel applies norm1's
affine and the SiLU in its epilogue; conv1 applies norm2, each row's batch modulation
and the SiLU to its output rows in its epilogue (``conv.conv_ln_silu``, for 128 hidden
channels; else the convolution and the LayerNorm kernel, the same bits); conv2 applies
the SiLU in its epilogue, and ``linear`` + ``skip_connection`` is one row-wise linear launch whose
residual epilogue adds the skip (``conv.dense_linear``; a gather convolution over the
one-offset identity plan for shapes it does not take, with the same bits; the skip's own
linear, when the channel count changes, is another such launch). The block runs on fp16
features (the reference's fp16 torso, ``convert_to_fp16``); weights of another dtype are
cast to fp16 for the launch.

Roundings: norm1/norm2 as the LayerNorm kernel (fp32 statistics and affine, one fp16
rounding, then two for the modulation); SiLU after a LayerNorm is the fp16
``x * sigmoid(x)`` (sigmoid and product each rounded); the convolutions and the linear
accumulate in fp32 and round once after bias, SiLU and the residual.
"""

from __future__ import annotations

import torch
from torch import nn

from . import conv as _conv
from . import kmap as _kmap
from . import spconv as _spconv
from .kernels import adaln_projection, layer_norm_modulate
from .nn import SparseConv3d, SparseDownsample, SparseTensor, SparseUpsample


def _plan_pair(conv: nn.Module, x: SparseTensor) -> tuple[_kmap.ConvPlan, _kmap.ConvPlan]:
    """The 3x3x3 plan of ``x``'s rows (through ``conv``'s kernel-map cache, so every
    convolution over the rows shares it) and the identity plan of the same rows."""
    data = conv._pairs(x.backend_data())
    if data.kmap is not None:
        return data.kmap.plan(), data.kmap.identity_plan()
    n = int(x.feats.shape[0])
    table = _spconv._table_from_pairs(data, n, 27)
    return _kmap.build_plan(table, n, data.indices), _kmap.identity_plan(n, x.device)


def _half(t: torch.Tensor | None) -> torch.Tensor | None:
    return None if t is None else t.detach().to(torch.float16).contiguous()


class SparseResBlock3d(nn.Module):
    """Residual block with timestep-embedding modulation and optional paired
    resampling (a factor-2 ``SparseDownsample`` or ``SparseUpsample`` before the
    convolutions)."""

    def __init__(
        self,
        channels: int,
        emb_channels: int,
        out_channels: int | None = None,
        downsample: bool = False,
        upsample: bool = False,
    ):
        super().__init__()
        if downsample and upsample:
            raise ValueError("cannot downsample and upsample in one block")
        self.channels = channels
        self.emb_channels = emb_channels
        self.out_channels = out_channels or channels
        self.hidden_channels = self.out_channels // 2
        self.downsample = downsample
        self.upsample = upsample
        self.norm1 = nn.LayerNorm(channels, elementwise_affine=True, eps=1e-6)
        self.norm2 = nn.LayerNorm(self.hidden_channels, elementwise_affine=False, eps=1e-6)
        self.conv1 = SparseConv3d(channels, self.hidden_channels, 3)
        self.conv2 = SparseConv3d(self.hidden_channels, self.hidden_channels, 3)
        self.linear = nn.Linear(self.hidden_channels, self.out_channels)
        nn.init.zeros_(self.linear.weight)
        nn.init.zeros_(self.linear.bias)
        self.emb_layers = nn.Sequential(nn.SiLU(), nn.Linear(emb_channels, 2 * self.hidden_channels, bias=True))
        self.skip_connection = (
            nn.Linear(channels, self.out_channels) if channels != self.out_channels else nn.Identity()
        )
        self.updown: nn.Module | None = None
        if downsample:
            self.updown = SparseDownsample(2)
        elif upsample:
            self.updown = SparseUpsample(2)

    def _modulation(self, embedding: torch.Tensor, batches: int) -> list[tuple[torch.Tensor, torch.Tensor]]:
        """``(fp16(1 + scale), shift)`` of each batch element from ``SiLU -> Linear``."""
        emb = embedding.reshape(embedding.shape[0], -1) if embedding.dim() > 1 else embedding.reshape(1, -1)
        if emb.shape[0] != batches:
            raise ValueError(f"embedding holds {emb.shape[0]} rows for {batches} batch elements")
        proj = self.emb_layers[1]
        return [adaln_projection(proj.weight.detach(), None if proj.bias is None else proj.bias.detach(), emb[b],
                                 apply_silu=True) for b in range(batches)]

    def forward(self, x: SparseTensor, embedding: torch.Tensor) -> SparseTensor:
        if x.feats.dtype != torch.float16 or x.feats.dim() != 2:
            raise NotImplementedError("the fused residual block takes fp16 feature rows [N, C] (the fp16 torso)")
        modulation = self._modulation(embedding, int(x.shape[0]))
        if self.updown is not None:
            x = self.updown(x)
        plan, rows = _plan_pair(self.conv1.conv, x)
        feats = x.feats.contiguous()
        h = layer_norm_modulate(feats, self.norm1.eps, weight=self.norm1.weight.detach(),
                                bias=self.norm1.bias.detach(), act="silu")
        c1, c2 = self.conv1.conv, self.conv2.conv
        w1 = _half(c1.weight).reshape(self.hidden_channels, 27, -1)
        if _conv.conv_ln_silu_supported(h.dtype, self.channels, self.hidden_channels, plan.kvol) and not _conv.HALO:
            # conv1 with norm2, the modulation of each row's batch and SiLU in its epilogue
            h = _conv.conv_ln_silu(h, plan, w1, _half(c1.bias), x.coords, torch.stack([m[0] for m in modulation]),
                                   torch.stack([m[1] for m in modulation]), self.norm2.eps)
        else:
            h = _conv.conv(h, plan, w1, _half(c1.bias))
            if len(modulation) == 1:
                scale1p, shift = modulation[0]
                h = layer_norm_modulate(h, self.norm2.eps, scale=scale1p, shift=shift, act="silu")
            else:
                h = torch.cat([layer_norm_modulate(h[span], self.norm2.eps, scale=s, shift=t, act="silu")
                               for span, (s, t) in zip(x.layout, modulation)])
        h = _conv.conv(h, plan, _half(c2.weight).reshape(self.hidden_channels, 27, -1), _half(c2.bias), act="silu")
        if isinstance(self.skip_connection, nn.Linear):
            sw, sb = _half(self.skip_connection.weight), _half(self.skip_connection.bias)
            if _conv.dense_linear_supported(feats.dtype, self.channels, self.out_channels):
                skip = _conv.dense_linear(feats, sw, sb)
            else:
                skip = _conv.conv(feats, rows, sw[:, None, :], sb)
        else:
            skip = feats
        lw, lb = _half(self.linear.weight), _half(self.linear.bias)
        if _conv.dense_linear_supported(h.dtype, self.hidden_channels, self.out_channels):
            out = _conv.dense_linear(h, lw, lb, residual=skip)
        else:
            out = _conv.conv(h, rows, lw[:, None, :], lb, residual=skip)
        return x.replace(out)
