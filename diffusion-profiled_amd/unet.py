"""The DDPM U-Net of fattorib/diffusion-profiled on the gfx950 FP8 path.

Module tree, parameter and buffer names, initialisation and forward arithmetic follow
diffusion/unet.py, so a reference ``state_dict`` loads unchanged (and vice versa). What runs
underneath differs:

* ``Conv2dFP8`` (diffusion/unet.py:32-94): registry shapes go through ``triton_conv2d_fp8``
  (the HIP kernels) with the same current/delayed scaling and window state machine; with
  ``UNetConfig.fp8_all_convs`` the other 3x3 convs whose channels are multiples of 128 use
  the general FP8 conv (current scaling) instead of the bf16 fallback.
* GroupNorm + SiLU (diffusion/unet.py:151, :157-159, :380-384) and the FiLM ``(w + 1) * h + b``
  run as one fused HIP kernel each way (``gn_silu``).
* With ``UNetConfig.fp8_linears`` the bias-free linears (time MLP, FiLM projection, qkv, out)
  and the 1x1 skip convs use the FP8 GEMM with current scaling.
* Attention (diffusion/unet.py:181-203): on the GPU the HIP self-attention kernels
  (``attention``: q, k, v read in place from the qkv projection, head dim 64, up to 256
  tokens), other shapes the reference's ``scaled_dot_product_attention`` limited to its fused
  kernels; ``_Attention`` (dense batched products, no transposed-view operands) serves the CPU.
  The attention LayerNorm, the residual joins, the decoder's upsample+concat and the encoder's
  downsample are HIP kernels too.

The torch ops left (the 3->128 and 128->3 convs whose channel counts the FP8 kernels do not
take, the time embedding's sinusoid) stay in PyTorch-ROCm, as in the reference.
"""
from __future__ import annotations

import math
from collections import deque
from dataclasses import asdict, dataclass
from functools import partial
from typing import Any

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import fp8_kernels as K
from . import grouped as GR
from .attention import self_attention_qkv
from .attention import supported as attn_supported
from .layer_norm import layer_norm_bf16, layer_norm_tee
from .residual import (downsample2, downsample2_tee, join_fp8_ok, residual_join,
                       upsample_concat)
from .layer_norm import supported as ln_supported
from .gn_silu import DROPOUT_SEEDS, dropout_ok as gn_dropout_ok, fp8_ok as gn_fp8_ok
from .gn_silu import group_norm_silu, group_norm_silu_film, group_norm_silu_tee
from .gn_silu import upcat_group_norm_silu_tee, upcat_ok
from .gn_silu import supported as gn_supported
from .thinconv import ImageConv2d


@dataclass
class UNetConfig:
    """diffusion/unet.py:13-28, plus three switches for the fused/FP8 sites of this build."""

    in_channels: int
    base_hidden: int
    scales: list[int]
    n_heads: int
    p_drop: float
    attn_resolutions: list[int]
    in_resolution: int
    n_resblocks: int
    fp8_convs_enabled: bool = False
    fp8_scaling_type: str = "current"
    fp8_amax_history: int = 1024
    fp8_all_convs: bool = False
    fp8_linears: bool = False
    fused_gn_silu: bool = True

    def as_dict(self):
        return asdict(self)


def _on_gpu(x: torch.Tensor) -> bool:
    return x.is_cuda


class _PreparedFP8Weight:
    """Mixin of the FP8 layers: records the FP8 path a layer takes on the GPU (so a
    weight_prep.WeightPrep plan can cover it) and hands out the step's prepared weight while
    that plan is active (between its run() at the start of UNet.forward and the forward's end)."""

    _fp8_mode: str | None = None
    _fp8_prepared = None
    _fp8_plan = None

    _fp8_frag = False

    def _note_fp8_mode(self, mode: str, w: torch.Tensor, x: torch.Tensor | None = None) -> None:
        """Record the layer's FP8 path; for a 3x3 conv whose input shape takes the halo-patch
        kernel, also that its prepared weight should be in that kernel's fragment layouts."""
        if self._fp8_mode is not None or not w.is_cuda or w.dtype != torch.float32:
            return
        dense = (w.is_contiguous(memory_format=torch.channels_last) if w.ndim == 4
                 else w.is_contiguous())
        if dense:
            self._fp8_mode = mode
            if x is not None and w.ndim == 4 and w.shape[2] == 3:
                n, cin, h, wd = x.shape
                self._fp8_frag = K.hconv_shape(n, cin, w.shape[0], h, wd)

    def _prepared(self, mode: str):
        plan = self._fp8_plan
        if self._fp8_prepared is None or self._fp8_mode != mode or plan is None or not plan.active:
            return None
        return self._fp8_prepared


class Conv2dFP8(_PreparedFP8Weight, nn.Module):
    """3x3 / stride 1 / pad 1 conv, FP8 when the shape allows (diffusion/unet.py:32-94).

    In delayed mode the window maxima and window/position updates run inside
    ``K.Conv2dFP8DelayedWindowed`` (same state machine, fewer launches);
    ``fused_window_update = False`` selects the reference's op-by-op form."""

    fused_window_update = True

    def __init__(
        self,
        in_channels: int,
        out_channels: int,
        fp8_convs_enabled: bool,
        scaling_type: str = "current",
        amax_history: int | None = None,
        fp8_all_convs: bool = False,
    ):
        super().__init__()
        self.conv = nn.Conv2d(in_channels, out_channels, (3, 3), stride=1, padding=1, bias=False)
        self.scaling_type = scaling_type
        self.fp8_convs_enabled = fp8_convs_enabled
        self.fp8_all_convs = fp8_all_convs
        assert self.scaling_type in ["current", "delayed"]
        if scaling_type == "delayed":
            assert amax_history is not None
            self.amax_history = amax_history
            self.register_buffer("amax_window_weights", torch.zeros(amax_history))
            self.register_buffer("amax_window_acts", torch.zeros(amax_history))
            self.register_buffer("amax_window_dy", torch.zeros(amax_history))
            self.register_buffer("window_pos", torch.zeros((), dtype=torch.long))

    def conv_fp8(self, x: torch.Tensor, weight: torch.Tensor) -> bool:
        """diffusion/unet.py:58-60: FP8 iff enabled and the shape is in the registry."""
        shape = (x.shape[1], weight.shape[0], x.shape[2], x.shape[3])
        return self.fp8_convs_enabled and shape in K.SUPPORTED_UNET_SHAPES

    def conv_fp8_general(self, x: torch.Tensor, weight: torch.Tensor) -> bool:
        return (self.fp8_convs_enabled and self.fp8_all_convs and x.shape[1] % 128 == 0
                and weight.shape[0] % 128 == 0)

    def fp8_handoffs(self, x_shape) -> tuple[K.Fp8Handoff, K.Fp8Handoff] | None:
        """Hand-offs (x, dy) for producers that write this conv's e4m3 operands, when an input
        of x_shape takes the delayed-scaling path with the step's prepared weight; else None."""
        if not (self.scaling_type == "delayed" and self.fused_window_update
                and self.fp8_convs_enabled) or "forward" in vars(self):
            return None                    # (an instance-level forward replaces this path)
        cout = self.conv.weight.shape[0]
        if (x_shape[1], cout, x_shape[2], x_shape[3]) not in K.SUPPORTED_UNET_SHAPES:
            return None
        pw = self._prepared("delayed")
        if pw is None:
            return None
        return (K.Fp8Handoff(pw.hist[0], pw.parts[0], pw.parts[1]),
                K.Fp8Handoff(pw.hist[2], pw.parts[2], pw.parts[3]))

    def forward(self, x: torch.Tensor, xq: torch.Tensor | None = None,
                dy_hand: K.Fp8Handoff | None = None) -> torch.Tensor:
        """xq: the e4m3 input its producer wrote (x is then a placeholder); dy_hand: the
        hand-off whose producer backward writes the e4m3 dy (see ``fp8_handoffs``)."""
        if xq is not None or dy_hand is not None:
            pw = self._prepared("delayed")
            assert pw is not None, "FP8 hand-off without the step's prepared weight"
            if xq is None:
                x = x.contiguous(memory_format=torch.channels_last)
            return K.Conv2dFP8DelayedPrepared.apply(
                x, self.conv.weight, pw.q, pw.qt, pw.scale, pw.hist, pw.parts, xq, dy_hand)
        if self.conv_fp8(x, self.conv.weight):
            x = x.contiguous(memory_format=torch.channels_last)
            if self.scaling_type == "current":
                return K.triton_conv2d_fp8(x, self.conv.weight)
            if self.fused_window_update and not torch.compiler.is_compiling():
                pw = self._prepared("delayed")
                if pw is not None:
                    return K.Conv2dFP8DelayedPrepared.apply(
                        x, self.conv.weight, pw.q, pw.qt, pw.scale, pw.hist, pw.parts)
                self._note_fp8_mode("delayed", self.conv.weight, x)
                return K.Conv2dFP8DelayedWindowed.apply(
                    x, self.conv.weight, self.amax_window_acts, self.amax_window_weights,
                    self.amax_window_dy, self.window_pos)
            with torch.no_grad():
                x_scale_hist = torch.max(self.amax_window_acts)
                w_scale_hist = torch.max(self.amax_window_weights)
            out, x_scale_curr, w_scale_curr = K.triton_conv2d_fp8(
                x, self.conv.weight, (x_scale_hist, w_scale_hist),
                (self.amax_window_dy, self.window_pos), do_delayed=True,
            )
            with torch.no_grad():
                window_idx = self.window_pos.unsqueeze(0)
                self.amax_window_weights.scatter_(0, window_idx, w_scale_curr.detach().unsqueeze(0))
                self.amax_window_acts.scatter_(0, window_idx, x_scale_curr.detach().unsqueeze(0))
                self.window_pos.add_(1).remainder_(self.amax_history)
            return out
        if self.conv_fp8_general(x, self.conv.weight):
            pw = self._prepared("current")
            if pw is not None:
                return K.Conv2dFP8GeneralPrepared.apply(x, self.conv.weight, pw.q, pw.qt,
                                                        pw.scale, 1, 1)
            self._note_fp8_mode("current", self.conv.weight, x)
            return K.conv2d_fp8(x, self.conv.weight, 1, 1)
        return self.conv(x)


class Conv1x1FP8(_PreparedFP8Weight, nn.Conv2d):
    """The bias-free 1x1 skip projection (diffusion/unet.py:137-139) with an FP8 path; the
    parameter is the nn.Conv2d ``weight`` so checkpoints are unchanged."""

    def __init__(self, in_channels: int, out_channels: int, fp8: bool):
        super().__init__(in_channels, out_channels, (1, 1), bias=False)
        self.fp8 = fp8

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.fp8 and _on_gpu(x) and self.in_channels % 128 == 0 and self.out_channels % 128 == 0:
            pw = self._prepared("current")
            if pw is not None:
                return K.Conv2dFP8GeneralPrepared.apply(x, self.weight, pw.q, pw.qt, pw.scale, 1, 0)
            self._note_fp8_mode("current", self.weight)
            return K.conv2d_fp8(x, self.weight, 1, 0)
        return super().forward(x)


class LinearFP8(_PreparedFP8Weight, nn.Linear):
    """nn.Linear with the FP8 GEMM (forward and both gradients) when enabled and shaped for it."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True, fp8: bool = False):
        super().__init__(in_features, out_features, bias=bias)
        self.fp8 = fp8

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.fp8 and _on_gpu(x) and K.linear_fp8_supported(self.in_features, self.out_features):
            pw = self._prepared("linear")
            if pw is not None:
                return K.LinearFP8Prepared.apply(x, self.weight, self.bias, pw.q, pw.qt, pw.scale,
                                                 self._fp8_plan.x_cache)
            self._note_fp8_mode("linear", self.weight)
            return K.LinearFP8Function.apply(x, self.weight, self.bias)
        return super().forward(x)


def norm_silu(norm: nn.GroupNorm, x: torch.Tensor, fused: bool, film_scale=None, film_shift=None):
    """silu(norm(x)) or silu(film_scale * norm(x) + film_shift); bf16 from the fused kernel."""
    if fused and _on_gpu(x) and gn_supported(x.shape[1], norm.num_groups):
        return group_norm_silu(x, norm.weight, norm.bias, norm.num_groups, norm.eps,
                               film_scale, film_shift)
    # autocast runs GroupNorm in float32 (diffusion/unet.py:151, :157); so does this path
    h = norm(x.float() if x.dtype in (torch.bfloat16, torch.float16) else x)
    if film_scale is not None:
        h = film_scale * h + film_shift
    return F.silu(h)


class TimeEmbed(nn.Module):
    """diffusion/unet.py:97-104. ``_pre``: this forward's projection, computed with the other
    blocks' in one grouped launch (UNet._group_films), taken by the next call."""

    _pre = None

    def __init__(self, embed_channels: int, channels: int, fp8: bool = False):
        super().__init__()
        self.mlp = LinearFP8(embed_channels, channels, bias=False, fp8=fp8)

    def forward(self, t: torch.Tensor):
        pre = self._pre
        if pre is not None:
            self._pre = None
            return pre[:, :, None, None]
        return self.mlp(t)[:, :, None, None]


def _conv_handoff(conv: Conv2dFP8, h: torch.Tensor, xh: K.Fp8Handoff | None,
                  dyh: K.Fp8Handoff | None) -> torch.Tensor:
    if xh is None and dyh is None:
        return conv(h)
    return conv(h, None if xh is None else xh.q, dyh)


class CatInput:
    """A decoder stage's input torch.concat([F.interpolate(a, scale_factor=2) if up else a, h],
    dim=1) (diffusion/unet.py:379-382), not yet formed: the stage's first residual block reads
    it through the fused upsample-and-concatenate GroupNorm where that applies, and forms it
    (upsample_concat) otherwise."""

    def __init__(self, a: torch.Tensor, h: torch.Tensor, up: bool):
        self.a, self.h, self.up = a, h, up
        n, ca, ha, wa = a.shape
        s = 2 if up else 1
        self.shape = torch.Size((n, ca + h.shape[1], ha * s, wa * s))
        self.is_cuda = a.is_cuda
        self.device = a.device

    def materialize(self) -> torch.Tensor:
        return upsample_concat(self.a, self.h, up=self.up)


class ResidualBlock(nn.Module):
    """diffusion/unet.py:107-161.

    With ``fp8_handoff`` (delayed scaling, weights prepared for the step) the producers write
    the e4m3 operands of the block's two FP8 convs directly, cast with the convs' window
    scales, instead of bf16 tensors that a separate pass casts: GN1 conv_1's input, GN2
    conv_2's input and, in its backward, conv_1's dy; the join's backward conv_2's dy. The
    bytes and window records are those of the unfused path."""

    fp8_handoff = True

    def __init__(self, config: UNetConfig, in_chann: int, out_chann: int, p_drop: float = 0.0):
        super().__init__()
        conv = partial(Conv2dFP8, fp8_convs_enabled=config.fp8_convs_enabled,
                       scaling_type=config.fp8_scaling_type, amax_history=config.fp8_amax_history,
                       fp8_all_convs=config.fp8_all_convs)
        self.conv_1 = conv(in_chann, out_chann)
        self.conv_2 = conv(out_chann, out_chann)
        self.norm1 = nn.GroupNorm(32, in_chann)
        self.norm2 = nn.GroupNorm(32, out_chann)
        self.t_embed_wb = TimeEmbed(4 * config.base_hidden, 2 * out_chann, fp8=config.fp8_linears)
        self.skip_connection: nn.Module = nn.Identity()
        if in_chann != out_chann:
            self.skip_connection = Conv1x1FP8(in_chann, out_chann, fp8=config.fp8_linears)
        self.dropout = nn.Dropout(p_drop)
        self.fused = config.fused_gn_silu
        self.reset_parameters()

    def reset_parameters(self):
        torch.nn.init.zeros_(self.conv_2.conv.weight)

    def forward(self, x: torch.Tensor | CatInput, t: torch.Tensor):
        cat = None
        if isinstance(x, CatInput):
            # the fused upsample-and-concatenate GroupNorm: bf16 sources, a 1x1 skip conv
            # (which reads the bf16 concatenation the kernel writes), the fused first norm
            if (self.fused and upcat_ok(x.a, x.h, x.up)
                    and gn_supported(x.shape[1], self.norm1.num_groups)
                    and isinstance(self.skip_connection, Conv1x1FP8)
                    and torch.is_autocast_enabled("cuda")):
                cat = x
            else:
                x = x.materialize()
        n, _, hh, ww = x.shape
        y_shape = (n, self.conv_1.conv.out_channels, hh, ww)     # conv_1's and conv_2's output
        gpu = self.fused and _on_gpu(x)
        g1, g2 = self.norm1.num_groups, self.norm2.num_groups
        fused1 = gpu and gn_supported(x.shape[1], g1) and gn_dropout_ok(x)
        wb = self.t_embed_wb(t)
        p_drop = self.dropout.p if self.training else 0.0
        fused2 = (gpu and wb.dtype == torch.bfloat16 and gn_supported(y_shape[1], g2)
                  and (p_drop == 0.0 or gn_dropout_ok(x)))
        c1 = self.conv_1.fp8_handoffs(x.shape) if gpu and self.fp8_handoff else None
        c2 = self.conv_2.fp8_handoffs(y_shape) if gpu and self.fp8_handoff else None
        x1 = c1[0] if c1 and fused1 and gn_fp8_ok(x.shape, g1, c1[0]) else None
        dy1 = c1[1] if c1 and fused2 and gn_fp8_ok(y_shape, g2, c1[1]) else None
        x2 = c2[0] if c2 and fused2 and gn_fp8_ok(y_shape, g2, c2[0]) else None
        if fused1:
            # the skip input's gradient is accumulated inside the GroupNorm backward
            # a 1x1 skip conv rounds its input to bf16 (FP8 path or autocast); the kernel
            # writes that copy as it reads x
            skip16 = (isinstance(self.skip_connection, Conv1x1FP8)
                      and torch.is_autocast_enabled("cuda"))
            if cat is not None:
                h, resid = upcat_group_norm_silu_tee(cat.a, cat.h, self.norm1.weight,
                                                     self.norm1.bias, g1, self.norm1.eps, x1)
            else:
                h, resid = group_norm_silu_tee(x, self.norm1.weight, self.norm1.bias, g1,
                                               self.norm1.eps, skip16, x1)
        else:
            if cat is not None:
                x = cat.materialize()
            resid, h = x, norm_silu(self.norm1, x, self.fused)
        x = _conv_handoff(self.conv_1, h, x1, dy1)
        if fused2:
            # the kernel reads (w, b) from wb, forms bf16(w + 1) itself and applies the dropout
            h = group_norm_silu_film(x, self.norm2.weight, self.norm2.bias, g2, self.norm2.eps,
                                     wb, p_drop, x2, dy1)
        else:
            w, b = torch.chunk(wb, chunks=2, dim=1)
            h = self.dropout(norm_silu(self.norm2, x, self.fused, w + 1, b))
        skip = self.skip_connection(resid)
        dy2 = c2[1] if c2 and join_fp8_ok(skip, y_shape) else None
        x = _conv_handoff(self.conv_2, h, x2, dy2)
        return residual_join(skip, x, dy2)


class _Attention(torch.autograd.Function):
    """softmax(q k^T / sqrt(d)) v over [B*heads, L, d] with dense batched products only.

    No operand of a batched product is a transposed view (transposes are materialised on the
    small [B, d, L] side, and the two products whose natural form has a transposed L x L
    operand are computed transposed). The softmax and its gradient take bf16 scores and
    work in float32 inside torch's kernels, so no float32 L x L tensor is written. The scale
    is folded into q (and k in the backward); for d a power of four it is a power of two and
    the fold is exact."""

    @staticmethod
    def forward(ctx: Any, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
        scale = 1.0 / math.sqrt(q.shape[-1])
        # autocast would run the softmax on a float32 copy of the scores
        with torch.autocast(device_type="cuda", enabled=False):
            qs = (q * scale).contiguous()
            k, v = k.contiguous(), v.contiguous()
            s = torch.bmm(qs, k.transpose(1, 2).contiguous())
            p = torch.softmax(s, dim=-1)
            o = torch.bmm(p, v)
        ctx.save_for_backward(qs, k, v, p)
        ctx.scale = scale
        return o

    @staticmethod
    def backward(ctx: Any, do: torch.Tensor):
        qs, k, v, p = ctx.saved_tensors
        with torch.autocast(device_type="cuda", enabled=False):
            do = do.to(qs.dtype).contiguous()
            dv = torch.bmm(do.transpose(1, 2).contiguous(), p).transpose(1, 2)   # (p^T do)
            dp = torch.bmm(do, v.transpose(1, 2).contiguous())
            ds = torch._softmax_backward_data(dp, p, -1, p.dtype)
            dq = torch.bmm(ds, (k * ctx.scale).contiguous())
            dk = torch.bmm(qs.transpose(1, 2).contiguous(), ds).transpose(1, 2)  # (ds^T qs)
        return dq, dk, dv


_GPU_SDPA = True  # False: the dense formulation below on the GPU too
_HIP_SDPA = True  # False: torch's fused SDPA kernels instead of the HIP self-attention


def _fused_sdpa():
    """SDPA restricted to the memory-efficient and flash kernels (preferred in that order)."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    backends = [SDPBackend.EFFICIENT_ATTENTION, SDPBackend.FLASH_ATTENTION]
    try:
        return sdpa_kernel(backends, set_priority=True)
    except TypeError:  # older torch: no priority argument
        return sdpa_kernel(backends)


class CHWAttention(nn.Module):
    """diffusion/unet.py:164-203."""

    def __init__(self, config: UNetConfig, hidden_size: int):
        super().__init__()
        self.config = config
        self.nh = config.n_heads
        self.qkv = LinearFP8(hidden_size, 3 * hidden_size, bias=False, fp8=config.fp8_linears)
        self.out = LinearFP8(hidden_size, hidden_size, bias=False, fp8=config.fp8_linears)
        self.norm = nn.LayerNorm(hidden_size)
        self.reset_parameters()

    def reset_parameters(self):
        torch.nn.init.zeros_(self.out.weight)

    # the skip path's gradient added inside the LayerNorm backward (LayerNormTee)
    ln_tee = True

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        resid = x
        b, c, h, w = x.shape
        seq = x.permute(0, 2, 3, 1).reshape(b, h * w, c)           # b (h w) c
        if _on_gpu(x) and ln_supported(c):
            # the bf16 tokens in, the bf16 the qkv projection would round to out (fp32 stats)
            if (self.ln_tee and seq.is_contiguous() and x.dtype in (torch.bfloat16, torch.float32)
                    and seq.data_ptr() % 16 == 0):
                seq, tokens = layer_norm_tee(seq, self.norm)
                resid = tokens.reshape(b, h, w, c).permute(0, 3, 1, 2)
            else:
                seq = layer_norm_bf16(seq, self.norm)
        else:
            seq = self.norm(seq)
        qkv = self.qkv(seq)
        q, k, v = torch.chunk(qkv, chunks=3, dim=-1)
        hd = c // self.nh

        def heads(t):                                              # b l (nh hd) -> (b nh) l hd
            return t.reshape(b, h * w, self.nh, hd).transpose(1, 2).reshape(b * self.nh, h * w, hd)

        dt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else q.dtype
        if _on_gpu(x) and _GPU_SDPA and _HIP_SDPA and dt == torch.bfloat16 \
                and attn_supported(h * w, c, self.nh):
            # the HIP kernel: q, k, v read in place from qkv, the output written as
            # "b l (nh hd)" (diffusion/unet.py:188-198 without the rearranges)
            o = self_attention_qkv(qkv, self.nh)
        elif _on_gpu(x) and _GPU_SDPA:
            # the reference's F.scaled_dot_product_attention (diffusion/unet.py:196), limited to
            # the fused (memory-efficient / flash) kernels: the math fallback would run bf16
            # batched products on transposed views
            def bnld(t):                                           # b l (nh hd) -> b nh l hd
                return t.reshape(b, h * w, self.nh, hd).transpose(1, 2).to(dt)
            with _fused_sdpa():
                o = F.scaled_dot_product_attention(bnld(q), bnld(k), bnld(v))
            o = o.transpose(1, 2).reshape(b, h * w, c)
        else:
            o = _Attention.apply(heads(q).to(dt), heads(k).to(dt), heads(v).to(dt))
            o = o.reshape(b, self.nh, h * w, hd).transpose(1, 2).reshape(b, h * w, c)
        o = self.out(o)
        return residual_join(o.reshape(b, h, w, c).permute(0, 3, 1, 2), resid)


class Stage(nn.Module):
    """diffusion/unet.py:206-242."""

    def __init__(self, config: UNetConfig, in_channels: int, hidden_channels: int,
                 out_channels: int, attention: bool = False, num_blocks: int = 2):
        super().__init__()
        self.num_blocks = num_blocks
        self.blocks = nn.ModuleList()
        self.attns = nn.ModuleList()
        self.blocks.append(ResidualBlock(config, in_channels, hidden_channels, p_drop=config.p_drop))
        self.attns.append(CHWAttention(config, hidden_channels) if attention else nn.Identity())
        for _ in range(num_blocks - 2):
            self.blocks.append(ResidualBlock(config, hidden_channels, hidden_channels, p_drop=config.p_drop))
            self.attns.append(CHWAttention(config, hidden_channels) if attention else nn.Identity())
        self.blocks.append(ResidualBlock(config, hidden_channels, out_channels, p_drop=config.p_drop))
        self.attns.append(CHWAttention(config, out_channels) if attention else nn.Identity())

    def forward(self, x: torch.Tensor, t: torch.Tensor):
        for block, attn in zip(self.blocks, self.attns):
            x = block(x, t)
            x = attn(x)
        return x


class _OutHead(nn.Sequential):
    """GroupNorm(32) + SiLU + 3x3 conv to image channels (diffusion/unet.py:325-329); the
    first two run as the fused kernel. Indices 0/1/2 keep the reference's state_dict keys."""

    def __init__(self, channs: int, out_channels: int, fused: bool):
        super().__init__(nn.GroupNorm(32, channs), nn.SiLU(),
                         ImageConv2d(channs, out_channels, kernel_size=(3, 3), padding=1,
                                     bias=False))
        self.fused = fused

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self[2](norm_silu(self[0], x, self.fused))


class UNet(nn.Module):
    """diffusion/unet.py:245-388."""

    # the encoder activations' two gradients summed inside the downsampling's backward
    down_tee = True
    # a decoder stage's upsample-and-concatenate read by its first GroupNorm (CatInput)
    upcat_gn = True

    def __init__(self, config: UNetConfig):
        super().__init__()
        self.config = config
        self.base_channs = config.base_hidden
        channs_1 = config.scales[0] * self.base_channs
        self.conv_in = ImageConv2d(config.in_channels, channs_1, kernel_size=(3, 3), padding=1,
                                   bias=False)

        down_stages: deque = deque()
        up_stages: deque = deque()
        res = config.in_resolution
        for i in range(0, len(config.scales) - 1):
            chann_curr = self.base_channs * config.scales[i]
            chann_next = self.base_channs * config.scales[i + 1]
            do_attn = res in config.attn_resolutions
            down_stages.append(Stage(config, chann_curr, chann_curr, chann_next, attention=do_attn,
                                     num_blocks=config.n_resblocks))
            up_stages.appendleft(Stage(config, chann_next + chann_next, chann_curr, chann_curr,
                                       attention=do_attn, num_blocks=config.n_resblocks + 1))
            res = res // 2

        mid_stage = config.scales[-1] * self.base_channs
        down_stages.append(Stage(config, mid_stage, mid_stage, mid_stage, num_blocks=config.n_resblocks))
        up_stages.appendleft(Stage(config, mid_stage + mid_stage, mid_stage, mid_stage,
                                   num_blocks=config.n_resblocks + 1))
        # attention=True in the middle whatever attn_resolutions says, as in the reference
        self.mid = Stage(config, mid_stage, mid_stage, mid_stage, attention=True,
                         num_blocks=config.n_resblocks)
        self.down_stages = nn.ModuleList(list(down_stages))
        self.up_stages = nn.ModuleList(list(up_stages))

        self.out = _OutHead(channs_1, self.config.in_channels, config.fused_gn_silu)
        fp8_lin = config.fp8_linears
        self.time_embed = nn.Sequential(
            LinearFP8(self.base_channs, 4 * self.config.base_hidden, bias=False, fp8=fp8_lin),
            nn.SiLU(),
            LinearFP8(4 * self.config.base_hidden, 4 * self.config.base_hidden, bias=False, fp8=fp8_lin),
            nn.SiLU(),
        )
        self.reset_parameters()
        self.downsample = partial(F.interpolate, scale_factor=0.5, mode="nearest")
        self.upsample = partial(F.interpolate, scale_factor=2.0, mode="nearest")
        half = self.base_channs // 2
        freqs = torch.exp(-torch.arange(half, dtype=torch.float32) * (math.log(10000.0) / half))
        self.register_buffer("freqs", freqs, persistent=False)

    def _timestep(self, t: torch.Tensor):
        emb = t[:, None].float() * self.freqs[None]
        emb = torch.cat([emb.sin(), emb.cos()], dim=1)
        if self.base_channs % 2 == 1:
            emb = F.pad(emb, (0, 1))
        return emb

    def reset_parameters(self):
        assert isinstance(self.out[-1], nn.Conv2d)
        torch.nn.init.zeros_(self.out[-1].weight)

    # Grouped FP8 weight preparation (weight_prep.WeightPrep): when enabled, the first GPU
    # forward records which layers run in FP8, the next builds the plan (outside graph capture)
    # and every forward from then on starts with the plan's three launches.
    weight_prep_enabled = False
    _wprep = None
    _fp8_seen = False

    def _weight_prep(self, x: torch.Tensor):
        if not self.weight_prep_enabled or not x.is_cuda or torch.compiler.is_compiling():
            # under torch.compile every FP8 layer takes its per-call path: the reference's op
            # API, registered as torch.library custom ops (ops.py), which the graph holds
            return None
        if self._wprep is None:
            if not self._fp8_seen or torch.cuda.is_current_stream_capturing():
                self._fp8_seen = True
                return None
            from .weight_prep import WeightPrep
            self._wprep = WeightPrep.from_model(self)
            if self._wprep is None:
                self.weight_prep_enabled = False
                return None
        self._wprep.run()
        self._wprep.active = True
        return self._wprep

    def forward(self, x: torch.Tensor, t: torch.Tensor) -> torch.Tensor:
        plan = self._weight_prep(x)
        n_drop = sum(1 for m in self.modules()
                     if isinstance(m, ResidualBlock) and m.training and m.dropout.p > 0.0)
        if n_drop and _on_gpu(x):
            DROPOUT_SEEDS.fill(x.device, n_drop)
        try:
            return self._forward(x, t)
        finally:
            DROPOUT_SEEDS.clear()
            if plan is not None:
                plan.active = False
                plan.x_cache.clear()

    # the FiLM projections of all residual blocks (the same t_emb) as one grouped FP8 op
    group_films = True

    def _group_films(self, t_emb: torch.Tensor) -> list:
        """Runs every block's FiLM projection in one GroupedLinearFP8 when all of them take the
        prepared FP8 linear path, leaving each result on its TimeEmbed; returns those modules."""
        if not self.group_films or not t_emb.is_cuda or t_emb.ndim != 2:
            return []
        embeds = [m.t_embed_wb for m in self.modules() if isinstance(m, ResidualBlock)]
        layers = []
        for e in embeds:
            lin = e.mlp
            if (not isinstance(lin, LinearFP8) or not lin.fp8 or "forward" in vars(lin)
                    or "forward" in vars(e) or lin.bias is not None):
                return []
            pw = lin._prepared("linear")
            if pw is None:
                return []
            layers.append((pw.q, pw.qt, pw.scale))
        if not GR.supported(t_emb.shape[0], t_emb.shape[1], [e.mlp.out_features for e in embeds]):
            return []
        outs = GR.grouped_linear_fp8(t_emb, layers, [e.mlp.weight for e in embeds])
        for e, o in zip(embeds, outs):
            e._pre = o
        return embeds

    def _forward(self, x: torch.Tensor, t: torch.Tensor) -> torch.Tensor:
        t_emb = self.time_embed(self._timestep(t))
        grouped = self._group_films(t_emb)
        try:
            return self._stages(x, t_emb)
        finally:
            for e in grouped:
                e._pre = None

    def _stages(self, x: torch.Tensor, t_emb: torch.Tensor) -> torch.Tensor:
        act = self.conv_in(x)
        hs = []
        for i, stage in enumerate(self.down_stages):
            if i > 0:
                # self.downsample(act): F.interpolate(scale 0.5, nearest), one pass on the GPU;
                # the skip copy's gradient (from the decoder's concatenation) is added inside
                # the downsampling's backward
                if self.down_tee:
                    act, hs[-1] = downsample2_tee(act)
                else:
                    act = downsample2(act)
            act = stage(act, t_emb)
            hs.append(act)
        act = self.mid(act, t_emb)
        for i, stage in enumerate(self.up_stages):
            h = hs.pop()
            # torch.concat([self.upsample(act) if i > 0 else act, h], dim=1): one pass on the
            # GPU, or none, read by the stage's first GroupNorm from act and h (CatInput)
            if self.upcat_gn and i > 0:
                act = stage(CatInput(act, h, True), t_emb)
            else:
                act = stage(upsample_concat(act, h, up=i > 0), t_emb)
        return self.out(act)


def cfg5_config(**overrides) -> UNetConfig:
    """The benchmark U-Net as the reference trains and profiles it (train.py:220-233,
    extra/profile_cuda_graph.py:121-133): ch 128, mults (1,2,2,2), 2 ResBlocks per level,
    attention at 16x16 and 8x8 plus the middle stage, dropout 0.2, delayed scaling; here
    every conv and linear whose channel counts are multiples of 128 runs in FP8."""
    kw: dict[str, Any] = dict(
        in_channels=3, base_hidden=128, scales=[1, 2, 2, 2], n_heads=4, p_drop=0.2,
        attn_resolutions=[16, 8], in_resolution=32, n_resblocks=2, fp8_convs_enabled=True,
        fp8_scaling_type="delayed", fp8_amax_history=1024, fp8_all_convs=True, fp8_linears=True,
        fused_gn_silu=True,
    )
    kw.update(overrides)
    return UNetConfig(**kw)
