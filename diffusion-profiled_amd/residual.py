"""The U-Net's residual join ``(a + b) / sqrt(2)`` (diffusion/unet.py:161, :203) in one HIP
pass, with torch's roundings: on two bf16 tensors (``dpa_residual_scale_bf16``), or on the fp32
residual stream with a bf16 branch (``dpa_residual_scale_f32``, fp32 result, and its
one-pass backward); other dtypes or layouts take the torch expression."""
from __future__ import annotations

import math
from typing import Any

import numpy as np
import torch

from . import _lib
from . import fp8_kernels as _fp8
from .fp8_kernels import FP8_DTYPE, Fp8Handoff, mark_amax_partials, placeholder

# torch divides by a CPU scalar as a product with the fp32 reciprocal of the scalar
INV_SQRT2 = float(np.float32(1.0) / np.float32(math.sqrt(2.0)))


def _stream(t: torch.Tensor) -> int:
    return _lib.current_stream(t)


def _same_dense(a: torch.Tensor, b: torch.Tensor) -> bool:
    if a.shape != b.shape or a.stride() != b.stride():
        return False
    if a.is_contiguous():
        return True
    return a.ndim == 4 and a.is_contiguous(memory_format=torch.channels_last)


def _scale(a: torch.Tensor, b: torch.Tensor | None) -> torch.Tensor:
    y = torch.empty_like(a)
    _lib.call("dpa_residual_scale_bf16", a.data_ptr(), None if b is None else b.data_ptr(),
              y.data_ptr(), a.numel(), INV_SQRT2, _stream(a))
    return y


def _bwd_fp8(g: torch.Tensor, hand: Fp8Handoff) -> torch.Tensor:
    """The join's backward writing b's gradient as the e4m3 dy of the conv that produced b
    (to hand.q); returns a's gradient (g's dtype). For a bf16 g, a's gradient holds the very
    bf16 values b's cast saw, so the cast's amax partials are recorded on it too (a 1x1 skip
    conv quantizing it next skips its amax pass; the partials stay in the conv's buffer until
    the next step's window records)."""
    ga = torch.empty_like(g)
    gbq = torch.empty_like(g, dtype=FP8_DTYPE)
    _lib.call("dpa_residual_scale_bwd_fp8", g.data_ptr(), _DT[g.dtype], ga.data_ptr(),
              gbq.data_ptr(), hand.scale.data_ptr(), hand.partials.data_ptr(),
              hand.partials.numel(), hand.count.data_ptr(), g.numel(), INV_SQRT2, _stream(g))
    hand.q = gbq
    if g.dtype == torch.bfloat16 and _fp8.PRODUCER_AMAX:
        mark_amax_partials(ga, hand.partials, _lib.query("dpa_residual_scale_fp8_partials",
                                                         g.numel()))
    return ga


def _bwd_amax(g: torch.Tensor) -> tuple[torch.Tensor | None, torch.Tensor]:
    """The plain join backward (bf16 g: the one bf16 gradient of both operands; fp32 g: the
    fp32 and the bf16 gradient) with amax partials of the bf16 gradient recorded on it, for a
    current-scaling FP8 GEMM that quantizes it next. Returns (fp32 gradient or None, bf16
    gradient)."""
    n = g.numel()
    count = _lib.query("dpa_residual_scale_fp8_partials", n)
    part = torch.empty(count, device=g.device, dtype=torch.int32)
    f32 = g.dtype == torch.float32
    ga = torch.empty_like(g) if f32 else None
    gb = torch.empty_like(g, dtype=torch.bfloat16)
    _lib.call("dpa_residual_scale_bwd_amax", g.data_ptr(), _DT[g.dtype],
              None if ga is None else ga.data_ptr(), gb.data_ptr(), part.data_ptr(), count, n,
              INV_SQRT2, _stream(g))
    return ga, mark_amax_partials(gb, part, count)


def _fp8_grad_ok(g: torch.Tensor, dtype: torch.dtype, hand: Fp8Handoff) -> bool:
    n = g.numel()
    return (g.dtype == dtype and n % 8 == 0 and g.data_ptr() % 16 == 0
            and 0 < _lib.query("dpa_residual_scale_fp8_partials", n) <= hand.partials.numel())


class ResidualScale(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, a: torch.Tensor, b: torch.Tensor,
                hand: Fp8Handoff | None = None) -> torch.Tensor:
        ctx.hand = hand
        return _scale(a, b)

    @staticmethod
    def backward(ctx: Any, g: torch.Tensor):
        g = g.contiguous(memory_format=torch.channels_last) if g.ndim == 4 else g.contiguous()
        hand = ctx.hand
        if hand is not None and _fp8_grad_ok(g, torch.bfloat16, hand):
            return _bwd_fp8(g, hand), placeholder(g.shape, torch.bfloat16, g.device), None
        if g.dtype != torch.bfloat16 or g.numel() % 8 != 0:
            gs = g / math.sqrt(2.0)
        elif _fp8.PRODUCER_AMAX and hand is None:
            gs = _bwd_amax(g)[1]
        else:
            gs = _scale(g, None)
        if hand is not None:             # unfused: cast b's gradient in a pass of its own
            hand.fill_from_bf16(gs)
            return gs, placeholder(g.shape, torch.bfloat16, g.device), None
        return gs, gs, None


class ResidualScaleF32(torch.autograd.Function):
    """a fp32, b bf16: (a + b) / sqrt(2) in fp32; gradients g / sqrt(2) in fp32 for a and
    rounded to bf16 for b."""

    @staticmethod
    def forward(ctx: Any, a: torch.Tensor, b: torch.Tensor,
                hand: Fp8Handoff | None = None) -> torch.Tensor:
        y = torch.empty_like(a)
        _lib.call("dpa_residual_scale_f32", a.data_ptr(), b.data_ptr(), y.data_ptr(), a.numel(),
                  INV_SQRT2, _stream(a))
        ctx.hand = hand
        return y

    @staticmethod
    def backward(ctx: Any, g: torch.Tensor):
        g = g.contiguous(memory_format=torch.channels_last) if g.ndim == 4 else g.contiguous()
        hand = ctx.hand
        if hand is not None and _fp8_grad_ok(g, torch.float32, hand):
            return _bwd_fp8(g, hand), placeholder(g.shape, torch.bfloat16, g.device), None
        if g.dtype != torch.float32:
            gs = g.float() / math.sqrt(2.0)
            ga, gb = gs, gs.to(torch.bfloat16)
        elif _fp8.PRODUCER_AMAX and hand is None and g.numel() % 8 == 0:
            ga, gb = _bwd_amax(g)
        else:
            ga = torch.empty_like(g)
            gb = torch.empty_like(g, dtype=torch.bfloat16)
            _lib.call("dpa_residual_scale_bwd_f32", g.data_ptr(), ga.data_ptr(), gb.data_ptr(),
                      g.numel(), INV_SQRT2, _stream(g))
        if hand is not None:             # unfused: cast b's gradient in a pass of its own
            hand.fill_from_bf16(gb)
            return ga, placeholder(g.shape, torch.bfloat16, g.device), None
        return ga, gb, None


def join_fp8_ok(a: torch.Tensor, b_shape) -> bool:
    """Whether residual_join(a, b) with a hand-off can run for a channels-last bf16 b of
    shape b_shape (b not formed yet)."""
    return (a.is_cuda and tuple(a.shape) == tuple(b_shape) and a.ndim == 4
            and a.is_contiguous(memory_format=torch.channels_last) and a.data_ptr() % 16 == 0
            and a.dtype in (torch.bfloat16, torch.float32) and a.numel() % 8 == 0)


def join_kernel_ok(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Whether residual_join(a, b) runs as one of the HIP Functions (b bf16)."""
    return (a.is_cuda and _same_dense(a, b) and a.data_ptr() % 16 == 0 and b.data_ptr() % 16 == 0
            and b.dtype == torch.bfloat16 and a.dtype in (torch.bfloat16, torch.float32)
            and a.numel() % 8 == 0)


def residual_join(a: torch.Tensor, b: torch.Tensor, hand: Fp8Handoff | None = None) -> torch.Tensor:
    """(a + b) / sqrt(2). With ``hand`` (b bf16, the output of a delayed-scaling FP8 conv, and
    ``join_kernel_ok``) the backward writes b's gradient to hand.q as that conv's e4m3 dy."""
    if hand is not None:
        if not join_kernel_ok(a, b):
            raise ValueError("FP8 hand-off through the residual join: no kernel for these operands")
        if a.dtype == torch.bfloat16:
            return ResidualScale.apply(a, b, hand)
        return ResidualScaleF32.apply(a, b, hand)
    if a.is_cuda and _same_dense(a, b) and a.data_ptr() % 16 == 0 and b.data_ptr() % 16 == 0:
        if a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16 and a.numel() % 8 == 0:
            return ResidualScale.apply(a, b)
        if a.numel() % 4 == 0:
            if a.dtype == torch.float32 and b.dtype == torch.bfloat16:
                return ResidualScaleF32.apply(a, b)
            if a.dtype == torch.bfloat16 and b.dtype == torch.float32:
                return ResidualScaleF32.apply(b, a)
    return (a + b) / math.sqrt(2.0)


_DT = {torch.bfloat16: 0, torch.float32: 1}  # include/dpa_fp8.h DPA_DTYPE_*


class UpsampleConcat(torch.autograd.Function):
    """cat([up(a), h], dim=1), fp32, NHWC, with up the 2x nearest upsampling (or identity):
    the decoder input of diffusion/unet.py:379-382 in one pass each way."""

    @staticmethod
    def forward(ctx: Any, a: torch.Tensor, h: torch.Tensor, up: bool) -> torch.Tensor:
        n, c1, ha, wa = a.shape
        _, c2, hh, wh = h.shape
        y = torch.empty((n, c1 + c2, hh, wh), device=a.device, dtype=torch.float32,
                        memory_format=torch.channels_last)
        _lib.call("dpa_upsample_concat_f32", a.data_ptr(), _DT[a.dtype], h.data_ptr(),
                  _DT[h.dtype], y.data_ptr(), n, hh, wh, c1, c2, int(up), _stream(a))
        ctx.meta = (a.shape, a.dtype, h.shape, h.dtype, int(up))
        return y

    @staticmethod
    def backward(ctx: Any, gy: torch.Tensor):
        a_shape, a_dtype, h_shape, h_dtype, up = ctx.meta
        gy = gy.float().contiguous(memory_format=torch.channels_last)
        ga = torch.empty(a_shape, device=gy.device, dtype=a_dtype, memory_format=torch.channels_last)
        gh = torch.empty(h_shape, device=gy.device, dtype=h_dtype, memory_format=torch.channels_last)
        n, c1 = a_shape[0], a_shape[1]
        c2, hh, wh = h_shape[1], h_shape[2], h_shape[3]
        _lib.call("dpa_upsample_concat_bwd_f32", gy.data_ptr(), ga.data_ptr(), _DT[a_dtype],
                  gh.data_ptr(), _DT[h_dtype], n, hh, wh, c1, c2, up, _stream(gy))
        return ga, gh, None


def upsample_concat(a: torch.Tensor, h: torch.Tensor, up: bool) -> torch.Tensor:
    """torch.concat([F.interpolate(a, scale_factor=2, mode="nearest") if up else a, h], 1) as
    autocast evaluates it (fp32 result)."""
    cl = torch.channels_last
    # the fused result is fp32: what autocast's fp32 interpolate and the promoting concat give
    f32_result = (up and torch.is_autocast_enabled("cuda")) or torch.float32 in (a.dtype, h.dtype)
    if (f32_result and a.is_cuda and a.dtype in _DT and h.dtype in _DT and a.ndim == 4 and h.ndim == 4
            and a.is_contiguous(memory_format=cl) and h.is_contiguous(memory_format=cl)
            and a.shape[1] % 4 == 0 and h.shape[1] % 4 == 0
            and a.shape[0] == h.shape[0]
            and a.shape[2] << int(up) == h.shape[2] and a.shape[3] << int(up) == h.shape[3]
            and a.data_ptr() % 16 == 0 and h.data_ptr() % 16 == 0):
        return UpsampleConcat.apply(a, h, up)
    import torch.nn.functional as F
    x = F.interpolate(a, scale_factor=2.0, mode="nearest") if up else a
    return torch.concat([x, h], dim=1)


class Downsample2(torch.autograd.Function):
    """F.interpolate(a, scale_factor=0.5, mode="nearest") as autocast evaluates it: fp32 out,
    gradient in a's dtype (zero off the sampled pixels); NHWC, one pass each way."""

    @staticmethod
    def forward(ctx: Any, a: torch.Tensor) -> torch.Tensor:
        n, c, h, w = a.shape
        y = torch.empty((n, c, h // 2, w // 2), device=a.device, dtype=torch.float32,
                        memory_format=torch.channels_last)
        _lib.call("dpa_downsample2_f32", a.data_ptr(), _DT[a.dtype], y.data_ptr(), n, h, w, c,
                  _stream(a))
        ctx.meta = (a.shape, a.dtype)
        return y

    @staticmethod
    def backward(ctx: Any, gy: torch.Tensor):
        shape, dtype = ctx.meta
        gy = gy.float().contiguous(memory_format=torch.channels_last)
        ga = torch.empty(shape, device=gy.device, dtype=dtype, memory_format=torch.channels_last)
        n, c, h, w = shape
        _lib.call("dpa_downsample2_bwd_f32", gy.data_ptr(), ga.data_ptr(), _DT[dtype], n, h, w, c,
                  _stream(gy))
        return ga


class Downsample2Tee(torch.autograd.Function):
    """(downsample2(a), a): the encoder activation that feeds both the next level (through the
    2x downsampling) and the decoder's concatenation (diffusion/unet.py:368-376). The backward
    adds the concatenation's gradient of a inside the downsampling's backward
    (dpa_downsample2_bwd_add_f32) instead of autograd's separate accumulation kernel: the same
    sum with the same roundings."""

    @staticmethod
    def forward(ctx: Any, a: torch.Tensor):
        y = Downsample2.forward(ctx, a)
        return y, a.view_as(a)

    @staticmethod
    def backward(ctx: Any, gy: torch.Tensor | None, gskip: torch.Tensor | None):
        shape, dtype = ctx.meta
        if gy is None:
            return gskip
        if (gskip is None or gskip.dtype != dtype
                or not gskip.is_contiguous(memory_format=torch.channels_last)
                or gskip.data_ptr() % 16 != 0):
            ga = Downsample2.backward(ctx, gy)
            return ga if gskip is None else ga + gskip
        gy = gy.float().contiguous(memory_format=torch.channels_last)
        ga = torch.empty(shape, device=gy.device, dtype=dtype, memory_format=torch.channels_last)
        n, c, h, w = shape
        _lib.call("dpa_downsample2_bwd_add_f32", gy.data_ptr(), gskip.data_ptr(), ga.data_ptr(),
                  _DT[dtype], n, h, w, c, _stream(gy))
        return ga


def _down_ok(a: torch.Tensor) -> bool:
    return ((torch.is_autocast_enabled("cuda") or a.dtype == torch.float32) and a.is_cuda
            and a.dtype in _DT and a.ndim == 4 and a.shape[1] % 4 == 0
            and a.shape[2] % 2 == 0 and a.shape[3] % 2 == 0
            and a.is_contiguous(memory_format=torch.channels_last) and a.data_ptr() % 16 == 0)


def downsample2(a: torch.Tensor) -> torch.Tensor:
    """F.interpolate(a, scale_factor=0.5, mode="nearest") (fp32 under autocast)."""
    if _down_ok(a):
        return Downsample2.apply(a)
    import torch.nn.functional as F
    return F.interpolate(a, scale_factor=0.5, mode="nearest")


def downsample2_tee(a: torch.Tensor):
    """(downsample2(a), a) with the second output's gradient added inside the downsampling's
    backward (Downsample2Tee); elsewhere (a, the plain downsampling)."""
    if _down_ok(a):
        return Downsample2Tee.apply(a)
    return downsample2(a), a
