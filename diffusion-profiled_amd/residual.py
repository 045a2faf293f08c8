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

# torch divides by a CPU scalar as a product with the fp32 reciprocal of the scalar
INV_SQRT2 = float(np.float32(1.0) / np.float32(math.sqrt(2.0)))


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


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


class ResidualScale(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        return _scale(a, b)

    @staticmethod
    def backward(ctx: Any, g: torch.Tensor):
        g = g.contiguous(memory_format=torch.channels_last) if g.ndim == 4 else g.contiguous()
        if g.dtype != torch.bfloat16 or g.numel() % 8 != 0:
            gs = g / math.sqrt(2.0)
        else:
            gs = _scale(g, None)
        return gs, gs


class ResidualScaleF32(torch.autograd.Function):
    """a fp32, b bf16: (a + b) / sqrt(2) in fp32; gradients g / sqrt(2) in fp32 for a and
    rounded to bf16 for b."""

    @staticmethod
    def forward(ctx: Any, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        y = torch.empty_like(a)
        _lib.call("dpa_residual_scale_f32", a.data_ptr(), b.data_ptr(), y.data_ptr(), a.numel(),
                  INV_SQRT2, _stream(a))
        return y

    @staticmethod
    def backward(ctx: Any, g: torch.Tensor):
        g = g.contiguous(memory_format=torch.channels_last) if g.ndim == 4 else g.contiguous()
        if g.dtype != torch.float32:
            gs = g.float() / math.sqrt(2.0)
            return gs, gs.to(torch.bfloat16)
        ga = torch.empty_like(g)
        gb = torch.empty_like(g, dtype=torch.bfloat16)
        _lib.call("dpa_residual_scale_bwd_f32", g.data_ptr(), ga.data_ptr(), gb.data_ptr(),
                  g.numel(), INV_SQRT2, _stream(g))
        return ga, gb


def residual_join(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """(a + b) / sqrt(2)."""
    if a.is_cuda and _same_dense(a, b) and a.data_ptr() % 16 == 0 and b.data_ptr() % 16 == 0:
        if a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16 and a.numel() % 8 == 0:
            return ResidualScale.apply(a, b)
        if a.numel() % 4 == 0:
            if a.dtype == torch.float32 and b.dtype == torch.bfloat16:
                return ResidualScaleF32.apply(a, b)
            if a.dtype == torch.bfloat16 and b.dtype == torch.float32:
                return ResidualScaleF32.apply(b, a)
    return (a + b) / math.sqrt(2.0)
