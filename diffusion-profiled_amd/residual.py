"""The U-Net's residual join ``(a + b) / sqrt(2)`` (diffusion/unet.py:161, :203) in one HIP
pass on bf16 tensors, with torch's roundings (``dpa_residual_scale_bf16``); other dtypes or
layouts take the torch expression."""
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


def residual_join(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """(a + b) / sqrt(2)."""
    if (a.is_cuda and a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16
            and a.numel() % 8 == 0 and _same_dense(a, b)
            and a.data_ptr() % 16 == 0 and b.data_ptr() % 16 == 0):
        return ResidualScale.apply(a, b)
    return (a + b) / math.sqrt(2.0)
