"""Torch fake-quant emulation of the FP8 training path: the test reference for the module
level (ResidualBlock, U-Net), run on the CPU.

Each FP8 site is replaced by the reference recipe written with plain torch ops: bf16 cast,
per-tensor scale RN(amax / 448) (1 if amax == 0), e4m3 cast of clamp(x / scale), an exact
float64 accumulation of the e4m3 products, then bf16(fp32(acc) * RN(scale_a * scale_b))
(diffusion/fp8_kernels.py:54-120, :246-247, :464-468). The backward quantizes dy the same
way and returns bf16 gradients (diffusion/fp8_kernels.py:874-913). GroupNorm + SiLU run as
torch float32 ops, with the bf16 rounding at the conv input that the reference's autocast
boundary performs (diffusion/fp8_kernels.py:835).
"""
from __future__ import annotations

import copy
import types

import torch
import torch.nn.functional as F

from conftest import dpa_mod

U = dpa_mod("unet")
FP8 = torch.float8_e4m3fn


def quant(t: torch.Tensor):
    """(e4m3 values as float64, fp32 scale) of bf16(t)."""
    tb = t.detach().to(torch.bfloat16).float()
    amax = tb.abs().max()
    s = amax / 448.0 if float(amax) > 0 else torch.tensor(1.0)
    q = (tb / s).clamp(-448.0, 448.0).to(FP8)
    return q.double(), s.float()


def epilogue(acc64: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor) -> torch.Tensor:
    return (acc64.float() * (sa * sb)).to(torch.bfloat16)


class FakeQuantConv(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, stride: int, pad: int):
        xq, xs = quant(x)
        wq, ws = quant(w)
        ctx.save_for_backward(xq, wq, xs, ws)
        ctx.cfg = (stride, pad, x.shape, w.shape)
        return epilogue(F.conv2d(xq, wq, stride=stride, padding=pad), xs, ws)

    @staticmethod
    def backward(ctx, dy):
        xq, wq, xs, ws = ctx.saved_tensors
        stride, pad, xshape, wshape = ctx.cfg
        dyq, dys = quant(dy)
        dx = epilogue(torch.nn.grad.conv2d_input(xshape, wq, dyq, stride=stride, padding=pad), dys, ws)
        dw = epilogue(torch.nn.grad.conv2d_weight(xq, wshape, dyq, stride=stride, padding=pad), xs, dys)
        return dx, dw, None, None


class FakeQuantLinear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w):
        lead = x.shape[:-1]
        xq, xs = quant(x.reshape(-1, x.shape[-1]))
        wq, ws = quant(w)
        ctx.save_for_backward(xq, wq, xs, ws)
        ctx.lead = lead
        return epilogue(xq @ wq.T, xs, ws).reshape(*lead, w.shape[0])

    @staticmethod
    def backward(ctx, dy):
        xq, wq, xs, ws = ctx.saved_tensors
        dyq, dys = quant(dy.reshape(-1, wq.shape[0]))
        dx = epilogue(dyq @ wq, dys, ws).reshape(*ctx.lead, wq.shape[1])
        dw = epilogue(dyq.T @ xq, xs, dys)
        return dx, dw


def _conv3x3_forward(self, x):
    return FakeQuantConv.apply(x, self.conv.weight, 1, 1)


def _conv1x1_forward(self, x):
    return FakeQuantConv.apply(x, self.weight, 1, 0)


def _linear_forward(self, x):
    assert self.bias is None
    return FakeQuantLinear.apply(x, self.weight)


def emulate(module: torch.nn.Module) -> torch.nn.Module:
    """CPU copy of ``module`` with every FP8 site replaced by its fake-quant emulation
    (current scaling) and the fused GroupNorm+SiLU by torch float32 ops."""
    em = copy.deepcopy(module).cpu()
    for m in em.modules():
        if isinstance(m, U.Conv2dFP8):
            m.forward = types.MethodType(_conv3x3_forward, m)
        elif isinstance(m, U.Conv1x1FP8):
            m.forward = types.MethodType(_conv1x1_forward, m)
        elif isinstance(m, U.LinearFP8):
            m.forward = types.MethodType(_linear_forward, m)
        if hasattr(m, "fused"):
            m.fused = False
    return em
