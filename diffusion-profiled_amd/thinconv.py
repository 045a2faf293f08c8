"""The U-Net's image-channel convolutions on the HIP library (csrc/thinconv.hip).

conv_in (diffusion/unet.py:255-257, 3 -> C) and the output head's conv (:325-329, C -> 3) are
plain nn.Conv2d(bias=False) layers that the reference runs in bf16 under autocast
(train.py:120, :136). ``ImageConv2d`` keeps the nn.Conv2d parameter (state dicts unchanged)
and, on the GPU under a bf16 autocast region, computes the conv as autocast would: x and the
weight rounded to bf16, fp32 accumulation, a bf16 output, and in the backward a bf16 input
gradient and the fp32 weight gradient fp32(bf16(dW)) (the bf16 conv gradient through the
cast's backward). Other cases (CPU, no autocast, unsupported shapes, an input that needs a
gradient on the thin side) run nn.Conv2d itself.
"""
from __future__ import annotations

from typing import Any

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib

DTYPE_BF16, DTYPE_F32 = 0, 1  # include/dpa_fp8.h DPA_DTYPE_*
_THIN = 3
_WIDE = (128, 256)


def _stream(t: torch.Tensor) -> int:
    return _lib.current_stream(t)


def shape_ok(n: int, cin: int, cout: int, h: int, w: int) -> bool:
    """The shapes csrc/thinconv.hip implements: one side 1-3 channels, the other 128 or 256;
    W in {16, 32, 64}, H a multiple of 64 / W."""
    thin_in = cin <= _THIN and cout in _WIDE
    thin_out = cout <= _THIN and cin in _WIDE
    return ((thin_in or thin_out) and w in (16, 32, 64) and h % (64 // w) == 0
            and n * h * w * max(cin, cout) < 2**31)


def _nhwc(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous(memory_format=torch.channels_last)


def _wargs(w: torch.Tensor) -> tuple:
    dt = DTYPE_F32 if w.dtype == torch.float32 else DTYPE_BF16
    return (w.data_ptr(), dt) + tuple(int(s) for s in w.stride())


class ThinConv2dFunction(torch.autograd.Function):
    """y = conv2d(bf16(x), bf16(w), padding=1) in bf16 (fp32 accumulation)."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        n, cin, h, wd = x.shape
        cout = w.shape[0]
        thin_in = cin <= _THIN
        xk = _nhwc(x if (thin_in and x.dtype == torch.float32) else x.to(torch.bfloat16))
        wk = w if w.dtype in (torch.float32, torch.bfloat16) else w.float()
        y = torch.empty((n, cout, h, wd), device=x.device, dtype=torch.bfloat16,
                        memory_format=torch.channels_last)
        xdt = DTYPE_F32 if xk.dtype == torch.float32 else DTYPE_BF16
        _lib.call("dpa_conv3x3_thin_fwd", xk.data_ptr(), xdt, *_wargs(wk), y.data_ptr(), n, h,
                  wd, cin, cout, _stream(x))
        ctx.save_for_backward(xk, wk)
        ctx.w_dtype = w.dtype
        return y

    @staticmethod
    def backward(ctx: Any, gy: torch.Tensor):
        xk, wk = ctx.saved_tensors
        n, h, wd = xk.shape[0], xk.shape[2], xk.shape[3]
        cin, cout = xk.shape[1], wk.shape[0]
        g = _nhwc(gy.to(torch.bfloat16))
        dx = dw = None
        if ctx.needs_input_grad[0]:
            if cout > _THIN:
                raise RuntimeError("ImageConv2d: no input gradient for a thin-input conv")
            dx = torch.empty((n, cin, h, wd), device=g.device, dtype=torch.bfloat16,
                             memory_format=torch.channels_last)
            _lib.call("dpa_conv3x3_thin_dgrad", g.data_ptr(), *_wargs(wk), dx.data_ptr(), n, h,
                      wd, cin, cout, _stream(g))
        if ctx.needs_input_grad[1]:
            ws_bytes = _lib.query("dpa_conv3x3_thin_wgrad_workspace_bytes", n, h, wd, cin, cout)
            ws = torch.empty(ws_bytes, device=g.device, dtype=torch.uint8)
            # [Cout][3][3][Cin] fp32 = the [Cout][Cin][3][3] weight in channels-last order
            dwk = torch.empty((cout, 3, 3, cin), device=g.device, dtype=torch.float32)
            xdt = DTYPE_F32 if xk.dtype == torch.float32 else DTYPE_BF16
            _lib.call("dpa_conv3x3_thin_wgrad", xk.data_ptr(), xdt, g.data_ptr(), dwk.data_ptr(),
                      n, h, wd, cin, cout, ws.data_ptr(), ws_bytes, _stream(g))
            dw = dwk.permute(0, 3, 1, 2)
            if ctx.w_dtype != torch.float32:
                dw = dw.to(ctx.w_dtype)
        return dx, dw


def _autocast_bf16(x: torch.Tensor) -> bool:
    return (torch.is_autocast_enabled(x.device.type)
            and torch.get_autocast_dtype(x.device.type) == torch.bfloat16)


class ImageConv2d(nn.Conv2d):
    """nn.Conv2d(cin, cout, 3, padding=1, bias=False) whose bf16 autocast forward and backward
    run the HIP kernels when one side has 1-3 channels (diffusion/unet.py:255-257, :325-329)."""

    use_hip = True

    def _hip_ok(self, x: torch.Tensor) -> bool:
        if not (self.use_hip and x.is_cuda and x.ndim == 4 and _autocast_bf16(x)):
            return False
        if (self.kernel_size != (3, 3) or self.stride != (1, 1) or self.padding != (1, 1)
                or self.dilation != (1, 1) or self.groups != 1 or self.bias is not None
                or self.padding_mode != "zeros"):
            return False
        n, cin, h, w = x.shape
        if cin <= _THIN and x.requires_grad:  # no thin-side input gradient kernel
            return False
        return shape_ok(n, cin, self.out_channels, h, w)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self._hip_ok(x):
            return ThinConv2dFunction.apply(x, self.weight)
        return F.conv2d(x, self.weight, self.bias, self.stride, self.padding, self.dilation,
                        self.groups)
