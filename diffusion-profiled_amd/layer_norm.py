"""LayerNorm on bf16 token rows with fp32 statistics, as an autograd Function (the HIP
library's dpa_layernorm_*).

Replaces the attention block's ``self.norm(seq)`` (diffusion/unet.py:174, :187), which
autocast runs in fp32 (on an fp32 copy of bf16 tokens, or on fp32 tokens of the fp32 residual
stream as they are) and whose result the qkv projection rounds back to bf16: here the kernel
reads the bf16 or fp32 tokens and writes that bf16 result; the input gradient comes back in
the tokens' dtype.
"""
from __future__ import annotations

from typing import Any

import torch

from . import _lib
from . import fp8_kernels as _fp8


def _stream(t: torch.Tensor) -> int:
    return _lib.current_stream(t)


def supported(c: int) -> bool:
    return c % 64 == 0 and c // 64 in (1, 2, 4, 8, 16)


DTYPE_BF16, DTYPE_F32 = 0, 1  # include/dpa_fp8.h DPA_DTYPE_*


class LayerNormBF16(torch.autograd.Function):
    """y = bf16(LayerNorm(x)) over the last axis; x bf16 or fp32 (rows contiguous),
    gamma/beta fp32."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, eps: float):
        c = x.shape[-1]
        xb = x.contiguous() if x.dtype == torch.float32 else x.to(torch.bfloat16).contiguous()
        rows = xb.numel() // c
        out = torch.empty_like(xb, dtype=torch.bfloat16)
        mean = torch.empty(rows, device=x.device, dtype=torch.float32)
        rstd = torch.empty(rows, device=x.device, dtype=torch.float32)
        g32, b32 = gamma.float().contiguous(), beta.float().contiguous()
        dt = DTYPE_F32 if xb.dtype == torch.float32 else DTYPE_BF16
        if _fp8.PRODUCER_AMAX:
            # the per-workgroup maxima of |out| for the qkv projection's e4m3 cast
            npart = _lib.query("dpa_layernorm_fwd_partials", rows, c)
            part = torch.empty(npart, device=x.device, dtype=torch.int32)
            _lib.call("dpa_layernorm_fwd_amax", xb.data_ptr(), dt, g32.data_ptr(),
                      b32.data_ptr(), out.data_ptr(), mean.data_ptr(), rstd.data_ptr(), rows, c,
                      float(eps), part.data_ptr(), _stream(xb))
            _fp8.mark_amax_partials(out, part, npart)
        else:
            _lib.call("dpa_layernorm_fwd_ex", xb.data_ptr(), dt, g32.data_ptr(), b32.data_ptr(),
                      out.data_ptr(), mean.data_ptr(), rstd.data_ptr(), rows, c, float(eps),
                      _stream(xb))
        ctx.save_for_backward(xb, g32, mean, rstd)
        ctx.x_dtype = x.dtype
        ctx.param_dtypes = (gamma.dtype, beta.dtype)
        return out

    @staticmethod
    def backward(ctx: Any, dout: torch.Tensor):
        xb, g32, mean, rstd = ctx.saved_tensors
        c = xb.shape[-1]
        rows = xb.numel() // c
        dout = dout.to(torch.bfloat16).contiguous()
        dx = torch.empty_like(xb)
        dgamma = torch.empty(c, device=xb.device, dtype=torch.float32)
        dbeta = torch.empty(c, device=xb.device, dtype=torch.float32)
        ws_bytes = _lib.query("dpa_layernorm_bwd_workspace_bytes", rows, c)
        ws = torch.empty(ws_bytes, device=xb.device, dtype=torch.uint8)
        dt = DTYPE_F32 if xb.dtype == torch.float32 else DTYPE_BF16
        _lib.call("dpa_layernorm_bwd_ex", xb.data_ptr(), dt, dout.data_ptr(), g32.data_ptr(),
                  mean.data_ptr(), rstd.data_ptr(), dx.data_ptr(), dgamma.data_ptr(),
                  dbeta.data_ptr(), ws.data_ptr(), ws_bytes, rows, c, _stream(xb))
        return (dx.to(ctx.x_dtype), dgamma.to(ctx.param_dtypes[0]),
                dbeta.to(ctx.param_dtypes[1]), None)


class LayerNormTee(torch.autograd.Function):
    """(bf16(LayerNorm(x)), x): the attention block's norm and its skip input
    (diffusion/unet.py:182-187, :201: the block input feeds the LayerNorm and the residual
    join). The backward adds the skip path's gradient of x into dx inside the LayerNorm kernel
    (dpa_layernorm_bwd_ex_add) instead of autograd's separate accumulation kernel: the same
    sum with the same roundings (fp32 + fp32, or bf16(dx) + bf16 rounded again)."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, eps: float):
        out = LayerNormBF16.forward(ctx, x, gamma, beta, eps)
        return out, x.view_as(x)

    @staticmethod
    def backward(ctx: Any, dout: torch.Tensor, dskip: torch.Tensor | None):
        xb, g32, mean, rstd = ctx.saved_tensors
        if dskip is None or dskip.dtype != xb.dtype or xb.dtype != ctx.x_dtype:
            dx, dgamma, dbeta, _ = LayerNormBF16.backward(ctx, dout)
            if dskip is not None:
                dx = dx + dskip.to(dx.dtype)
            return dx, dgamma, dbeta, None
        c = xb.shape[-1]
        rows = xb.numel() // c
        dout = dout.to(torch.bfloat16).contiguous()
        add = dskip.contiguous()
        dx = torch.empty_like(xb)
        dgamma = torch.empty(c, device=xb.device, dtype=torch.float32)
        dbeta = torch.empty(c, device=xb.device, dtype=torch.float32)
        ws_bytes = _lib.query("dpa_layernorm_bwd_workspace_bytes", rows, c)
        ws = torch.empty(ws_bytes, device=xb.device, dtype=torch.uint8)
        dt = DTYPE_F32 if xb.dtype == torch.float32 else DTYPE_BF16
        _lib.call("dpa_layernorm_bwd_ex_add", xb.data_ptr(), dt, dout.data_ptr(),
                  g32.data_ptr(), mean.data_ptr(), rstd.data_ptr(), add.data_ptr(),
                  dx.data_ptr(), dgamma.data_ptr(), dbeta.data_ptr(), ws.data_ptr(), ws_bytes,
                  rows, c, _stream(xb))
        return (dx, dgamma.to(ctx.param_dtypes[0]), dbeta.to(ctx.param_dtypes[1]), None)


def layer_norm_bf16(x: torch.Tensor, norm: torch.nn.LayerNorm) -> torch.Tensor:
    return LayerNormBF16.apply(x, norm.weight, norm.bias, norm.eps)


def layer_norm_tee(x: torch.Tensor, norm: torch.nn.LayerNorm):
    """(bf16(norm(x)), x) with the skip gradient added inside the LayerNorm backward; x a
    contiguous bf16 or fp32 token view."""
    return LayerNormTee.apply(x, norm.weight, norm.bias, norm.eps)
