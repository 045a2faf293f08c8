"""The reference's FP8 op API (diffusion/fp8_kernels.py:518-808) as torch.library custom ops.

The reference compiles the model that calls its FP8 ops (train.py:252) and its training step
(diffusion/ddpm.py:208). A ctypes call inside a Python function is opaque to Dynamo and
breaks the graph there; a custom op is one node of the graph, with a fake implementation
that gives AOTAutograd and Inductor the outputs' shapes, dtypes and strides without touching
the device. Each op's body is the C-ABI launch sequence of ``fp8_kernels`` (fresh outputs
from torch's caching allocator, launches on torch's current stream), so eager calls, graph
capture and compiled graphs run the same kernels. The ops are CUDA-only: a CPU tensor raises
instead of falling back.

Namespace ``dpa_fp8``:

=================  ====================================================================
``quantize``        current scaling: (e4m3 q, fp32 scale)  (fp8_kernels.py:559-601)
``quantize_delayed``  cast with prev_scale, return the current scale  (:518-556)
``conv_fwd``        e4m3 conv forward, any supported (k, stride, pad)  (:604-639)
``conv_dgrad``      e4m3 conv data gradient  (:671-709)
``conv_wgrad``      e4m3 conv weight gradient  (:723-808)
``gemm``            e4m3 GEMM x @ w^T (the FP8 linear; no reference kernel)
``gemm_dgrad``      its data gradient dy @ w
``gemm_wgrad``      its weight gradient dy^T @ x
``conv2d_fp8``      current-scaling conv with autograd (``triton_conv2d_fp8``'s current mode,
                    :822-923), saving the e4m3 operands as the reference does
``linear_fp8``      current-scaling FP8 linear with autograd
=================  ====================================================================

The two autograd ops return the saved e4m3 tensors and scales as extra outputs (a custom
op's autograd context only sees its inputs and outputs); ``fp8_kernels`` returns only the
first output to callers.
"""
from typing import Optional

import torch

from . import fp8_kernels as K

_CL = torch.channels_last
_BF16 = torch.bfloat16


def _empty_cl(shape, device, dtype=_BF16) -> torch.Tensor:
    return torch.empty(shape, device=device, dtype=dtype, memory_format=_CL)


# ---- quantization --------------------------------------------------------------------
@torch.library.custom_op("dpa_fp8::quantize", mutates_args=(), device_types="cuda")
def quantize(tensor: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    q, s = K._quantize_impl(tensor, None)
    return q, s


@quantize.register_fake
def _quantize_fake(tensor):
    t = tensor if K._dense(tensor) else tensor.contiguous()
    return (torch.empty_like(t, dtype=K.FP8_DTYPE, memory_format=torch.preserve_format),
            t.new_empty((), dtype=torch.float32))


@torch.library.custom_op("dpa_fp8::quantize_delayed", mutates_args=(), device_types="cuda")
def quantize_delayed(tensor: torch.Tensor, prev_scale: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    q, s = K._quantize_impl(tensor, prev_scale)
    return q, s


@quantize_delayed.register_fake
def _quantize_delayed_fake(tensor, prev_scale):
    return _quantize_fake(tensor)


# ---- convolution ---------------------------------------------------------------------
@torch.library.custom_op("dpa_fp8::conv_fwd", mutates_args=(), device_types="cuda")
def conv_fwd(x: torch.Tensor, weight: torch.Tensor, x_scale: torch.Tensor,
             weight_scale: torch.Tensor, stride: int, padding: int) -> torch.Tensor:
    return K.conv2d_fp8_fwd_general(x, weight, x_scale, weight_scale, stride, padding)


@conv_fwd.register_fake
def _conv_fwd_fake(x, weight, x_scale, weight_scale, stride, padding):
    batch, _, height, width = x.shape
    cout, _, kh, _ = weight.shape
    oh, ow = K._out_hw(height, width, kh, stride, padding)
    return _empty_cl((batch, cout, oh, ow), x.device)


@torch.library.custom_op("dpa_fp8::conv_dgrad", mutates_args=(), device_types="cuda")
def conv_dgrad(dy: torch.Tensor, weight: torch.Tensor, dy_scale: torch.Tensor,
               weight_scale: torch.Tensor, height: int, width: int, stride: int,
               padding: int) -> torch.Tensor:
    return K.conv2d_fp8_dgrad_general(dy, weight, dy_scale, weight_scale, (height, width),
                                      stride, padding)


@conv_dgrad.register_fake
def _conv_dgrad_fake(dy, weight, dy_scale, weight_scale, height, width, stride, padding):
    return _empty_cl((dy.shape[0], weight.shape[1], height, width), dy.device)


@torch.library.custom_op("dpa_fp8::conv_wgrad", mutates_args=(), device_types="cuda")
def conv_wgrad(x: torch.Tensor, dy: torch.Tensor, x_scale: torch.Tensor, dy_scale: torch.Tensor,
               kernel_size: int, stride: int, padding: int, split_k: int,
               out_f32: bool) -> torch.Tensor:
    """split_k <= 0: the library's choice."""
    return K.conv2d_fp8_wgrad_general(x, dy, x_scale, dy_scale, kernel_size, stride, padding,
                                      split_k if split_k > 0 else None, out_f32)


@conv_wgrad.register_fake
def _conv_wgrad_fake(x, dy, x_scale, dy_scale, kernel_size, stride, padding, split_k, out_f32):
    return _empty_cl((dy.shape[1], x.shape[1], kernel_size, kernel_size), x.device,
                     torch.float32 if out_f32 else _BF16)


# ---- GEMM (the FP8 linear) -------------------------------------------------------------
@torch.library.custom_op("dpa_fp8::gemm", mutates_args=(), device_types="cuda")
def gemm(a: torch.Tensor, b: torch.Tensor, a_scale: torch.Tensor, b_scale: torch.Tensor,
         bias: Optional[torch.Tensor]) -> torch.Tensor:
    return K.linear_fp8_prequantized(a, b, a_scale, b_scale, bias)


@gemm.register_fake
def _gemm_fake(a, b, a_scale, b_scale, bias):
    return a.new_empty((a.shape[0], b.shape[0]), dtype=_BF16)


@torch.library.custom_op("dpa_fp8::gemm_dgrad", mutates_args=(), device_types="cuda")
def gemm_dgrad(dy: torch.Tensor, weight: torch.Tensor, dy_scale: torch.Tensor,
               weight_scale: torch.Tensor) -> torch.Tensor:
    return K.linear_fp8_dgrad_prequantized(dy, weight, dy_scale, weight_scale)


@gemm_dgrad.register_fake
def _gemm_dgrad_fake(dy, weight, dy_scale, weight_scale):
    return dy.new_empty((dy.shape[0], weight.shape[1]), dtype=_BF16)


@torch.library.custom_op("dpa_fp8::gemm_wgrad", mutates_args=(), device_types="cuda")
def gemm_wgrad(x: torch.Tensor, dy: torch.Tensor, x_scale: torch.Tensor, dy_scale: torch.Tensor,
               out_f32: bool) -> torch.Tensor:
    return K.linear_fp8_wgrad_prequantized(x, dy, x_scale, dy_scale, out_f32)


@gemm_wgrad.register_fake
def _gemm_wgrad_fake(x, dy, x_scale, dy_scale, out_f32):
    return x.new_empty((dy.shape[1], x.shape[1]), dtype=torch.float32 if out_f32 else _BF16)


# ---- current-scaling conv and linear with autograd --------------------------------------
@torch.library.custom_op("dpa_fp8::conv2d_fp8", mutates_args=(), device_types="cuda")
def conv2d_fp8(x: torch.Tensor, weight: torch.Tensor, stride: int, padding: int
               ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(y, e4m3 x, e4m3 w, x scale, w scale): bf16 casts of x and the weight, current-scaling
    quantization, forward (diffusion/fp8_kernels.py:835-866 in current mode)."""
    xb = x.to(_BF16).contiguous(memory_format=_CL)
    wb = weight.to(_BF16).contiguous(memory_format=_CL)
    xq, xs = K._quantize_impl(xb, None)
    wq, ws = K._quantize_impl(wb, None)
    y = K.conv2d_fp8_fwd_general(xq, wq, xs, ws, stride, padding)
    return y, xq, wq, xs, ws


@conv2d_fp8.register_fake
def _conv2d_fp8_fake(x, weight, stride, padding):
    batch, cin, height, width = x.shape
    cout, _, kh, kw = weight.shape
    oh, ow = K._out_hw(height, width, kh, stride, padding)
    scalar = x.new_empty((), dtype=torch.float32)
    return (_empty_cl((batch, cout, oh, ow), x.device),
            _empty_cl((batch, cin, height, width), x.device, K.FP8_DTYPE),
            _empty_cl((cout, cin, kh, kw), x.device, K.FP8_DTYPE), scalar, scalar.clone())


def _conv2d_fp8_setup(ctx, inputs, output):
    x, weight, stride, padding = inputs
    _, xq, wq, xs, ws = output
    ctx.save_for_backward(xq, wq, xs, ws)
    ctx.geom = (x.shape[2], x.shape[3], stride, padding)
    ctx.x_dtype, ctx.w_dtype = x.dtype, weight.dtype


def _conv2d_fp8_backward(ctx, dy, *_unused):
    """diffusion/fp8_kernels.py:874-913 in current mode: dy to bf16, its own scale, then the
    data and weight gradients from the saved e4m3 operands; returned in the inputs' dtypes
    (what autograd's cast of the reference's bf16 gradients gives)."""
    xq, wq, xs, ws = ctx.saved_tensors
    height, width, stride, padding = ctx.geom
    dyq, dys = quantize(dy.to(_BF16).contiguous(memory_format=_CL))
    dx = dw = None
    if ctx.needs_input_grad[0]:
        dx = conv_dgrad(dyq, wq, dys, ws, height, width, stride, padding).to(ctx.x_dtype)
    if ctx.needs_input_grad[1]:
        dw = conv_wgrad(xq, dyq, xs, dys, wq.shape[2], stride, padding, 0,
                        ctx.w_dtype == torch.float32)
        dw = dw.to(ctx.w_dtype)
    return dx, dw, None, None


conv2d_fp8.register_autograd(_conv2d_fp8_backward, setup_context=_conv2d_fp8_setup)


@torch.library.custom_op("dpa_fp8::linear_fp8", mutates_args=(), device_types="cuda")
def linear_fp8(x: torch.Tensor, weight: torch.Tensor
               ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(y [..., N], e4m3 x [M, K], e4m3 w, x scale, w scale) of y = x @ w^T with current
    scaling of bf16(x) and bf16(w)."""
    k = weight.shape[1]
    x2 = x.to(_BF16).reshape(-1, k).contiguous()
    xq, xs = K._quantize_impl(x2, None)
    wq, ws = K._quantize_impl(weight.to(_BF16).contiguous(), None)
    y = K.linear_fp8_prequantized(xq, wq, xs, ws, None)
    return y.reshape(*x.shape[:-1], weight.shape[0]), xq, wq, xs, ws


@linear_fp8.register_fake
def _linear_fp8_fake(x, weight):
    n, k = weight.shape
    m = x.numel() // k
    scalar = x.new_empty((), dtype=torch.float32)
    return (x.new_empty((*x.shape[:-1], n), dtype=_BF16), x.new_empty((m, k), dtype=K.FP8_DTYPE),
            weight.new_empty((n, k), dtype=K.FP8_DTYPE), scalar, scalar.clone())


def _linear_fp8_setup(ctx, inputs, output):
    x, weight = inputs
    _, xq, wq, xs, ws = output
    ctx.save_for_backward(xq, wq, xs, ws)
    ctx.lead = tuple(x.shape[:-1])
    ctx.x_dtype, ctx.w_dtype = x.dtype, weight.dtype


def _linear_fp8_backward(ctx, dy, *_unused):
    xq, wq, xs, ws = ctx.saved_tensors
    n, k = wq.shape
    dyq, dys = quantize(dy.to(_BF16).reshape(-1, n).contiguous())
    dx = dw = None
    if ctx.needs_input_grad[0]:
        dx = gemm_dgrad(dyq, wq, dys, ws).reshape(*ctx.lead, k).to(ctx.x_dtype)
    if ctx.needs_input_grad[1]:
        dw = gemm_wgrad(xq, dyq, xs, dys, ctx.w_dtype == torch.float32).to(ctx.w_dtype)
    return dx, dw


linear_fp8.register_autograd(_linear_fp8_backward, setup_context=_linear_fp8_setup)
