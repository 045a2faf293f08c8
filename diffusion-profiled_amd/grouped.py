"""FP8 linear layers that share one input, run as one group: the FiLM projections of the
U-Net's residual blocks (diffusion/unet.py:101-104 TimeEmbed at :135 -- every block projects
the same time embedding to its FiLM (w, b)). Per layer the arithmetic is the per-layer FP8
recipe of ``LinearFP8Prepared`` with the layer's own per-tensor scales; one HIP launch per
direction covers every layer (the input's and the gradients' quantization, the forward, the
weight gradients and the summed input gradient), instead of four per layer. The input
gradient sums the layers in fp32 before its one bf16 rounding (per-layer gradients are
rounded to bf16 each and summed by autograd in bf16)."""
from __future__ import annotations

import ctypes
from typing import Any

import torch
from torch.amp.autocast_mode import custom_bwd, custom_fwd

from . import _lib
from .fp8_kernels import FP8_DTYPE

MAX_LAYERS = 32


def _stream(t: torch.Tensor) -> int:
    return _lib.current_stream(t)


def supported(m: int, k: int, ns) -> bool:
    """Shapes the grouped kernels implement: M (rows of x) % 128, K % 128, every n_i % 128."""
    return (0 < len(ns) <= MAX_LAYERS and m > 0 and m % 128 == 0 and k > 0 and k % 128 == 0
            and all(n > 0 and n % 128 == 0 for n in ns))


def _ptrs(ts) -> ctypes.Array:
    return (ctypes.c_void_p * len(ts))(*[t.data_ptr() for t in ts])


def _ints(vals) -> ctypes.Array:
    return (ctypes.c_int * len(vals))(*vals)


def grouped_quantize(srcs, want_q: bool = True, want_qt: bool = True):
    """Per-tensor current-scaling e4m3 of each bf16 [R, n_i] in srcs, concatenated along the
    columns: (q [R, sum n_i] or None, q^T [sum n_i, R] or None, scales fp32 [len(srcs)])."""
    r = srcs[0].shape[0]
    ns = [s.shape[1] for s in srcs]
    dev = srcs[0].device
    tot = sum(ns)
    q = torch.empty((r, tot), device=dev, dtype=FP8_DTYPE) if want_q else None
    qt = torch.empty((tot, r), device=dev, dtype=FP8_DTYPE) if want_qt else None
    scales = torch.empty(len(srcs), device=dev, dtype=torch.float32)
    src_arr, n_arr = _ptrs(srcs), _ints(ns)
    _lib.call("dpa_grouped_quantize_fp8_bf16", ctypes.addressof(src_arr), ctypes.addressof(n_arr),
              len(srcs), r, None if q is None else q.data_ptr(),
              None if qt is None else qt.data_ptr(), scales.data_ptr(), _stream(srcs[0]))
    return q, qt, scales


class GroupedLinearFP8(torch.autograd.Function):
    """y_i = x @ w_i^T for the layers of ``layers`` (prepared e4m3 weights: per layer
    (w_q [n_i, K], w_q^T [K, n_i], w_scale [1])); ``weights`` are the layers' fp32 parameters,
    which receive the gradients. x: [M, K] (any float dtype; used as bf16)."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx: Any, x: torch.Tensor, layers: tuple, *weights: torch.Tensor):
        x2 = x.to(torch.bfloat16).contiguous()
        m, k = x2.shape
        ns = [wq.shape[0] for wq, _, _ in layers]
        xq, xqt, xs = grouped_quantize([x2])
        ys = [torch.empty((m, n), device=x.device, dtype=torch.bfloat16) for n in ns]
        w_arr = _ptrs([wq for wq, _, _ in layers])
        s_arr = _ptrs([ws for _, _, ws in layers])
        y_arr, n_arr = _ptrs(ys), _ints(ns)
        _lib.call("dpa_grouped_linear_fwd_fp8", xq.data_ptr(), xs.data_ptr(),
                  ctypes.addressof(w_arr), ctypes.addressof(s_arr), ctypes.addressof(y_arr),
                  ctypes.addressof(n_arr), len(ns), m, k, _stream(x2))
        ctx.layers = layers
        ctx.x_dtype = x.dtype
        ctx.save_for_backward(xqt, xs)
        return tuple(ys)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx: Any, *dys: torch.Tensor):
        xqt, xs = ctx.saved_tensors
        layers = ctx.layers
        k, m = xqt.shape
        ns = [wq.shape[0] for wq, _, _ in layers]
        dev = xqt.device
        d16 = [torch.zeros((m, n), device=dev, dtype=torch.bfloat16) if d is None
               else d.to(torch.bfloat16).reshape(m, n).contiguous() for d, n in zip(dys, ns)]
        dyq, dyqt, dys_scale = grouped_quantize(d16)
        n_arr = _ints(ns)
        # input gradient: one partial per layer, summed in layer order
        dx = torch.empty((m, k), device=dev, dtype=torch.bfloat16)
        ws_bytes = _lib.query("dpa_grouped_linear_dgrad_workspace_bytes", len(ns), m, k)
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
        wt_arr = _ptrs([wt for _, wt, _ in layers])
        s_arr = _ptrs([w_s for _, _, w_s in layers])
        _lib.call("dpa_grouped_linear_dgrad_fp8", dyq.data_ptr(), dys_scale.data_ptr(),
                  ctypes.addressof(wt_arr), ctypes.addressof(s_arr), dx.data_ptr(),
                  ctypes.addressof(n_arr), len(ns), m, k, ws.data_ptr(), ws_bytes, _stream(dx))
        # weight gradients: fp32 tensors holding the bf16 values (the fp32 master weights')
        dws = [torch.empty((n, k), device=dev, dtype=torch.float32) for n in ns]
        dw_arr = _ptrs(dws)
        _lib.call("dpa_grouped_linear_wgrad_fp8_f32", xqt.data_ptr(), xs.data_ptr(),
                  dyqt.data_ptr(), dys_scale.data_ptr(), ctypes.addressof(dw_arr),
                  ctypes.addressof(n_arr), len(ns), m, k, _stream(dx))
        return (dx.to(ctx.x_dtype), None, *dws)


def grouped_linear_fp8(x: torch.Tensor, layers, weights):
    return GroupedLinearFP8.apply(x, tuple(layers), *weights)
