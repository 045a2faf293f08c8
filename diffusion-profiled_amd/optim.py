"""The training step's optimizer tail as one fused pass (the HIP library's dpa_adamw_ema_step).

The reference step (train.py:104-149) ends with ``clip_grad_norm_(params, max_norm)``,
``AdamW(fused=True, capturable=True).step()`` (train.py:253) and the EMA update of
``EWMAWrapper`` (diffusion/ddpm.py:10-30). ``FusedAdamWEMA`` does all three: a gradient-norm
pass, a one-block finalize (clip coefficient, step count, bias corrections) and one update
pass that applies the clipped AdamW update and the EMA of every parameter and float buffer;
integer buffers of the EMA copy are copied as ``EWMAWrapper.update`` does.
"""
from __future__ import annotations

import ctypes
from ctypes import c_int64, c_void_p

import torch

from . import _lib


class DpaOptTensor(ctypes.Structure):
    """include/dpa_fp8.h ``DpaOptTensor``."""

    _fields_ = [("param", c_void_p), ("grad", c_void_p), ("exp_avg", c_void_p),
                ("exp_avg_sq", c_void_p), ("ema", c_void_p), ("n", c_int64)]


class FusedAdamWEMA:
    """AdamW (decoupled weight decay, torch defaults) with gradient-norm clipping and the EMA of
    ``ema_model`` folded in. ``fuses_clip_and_ema`` tells the training step not to run
    ``clip_grad_norm_`` and the EMA update itself."""

    fuses_clip_and_ema = True

    def __init__(self, model: torch.nn.Module, ema_model: torch.nn.Module | None, lr: float,
                 betas=(0.9, 0.999), eps: float = 1e-8, weight_decay: float = 1e-2,
                 max_norm: float = 1.0, ema_beta: float = 0.9999):
        self.lr, self.betas, self.eps, self.wd = float(lr), betas, float(eps), float(weight_decay)
        self.max_norm, self.ema_beta = float(max_norm), float(ema_beta)
        named = dict(model.named_parameters())
        self.params = list(named.values())
        dev = self.params[0].device
        for p in self.params:
            dense = (p.is_contiguous(memory_format=torch.channels_last) if p.ndim == 4
                     else p.is_contiguous())
            assert p.dtype == torch.float32 and dense, "fp32 dense parameters"
        self.exp_avg = [torch.zeros_like(p) for p in self.params]
        self.exp_avg_sq = [torch.zeros_like(p) for p in self.params]
        self.step_t = torch.zeros((), device=dev, dtype=torch.float32)
        self.ema_params = [None] * len(self.params)
        self.ema_float_buffers: list[tuple[torch.Tensor, torch.Tensor]] = []
        self.ema_int_buffers: list[tuple[torch.Tensor, torch.Tensor]] = []
        if ema_model is not None:
            ema_named = dict(ema_model.named_parameters())
            self.ema_params = [ema_named[k] for k in named]
            src_buf = dict(model.named_buffers())
            for k, eb in ema_model.named_buffers():
                if k not in src_buf or k not in ema_model.state_dict():
                    continue
                (self.ema_float_buffers if eb.is_floating_point() else self.ema_int_buffers).append(
                    (eb, src_buf[k]))
        self._ws = None

    def zero_grad(self, set_to_none: bool = True) -> None:
        for p in self.params:
            if set_to_none:
                p.grad = None
            elif p.grad is not None:
                p.grad.zero_()

    def _table(self):
        entries = []
        for p, m, v, e in zip(self.params, self.exp_avg, self.exp_avg_sq, self.ema_params):
            g = p.grad
            if g is not None:
                assert g.dtype == torch.float32, "fp32 gradients"
                if g.stride() != p.stride():
                    # the kernels walk gradient and parameter as one flat range each: give the
                    # gradient the parameter's layout (torch's AdamW accepts any strides)
                    g = torch.empty_like(p).copy_(g)
                    p.grad = g
                entries.append((p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(),
                                None if e is None else e.data_ptr(), p.numel()))
            elif e is not None:
                entries.append((p.data_ptr(), None, None, None, e.data_ptr(), p.numel()))
        for eb, sb in self.ema_float_buffers:
            if eb.dtype == torch.float32 and sb.dtype == torch.float32 and eb.is_contiguous() \
                    and sb.is_contiguous():
                entries.append((sb.data_ptr(), None, None, None, eb.data_ptr(), sb.numel()))
        arr = (DpaOptTensor * len(entries))()
        for a, (p, g, m, v, e, n) in zip(arr, entries):
            a.param, a.grad, a.exp_avg, a.exp_avg_sq, a.ema, a.n = p, g, m, v, e, n
        return arr, len(entries)

    @torch.no_grad()
    def step(self) -> None:
        arr, count = self._table()
        addr = ctypes.addressof(arr)
        ws_bytes = _lib.load().dpa_adamw_ema_workspace_bytes(addr, count)
        if self._ws is None or self._ws.numel() < ws_bytes:
            self._ws = torch.empty(ws_bytes, device=self.step_t.device, dtype=torch.uint8)
        stream = _lib.current_stream(self.step_t)
        _lib.check(_lib.load().dpa_adamw_ema_step(
            addr, count, self.step_t.data_ptr(), self.lr, self.betas[0], self.betas[1], self.eps,
            self.wd, self.max_norm, self.ema_beta, self._ws.data_ptr(), ws_bytes, stream),
            "dpa_adamw_ema_step")
        if self.ema_int_buffers:
            torch._foreach_copy_([e for e, _ in self.ema_int_buffers],
                                 [s for _, s in self.ema_int_buffers])
