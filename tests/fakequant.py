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


# ---------------------------------------------------------------------------------------
# GPU emulation of a whole model's recipe, current and delayed scaling, for training runs
# ---------------------------------------------------------------------------------------
def _div32(a: torch.Tensor, b) -> torch.Tensor:
    """RN32(a / b), the IEEE fp32 quotient. Formed in fp64 and rounded once to fp32 (exact:
    53 >= 2 * 24 + 2 bits makes the double rounding harmless): torch's fp32 division on these
    GPUs is not correctly rounded, which moves exact e4m3 ties (x / scale landing on a
    rounding midpoint, common when the scale has few significant bits)."""
    return (a.double() / (b.double() if torch.is_tensor(b) else b)).float()


def _scale_of(v: torch.Tensor) -> torch.Tensor:
    """RN32(amax / 448), or 1 when amax == 0 (diffusion/fp8_kernels.py:90-102); v fp32."""
    amax = v.abs().max()
    return torch.where(amax > 0, _div32(amax, 448.0), torch.ones_like(amax))


def _cast(v: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """e4m3 values (as fp32) of clamp(v / s, +-448) with the reference's min-then-max order
    (diffusion/fp8_kernels.py:84-85, :118-119): a NaN quotient (0 / 0 under an empty history)
    becomes +448, as Triton's minimum/maximum return the non-NaN operand, and +-inf clamps
    to +-448 (written as nan_to_num then clamp: no host constants, so it can be captured)."""
    r = torch.nan_to_num(_div32(v, s), nan=448.0).clamp(-448.0, 448.0)
    return r.to(FP8).float()


def _epi(acc: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor) -> torch.Tensor:
    return (acc.float() * (sa * sb)).to(torch.bfloat16)


def _fp32():
    """The model runs under autocast; the emulated products must not: they accumulate in
    fp32 (as the reference's kernels do) before the scale and the bf16 rounding."""
    return torch.autocast("cuda", enabled=False)


def _cols(x64: torch.Tensor, k: int, stride: int, pad: int) -> torch.Tensor:
    """im2col of an fp64 NCHW tensor as a 2-D [C*k*k, N*L] matrix (a copy)."""
    n, c = x64.shape[:2]
    cols = F.unfold(x64, k, padding=pad, stride=stride)            # [N, C*k*k, L]
    return cols.permute(1, 0, 2).reshape(c * k * k, -1)


def _conv_fwd64(xq, wq, stride: int, pad: int) -> torch.Tensor:
    """Exact convolution of e4m3 values: unfold + one fp64 GEMM (every product is a multiple
    of 2^-18 below 2^18 and the sums stay far inside 53 bits, so no rounding occurs)."""
    n, _, h, w = xq.shape
    o, _, k, _ = wq.shape
    p_, q_ = (h + 2 * pad - k) // stride + 1, (w + 2 * pad - k) // stride + 1
    y = wq.double().reshape(o, -1) @ _cols(xq.double(), k, stride, pad)   # [O, N*L]
    return y.reshape(o, n, p_, q_).permute(1, 0, 2, 3)


def _conv_dgrad64(dyq, wq, xshape, stride: int, pad: int) -> torch.Tensor:
    n, c, h, w = xshape
    o, _, k, _ = wq.shape
    dyc = dyq.double().permute(1, 0, 2, 3).reshape(o, -1)                 # [O, N*L]
    dcols = wq.double().reshape(o, -1).t().contiguous() @ dyc              # [C*k*k, N*L]
    dcols = dcols.reshape(c * k * k, n, -1).permute(1, 0, 2).contiguous()
    return F.fold(dcols, (h, w), k, padding=pad, stride=stride)


def _conv_wgrad64(xq, dyq, wshape, stride: int, pad: int) -> torch.Tensor:
    o, c, k, _ = wshape
    dyc = dyq.double().permute(1, 0, 2, 3).reshape(o, -1)                 # [O, N*L]
    cols = _cols(xq.double(), k, stride, pad)                             # [C*k*k, N*L]
    return (dyc @ cols.t().contiguous()).reshape(o, c, k, k)


class GpuFakeQuantConv(torch.autograd.Function):
    """Current scaling on the GPU: bf16 operands, e4m3 casts by torch, fp32 convolution of
    the e4m3 values, the reference's epilogue. x may be fp32 or bf16 (cast to bf16 first,
    diffusion/fp8_kernels.py:835-836)."""

    @staticmethod
    def forward(ctx, x, w, stride: int, pad: int):
        xb = x.detach().to(torch.bfloat16).float()
        wb = w.detach().to(torch.bfloat16).float()
        xs, ws = _scale_of(xb), _scale_of(wb)
        xq, wq = _cast(xb, xs), _cast(wb, ws)
        ctx.save_for_backward(xq, wq, xs, ws)
        ctx.cfg = (stride, pad)
        with _fp32():
            y = _epi(_conv_fwd64(xq, wq, stride, pad), xs, ws)
        return y.contiguous(memory_format=torch.channels_last)

    @staticmethod
    def backward(ctx, dy):
        xq, wq, xs, ws = ctx.saved_tensors
        stride, pad = ctx.cfg
        db = dy.to(torch.bfloat16).float()
        dys = _scale_of(db)
        dyq = _cast(db, dys)
        dx = _epi(_conv_dgrad64(dyq, wq, xq.shape, stride, pad), dys, ws)
        dw = _epi(_conv_wgrad64(xq, dyq, wq.shape, stride, pad), xs, dys)
        return (dx.contiguous(memory_format=torch.channels_last),
                dw.contiguous(memory_format=torch.channels_last), None, None)


class GpuFakeQuantConvDelayed(torch.autograd.Function):
    """Delayed scaling of one Conv2dFP8 (diffusion/unet.py:69-91 and
    diffusion/fp8_kernels.py:845-889) written with torch ops on the module's own buffers:
    x and w are cast with the maxima of their windows, dy with the maximum of its window read
    at forward time; the current x / w scales go to slot window_pos, which then advances; the
    backward writes the current dy scale at the advanced position."""

    @staticmethod
    def forward(ctx, x, w, mod):
        with torch.no_grad():
            xs_h = mod.amax_window_acts.max()
            ws_h = mod.amax_window_weights.max()
            dys_h = mod.amax_window_dy.max()
            xb = x.detach().to(torch.bfloat16).float()
            wb = w.detach().to(torch.bfloat16).float()
            xq, wq = _cast(xb, xs_h), _cast(wb, ws_h)
            idx = mod.window_pos.unsqueeze(0)
            mod.amax_window_weights.scatter_(0, idx, _scale_of(wb).unsqueeze(0))
            mod.amax_window_acts.scatter_(0, idx, _scale_of(xb).unsqueeze(0))
            mod.window_pos.add_(1).remainder_(mod.amax_history)
        ctx.save_for_backward(xq, wq, xs_h, ws_h, dys_h)
        ctx.mod = mod
        with _fp32():
            y = _epi(_conv_fwd64(xq, wq, 1, 1), xs_h, ws_h)
        return y.contiguous(memory_format=torch.channels_last)

    @staticmethod
    def backward(ctx, dy):
        xq, wq, xs_h, ws_h, dys_h = ctx.saved_tensors
        mod = ctx.mod
        db = dy.to(torch.bfloat16).float()
        with torch.no_grad():
            dyq = _cast(db, dys_h)
            mod.amax_window_dy.scatter_(0, mod.window_pos.unsqueeze(0), _scale_of(db).unsqueeze(0))
        dx = _epi(_conv_dgrad64(dyq, wq, xq.shape, 1, 1), dys_h, ws_h)
        dw = _epi(_conv_wgrad64(xq, dyq, wq.shape, 1, 1), xs_h, dys_h)
        return (dx.contiguous(memory_format=torch.channels_last),
                dw.contiguous(memory_format=torch.channels_last), None)


class GpuFakeQuantLinear(torch.autograd.Function):
    """Current-scaling FP8 linear on the GPU (the recipe applied to nn.Linear)."""

    @staticmethod
    def forward(ctx, x, w):
        lead = x.shape[:-1]
        xb = x.detach().reshape(-1, x.shape[-1]).to(torch.bfloat16).float()
        wb = w.detach().to(torch.bfloat16).float()
        xs, ws = _scale_of(xb), _scale_of(wb)
        xq, wq = _cast(xb, xs), _cast(wb, ws)
        ctx.save_for_backward(xq, wq, xs, ws)
        ctx.lead = lead
        with _fp32():
            return _epi(xq.double() @ wq.double().t().contiguous(), xs, ws).reshape(*lead, w.shape[0])

    @staticmethod
    def backward(ctx, dy):
        xq, wq, xs, ws = ctx.saved_tensors
        db = dy.reshape(-1, wq.shape[0]).to(torch.bfloat16).float()
        dys = _scale_of(db)
        dyq = _cast(db, dys)
        dx = _epi(dyq.double() @ wq.double(), dys, ws).reshape(*ctx.lead, wq.shape[1])
        dw = _epi(dyq.double().t().contiguous() @ xq.double(), xs, dys)
        return dx, dw


def _gpu_conv3x3(self, x):
    if self.conv_fp8(x, self.conv.weight):
        if self.scaling_type == "delayed":
            return GpuFakeQuantConvDelayed.apply(x, self.conv.weight, self)
        return GpuFakeQuantConv.apply(x, self.conv.weight, 1, 1)
    if self.conv_fp8_general(x, self.conv.weight):
        return GpuFakeQuantConv.apply(x, self.conv.weight, 1, 1)
    return self.conv(x)


def _gpu_conv1x1(self, x):
    if self.fp8 and self.in_channels % 128 == 0 and self.out_channels % 128 == 0:
        return GpuFakeQuantConv.apply(x, self.weight, 1, 0)
    return torch.nn.Conv2d.forward(self, x)


def _gpu_linear(self, x):
    if self.fp8 and self.in_features % 128 == 0 and self.out_features % 128 == 0:
        assert self.bias is None
        return GpuFakeQuantLinear.apply(x, self.weight)
    return torch.nn.Linear.forward(self, x)


def emulate_on_gpu(model: torch.nn.Module) -> torch.nn.Module:
    """Turn ``model`` (in place, on the GPU) into the torch emulation of its FP8 recipe: every
    FP8 site runs the fake-quant autograd functions above (the registry 3x3 convs with the
    module's own scaling type and windows, every other FP8 conv and linear with current
    scaling, as the HIP model does), GroupNorm+SiLU run as torch float32 ops and no grouped
    weight preparation is used. Products of e4m3 values are exact (fp64 GEMMs over im2col
    matrices), as in the CPU oracle, so the result does not depend on a library's choice of
    convolution algorithm."""
    model.weight_prep_enabled = False
    for m in model.modules():
        if isinstance(m, U.Conv2dFP8):
            m.forward = types.MethodType(_gpu_conv3x3, m)
        elif isinstance(m, U.Conv1x1FP8):
            m.forward = types.MethodType(_gpu_conv1x1, m)
        elif isinstance(m, U.LinearFP8):
            m.forward = types.MethodType(_gpu_linear, m)
        if hasattr(m, "fused"):
            m.fused = False
    return model
