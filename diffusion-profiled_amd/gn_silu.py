"""Fused GroupNorm(+FiLM)+SiLU on the HIP library, as an autograd Function.

Replaces the two Inductor-fused chains of the reference ResidualBlock
(diffusion/unet.py:151 ``F.silu(self.norm1(x))`` and :157-159
``F.silu((w + 1) * self.norm2(x) + b)``). The output is bf16, which is exactly what the FP8
conv consumes after its ``x.to(torch.bfloat16)`` (diffusion/fp8_kernels.py:835). An fp32 input
(the residual stream below the first level and the decoder's concatenations are fp32 under
autocast, as in the reference) is normalised as it is, as autocast's fp32 GroupNorm does, and
its gradient is returned in fp32 by the kernels, for images of up to 8192 pixels (the
resident form up to 1024 pixels, the chunked form above); other inputs are cast to bf16 first.
"""
from __future__ import annotations

from typing import Any

import torch

from . import _lib
from . import fp8_kernels as _fp8
from .fp8_kernels import FP8_DTYPE, Fp8Handoff, placeholder


def _stream(t: torch.Tensor) -> int:
    return _lib.current_stream(t)


DTYPE_BF16, DTYPE_F32 = 0, 1  # include/dpa_fp8.h DPA_DTYPE_*


def f32_input_ok(x: torch.Tensor) -> bool:
    """fp32 x that the kernels read directly: resident (<= 1024 pixels) or chunked form
    (<= 8192 pixels)."""
    hw = x.shape[2] * x.shape[3]
    return x.dtype == torch.float32 and hw <= 64 * 128


def _prep_x(x: torch.Tensor) -> tuple[torch.Tensor, int]:
    """x as the kernels read it (channels-last) and its DTYPE_*."""
    if f32_input_ok(x):
        return x.contiguous(memory_format=torch.channels_last), DTYPE_F32
    return x.to(torch.bfloat16).contiguous(memory_format=torch.channels_last), DTYPE_BF16


def supported(c: int, groups: int) -> bool:
    """Shapes the fused kernel implements (all GroupNorms of the reference U-Net)."""
    if c % groups != 0 or c % 64 != 0:
        return False
    cpg = c // groups
    return cpg >= 4 and 64 % cpg == 0


def gn_silu_fwd(x, gamma, beta, groups, eps, film_scale=None, film_shift=None, x_bf16=None):
    """Returns (out bf16 channels-last, mean [N*G], rstd [N*G]); with x_bf16 (fp32 x) the
    kernel also writes bf16(x) there."""
    n, c, h, w = x.shape
    x, _ = _prep_x(x)
    out = torch.empty_like(x, dtype=torch.bfloat16, memory_format=torch.channels_last)
    mean = torch.empty(n * groups, device=x.device, dtype=torch.float32)
    rstd = torch.empty(n * groups, device=x.device, dtype=torch.float32)
    gamma = gamma.float().contiguous()
    beta = beta.float().contiguous()
    fs = fb = None
    if film_scale is not None:
        fs = film_scale.float().reshape(n, c).contiguous()
        fb = film_shift.float().reshape(n, c).contiguous()
    _fwd_call(x, gamma, beta, fs, fb, None, out, mean, rstd, groups, eps, x_bf16=x_bf16)
    return out, mean, rstd


def dropout_ok(x: torch.Tensor) -> bool:
    """Images whose GroupNorm+SiLU kernels also apply dropout (the resident and chunked forms,
    up to 8192 pixels)."""
    hw = x.shape[2] * x.shape[3]
    return hw <= 64 * 128


def new_dropout_seed(device) -> torch.Tensor:
    """A fresh dropout seed in device memory, drawn from torch's generator (so it follows
    torch.manual_seed and is redrawn on each replay of a captured graph)."""
    return torch.randint(0, 2**62, (1,), device=device, dtype=torch.int64)


class DropoutSeeds:
    """Seeds for the dropout layers of one forward pass, drawn by one randint launch (instead of
    one per layer): the model fills it before its forward and clears it after; each fused
    dropout takes the next seed, or draws its own when none is left."""

    def __init__(self):
        self.seeds: torch.Tensor | None = None
        self.next = 0

    def fill(self, device, count: int) -> None:
        self.seeds = torch.randint(0, 2**62, (count,), device=device, dtype=torch.int64)
        self.next = 0

    def clear(self) -> None:
        self.seeds, self.next = None, 0

    def take(self, device) -> torch.Tensor:
        s = self.seeds
        if s is not None and self.next < s.numel() and s.device == torch.device(device):
            self.next += 1
            return s[self.next - 1:self.next]
        return new_dropout_seed(device)


DROPOUT_SEEDS = DropoutSeeds()


def _xb_partials(x_bf16, groups):
    """Room for the amax partials of the bf16 copy of x (one per workgroup of the launch that
    writes it), or None when that copy is not written or no form records them."""
    if x_bf16 is None or not _fp8.PRODUCER_AMAX:
        return None
    n, c, h, w = x_bf16.shape
    count = _lib.query("dpa_gn_silu_fp8_partials", n, h * w, c, groups)
    if count <= 0:
        return None
    return torch.empty(count, device=x_bf16.device, dtype=torch.int32)


def _fwd_call(x, gamma, beta, fs, fb, wb, out, mean, rstd, groups, eps, seed=None, p_drop=0.0,
              x_bf16=None):
    """The workspace form of the forward (chunked for images of 1025+ pixels); x bf16 or fp32;
    seed: dropout seed tensor (int64 [1]) or None. A bf16 copy x_bf16 of an fp32 x carries the
    amax partials its writer left (for the current-scaling 1x1 skip conv that reads it)."""
    n, c, h, w = x.shape
    ws_bytes = _lib.query("dpa_gn_silu_fwd_workspace_bytes", n, h * w, c, groups)
    ws = torch.empty(ws_bytes, device=x.device, dtype=torch.uint8) if ws_bytes else None
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    dt = DTYPE_F32 if x.dtype == torch.float32 else DTYPE_BF16
    xbp = _xb_partials(x_bf16, groups)
    args = (x.data_ptr(), dt, gamma.data_ptr(), beta.data_ptr(), p(fs), p(fb), p(wb),
            out.data_ptr(), mean.data_ptr(), rstd.data_ptr(), p(ws), ws_bytes, n, h * w, c,
            groups, float(eps), p(seed), float(p_drop), p(x_bf16))
    if xbp is None:
        _lib.call("dpa_gn_silu_fwd_ex", *args, _stream(x))
    else:
        _lib.call("dpa_gn_silu_fwd_ex_amax", *args, xbp.data_ptr(), xbp.numel(), _stream(x))
        _fp8.mark_amax_partials(x_bf16, xbp, xbp.numel())


def fp8_ok(shape, groups: int, hand: Fp8Handoff) -> bool:
    """Whether the kernels can write this GroupNorm's output (or bf16 dx) as the e4m3 operand
    of a delayed-scaling conv: a form with the fused cast for the image size, and room for its
    amax partials in the conv's buffer."""
    n, c, h, w = shape
    need = _lib.query("dpa_gn_silu_fp8_partials", n, h * w, c, groups)
    return 0 < need <= hand.partials.numel()


def _fwd_fp8_call(x, gamma, beta, wb, hand: Fp8Handoff, mean, rstd, groups, eps, seed=None,
                  p_drop=0.0, x_bf16=None) -> None:
    """The forward writing e4m3(out / hand.scale) to hand.q (no bf16 output) and its amax
    partials to the hand-off's buffers."""
    n, c, h, w = x.shape
    q = torch.empty_like(x, dtype=FP8_DTYPE, memory_format=torch.channels_last)
    ws_bytes = _lib.query("dpa_gn_silu_fwd_workspace_bytes", n, h * w, c, groups)
    ws = torch.empty(ws_bytes, device=x.device, dtype=torch.uint8) if ws_bytes else None
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    dt = DTYPE_F32 if x.dtype == torch.float32 else DTYPE_BF16
    xbp = _xb_partials(x_bf16, groups)
    args = (x.data_ptr(), dt, gamma.data_ptr(), beta.data_ptr(), None, None, p(wb), q.data_ptr(),
            hand.scale.data_ptr(), hand.partials.data_ptr(), hand.partials.numel(),
            hand.count.data_ptr(), mean.data_ptr(), rstd.data_ptr(), p(ws), ws_bytes, n, h * w,
            c, groups, float(eps), p(seed), float(p_drop), p(x_bf16))
    if xbp is None:
        _lib.call("dpa_gn_silu_fwd_fp8", *args, _stream(x))
    else:
        _lib.call("dpa_gn_silu_fwd_fp8_amax", *args, xbp.data_ptr(), xbp.numel(), _stream(x))
        _fp8.mark_amax_partials(x_bf16, xbp, xbp.numel())
    hand.q = q


def gn_silu_bwd(x, dout, gamma, beta, mean, rstd, groups, film_scale=None, film_shift=None,
                dx_add=None):
    """Returns (dx in x's dtype (bf16 or fp32), dgamma, dbeta, dfilm_scale [N,C] | None,
    dfilm_shift | None); dx_add (x's dtype, channels-last) is added to dx by the kernel."""
    n, c, h, w = x.shape
    x = x.contiguous(memory_format=torch.channels_last)
    dout = dout.to(torch.bfloat16).contiguous(memory_format=torch.channels_last)
    dx = torch.empty_like(x, memory_format=torch.channels_last)
    dgamma = torch.empty(c, device=x.device, dtype=torch.float32)
    dbeta = torch.empty(c, device=x.device, dtype=torch.float32)
    fs = fb = dfs = dfb = None
    if film_scale is not None:
        fs = film_scale.float().reshape(n, c).contiguous()
        fb = film_shift.float().reshape(n, c).contiguous()
        dfs = torch.empty((n, c), device=x.device, dtype=torch.float32)
        dfb = torch.empty((n, c), device=x.device, dtype=torch.float32)
    ws_bytes = _lib.query("dpa_gn_silu_bwd_workspace_bytes", n, h * w, c, groups)
    ws = torch.empty(ws_bytes, device=x.device, dtype=torch.uint8)
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    dt = DTYPE_F32 if x.dtype == torch.float32 else DTYPE_BF16
    _lib.call(
        "dpa_gn_silu_bwd_ex",
        x.data_ptr(), dt, dout.data_ptr(), gamma.float().contiguous().data_ptr(),
        beta.float().contiguous().data_ptr(), p(fs), p(fb), None, mean.data_ptr(),
        rstd.data_ptr(), dx.data_ptr(), p(dx_add),
        DTYPE_BF16 if dx_add is not None and dx_add.dtype == torch.bfloat16 else DTYPE_F32,
        dgamma.data_ptr(), dbeta.data_ptr(), p(dfs),
        p(dfb), None, ws.data_ptr(), ws_bytes, n, h * w, c, groups, None, 0.0, _stream(x),
    )
    return dx, dgamma, dbeta, dfs, dfb


class GroupNormSiLU(torch.autograd.Function):
    """silu(GroupNorm(x)) or silu(film_scale * GroupNorm(x) + film_shift), bf16 out.

    x: bf16 or fp32 [N, C, H, W] (any memory format; used channels-last). gamma/beta: fp32 [C].
    film_scale/film_shift: [N, C, 1, 1] or None (the reference's ``w + 1`` and ``b``)."""

    @staticmethod
    def forward(ctx: Any, x, gamma, beta, groups: int, eps: float, film_scale=None, film_shift=None):
        xb, _ = _prep_x(x)
        out, mean, rstd = gn_silu_fwd(xb, gamma, beta, groups, eps, film_scale, film_shift)
        ctx.groups = groups
        ctx.has_film = film_scale is not None
        ctx.x_dtype = x.dtype
        ctx.film_dtypes = (film_scale.dtype, film_shift.dtype) if ctx.has_film else None
        ctx.save_for_backward(xb, gamma, beta, mean, rstd, film_scale, film_shift)
        return out

    @staticmethod
    def backward(ctx: Any, dout):
        xb, gamma, beta, mean, rstd, fs, fb = ctx.saved_tensors
        dx, dgamma, dbeta, dfs, dfb = gn_silu_bwd(xb, dout, gamma, beta, mean, rstd, ctx.groups, fs, fb)
        n, c = xb.shape[0], xb.shape[1]
        gfs = gfb = None
        if ctx.has_film:
            gfs = dfs.reshape(fs.shape).to(ctx.film_dtypes[0])
            gfb = dfb.reshape(fb.shape).to(ctx.film_dtypes[1])
        return dx.to(ctx.x_dtype), dgamma.to(gamma.dtype), dbeta.to(beta.dtype), None, None, gfs, gfb


class GroupNormSiLUTee(torch.autograd.Function):
    """(silu(GroupNorm(x)), x): the residual block's first norm and its skip input
    (diffusion/unet.py:149-151). The backward adds the skip path's gradient of x into dx inside
    the GroupNorm kernel instead of autograd's separate accumulation kernel (same sum, same
    roundings). With skip_bf16 and an fp32 x the second output is x.to(bfloat16), written by
    the GroupNorm kernel as it reads x (what the 1x1 skip conv rounds its input to), and its
    bf16 gradient is added to the fp32 dx as autograd would (cast, then one fp32 add)."""

    @staticmethod
    def forward(ctx: Any, x, gamma, beta, groups: int, eps: float, skip_bf16: bool = False,
                hand: Fp8Handoff | None = None):
        xb, _ = _prep_x(x)
        x16 = None
        if skip_bf16 and xb.dtype == torch.float32 and dropout_ok(xb):
            x16 = torch.empty_like(xb, dtype=torch.bfloat16, memory_format=torch.channels_last)
        if hand is None:
            out, mean, rstd = gn_silu_fwd(xb, gamma, beta, groups, eps, x_bf16=x16)
        else:
            # the e4m3 conv input goes to hand.q; autograd carries a placeholder for it
            n = xb.shape[0]
            mean = torch.empty(n * groups, device=xb.device, dtype=torch.float32)
            rstd = torch.empty(n * groups, device=xb.device, dtype=torch.float32)
            _fwd_fp8_call(xb, gamma.float().contiguous(), beta.float().contiguous(), None, hand,
                          mean, rstd, groups, eps, x_bf16=x16)
            out = placeholder(xb.shape, torch.bfloat16, xb.device)
        ctx.groups = groups
        ctx.x_dtype = x.dtype
        ctx.save_for_backward(xb, gamma, beta, mean, rstd)
        if x16 is not None:
            return out, x16
        return out, (x.to(torch.bfloat16) if skip_bf16 else x.view_as(x))

    @staticmethod
    def backward(ctx: Any, dout, dskip):
        xb, gamma, beta, mean, rstd = ctx.saved_tensors
        add = None
        if (dskip is not None and xb.dtype == ctx.x_dtype and dropout_ok(xb)
                and (dskip.dtype == xb.dtype
                     or (dskip.dtype == torch.bfloat16 and xb.dtype == torch.float32))):
            add = dskip.contiguous(memory_format=torch.channels_last)
        dx, dgamma, dbeta, _, _ = gn_silu_bwd(xb, dout, gamma, beta, mean, rstd, ctx.groups,
                                              dx_add=add)
        dx = dx.to(ctx.x_dtype)
        if dskip is not None and add is None:
            dx = dx + dskip.to(dx.dtype)
        return dx, dgamma.to(gamma.dtype), dbeta.to(beta.dtype), None, None, None, None


def group_norm_silu_tee(x, gamma, beta, groups: int, eps: float = 1e-5, skip_bf16: bool = False,
                        hand: Fp8Handoff | None = None):
    """With ``hand`` the first output is a placeholder and the e4m3 conv input is ``hand.q``."""
    return GroupNormSiLUTee.apply(x, gamma, beta, groups, eps, skip_bf16, hand)


def upcat_ok(a: torch.Tensor, h: torch.Tensor, up: bool) -> bool:
    """Whether cat([up2(a), h], 1) can feed the fused upsample-and-concatenate GroupNorm
    (dpa_upcat_gn_silu_fwd): channels-last on the GPU, a bf16, 32x32 images with h bf16 or
    16x16 images with h bf16 or fp32, channel counts multiples of 64."""
    cl = torch.channels_last
    if not (up and a.is_cuda and h.is_cuda and a.dtype == torch.bfloat16
            and h.dtype in (torch.bfloat16, torch.float32) and a.ndim == 4 and h.ndim == 4):
        return False
    n, ca, ha, wa = a.shape
    nh, ch, hh, wh = h.shape
    size_ok = (hh == wh == 32 and h.dtype == torch.bfloat16) or hh == wh == 16
    return (n == nh and hh == 2 * ha and wh == 2 * wa and size_ok and ca % 64 == 0
            and ch % 64 == 0 and a.is_contiguous(memory_format=cl)
            and h.is_contiguous(memory_format=cl) and a.data_ptr() % 16 == 0
            and h.data_ptr() % 16 == 0)


_DT_H = {torch.bfloat16: DTYPE_BF16, torch.float32: DTYPE_F32}


class UpcatGroupNormSiLUTee(torch.autograd.Function):
    """GroupNormSiLUTee on x = cat([up2(a), h], 1), the fp32 decoder-stage input of
    diffusion/unet.py:379-382, with skip_bf16: (silu(GroupNorm(x)), x.to(bfloat16)). The
    kernels read a and h where x would be read, so the fp32 concatenation is never
    formed; the backward returns the gradients of a and h that the upsample-and-concatenate's
    backward would form from the GroupNorm's fp32 dx plus the bf16 skip-path gradient. Every
    output and gradient is bit-identical to upsample_concat followed by GroupNormSiLUTee."""

    @staticmethod
    def forward(ctx: Any, a, h, gamma, beta, groups: int, eps: float,
                hand: Fp8Handoff | None = None):
        n, ca, _, _ = a.shape
        _, ch, hh, wh = h.shape
        c = ca + ch
        cl = torch.channels_last
        x16 = torch.empty((n, c, hh, wh), device=a.device, dtype=torch.bfloat16, memory_format=cl)
        xbp = _xb_partials(x16, groups)
        mean = torch.empty(n * groups, device=a.device, dtype=torch.float32)
        rstd = torch.empty(n * groups, device=a.device, dtype=torch.float32)
        g32, b32 = gamma.float().contiguous(), beta.float().contiguous()
        p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        if hand is None:
            out = torch.empty((n, c, hh, wh), device=a.device, dtype=torch.bfloat16,
                              memory_format=cl)
            q = None
            qargs = (None, None, 0, None)
        else:
            out = None
            q = torch.empty((n, c, hh, wh), device=a.device, dtype=FP8_DTYPE, memory_format=cl)
            qargs = (hand.scale.data_ptr(), hand.partials.data_ptr(), hand.partials.numel(),
                     hand.count.data_ptr())
        _lib.call("dpa_upcat_gn_silu_fwd", a.data_ptr(), h.data_ptr(), _DT_H[h.dtype], n, hh,
                  wh, ca, ch, g32.data_ptr(), b32.data_ptr(), p(out), p(q), *qargs, mean.data_ptr(),
                  rstd.data_ptr(), x16.data_ptr(), p(xbp), 0 if xbp is None else xbp.numel(),
                  groups, float(eps), _stream(a))
        if xbp is not None:
            _fp8.mark_amax_partials(x16, xbp, xbp.numel())
        if hand is not None:
            hand.q = q
            out = placeholder((n, c, hh, wh), torch.bfloat16, a.device)
        ctx.groups = groups
        ctx.save_for_backward(a, h, gamma, beta, mean, rstd)
        return out, x16

    @staticmethod
    def backward(ctx: Any, dout, dskip):
        a, h, gamma, beta, mean, rstd = ctx.saved_tensors
        n, ca, _, _ = a.shape
        _, ch, hh, wh = h.shape
        c = ca + ch
        cl = torch.channels_last
        dout = dout.to(torch.bfloat16).contiguous(memory_format=cl)
        add = None
        if dskip is not None:
            # the skip input is the bf16 copy, so its gradient is bf16
            add = dskip.to(torch.bfloat16).contiguous(memory_format=cl)
        ga = torch.empty_like(a, memory_format=cl)
        gh = torch.empty_like(h, memory_format=cl)
        dgamma = torch.empty(c, device=a.device, dtype=torch.float32)
        dbeta = torch.empty(c, device=a.device, dtype=torch.float32)
        ws_bytes = 2 * n * c * 4
        ws = torch.empty(ws_bytes, device=a.device, dtype=torch.uint8)
        _lib.call("dpa_upcat_gn_silu_bwd", a.data_ptr(), h.data_ptr(), _DT_H[h.dtype], n, hh,
                  wh, ca, ch, dout.data_ptr(), gamma.float().contiguous().data_ptr(),
                  beta.float().contiguous().data_ptr(), mean.data_ptr(), rstd.data_ptr(),
                  None if add is None else add.data_ptr(), ga.data_ptr(), gh.data_ptr(),
                  dgamma.data_ptr(), dbeta.data_ptr(), ws.data_ptr(), ws_bytes, ctx.groups,
                  _stream(a))
        return ga, gh, dgamma.to(gamma.dtype), dbeta.to(beta.dtype), None, None, None


def upcat_group_norm_silu_tee(a, h, gamma, beta, groups: int, eps: float = 1e-5,
                              hand: Fp8Handoff | None = None):
    """group_norm_silu_tee(upsample_concat(a, h, True), ..., skip_bf16=True) without the fp32
    concatenation (upcat_ok(a, h, True) must hold)."""
    return UpcatGroupNormSiLUTee.apply(a, h, gamma, beta, groups, eps, hand)


class GroupNormSiLUFilm(torch.autograd.Function):
    """silu(bf16(w + 1) * GroupNorm(x) + b) with (w, b) = chunk(film_wb, 2, dim=1), the time
    projection of diffusion/unet.py:157-159, read by the kernel in bf16; the backward returns
    the gradient of film_wb [N, 2C, 1, 1] (bf16) directly. With p_drop > 0 the output also
    takes the dropout of diffusion/unet.py:160 (mask from a counter hash of a seed drawn here;
    the backward recomputes it from the same seed)."""

    @staticmethod
    def forward(ctx: Any, x, gamma, beta, groups: int, eps: float, film_wb, p_drop: float = 0.0,
                hand: Fp8Handoff | None = None, dx_hand: Fp8Handoff | None = None):
        n, c, h, w = x.shape
        xb, _ = _prep_x(x)
        wb = film_wb.contiguous()
        assert wb.dtype == torch.bfloat16 and wb.numel() == n * 2 * c
        mean = torch.empty(n * groups, device=x.device, dtype=torch.float32)
        rstd = torch.empty(n * groups, device=x.device, dtype=torch.float32)
        g32, b32 = gamma.float().contiguous(), beta.float().contiguous()
        seed = DROPOUT_SEEDS.take(x.device) if p_drop > 0.0 else None
        if seed is not None and not dropout_ok(x):
            raise ValueError(f"fused dropout: no kernel form for {h}x{w} images")
        if dx_hand is not None and not (xb.dtype == torch.bfloat16
                                        and fp8_ok(xb.shape, groups, dx_hand)):
            raise ValueError("FP8 hand-off of dx: needs a bf16 x and a fused-cast form")
        if hand is None:
            out = torch.empty_like(xb, dtype=torch.bfloat16, memory_format=torch.channels_last)
            _fwd_call(xb, g32, b32, None, None, wb, out, mean, rstd, groups, eps, seed, p_drop)
        else:
            _fwd_fp8_call(xb, g32, b32, wb, hand, mean, rstd, groups, eps, seed, p_drop)
            out = placeholder(xb.shape, torch.bfloat16, xb.device)
        ctx.groups = groups
        ctx.x_dtype = x.dtype
        ctx.wb_shape = film_wb.shape
        ctx.p_drop = p_drop
        ctx.dx_hand = dx_hand
        ctx.save_for_backward(xb, gamma, beta, mean, rstd, wb, seed)
        return out

    @staticmethod
    def backward(ctx: Any, dout):
        xb, gamma, beta, mean, rstd, wb, seed = ctx.saved_tensors
        n, c, h, w = xb.shape
        dout = dout.to(torch.bfloat16).contiguous(memory_format=torch.channels_last)
        dx = torch.empty_like(xb, memory_format=torch.channels_last)
        dgamma = torch.empty(c, device=xb.device, dtype=torch.float32)
        dbeta = torch.empty(c, device=xb.device, dtype=torch.float32)
        dwb = torch.empty(ctx.wb_shape, device=xb.device, dtype=torch.bfloat16)
        ws_bytes = _lib.query("dpa_gn_silu_bwd_workspace_bytes", n, h * w, c, ctx.groups)
        ws = torch.empty(ws_bytes, device=xb.device, dtype=torch.uint8)
        dt = DTYPE_F32 if xb.dtype == torch.float32 else DTYPE_BF16
        hand = ctx.dx_hand
        if hand is not None:
            # dx is the dy of the delayed-scaling conv that produced x: written as its e4m3
            # operand, autograd gets a placeholder
            dxq = torch.empty_like(xb, dtype=FP8_DTYPE, memory_format=torch.channels_last)
            _lib.call(
                "dpa_gn_silu_bwd_fp8",
                xb.data_ptr(), dout.data_ptr(), gamma.float().contiguous().data_ptr(),
                beta.float().contiguous().data_ptr(), None, None, wb.data_ptr(),
                mean.data_ptr(), rstd.data_ptr(), dxq.data_ptr(), hand.scale.data_ptr(),
                hand.partials.data_ptr(), hand.partials.numel(), hand.count.data_ptr(),
                dgamma.data_ptr(), dbeta.data_ptr(), None, None, dwb.data_ptr(), ws.data_ptr(),
                ws_bytes, n, h * w, c, ctx.groups, None if seed is None else seed.data_ptr(),
                float(ctx.p_drop), _stream(xb),
            )
            hand.q = dxq
            return (placeholder(xb.shape, xb.dtype, xb.device), dgamma.to(gamma.dtype),
                    dbeta.to(beta.dtype), None, None, dwb, None, None, None)
        _lib.call(
            "dpa_gn_silu_bwd_ex",
            xb.data_ptr(), dt, dout.data_ptr(), gamma.float().contiguous().data_ptr(),
            beta.float().contiguous().data_ptr(), None, None, wb.data_ptr(), mean.data_ptr(),
            rstd.data_ptr(), dx.data_ptr(), None, DTYPE_BF16, dgamma.data_ptr(),
            dbeta.data_ptr(), None, None,
            dwb.data_ptr(), ws.data_ptr(), ws_bytes, n, h * w, c, ctx.groups,
            None if seed is None else seed.data_ptr(), float(ctx.p_drop), _stream(xb),
        )
        return (dx.to(ctx.x_dtype), dgamma.to(gamma.dtype), dbeta.to(beta.dtype), None, None, dwb,
                None, None, None)


def group_norm_silu_film(x, gamma, beta, groups: int, eps: float, film_wb, p_drop: float = 0.0,
                         hand: Fp8Handoff | None = None, dx_hand: Fp8Handoff | None = None):
    """With ``hand`` the output is a placeholder and the e4m3 conv input is ``hand.q``; with
    ``dx_hand`` the backward writes the e4m3 dx there (the dy of the conv producing x)."""
    return GroupNormSiLUFilm.apply(x, gamma, beta, groups, eps, film_wb, float(p_drop), hand,
                                   dx_hand)


def group_norm_silu(x, gamma, beta, groups: int, eps: float = 1e-5, film_scale=None, film_shift=None):
    return GroupNormSiLU.apply(x, gamma, beta, groups, eps, film_scale, film_shift)
