"""CPU restatement of the reference FP8 recipe (fattorib/diffusion-profiled).

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker / CPU baseline. The
product path (``diffusion-profiled_amd``) never calls it.

Each function cites the reference lines it restates. Integer/bit work is numpy; the
convolutions use torch CPU float64 on dequantized e4m3 values, where the accumulation is
exact (every e4m3 value is k * 2^-9 with |k| < 2^18, so a product is a multiple of 2^-18 below
2^36 and <= 2^17 of them sum exactly in 53 bits), making the result independent of order.

What pins each function (see tests/test_oracle_*.py):
  f32_to_e4m3_rne   torch's float8_e4m3fn conversion over every fp32 in [-464, 464] (C port
                    exhaustively, this numpy version on all boundaries + random) and the
                    known answers 1.0625->0x38, 1.1875->0x3a, 2^-10->0, 3*2^-11->1, 464->0x7e.
  scale / cast      closed form; all 65536 bf16 inputs x every reachable scale by the C port.
  conv fwd/dgrad/   torch.nn.functional.conv2d / torch.nn.grad.conv2d_input / conv2d_weight
  wgrad, gemm       in float64, cross-checked by brute-force loops on tiny shapes, transpose
                    identities (<dgrad(dy), x> == <dy, fwd(x)>), and stride/pad special cases.
  gn_silu fwd/bwd   torch.nn.functional.group_norm + silu in float64 and autograd.
  DelayedScaling    scripted sequences (window writes, one-slot dy offset, max-of-window).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

FP8_MAX = np.float32(448.0)  # torch.finfo(torch.float8_e4m3fn).max, fp8_kernels.py:12
AMAX_HISTORY = 1024  # diffusion/unet.py:25


# ---------------------------------------------------------------------------------------
# bit-level conversions
# ---------------------------------------------------------------------------------------
def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(f: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 round-to-nearest-even (torch's .to(bfloat16)); NaN -> quiet NaN."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r = np.where(nan, ((u >> 16) & 0x8000).astype(np.uint16) | np.uint16(0x7FC0), r)
    return r.astype(np.uint16)


_E4M3_TABLE = None


def e4m3_to_f32(q: np.ndarray) -> np.ndarray:
    """Decode OCP e4m3 (float8_e4m3fn) bytes: bias 7, subnormals k*2^-9, 0x7f/0xff NaN."""
    global _E4M3_TABLE
    if _E4M3_TABLE is None:
        t = np.zeros(256, dtype=np.float32)
        for b in range(256):
            s = -1.0 if b & 0x80 else 1.0
            e = (b >> 3) & 0xF
            m = b & 7
            if e == 15 and m == 7:
                t[b] = np.nan
            elif e == 0:
                t[b] = s * m * 2.0**-9
            else:
                t[b] = s * (1 + m / 8.0) * 2.0 ** (e - 7)
        _E4M3_TABLE = t
    return _E4M3_TABLE[np.asarray(q, dtype=np.uint8)]


def f32_to_e4m3_rne(v: np.ndarray) -> np.ndarray:
    """fp32 -> e4m3 bytes, round to nearest even. |v| > 464 or NaN -> 0x7f|sign (NaN);
    448 < |v| <= 464 rounds to 448 (0x7e). Same rule as torch's CPU conversion."""
    b = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32)
    sign = ((b >> 24) & 0x80).astype(np.uint32)
    a = (b & 0x7FFFFFFF).astype(np.uint32)
    out = np.zeros(a.shape, dtype=np.uint32)
    big = a > 0x43E80000
    normal = (a >= 0x3C800000) & ~big
    sub = a < 0x3C800000
    # normal: round the 23-bit mantissa to 3 bits (RNE), rebias 127 -> 7
    an = a[normal].astype(np.uint64)
    rn = an + 0x7FFFF + ((an >> 20) & 1)
    out[normal] = ((rn >> 20) - 0x3C0).astype(np.uint32)
    # subnormal: nearest multiple of 2^-9, ties to even, exact in integer arithmetic
    asub = a[sub].astype(np.int64)
    e = (asub >> 23) - 127
    mant = (asub & 0x7FFFFF) | 0x800000
    s = 14 - e
    res = np.zeros(asub.shape, dtype=np.int64)
    ok = (e >= -126) & (s <= 24)
    sh = s[ok]
    mm = mant[ok]
    m = mm >> sh
    rem = mm & ((np.int64(1) << sh) - 1)
    half = np.int64(1) << (sh - 1)
    m = m + ((rem > half) | ((rem == half) & ((m & 1) == 1))).astype(np.int64)
    res[ok] = m
    out[sub] = res.astype(np.uint32)
    out[big] = 0x7F
    return (sign | out).astype(np.uint8)


# ---------------------------------------------------------------------------------------
# scale and cast (diffusion/fp8_kernels.py:54-120, :518-601)
# ---------------------------------------------------------------------------------------
def amax_bf16(x_bits: np.ndarray) -> np.float32:
    """max |x| over a bf16 tensor (partial_amax_kernel :54-64 + finalize max :100)."""
    xb = np.asarray(x_bits, dtype=np.uint16).reshape(-1)
    if xb.size == 0:
        return np.float32(0.0)
    m = np.max(xb & np.uint16(0x7FFF))
    return bf16_bits_to_f32(np.array([m], dtype=np.uint16))[0]


def scale_from_amax(amax: np.float32) -> np.float32:
    """tl.where(amax > 0, amax / FP8_MAX, 1.0)  (fp8_kernels.py:101); IEEE fp32 division."""
    amax = np.float32(amax)
    if amax > 0:
        return np.float32(amax / FP8_MAX)
    return np.float32(1.0)


def cast_e4m3(x_bits: np.ndarray, scale: np.float32) -> np.ndarray:
    """q = e4m3(max(-448, min(f32(x) / scale, 448)))  (quantize_fp8_kernel :116-120).

    The clamp follows the kernel's order with IEEE minNum/maxNum (np.fmin / np.fmax), so a
    NaN quotient maps to +448; NaN/Inf inputs are outside the parity contract."""
    x = bf16_bits_to_f32(x_bits)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        s = (x / np.float32(scale)).astype(np.float32)
    s = np.fmax(-FP8_MAX, np.fmin(s, FP8_MAX)).astype(np.float32)
    return f32_to_e4m3_rne(s)


def quantize_fp8(x_bits: np.ndarray) -> tuple[np.ndarray, np.float32]:
    """Current scaling: partial amax -> finalize -> cast (fp8_kernels.py:559-601)."""
    scale = scale_from_amax(amax_bf16(x_bits))
    return cast_e4m3(x_bits, scale), scale


def quantize_fp8_delayed(x_bits: np.ndarray, prev_scale: np.float32) -> tuple[np.ndarray, np.float32]:
    """Delayed scaling: cast with prev_scale, return the current scale (:518-556, :69-87)."""
    return cast_e4m3(x_bits, prev_scale), scale_from_amax(amax_bf16(x_bits))


def reachable_scales() -> np.ndarray:
    """Every scale current scaling can produce from bf16 data: RN32(a / 448) for each positive
    finite bf16 magnitude a, plus 1.0 (amax == 0). Sorted, unique."""
    mags = np.arange(1, 0x7F80, dtype=np.uint16)
    s = (bf16_bits_to_f32(mags) / FP8_MAX).astype(np.float32)
    return np.unique(np.concatenate([s, np.array([1.0], dtype=np.float32)]))


# ---------------------------------------------------------------------------------------
# FP8 convolution / GEMM (diffusion/fp8_kernels.py:142-468), exact accumulation
# ---------------------------------------------------------------------------------------
def _deq64(q_nhwc: np.ndarray) -> torch.Tensor:
    """e4m3 NHWC bytes -> float64 NCHW tensor (exact)."""
    f = e4m3_to_f32(q_nhwc).astype(np.float64)
    return torch.from_numpy(np.ascontiguousarray(f)).permute(0, 3, 1, 2)


def _deq64_w(q_ohwi: np.ndarray) -> torch.Tensor:
    f = e4m3_to_f32(q_ohwi).astype(np.float64)
    return torch.from_numpy(np.ascontiguousarray(f)).permute(0, 3, 1, 2)


def _epilogue(acc64: np.ndarray, sa: np.float32, sb: np.float32, bias: np.ndarray | None = None) -> np.ndarray:
    """bf16(RN32(RN32(acc) * RN32(sa * sb)) [+ bias]) — tl.store(acc * (xs * ws)) (:246-247)."""
    scale = np.float32(np.float32(sa) * np.float32(sb))
    v = (acc64.astype(np.float32) * scale).astype(np.float32)
    if bias is not None:
        v = (v + bias.astype(np.float32)).astype(np.float32)
    return f32_to_bf16_bits(v)


def conv2d_fwd(xq: np.ndarray, wq: np.ndarray, xs, ws, stride: int = 1, pad: int = 1,
               bias: np.ndarray | None = None) -> np.ndarray:
    """y[n,oh,ow,oc] = bf16(xs*ws * sum_{kh,kw,ic} xq[n, oh*st+kh-pad, ow*st+kw-pad, ic] *
    wq[oc,kh,kw,ic]) with zero padding (conv2d_fwd_fp8_kernel :201-247; stride/1x1 are the
    same recipe). xq NHWC bytes, wq OHWI bytes; returns NHWC bf16 bits."""
    acc = F.conv2d(_deq64(xq), _deq64_w(wq), stride=stride, padding=pad)
    acc = acc.permute(0, 2, 3, 1).contiguous().numpy()
    return _epilogue(acc, xs, ws, bias)


def conv2d_dgrad(dyq: np.ndarray, wq: np.ndarray, dys, ws, input_hw: tuple[int, int],
                 stride: int = 1, pad: int = 1) -> np.ndarray:
    """dx[n,ih,iw,ic] = bf16(dys*ws * sum dyq[n,oh,ow,oc] wq[oc,kh,kw,ic]) over
    ih = oh*st + kh - pad (conv2d_dx_fp8_kernel :278-318)."""
    dy = _deq64(dyq)
    w = _deq64_w(wq)
    n = dy.shape[0]
    cin = w.shape[1]
    acc = torch.nn.grad.conv2d_input((n, cin, *input_hw), w, dy, stride=stride, padding=pad)
    acc = acc.permute(0, 2, 3, 1).contiguous().numpy()
    return _epilogue(acc, dys, ws)


def conv2d_wgrad(xq: np.ndarray, dyq: np.ndarray, xs, dys, kernel_size: int = 3,
                 stride: int = 1, pad: int = 1) -> np.ndarray:
    """dw[oc,kh,kw,ic] = bf16(xs*dys * sum_{n,oh,ow} dyq[n,oh,ow,oc] xq[n,oh*st+kh-pad,..,ic])
    (conv2d_dw_fp8_kernel :400-443 + conv2d_dw_reduce_fp8_kernel :457-468); OHWI bf16 bits."""
    x = _deq64(xq)
    dy = _deq64(dyq)
    cout = dy.shape[1]
    acc = torch.nn.grad.conv2d_weight(x, (cout, x.shape[1], kernel_size, kernel_size), dy,
                                      stride=stride, padding=pad)
    acc = acc.permute(0, 2, 3, 1).contiguous().numpy()
    return _epilogue(acc, xs, dys)


def gemm(aq: np.ndarray, bq: np.ndarray, sa, sb, bias: np.ndarray | None = None) -> np.ndarray:
    """c = bf16(sa*sb * aq[M,K] @ bq[N,K]^T [+ bias]) — the FP8 linear recipe."""
    a = torch.from_numpy(e4m3_to_f32(aq).astype(np.float64))
    b = torch.from_numpy(e4m3_to_f32(bq).astype(np.float64))
    return _epilogue((a @ b.T).numpy(), sa, sb, bias)


# ---------------------------------------------------------------------------------------
# GroupNorm (+FiLM) + SiLU (diffusion/unet.py:132-133, :151, :157-159)
# ---------------------------------------------------------------------------------------
def _gn_input_f64(x: np.ndarray) -> np.ndarray:
    """GroupNorm input as float64: NHWC bf16 bits (uint16) or fp32 values (the fp32 residual
    stream, which autocast's float32 GroupNorm reads as it is)."""
    if x.dtype == np.float32:
        return x.astype(np.float64)
    return bf16_bits_to_f32(x).astype(np.float64)


def splitmix64(seed: int, idx: np.ndarray) -> np.ndarray:
    """splitmix64 output for state seed + idx * 0x9E3779B97F4A7C15 (Steele, Lea and Flood,
    "Fast splittable pseudorandom number generators", OOPSLA 2014; Vigna's finaliser
    constants), uint64 with wrap-around."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed & (2**64 - 1)) + idx.astype(np.uint64) * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def dropout_keep(seed: int, n: int, p: float) -> np.ndarray:
    """Keep mask of the fused dropout over n elements (NHWC index order): element idx is kept
    when the 16-bit quarter idx % 4 of splitmix64(seed, idx // 4) (bits 16 (idx % 4) up to
    16 (idx % 4) + 15) is >= floor(p * 2^16). The reference draws its mask from torch's
    Philox generator (diffusion/unet.py:160 nn.Dropout), which no restatement reproduces;
    this mask has the keep probability 1 - floor(p * 2^16) / 2^16, within 2^-16 of 1 - p. p
    is taken as the fp32 value the C ABI receives (``float drop_p``): the threshold is
    floor(fp32(p) * 2^16), computed exactly in double."""
    keep_from = int(float(np.float32(p)) * 65536.0)
    idx = np.arange(n, dtype=np.uint64)
    z = splitmix64(seed, idx >> np.uint64(2))
    quarter = (z >> (np.uint64(16) * (idx & np.uint64(3)))) & np.uint64(0xFFFF)
    return quarter >= np.uint64(keep_from)


def dropout_scale(p: float) -> np.float32:
    """1 / (1 - p) as torch's dropout kernel forms it: 1 - p rounded to fp32, its reciprocal
    taken in double and rounded to fp32; p is the fp32 value the C ABI receives."""
    return np.float32(1.0 / float(np.float32(1.0 - float(np.float32(p)))))


def gn_silu_fwd(x_bits: np.ndarray, gamma: np.ndarray, beta: np.ndarray, groups: int,
                eps: float = 1e-5, film_scale: np.ndarray | None = None,
                film_shift: np.ndarray | None = None, drop: tuple[int, float] | None = None
                ) -> np.ndarray:
    """bf16( silu( [fs *] GroupNorm(x) [+ fb] ) ) evaluated in float64, then rounded to fp32
    and bf16. x NHWC bf16 bits or fp32 values; gamma/beta fp32 [C]; film [N, C]; drop =
    (seed, p): the fp32 SiLU output is dropped or scaled by dropout_scale(p) in fp32 before the
    bf16 rounding (dropout on autocast's fp32 SiLU output, diffusion/unet.py:160). Returns NHWC
    bf16 bits."""
    x = torch.from_numpy(_gn_input_f64(x_bits)).permute(0, 3, 1, 2)
    z = F.group_norm(x, groups, torch.from_numpy(gamma.astype(np.float64)),
                     torch.from_numpy(beta.astype(np.float64)), eps)
    if film_scale is not None:
        fs = torch.from_numpy(film_scale.astype(np.float64))[:, :, None, None]
        fb = torch.from_numpy(film_shift.astype(np.float64))[:, :, None, None]
        z = fs * z + fb
    out = F.silu(z).permute(0, 2, 3, 1).contiguous().numpy().astype(np.float32)
    if drop is not None:
        keep = dropout_keep(drop[0], out.size, drop[1]).reshape(out.shape)
        out = np.where(keep, out * dropout_scale(drop[1]), np.float32(0.0)).astype(np.float32)
    return f32_to_bf16_bits(out)


def gn_silu_bwd(x_bits: np.ndarray, dout_bits: np.ndarray, gamma: np.ndarray, beta: np.ndarray,
                groups: int, eps: float = 1e-5, film_scale: np.ndarray | None = None,
                film_shift: np.ndarray | None = None, drop: tuple[int, float] | None = None):
    """Autograd of gn_silu_fwd in float64 (x and drop as there: the incoming gradient is
    masked and scaled in fp32 first). Returns (dx NHWC float64, dgamma, dbeta, dfilm_scale
    [N,C] | None, dfilm_shift | None)."""
    x = torch.from_numpy(_gn_input_f64(x_bits)).permute(0, 3, 1, 2)
    x.requires_grad_(True)
    g = torch.from_numpy(gamma.astype(np.float64)).requires_grad_(True)
    b = torch.from_numpy(beta.astype(np.float64)).requires_grad_(True)
    z = F.group_norm(x, groups, g, b, eps)
    fs = fb = None
    if film_scale is not None:
        fs = torch.from_numpy(film_scale.astype(np.float64)).requires_grad_(True)
        fb = torch.from_numpy(film_shift.astype(np.float64)).requires_grad_(True)
        z = fs[:, :, None, None] * z + fb[:, :, None, None]
    out = F.silu(z)
    d32 = bf16_bits_to_f32(dout_bits)
    if drop is not None:
        keep = dropout_keep(drop[0], d32.size, drop[1]).reshape(d32.shape)
        d32 = np.where(keep, d32 * dropout_scale(drop[1]), np.float32(0.0)).astype(np.float32)
    d = torch.from_numpy(d32.astype(np.float64)).permute(0, 3, 1, 2)
    out.backward(d)
    dx = x.grad.permute(0, 2, 3, 1).contiguous().numpy()
    res = [dx, g.grad.numpy(), b.grad.numpy()]
    res += [fs.grad.numpy(), fb.grad.numpy()] if fs is not None else [None, None]
    return tuple(res)


# ---------------------------------------------------------------------------------------
# delayed-scaling state machine (diffusion/unet.py:50-56, :69-91; fp8_kernels.py:845-889)
# ---------------------------------------------------------------------------------------
class DelayedScaling:
    """Windows of *scales* (amax/448 values) for acts, weights and dy, plus window_pos.

    forward(x, w):  xs_h = max(win_acts), ws_h = max(win_w), dys_h = max(win_dy) (read in
                    forward, :849); q = cast with the historical scales; the current scales
                    are written at window_pos, then window_pos = (window_pos + 1) % H.
    backward(dy):   cast dy with dys_h; the current dy scale is written at the ALREADY
                    advanced window_pos (one slot ahead of acts/weights).
    """

    def __init__(self, history: int = AMAX_HISTORY):
        self.history = history
        self.win_acts = np.zeros(history, dtype=np.float32)
        self.win_weights = np.zeros(history, dtype=np.float32)
        self.win_dy = np.zeros(history, dtype=np.float32)
        self.pos = 0
        self._dy_hist = None

    def forward(self, x_bits, w_bits):
        xs_h = np.float32(self.win_acts.max())
        ws_h = np.float32(self.win_weights.max())
        self._dy_hist = np.float32(self.win_dy.max())
        xq, xs_cur = quantize_fp8_delayed(x_bits, xs_h)
        wq, ws_cur = quantize_fp8_delayed(w_bits, ws_h)
        self.win_weights[self.pos] = ws_cur
        self.win_acts[self.pos] = xs_cur
        self.pos = (self.pos + 1) % self.history
        return xq, wq, xs_h, ws_h, xs_cur, ws_cur

    def backward(self, dy_bits):
        dyq, dys_cur = quantize_fp8_delayed(dy_bits, self._dy_hist)
        self.win_dy[self.pos] = dys_cur
        return dyq, self._dy_hist, dys_cur
