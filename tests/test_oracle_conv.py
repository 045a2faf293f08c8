"""Pins the oracle's FP8 conv/GEMM/GroupNorm restatements (CPU only).

Brute-force loops over the reference's index formulas (diffusion/fp8_kernels.py:201-247,
:278-318, :400-468) on tiny shapes, adjoint identities between fwd/dgrad/wgrad (a transposed
operand or a wrong tap sign breaks them), the bf16 epilogue rounding, and GroupNorm+SiLU
against a direct numpy formula and finite differences.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8_oracle as O


def rand_e4m3(shape, rng, zero_frac=0.1):
    """Random finite e4m3 bytes (no NaN), some zeros."""
    q = rng.integers(0, 256, size=shape, dtype=np.int64).astype(np.uint8)
    q = np.where((q & 0x7F) == 0x7F, q ^ 0x01, q)
    q = np.where(rng.random(shape) < zero_frac, 0, q).astype(np.uint8)
    return q


def brute_fwd(x, w, stride, pad):
    """x [N,H,W,C] float, w [K,R,S,C] -> [N,P,Q,K], straight from the index formula."""
    n_, h, wd, c = x.shape
    k, r_, s_, _ = w.shape
    p = (h + 2 * pad - r_) // stride + 1
    q = (wd + 2 * pad - s_) // stride + 1
    y = np.zeros((n_, p, q, k))
    for n in range(n_):
        for oh in range(p):
            for ow in range(q):
                for r in range(r_):
                    for s in range(s_):
                        ih, iw = oh * stride + r - pad, ow * stride + s - pad
                        if 0 <= ih < h and 0 <= iw < wd:
                            y[n, oh, ow] += w[:, r, s, :] @ x[n, ih, iw]
    return y


def brute_dgrad(dy, w, h, wd, stride, pad):
    n_, p, q, k = dy.shape
    _, r_, s_, c = w.shape
    dx = np.zeros((n_, h, wd, c))
    for n in range(n_):
        for ih in range(h):
            for iw in range(wd):
                for r in range(r_):
                    for s in range(s_):
                        eh, ew = ih + pad - r, iw + pad - s
                        if eh % stride or ew % stride:
                            continue
                        oh, ow = eh // stride, ew // stride
                        if 0 <= oh < p and 0 <= ow < q:
                            dx[n, ih, iw] += dy[n, oh, ow] @ w[:, r, s, :]
    return dx


def brute_wgrad(x, dy, r_, s_, stride, pad):
    n_, h, wd, c = x.shape
    _, p, q, k = dy.shape
    dw = np.zeros((k, r_, s_, c))
    for n in range(n_):
        for oh in range(p):
            for ow in range(q):
                for r in range(r_):
                    for s in range(s_):
                        ih, iw = oh * stride + r - pad, ow * stride + s - pad
                        if 0 <= ih < h and 0 <= iw < wd:
                            dw[:, r, s, :] += np.outer(dy[n, oh, ow], x[n, ih, iw])
    return dw


CASES = [(3, 1, 1), (3, 2, 1), (1, 1, 0)]  # (k, stride, pad)


@pytest.mark.parametrize("k,stride,pad", CASES)
@pytest.mark.parametrize("hw", [(5, 5), (4, 6), (8, 8)])
def test_conv_fwd_dgrad_wgrad_vs_brute_force(k, stride, pad, hw):
    rng = np.random.default_rng(10 + k + stride + hw[0])
    n, c, kout = 2, 8, 6
    h, wd = hw
    xq = rand_e4m3((n, h, wd, c), rng)
    wq = rand_e4m3((kout, k, k, c), rng)
    x = O.e4m3_to_f32(xq).astype(np.float64)
    w = O.e4m3_to_f32(wq).astype(np.float64)
    xs, ws = np.float32(0.0123), np.float32(1.5)
    y = O.conv2d_fwd(xq, wq, xs, ws, stride, pad)
    np.testing.assert_array_equal(y, O._epilogue(brute_fwd(x, w, stride, pad), xs, ws))
    p, q = y.shape[1], y.shape[2]
    dyq = rand_e4m3((n, p, q, kout), rng)
    dy = O.e4m3_to_f32(dyq).astype(np.float64)
    dx = O.conv2d_dgrad(dyq, wq, xs, ws, (h, wd), stride, pad)
    np.testing.assert_array_equal(dx, O._epilogue(brute_dgrad(dy, w, h, wd, stride, pad), xs, ws))
    dw = O.conv2d_wgrad(xq, dyq, xs, ws, k, stride, pad)
    np.testing.assert_array_equal(dw, O._epilogue(brute_wgrad(x, dy, k, k, stride, pad), xs, ws))


def test_adjoint_identities():
    """<dgrad(dy), x> == <dy, fwd(x)> == <wgrad(x, dy), w> in float64."""
    rng = np.random.default_rng(3)
    for k, stride, pad in CASES:
        xq = rand_e4m3((2, 8, 8, 16), rng)
        wq = rand_e4m3((8, k, k, 16), rng)
        x64 = O._deq64(xq)
        w64 = O._deq64_w(wq)
        y = torch.nn.functional.conv2d(x64, w64, stride=stride, padding=pad)
        dyq = rand_e4m3(tuple(y.permute(0, 2, 3, 1).shape), rng)
        dy64 = O._deq64(dyq)
        dx = torch.nn.grad.conv2d_input(x64.shape, w64, dy64, stride=stride, padding=pad)
        dw = torch.nn.grad.conv2d_weight(x64, w64.shape, dy64, stride=stride, padding=pad)
        a = float((dx * x64).sum())
        b = float((dy64 * y).sum())
        c = float((dw * w64).sum())
        # equal up to the float64 rounding of the final dot products (a transposed operand
        # or a flipped tap changes them at O(1))
        assert abs(a - b) <= 1e-12 * abs(b) and abs(c - b) <= 1e-12 * abs(b)


def test_epilogue_rounding():
    # acc * scale rounded to fp32, then bf16 RNE: 1 + 2^-8 is a tie -> even (1.0)
    acc = np.array([1.0 + 2.0**-8, 1.0 + 3 * 2.0**-8, -2.0], dtype=np.float64)
    out = O._epilogue(acc, np.float32(1.0), np.float32(1.0))
    np.testing.assert_array_equal(out, np.array([0x3F80, 0x3F82, 0xC000], dtype=np.uint16))
    # scale product rounded in fp32 before the multiply (xs * ws)
    xs, ws = np.float32(1 / 3), np.float32(3.0)
    assert O._epilogue(np.array([1.0]), xs, ws)[0] == O.f32_to_bf16_bits(np.array([np.float32(xs * ws)]))[0]


def test_gemm_vs_numpy():
    rng = np.random.default_rng(4)
    aq = rand_e4m3((33, 64), rng)
    bq = rand_e4m3((16, 64), rng)
    a = O.e4m3_to_f32(aq).astype(np.float64)
    b = O.e4m3_to_f32(bq).astype(np.float64)
    bias = rng.standard_normal(16).astype(np.float32)
    np.testing.assert_array_equal(O.gemm(aq, bq, 0.5, 0.25, bias), O._epilogue(a @ b.T, 0.5, 0.25, bias))


def _gn_numpy(x, gamma, beta, groups, eps, fs=None, fb=None):
    n, h, w, c = x.shape
    xg = x.reshape(n, h * w, groups, c // groups)
    mean = xg.mean(axis=(1, 3), keepdims=True)
    var = ((xg - mean) ** 2).mean(axis=(1, 3), keepdims=True)
    z = ((xg - mean) / np.sqrt(var + eps)).reshape(n, h, w, c) * gamma + beta
    if fs is not None:
        z = fs[:, None, None, :] * z + fb[:, None, None, :]
    return z / (1 + np.exp(-z))


@pytest.mark.parametrize("film", [False, True])
def test_gn_silu_fwd_vs_numpy(film):
    rng = np.random.default_rng(5)
    n, h, w, c, g = 2, 4, 4, 64, 8
    xb = O.f32_to_bf16_bits(rng.standard_normal((n, h, w, c)).astype(np.float32))
    gamma = rng.standard_normal(c).astype(np.float32)
    beta = rng.standard_normal(c).astype(np.float32)
    fs = fb = None
    if film:
        fs = rng.standard_normal((n, c)).astype(np.float32)
        fb = rng.standard_normal((n, c)).astype(np.float32)
    got = O.gn_silu_fwd(xb, gamma, beta, g, 1e-5, fs, fb)
    ref = _gn_numpy(O.bf16_bits_to_f32(xb).astype(np.float64), gamma, beta, g, 1e-5, fs, fb)
    np.testing.assert_array_equal(got, O.f32_to_bf16_bits(ref.astype(np.float32)))


def test_gn_silu_bwd_finite_differences():
    rng = np.random.default_rng(6)
    n, h, w, c, g = 1, 2, 2, 8, 2
    xb = O.f32_to_bf16_bits(rng.standard_normal((n, h, w, c)).astype(np.float32))
    gamma = rng.standard_normal(c).astype(np.float32)
    beta = rng.standard_normal(c).astype(np.float32)
    fs = rng.standard_normal((n, c)).astype(np.float32)
    fb = rng.standard_normal((n, c)).astype(np.float32)
    db = O.f32_to_bf16_bits(rng.standard_normal((n, h, w, c)).astype(np.float32))
    d = O.bf16_bits_to_f32(db).astype(np.float64)
    dx, dg, dbt, dfs, dfb = O.gn_silu_bwd(xb, db, gamma, beta, g, 1e-5, fs, fb)
    x = O.bf16_bits_to_f32(xb).astype(np.float64)
    eps = 1e-6

    def loss(xv=x, gv=gamma, bv=beta, fsv=fs, fbv=fb):
        return float((_gn_numpy(xv, gv.astype(np.float64), bv.astype(np.float64), g, 1e-5,
                                fsv.astype(np.float64), fbv.astype(np.float64)) * d).sum())

    for idx in [(0, 0, 0, 0), (0, 1, 1, 5), (0, 1, 0, 7)]:
        xp = x.copy(); xp[idx] += eps
        xm = x.copy(); xm[idx] -= eps
        assert abs((loss(xv=xp) - loss(xv=xm)) / (2 * eps) - dx[idx]) < 1e-6
    for j in (0, 3):
        gp = gamma.astype(np.float64).copy(); gp[j] += eps
        gm = gamma.astype(np.float64).copy(); gm[j] -= eps
        assert abs((loss(gv=gp) - loss(gv=gm)) / (2 * eps) - dg[j]) < 1e-6
        fp = fs.astype(np.float64).copy(); fp[0, j] += eps
        fm = fs.astype(np.float64).copy(); fm[0, j] -= eps
        assert abs((loss(fsv=fp) - loss(fsv=fm)) / (2 * eps) - dfs[0, j]) < 1e-6
        bp = beta.astype(np.float64).copy(); bp[j] += eps
        bm = beta.astype(np.float64).copy(); bm[j] -= eps
        assert abs((loss(bv=bp) - loss(bv=bm)) / (2 * eps) - dbt[j]) < 1e-6
        sp = fb.astype(np.float64).copy(); sp[0, j] += eps
        sm = fb.astype(np.float64).copy(); sm[0, j] -= eps
        assert abs((loss(fbv=sp) - loss(fbv=sm)) / (2 * eps) - dfb[0, j]) < 1e-6
    assert dbt.shape == (c,) and dfb.shape == (n, c)
    # a planted mistake (the FiLM shift's gradient taken as the beta gradient) is caught
    assert np.abs(dfb[0] - dbt).max() > 1e-3
