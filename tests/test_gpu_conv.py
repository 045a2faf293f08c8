"""GPU parity of the FP8 conv (fwd / dgrad / wgrad) and GEMM against the oracle, through
the reference-named Python ops and the C ABI beneath them.

Reduced batch at every registry shape (the oracle accumulates exactly in float64), stride-2
and 1x1 variants, ragged pixel counts, and the full BASELINE sizes through size-independent
properties: batch independence (image i of a batched conv equals the conv of image i alone,
bit for bit) plus a float32 torch reference on the GPU.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import assert_bf16_close, bits, dpa_mod, kaiming_uniform_bf16, nhwc_bits, randn_bf16
from oracle import fp8_oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K():
    return dpa_mod("fp8_kernels")


def cl(t: torch.Tensor) -> torch.Tensor:
    return t.cuda().contiguous(memory_format=torch.channels_last)


def quantized_inputs(K, n, cin, cout, h, w, k=3, stride=1, pad=1, seed=0):
    x = randn_bf16((n, cin, h, w), seed=seed)
    wt = kaiming_uniform_bf16((cout, cin, k, k), seed=seed + 1)
    p, q = (h + 2 * pad - k) // stride + 1, (w + 2 * pad - k) // stride + 1
    dy = randn_bf16((n, cout, p, q), seed=seed + 2, std=1e-2)
    xq, xs = K.quantize_fp8(cl(x))
    wq, ws = K.quantize_fp8(cl(wt))
    dyq, dys = K.quantize_fp8(cl(dy))
    # the quantized operands themselves are bit-exact (checked in depth in test_gpu_quant)
    q_ref, s_ref = O.quantize_fp8(nhwc_bits(x))
    assert np.float32(xs.item()) == s_ref
    np.testing.assert_array_equal(nhwc_bits(xq.cpu().view(torch.uint8)), q_ref)
    return xq, xs, wq, ws, dyq, dys


def f32(t):
    return np.float32(t.item())


def run_all_three(K, n, cin, cout, h, w, k=3, stride=1, pad=1, seed=0, use_reference_names=True):
    xq, xs, wq, ws, dyq, dys = quantized_inputs(K, n, cin, cout, h, w, k, stride, pad, seed)
    if use_reference_names:
        y = K.conv2d_fwd_fp8_prequantized(xq, wq, xs, ws)
        dx = K.conv2d_bwd_input_fp8_prequantized(dyq, wq, dys, ws)
        dw = K.conv2d_bwd_weight_fp8_prequantized(xq, dyq, xs, dys)
    else:
        y = K.conv2d_fp8_fwd_general(xq, wq, xs, ws, stride, pad)
        dx = K.conv2d_fp8_dgrad_general(dyq, wq, dys, ws, (h, w), stride, pad)
        dw = K.conv2d_fp8_wgrad_general(xq, dyq, xs, dys, k, stride, pad)
    torch.cuda.synchronize()
    xb, wb, db = (nhwc_bits(t.cpu().view(torch.uint8)) for t in (xq, wq, dyq))
    y_ref = O.conv2d_fwd(xb, wb, f32(xs), f32(ws), stride, pad)
    dx_ref = O.conv2d_dgrad(db, wb, f32(dys), f32(ws), (h, w), stride, pad)
    dw_ref = O.conv2d_wgrad(xb, db, f32(xs), f32(dys), k, stride, pad)
    assert y.is_contiguous(memory_format=torch.channels_last) and y.dtype == torch.bfloat16
    assert dx.shape == (n, cin, h, w) and dw.shape == (cout, cin, k, k)
    tag = f"{(n, cin, cout, h, w, k, stride)}"
    e1 = assert_bf16_close(nhwc_bits(y.cpu()), y_ref, "fwd " + tag)
    e2 = assert_bf16_close(nhwc_bits(dx.cpu()), dx_ref, "dgrad " + tag)
    e3 = assert_bf16_close(nhwc_bits(dw.cpu()), dw_ref, "wgrad " + tag)
    # fp32 accumulation differs from the exact sum only at bf16 rounding ties
    assert min(e1, e2) > 0.97, (e1, e2)
    assert e3 > 0.9, e3


REGISTRY = [
    (128, 128, 32, 32), (128, 256, 32, 32), (256, 256, 16, 16), (512, 256, 16, 16),
    (256, 256, 8, 8), (512, 256, 8, 8), (512, 128, 32, 32), (256, 256, 32, 32), (256, 256, 4, 4),
]


@pytest.mark.parametrize("shape", REGISTRY, ids=lambda s: "x".join(map(str, s)))
def test_registry_shapes_reduced_batch(K, shape):
    cin, cout, h, w = shape
    run_all_three(K, 2, cin, cout, h, w, seed=sum(shape))


@pytest.mark.parametrize(
    "n,cin,cout,h,w,k,stride,pad",
    [
        (2, 256, 256, 16, 16, 3, 2, 1),   # cfg3 stride-2 downsample
        (3, 256, 256, 9, 7, 3, 2, 1),     # odd sizes, ragged pixel count
        (2, 128, 256, 32, 32, 1, 1, 0),   # cfg3 1x1 residual projection
        (2, 512, 256, 16, 16, 1, 1, 0),
        (3, 128, 128, 7, 9, 3, 1, 1),     # ragged M (189 pixels)
        (1, 128, 128, 1, 1, 3, 1, 1),     # single pixel: only the centre tap is in range
    ],
)
def test_general_convs(K, n, cin, cout, h, w, k, stride, pad):
    run_all_three(K, n, cin, cout, h, w, k, stride, pad, seed=n + h, use_reference_names=False)


def test_gemm_cfg1_full_size(K):
    """cfg1: X bf16 [32768, 256], W [768, 256], per-tensor e4m3, bf16 out — vs the exact oracle."""
    x = randn_bf16((32768, 256), seed=0)
    wt = kaiming_uniform_bf16((768, 256), seed=1)
    xq, xs = K.quantize_fp8_tensor(x.cuda())
    wq, ws = K.quantize_fp8_tensor(wt.cuda())
    y = K.linear_fp8_prequantized(xq, wq, xs, ws)
    torch.cuda.synchronize()
    y_ref = O.gemm(bits(xq.cpu()), bits(wq.cpu()), f32(xs), f32(ws))
    frac = assert_bf16_close(bits(y.cpu()), y_ref, "gemm cfg1")
    assert frac > 0.97
    # the fused path gives the same bytes
    y2 = K.linear_fp8(x.cuda(), wt.cuda())
    np.testing.assert_array_equal(bits(y2.cpu()), bits(y.cpu()))


def test_gemm_bias_and_ragged_m(K):
    x = randn_bf16((300, 384), seed=3)
    wt = kaiming_uniform_bf16((256, 384), seed=4)
    bias = torch.randn(256, generator=torch.Generator().manual_seed(5))
    xq, xs = K.quantize_fp8_tensor(x.cuda())
    wq, ws = K.quantize_fp8_tensor(wt.cuda())
    y = K.linear_fp8_prequantized(xq, wq, xs, ws, bias.cuda())
    torch.cuda.synchronize()
    y_ref = O.gemm(bits(xq.cpu()), bits(wq.cpu()), f32(xs), f32(ws), bias.numpy())
    assert_bf16_close(bits(y.cpu()), y_ref, "gemm bias")


def test_cfg2_full_size_properties(K):
    """cfg2 at full size (B=128, 32x32, 128->128): batch independence (bit-exact), the first
    images against the exact oracle, and all outputs against a float32 torch reference."""
    n, c, h, w = 128, 128, 32, 32
    xq, xs, wq, ws, dyq, dys = quantized_inputs(K, n, c, c, h, w, seed=0)
    y = K.conv2d_fwd_fp8_prequantized(xq, wq, xs, ws)
    dx = K.conv2d_bwd_input_fp8_prequantized(dyq, wq, dys, ws)
    dw = K.conv2d_bwd_weight_fp8_prequantized(xq, dyq, xs, dys)
    torch.cuda.synchronize()
    # batch independence for fwd/dgrad: image 5 alone gives the same bytes
    y5 = K.conv2d_fp8_fwd_general(xq[5:6], wq, xs, ws)
    dx5 = K.conv2d_fp8_dgrad_general(dyq[5:6], wq, dys, ws, (h, w))
    np.testing.assert_array_equal(bits(y5.cpu()), bits(y[5:6].cpu()))
    np.testing.assert_array_equal(bits(dx5.cpu()), bits(dx[5:6].cpu()))
    # exact oracle on two images
    xb, wb, db = (nhwc_bits(t.cpu().view(torch.uint8)) for t in (xq[:2], wq, dyq[:2]))
    assert_bf16_close(nhwc_bits(y[:2].cpu()), O.conv2d_fwd(xb, wb, f32(xs), f32(ws)), "cfg2 fwd")
    assert_bf16_close(nhwc_bits(dx[:2].cpu()), O.conv2d_dgrad(db, wb, f32(dys), f32(ws), (h, w)), "cfg2 dgrad")
    # float32 GPU reference of the dequantized operands, all outputs
    torch.backends.cudnn.allow_tf32 = False
    xf = xq.float() * xs
    wf = wq.float() * ws
    dyf = dyq.float() * dys
    y_t = F.conv2d(xf, wf, padding=1)
    dx_t = torch.nn.grad.conv2d_input(xf.shape, wf, dyf, padding=1)
    dw_t = torch.nn.grad.conv2d_weight(xf, wf.shape, dyf, padding=1)
    for got, ref, name in ((y, y_t, "fwd"), (dx, dx_t, "dgrad"), (dw, dw_t, "wgrad")):
        err = (got.float() - ref).norm() / ref.norm()
        assert err < 1e-2, (name, float(err))


def test_wgrad_split_invariance(K):
    """The split count changes only fp32 summation order: results agree within tolerance."""
    xq, xs, wq, ws, dyq, dys = quantized_inputs(K, 8, 128, 128, 32, 32, seed=9)
    a = K.conv2d_bwd_weight_fp8_prequantized(xq, dyq, xs, dys, split_k=1)
    b = K.conv2d_bwd_weight_fp8_prequantized(xq, dyq, xs, dys, split_k=7)
    c = K.conv2d_bwd_weight_fp8_prequantized(xq, dyq, xs, dys)
    torch.cuda.synchronize()
    ref = nhwc_bits(a.cpu())
    assert_bf16_close(nhwc_bits(b.cpu()), ref, "split 7 vs 1")
    assert_bf16_close(nhwc_bits(c.cpu()), ref, "default vs 1")


@pytest.mark.parametrize("n,h,w,split_k", [(3, 16, 16, 2), (3, 16, 16, 5), (3, 32, 32, 5),
                                           (2, 32, 32, 1)])
def test_wgrad_three_tap_splits_across_images(K, n, h, w, split_k):
    """3x3 stride-1 wgrad of 16/32-wide images (three taps per workgroup): pixel splits that
    start and end inside an image and cross image boundaries, against the exact oracle."""
    xq, xs, wq, ws, dyq, dys = quantized_inputs(K, n, 128, 256, h, w, seed=n + h + split_k)
    dw = K.conv2d_fp8_wgrad_general(xq, dyq, xs, dys, 3, 1, 1, split_k)
    torch.cuda.synchronize()
    xb, db = (nhwc_bits(t.cpu().view(torch.uint8)) for t in (xq, dyq))
    dw_ref = O.conv2d_wgrad(xb, db, f32(xs), f32(dys), 3, 1, 1)
    frac = assert_bf16_close(nhwc_bits(dw.cpu()), dw_ref, f"wgrad split {split_k}")
    assert frac > 0.9, frac


def test_zero_weight_gives_zero_output(K):
    """conv_2 is zero-initialised in the reference (diffusion/unet.py:146): scale 1, y == 0."""
    x = randn_bf16((2, 256, 16, 16), seed=1)
    wz = torch.zeros((256, 256, 3, 3), dtype=torch.bfloat16)
    y = K.conv2d_fwd_fp8(cl(x), cl(wz))
    torch.cuda.synchronize()
    assert not bits(y.cpu()).any()


SPLIT_SHAPES = [
    (128, 256, 256, 4, 4, 3, 1, 1),   # U-Net 4x4 level: 16 output tiles, 3-way K split
    (32, 512, 256, 8, 8, 3, 1, 1),    # 8x8, 512 -> 256
    (16, 256, 256, 8, 8, 3, 2, 1),    # stride-2 downsample; dgrad parity classes split too
    (24, 1024, 128, 4, 4, 1, 1, 0),   # 1x1 projection, ragged last tile (384 pixels)
    (5, 128, 256, 3, 5, 3, 1, 1),     # ragged, 9 K-steps: 3-way split
]


@pytest.mark.parametrize("n,cin,cout,h,w,k,stride,pad", SPLIT_SHAPES)
def test_split_k_conv_matches_single_pass_and_oracle(K, n, cin, cout, h, w, k, stride, pad):
    """Launches too small to fill the GPU split their K range (fp32 partials reduced in split
    order): fwd and dgrad against the exact oracle, and against the single-pass kernel."""
    L = dpa_mod("_lib")
    geom = (n, h, w, cin, cout, k, k, stride, pad)
    assert L.query("dpa_conv2d_fwd_split_workspace_bytes", *geom) > 0
    xq, xs, wq, ws, dyq, dys = quantized_inputs(K, n, cin, cout, h, w, k, stride, pad, seed=n + h)
    y = K.conv2d_fp8_fwd_general(xq, wq, xs, ws, stride, pad)
    y1 = K.conv2d_fp8_fwd_general(xq, wq, xs, ws, stride, pad, split=False)
    dx = K.conv2d_fp8_dgrad_general(dyq, wq, dys, ws, (h, w), stride, pad)
    dx1 = K.conv2d_fp8_dgrad_general(dyq, wq, dys, ws, (h, w), stride, pad, split=False)
    torch.cuda.synchronize()
    xb, wb, db = (nhwc_bits(t.cpu().view(torch.uint8)) for t in (xq, wq, dyq))
    y_ref = O.conv2d_fwd(xb, wb, f32(xs), f32(ws), stride, pad)
    dx_ref = O.conv2d_dgrad(db, wb, f32(dys), f32(ws), (h, w), stride, pad)
    tag = f"{geom}"
    for got, ref, name in ((y, y_ref, "fwd"), (y1, y_ref, "fwd single"), (dx, dx_ref, "dgrad"),
                           (dx1, dx_ref, "dgrad single")):
        frac = assert_bf16_close(nhwc_bits(got.cpu()), ref, f"{name} {tag}")
        assert frac > 0.97, (name, frac)
    assert_bf16_close(nhwc_bits(y.cpu()), nhwc_bits(y1.cpu()), "fwd split vs single " + tag)


def test_split_k_gemm_and_linear_dgrad(K):
    """A 128-row GEMM (the U-Net's time-embedding shape class) with bias, split 4 ways, and
    the linear's data gradient, against the oracle and the single-pass kernel."""
    L = dpa_mod("_lib")
    m, k, n = 128, 1024, 512
    assert L.query("dpa_gemm_split_workspace_bytes", m, n, k) > 0
    x = randn_bf16((m, k), seed=11)
    wt = kaiming_uniform_bf16((n, k), seed=12)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(13))
    dy = randn_bf16((m, n), seed=14, std=1e-2)
    xq, xs = K.quantize_fp8_tensor(x.cuda())
    wq, ws = K.quantize_fp8_tensor(wt.cuda())
    dyq, dys = K.quantize_fp8_tensor(dy.cuda())
    y = K.linear_fp8_prequantized(xq, wq, xs, ws, bias.cuda())
    y1 = K.linear_fp8_prequantized(xq, wq, xs, ws, bias.cuda(), split=False)
    dx = K.linear_fp8_dgrad_prequantized(dyq, wq, dys, ws)
    dx1 = K.linear_fp8_dgrad_prequantized(dyq, wq, dys, ws, split=False)
    torch.cuda.synchronize()
    y_ref = O.gemm(bits(xq.cpu()), bits(wq.cpu()), f32(xs), f32(ws), bias.numpy())
    wT = np.ascontiguousarray(bits(wq.cpu()).T)
    dx_ref = O.gemm(bits(dyq.cpu()), wT, f32(dys), f32(ws))
    for got, ref, name in ((y, y_ref, "gemm"), (y1, y_ref, "gemm single"), (dx, dx_ref, "dgrad"),
                           (dx1, dx_ref, "dgrad single")):
        frac = assert_bf16_close(bits(got.cpu()), ref, name)
        assert frac > 0.97, (name, frac)


def frag_layout_reference(wq_ohwi: np.ndarray, transpose: bool) -> np.ndarray:
    """The fragment-native weight layout restated with numpy from its definition: 2 KB blocks,
    block (kc * T + t) * (rows / 16) + rb holds at byte h * 1024 + l * 16 + b row 16 rb + l % 16,
    K byte 128 kc + 32 (l // 16) + 16 h + b of tap t; forward rows = Cout, K = Cin; data
    gradient rows = Cin, K = Cout with the taps mirrored."""
    cout, kh, kw, cin = wq_ohwi.shape
    t_ = kh * kw
    w = wq_ohwi.reshape(cout, t_, cin)
    if transpose:
        w = w[:, ::-1, :].transpose(2, 1, 0)      # [Cin][T][Cout], taps mirrored
    rows, _, k = w.shape
    # [rows, T, K] -> [kc, t, rb, h, fq, frow, b]
    v = w.reshape(rows // 16, 16, t_, k // 128, 4, 2, 16)   # rb, frow, t, kc, fq, h, b
    v = v.transpose(3, 2, 0, 5, 4, 1, 6)                      # kc, t, rb, h, fq, frow, b
    return np.ascontiguousarray(v).reshape(-1)


@pytest.mark.parametrize("cout,cin", [(128, 128), (256, 128), (256, 512), (128, 256)])
def test_weight_frag_layout_bytes(cout, cin):
    """dpa_weight_frag_fp8 permutes the OHWI e4m3 bytes into the fragment layout (forward)
    and the transposed, mirrored one (data gradient), bit for bit."""
    L = dpa_mod("_lib")
    rng = np.random.default_rng(cout + cin)
    wq = rng.integers(0, 256, size=(cout, 3, 3, cin), dtype=np.uint8)
    wq[(wq & 0x7F) == 0x7F] = 0   # no NaN codes needed; the layout only moves bytes
    d = torch.from_numpy(wq.copy()).cuda()
    wf = torch.empty(d.numel(), dtype=torch.uint8, device="cuda")
    wt = torch.empty_like(wf)
    assert L.query("dpa_weight_frag_bytes", cout, 3, 3, cin) == d.numel()
    L.call("dpa_weight_frag_fp8", d.data_ptr(), wf.data_ptr(), wt.data_ptr(), cout, 3, 3, cin,
           torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(wf.cpu().numpy(), frag_layout_reference(wq, False))
    np.testing.assert_array_equal(wt.cpu().numpy(), frag_layout_reference(wq, True))


HCONV_SHAPES = [(128, 128, 32, 32), (128, 256, 32, 32), (256, 256, 16, 16), (512, 256, 16, 16),
                (512, 128, 32, 32), (256, 256, 32, 32)]


@pytest.mark.parametrize("shape", HCONV_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_fragment_weight_convs_vs_oracle(K, shape):
    """dpa_conv2d_fwd_fp8_wf / dpa_conv2d_dgrad_fp8_wf with the weight prepared by
    dpa_weight_frag_fp8: against the exact oracle, and bit-identical to the OHWI entries
    (the same kernel arithmetic; only the weight fetch differs)."""
    L = dpa_mod("_lib")
    cin, cout, h, w = shape
    n = 2
    xq, xs, wq, ws, dyq, dys = quantized_inputs(K, n, cin, cout, h, w, seed=sum(shape) + 7)
    stream = torch.cuda.current_stream().cuda_stream
    wf = torch.empty(wq.numel(), dtype=torch.uint8, device="cuda")
    wt = torch.empty_like(wf)
    L.call("dpa_weight_frag_fp8", wq.data_ptr(), wf.data_ptr(), wt.data_ptr(), cout, 3, 3, cin,
           stream)
    y = torch.empty((n, cout, h, w), dtype=torch.bfloat16, device="cuda",
                    memory_format=torch.channels_last)
    dx = torch.empty((n, cin, h, w), dtype=torch.bfloat16, device="cuda",
                     memory_format=torch.channels_last)
    L.call("dpa_conv2d_fwd_fp8_wf", xq.data_ptr(), wf.data_ptr(), xs.data_ptr(), ws.data_ptr(),
           None, y.data_ptr(), n, h, w, cin, cout, stream)
    L.call("dpa_conv2d_dgrad_fp8_wf", dyq.data_ptr(), wt.data_ptr(), dys.data_ptr(),
           ws.data_ptr(), dx.data_ptr(), n, h, w, cin, cout, stream)
    y_ohwi = K.conv2d_fwd_fp8_prequantized(xq, wq, xs, ws)
    dx_ohwi = K.conv2d_bwd_input_fp8_prequantized(dyq, wq, dys, ws)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y_ohwi.view(torch.int16))
    assert torch.equal(dx.view(torch.int16), dx_ohwi.view(torch.int16))
    xb, wb, db = (nhwc_bits(t.cpu().view(torch.uint8)) for t in (xq, wq, dyq))
    tag = f"{shape}"
    e1 = assert_bf16_close(nhwc_bits(y.cpu()), O.conv2d_fwd(xb, wb, f32(xs), f32(ws)), "fwd_wf " + tag)
    e2 = assert_bf16_close(nhwc_bits(dx.cpu()), O.conv2d_dgrad(db, wb, f32(dys), f32(ws), (h, w)),
                           "dgrad_wf " + tag)
    assert min(e1, e2) > 0.97, (e1, e2)


def test_fragment_weight_entries_refuse_other_shapes():
    """The _wf entries serve only the halo-patch shapes (W 16 or 32, rows a multiple of the
    tile's row count); other shapes and misaligned outputs return an error before any launch.
    The pointers are real buffers large enough for every call, so a call that were accepted
    by mistake would fail the assertion, not read unmapped memory."""
    L = dpa_mod("_lib").load(build_if_missing=False)
    mb = 1 << 20
    buf = torch.zeros(3 * mb, device="cuda", dtype=torch.uint8)
    sc = torch.ones(2, device="cuda", dtype=torch.float32)
    act, wgt, out, s, nul = buf.data_ptr(), buf.data_ptr() + mb, buf.data_ptr() + 2 * mb, sc.data_ptr(), None
    assert L.dpa_conv2d_fwd_fp8_wf(act, wgt, s, s, nul, out, 2, 8, 8, 256, 256, nul) == -4
    assert L.dpa_conv2d_dgrad_fp8_wf(act, wgt, s, s, out, 2, 10, 32, 128, 128, nul) == -4
    assert L.dpa_conv2d_fwd_fp8_wf(act, wgt, s, s, nul, out + 8, 2, 32, 32, 128, 128, nul) == -3
    assert L.dpa_weight_frag_fp8(wgt, act, nul, 100, 3, 3, 128, nul) == -4
    torch.cuda.synchronize()
