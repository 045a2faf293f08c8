"""The fused residual join (a + b) / sqrt(2) (residual.residual_join, dpa_residual_scale_bf16)
equals torch's bf16 expression of diffusion/unet.py:161 / :203 bit for bit, forward and
backward, on channels-last and contiguous tensors."""
from __future__ import annotations

import math

import pytest
import torch

from conftest import dpa_mod

pytestmark = pytest.mark.gpu

R = dpa_mod("residual")


@pytest.mark.parametrize("shape,cl", [((4, 128, 32, 32), True), ((3, 256, 8, 8), True),
                                      ((128, 512), False), ((2, 256, 4, 4), True)])
def test_residual_join_bit_exact(shape, cl):
    g = torch.Generator().manual_seed(sum(shape))
    a = (torch.randn(shape, generator=g) * 3).to(torch.bfloat16).cuda()
    b = (torch.randn(shape, generator=g) * 0.5).to(torch.bfloat16).cuda()
    gy = (torch.randn(shape, generator=g) * 1e-2).to(torch.bfloat16).cuda()
    if cl:
        a, b, gy = (t.contiguous(memory_format=torch.channels_last) for t in (a, b, gy))
    a1, b1 = a.clone().requires_grad_(), b.clone().requires_grad_()
    a2, b2 = a.clone().requires_grad_(), b.clone().requires_grad_()
    y1 = R.residual_join(a1, b1)
    y2 = (a2 + b2) / math.sqrt(2.0)
    y1.backward(gy)
    y2.backward(gy)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert torch.equal(a1.grad, a2.grad) and torch.equal(b1.grad, b2.grad)


@pytest.mark.parametrize("shape,cl,swap", [((4, 256, 16, 16), True, False),
                                           ((3, 256, 8, 8), True, True),
                                           ((2, 256, 4, 4), True, False),
                                           ((128, 4, 256), False, True)])
def test_residual_join_fp32_stream_bit_exact(shape, cl, swap):
    """fp32 skip path + bf16 branch (the residual stream below the first level): torch's
    promoted fp32 add and scalar division, and autograd's gradients (fp32 for the fp32
    operand, rounded to bf16 for the bf16 one), bit for bit, in either operand order."""
    g = torch.Generator().manual_seed(sum(shape) + 1)
    a = (torch.randn(shape, generator=g) * 3).cuda()                       # fp32, full mantissa
    b = (torch.randn(shape, generator=g) * 0.5).to(torch.bfloat16).cuda()
    gy = (torch.randn(shape, generator=g) * 1e-2).cuda()
    if cl:
        a, b, gy = (t.contiguous(memory_format=torch.channels_last) for t in (a, b, gy))
    a1, b1 = a.clone().requires_grad_(), b.clone().requires_grad_()
    a2, b2 = a.clone().requires_grad_(), b.clone().requires_grad_()
    y1 = R.residual_join(b1, a1) if swap else R.residual_join(a1, b1)
    y2 = (b2 + a2) / math.sqrt(2.0) if swap else (a2 + b2) / math.sqrt(2.0)
    assert y1.dtype == torch.float32
    y1.backward(gy)
    y2.backward(gy)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert a1.grad.dtype == torch.float32 and b1.grad.dtype == torch.bfloat16
    assert torch.equal(a1.grad, a2.grad) and torch.equal(b1.grad, b2.grad)


@pytest.mark.parametrize("n,c1,c2,h,w,up,a32,h32", [
    (4, 256, 256, 32, 32, True, False, False),   # decoder top level: bf16 act, bf16 skip
    (4, 256, 256, 16, 16, True, False, True),    # bf16 act, fp32 skip
    (3, 256, 256, 8, 8, True, True, True),
    (2, 256, 256, 4, 4, False, True, True),      # first decoder stage: no upsampling
    (2, 128, 64, 6, 10, True, True, False),      # odd channel split, non-square
])
def test_upsample_concat_bit_exact(n, c1, c2, h, w, up, a32, h32):
    """cat([F.interpolate(a, 2x nearest), h], 1) as the U-Net evaluates it under autocast
    (diffusion/unet.py:379-382): the fp32 output and both gradients (the upsampling's summed
    in torch's order, each cast to its operand's dtype) bit for bit."""
    g = torch.Generator().manual_seed(n * 100 + c1 + h)
    hl, wl = (h // 2, w // 2) if up else (h, w)
    a = torch.randn((n, c1, hl, wl), generator=g) * 2
    hh = torch.randn((n, c2, h, w), generator=g)
    gy = torch.randn((n, c1 + c2, h, w), generator=g) * 1e-2
    a = a.cuda().to(torch.float32 if a32 else torch.bfloat16).contiguous(memory_format=torch.channels_last)
    hh = hh.cuda().to(torch.float32 if h32 else torch.bfloat16).contiguous(memory_format=torch.channels_last)
    gy = gy.cuda().contiguous(memory_format=torch.channels_last)
    a1, h1 = a.clone().requires_grad_(), hh.clone().requires_grad_()
    a2, h2 = a.clone().requires_grad_(), hh.clone().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y1 = R.upsample_concat(a1, h1, up)
        x2 = torch.nn.functional.interpolate(a2, scale_factor=2.0, mode="nearest") if up else a2
        y2 = torch.concat([x2, h2], dim=1)
    assert y1.dtype == y2.dtype == torch.float32
    y1.backward(gy)
    y2.backward(gy)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert a1.grad.dtype == a.dtype and h1.grad.dtype == hh.dtype
    assert torch.equal(a1.grad, a2.grad) and torch.equal(h1.grad, h2.grad)


@pytest.mark.parametrize("n,c,h,w,a32", [(4, 128, 32, 32, False), (4, 256, 16, 16, True),
                                         (3, 256, 8, 8, True), (2, 64, 6, 10, False)])
def test_downsample2_bit_exact(n, c, h, w, a32):
    """F.interpolate(a, scale_factor=0.5, mode="nearest") under autocast (diffusion/unet.py:
    370-373): fp32 output and the input gradient (in a's dtype) bit for bit."""
    g = torch.Generator().manual_seed(n + c + h)
    a = (torch.randn((n, c, h, w), generator=g) * 2).cuda()
    a = a.to(torch.float32 if a32 else torch.bfloat16).contiguous(memory_format=torch.channels_last)
    gy = (torch.randn((n, c, h // 2, w // 2), generator=g) * 1e-2).cuda().contiguous(
        memory_format=torch.channels_last)
    a1, a2 = a.clone().requires_grad_(), a.clone().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y1 = R.downsample2(a1)
        y2 = torch.nn.functional.interpolate(a2, scale_factor=0.5, mode="nearest")
    assert y1.dtype == y2.dtype == torch.float32
    y1.backward(gy)
    y2.backward(gy)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert a1.grad.dtype == a.dtype and torch.equal(a1.grad, a2.grad)


@pytest.mark.parametrize("n,c,h,w,a32", [(4, 128, 32, 32, False), (4, 256, 16, 16, True),
                                         (3, 256, 8, 8, True), (2, 64, 6, 10, False)])
def test_downsample2_tee_equals_autograd_sum(n, c, h, w, a32):
    """An activation read by the downsampling and by a second consumer (the decoder's
    concatenation, diffusion/unet.py:368-376): the tee's input gradient, summed inside the
    downsampling's backward, equals interpolate + autograd's accumulation bit for bit,
    including the sign of zero where the second gradient is -0."""
    g = torch.Generator().manual_seed(3 * n + c + h + w)
    a = (torch.randn((n, c, h, w), generator=g) * 2).cuda()
    a = a.to(torch.float32 if a32 else torch.bfloat16).contiguous(memory_format=torch.channels_last)
    gy = (torch.randn((n, c, h // 2, w // 2), generator=g) * 1e-2).cuda().contiguous(
        memory_format=torch.channels_last)
    gs = (torch.randn((n, c, h, w), generator=g) * 1e-2).cuda().to(a.dtype)
    gs[0, 0] = -0.0  # -0 beside the downsampling's +0 off the sampled pixels
    gs = gs.contiguous(memory_format=torch.channels_last)
    a1, a2 = a.clone().requires_grad_(), a.clone().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y1, s1 = R.downsample2_tee(a1)
        y2 = torch.nn.functional.interpolate(a2, scale_factor=0.5, mode="nearest")
        s2 = a2
    assert y1.dtype == y2.dtype == torch.float32 and torch.equal(y1, y2)
    assert torch.equal(s1, a)
    torch.autograd.backward([y1, s1], [gy, gs])
    torch.autograd.backward([y2, s2], [gy, gs])
    torch.cuda.synchronize()
    assert a1.grad.dtype == a.dtype
    b1 = a1.grad.view(torch.int16 if a.dtype == torch.bfloat16 else torch.int32)
    b2 = a2.grad.view(torch.int16 if a.dtype == torch.bfloat16 else torch.int32)
    assert torch.equal(b1, b2)
    # only the downsampling's gradient (the skip copy unused): the plain backward
    a3 = a.clone().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y3, _ = R.downsample2_tee(a3)
    y3.backward(gy)
    a4 = a.clone().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y4 = R.downsample2(a4)
    y4.backward(gy)
    torch.cuda.synchronize()
    assert torch.equal(a3.grad, a4.grad)
