"""The image-channel convolutions (csrc/thinconv.hip): the U-Net's conv_in (3 -> C) and output
conv (C -> 3), diffusion/unet.py:255-257 and :325-329, which the reference runs in bf16 under
autocast (train.py:120, :136).

Oracle: float64 convolutions (torch on the CPU) of the bf16-rounded operands. The kernels
accumulate in fp32 and round once to bf16, so every output must lie within half a bf16 ulp of
the exact value plus the fp32 summation error (bounded by K * 2^-24 times the sum of the
magnitudes of the terms), and at least 99 % of them must equal the exact value rounded to
bf16. Weight gradients: fp32(bf16(sum)), the same bound. Then the module under autocast
against nn.Conv2d's own bf16 path (MIOpen), a full cfg5-size step, and graph replays.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from conftest import dpa_mod

pytestmark = pytest.mark.gpu

T = dpa_mod("thinconv")


def cl(t):
    return t.contiguous(memory_format=torch.channels_last)


def bf(t):
    return t.to(torch.bfloat16).double()


def check_close(ours, exact, abs_sum, k, what):
    """ours vs the exact float64 result: half a bf16 ulp + the fp32 summation bound, and
    >= 99 % equal to bf16(exact)."""
    ours = ours.double().cpu()
    exact = exact.cpu()
    bound = exact.abs() * 2.0**-8 + abs_sum.cpu() * (k * 2.0**-24) + 1e-30
    err = (ours - exact).abs()
    assert bool((err <= bound).all()), (what, float((err / bound).max()))
    same = (ours == exact.to(torch.bfloat16).double()).double().mean().item()
    assert same >= 0.99, (what, same)


def grads_exact(x64, w64, gy64):
    dx = torch.nn.grad.conv2d_input(x64.shape, w64, gy64, padding=1)
    dw = torch.nn.grad.conv2d_weight(x64, w64.shape, gy64, padding=1)
    adx = torch.nn.grad.conv2d_input(x64.shape, w64.abs(), gy64.abs(), padding=1)
    adw = torch.nn.grad.conv2d_weight(x64.abs(), w64.shape, gy64.abs(), padding=1)
    return dx, dw, adx, adw


CASES = [  # (n, cin, cout, h, w, x fp32)
    (4, 3, 128, 32, 32, True),     # conv_in, fp32 image under autocast
    (4, 3, 128, 32, 32, False),
    (2, 1, 256, 16, 16, True),
    (4, 2, 128, 16, 16, False),
    (4, 128, 3, 32, 32, False),    # the output head's conv
    (2, 256, 3, 16, 16, False),
    (4, 128, 1, 32, 32, False),
    (1, 128, 2, 2, 64, False),
]


@pytest.mark.parametrize("n,cin,cout,h,w,xf32", CASES)
def test_thin_conv_vs_float64(n, cin, cout, h, w, xf32):
    print(f"thin conv n={n} cin={cin} cout={cout} {h}x{w} xf32={xf32}", flush=True)
    g = torch.Generator().manual_seed(n * 1000 + cin * 7 + cout)
    x = torch.randn((n, cin, h, w), generator=g)
    wt = torch.randn((cout, cin, 3, 3), generator=g) / (3 * cin) ** 0.5
    gy = torch.randn((n, cout, h, w), generator=g)
    x_dev = cl(x.cuda() if xf32 else x.cuda().to(torch.bfloat16)).requires_grad_(cin > 3)
    w_dev = cl(wt.cuda()).requires_grad_()
    y = T.ThinConv2dFunction.apply(x_dev, w_dev)
    assert y.dtype == torch.bfloat16 and y.is_contiguous(memory_format=torch.channels_last)
    y.backward(cl(gy.cuda().to(torch.bfloat16)))
    torch.cuda.synchronize()

    x64, w64, gy64 = bf(x), bf(wt), bf(gy)
    k = 9 * cin
    exact = F.conv2d(x64, w64, padding=1)
    check_close(y, exact, F.conv2d(x64.abs(), w64.abs(), padding=1), k, "y")
    dx, dw, adx, adw = grads_exact(x64, w64, gy64)
    assert w_dev.grad.dtype == torch.float32
    check_close(w_dev.grad, dw, adw, n * h * w, "dw")
    if cin > 3:
        assert x_dev.grad.dtype == torch.bfloat16
        check_close(x_dev.grad, dx, adx, 9 * cout, "dx")


def test_weight_strides_contiguous_and_channels_last():
    """The kernels read the weight at its own element strides."""
    g = torch.Generator().manual_seed(5)
    x = cl(torch.randn((2, 128, 32, 32), generator=g).cuda().to(torch.bfloat16))
    wt = torch.randn((3, 128, 3, 3), generator=g).cuda() / 34.0
    ya = T.ThinConv2dFunction.apply(x, wt.contiguous())
    yb = T.ThinConv2dFunction.apply(x, cl(wt))
    assert torch.equal(ya, yb)


def test_shape_gate():
    assert T.shape_ok(128, 3, 128, 32, 32) and T.shape_ok(128, 128, 3, 32, 32)
    assert not T.shape_ok(128, 3, 64, 32, 32)      # wide side 128 or 256
    assert not T.shape_ok(128, 4, 128, 32, 32)     # thin side 1-3
    assert not T.shape_ok(128, 3, 128, 30, 30)     # W in {16, 32, 64}
    assert not T.shape_ok(128, 128, 3, 31, 32)     # H a multiple of 64 / W


def _module_pair(cin, cout, seed):
    torch.manual_seed(seed)
    m = T.ImageConv2d(cin, cout, (3, 3), padding=1, bias=False).cuda()
    m = m.to(memory_format=torch.channels_last)
    ref = torch.nn.Conv2d(cin, cout, (3, 3), padding=1, bias=False).cuda()
    ref = ref.to(memory_format=torch.channels_last)
    with torch.no_grad():
        ref.weight.copy_(m.weight)
    return m, ref


@pytest.mark.parametrize("cin,cout", [(3, 128), (128, 3)])
def test_module_under_autocast_vs_torch_conv(cin, cout):
    """ImageConv2d at cfg5 size (batch 128, 32x32) under bf16 autocast against nn.Conv2d's
    own bf16 path: the same dtypes and layouts, outputs and gradients within one bf16 ulp
    (both accumulate in fp32, in different orders)."""
    print(f"module {cin}->{cout}", flush=True)
    m, ref = _module_pair(cin, cout, 11)
    g = torch.Generator().manual_seed(12)
    x0 = torch.randn((128, cin, 32, 32), generator=g)
    gy = cl(torch.randn((128, cout, 32, 32), generator=g).cuda().to(torch.bfloat16))
    outs = []
    for mod in (m, ref):
        if cin == 3:
            x = cl(x0.cuda())                         # the fp32 image
        else:
            x = cl(x0.cuda().to(torch.bfloat16)).requires_grad_()
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = mod(x)
        y.backward(gy)
        outs.append((y, x.grad, mod.weight.grad))
    torch.cuda.synchronize()
    (ya, dxa, dwa), (yb, dxb, dwb) = outs
    assert ya.dtype == yb.dtype == torch.bfloat16
    assert dwa.dtype == dwb.dtype == torch.float32
    ulp = 2.0**-7
    assert float((ya.float() - yb.float()).abs().max()) <= ulp * float(yb.float().abs().max())
    rel = float((dwa - dwb).norm() / dwb.norm())
    assert rel < 4e-3, rel
    if dxb is not None:
        assert dxa.dtype == torch.bfloat16
        assert float((dxa.float() - dxb.float()).abs().max()) <= ulp * float(dxb.float().abs().max())


def test_forward_is_batch_independent():
    """Forward and data gradient are per pixel: the first images of a batch-128 call equal a
    batch-4 call bit for bit."""
    g = torch.Generator().manual_seed(21)
    x = cl(torch.randn((128, 128, 32, 32), generator=g).cuda().to(torch.bfloat16))
    wt = cl(torch.randn((3, 128, 3, 3), generator=g).cuda() / 34.0)
    y_all = T.ThinConv2dFunction.apply(x, wt)
    y_4 = T.ThinConv2dFunction.apply(cl(x[:4]), wt)
    assert torch.equal(y_all[:4], y_4)
    xi = cl(torch.randn((128, 3, 32, 32), generator=g).cuda())
    wi = cl(torch.randn((128, 3, 3, 3), generator=g).cuda() / 5.0)
    assert torch.equal(T.ThinConv2dFunction.apply(xi, wi)[:4],
                       T.ThinConv2dFunction.apply(cl(xi[:4]), wi))


def test_graph_replays_match_eager():
    """Captured forward + backward of both convs replayed several times, with eager work in
    between: every replay equals the eager results (no memset nodes, deterministic sums)."""
    mi, _ = _module_pair(3, 128, 31)
    mo, _ = _module_pair(128, 3, 32)
    g = torch.Generator().manual_seed(33)
    x = cl(torch.randn((32, 3, 32, 32), generator=g).cuda())
    gy = cl(torch.randn((32, 3, 32, 32), generator=g).cuda().to(torch.bfloat16))

    def step():
        for p in (mi.weight, mo.weight):
            p.grad = None
        with torch.autocast("cuda", dtype=torch.bfloat16):
            h = mi(x)
            y = mo(h)
        y.backward(gy)
        return y.detach().clone(), mi.weight.grad.clone(), mo.weight.grad.clone()

    eager = step()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step()
    for _ in range(3):
        _ = torch.randn((1024, 1024), device="cuda") @ torch.randn((1024, 1024), device="cuda")
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(static, eager):
            assert torch.equal(a, b)
