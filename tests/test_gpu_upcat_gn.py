"""A decoder stage's first GroupNorm+SiLU fused with the upsample-and-concatenate before it
(diffusion/unet.py:379-382 feeding :151): dpa_upcat_gn_silu_fwd / _bwd read the two bf16
sources where the fp32 concatenation would be read, and write the sources' gradients where its
gradient would be written. Each output and gradient must equal, bit for bit, the unfused path
it replaces -- dpa_upsample_concat_f32 (pinned against torch's interpolate + cat) followed by
the GroupNorm tee on the fp32 result (pinned against the float64 oracle) -- including the bf16
copy for the 1x1 skip conv, its amax partials and the FP8 hand-off bytes of conv_1's input.
"""
from __future__ import annotations

import pytest
import torch

from conftest import dpa_mod

pytestmark = pytest.mark.gpu

GROUPS = 32
K = dpa_mod("fp8_kernels")
G = dpa_mod("gn_silu")
R = dpa_mod("residual")

CASES = [
    # (n, channels of a (upsampled), channels of h, image side, h fp32)
    (3, 256, 256, 32, False),   # the U-Net's 32x32 decoder stage: 256 + 256, bf16
    (2, 128, 384, 32, False),
    (2, 64, 64, 32, False),     # C = 128: four channels per group
    (3, 256, 256, 16, True),    # the 16x16 stage: a bf16, h fp32
    (2, 128, 384, 16, True),
    (2, 128, 128, 16, False),   # h bf16 at 16x16
]


def cl(t):
    return t.cuda().contiguous(memory_format=torch.channels_last)


def inputs(n, ca, ch, seed, side=32, h32=False):
    g = torch.Generator().manual_seed(seed)
    a = cl((torch.randn((n, ca, side // 2, side // 2), generator=g) * 1.5 + 0.3).to(torch.bfloat16))
    h = torch.randn((n, ch, side, side), generator=g) * 0.7 - 0.2
    h = cl(h if h32 else h.to(torch.bfloat16))
    c = ca + ch
    gamma = (1.0 + 0.2 * torch.randn(c, generator=g)).cuda()
    beta = (0.1 * torch.randn(c, generator=g)).cuda()
    dout = cl((1e-2 * torch.randn((n, c, side, side), generator=g)).to(torch.bfloat16))
    dskip = cl((1e-2 * torch.randn((n, c, side, side), generator=g)).to(torch.bfloat16))
    return a, h, gamma, beta, dout, dskip


def run(fused: bool, a, h, gamma, beta, dout, dskip, hand=None):
    a, h = a.clone().requires_grad_(), h.clone().requires_grad_()
    gamma, beta = gamma.clone().requires_grad_(), beta.clone().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        if fused:
            assert G.upcat_ok(a, h, True)
            y, x16 = G.upcat_group_norm_silu_tee(a, h, gamma, beta, GROUPS, 1e-5, hand)
        else:
            x = R.upsample_concat(a, h, True)
            assert x.dtype == torch.float32  # autocast's fp32 interpolate and concatenation
            y, x16 = G.group_norm_silu_tee(x, gamma, beta, GROUPS, 1e-5, True, hand)
    rec = getattr(x16, "_dpa_amax", None)  # (partials, count, ...) its producer left
    parts = None if rec is None else rec[0][:rec[1]].clone()
    torch.autograd.backward([y, x16], [dout, dskip])
    torch.cuda.synchronize()
    return y, x16, parts, a.grad, h.grad, gamma.grad, beta.grad


@pytest.mark.parametrize("n,ca,ch,side,h32", CASES, ids=lambda v: str(v))
def test_upcat_gn_equals_upsample_concat_then_gn(n, ca, ch, side, h32):
    a, h, gamma, beta, dout, dskip = inputs(n, ca, ch, n * 7 + ca + ch + side, side, h32)
    got = run(True, a, h, gamma, beta, dout, dskip)
    ref = run(False, a, h, gamma, beta, dout, dskip)
    names = ["y", "x16", "x16 amax partials", "grad a", "grad h", "dgamma", "dbeta"]
    for name, g_, r_ in zip(names, got, ref):
        if g_ is None and r_ is None:
            continue
        assert g_.dtype == r_.dtype and g_.shape == r_.shape, name
        assert torch.equal(g_, r_), name
    # the skip path's gradient reaches both sources: without it the gradients differ
    bare = run(True, a, h, gamma, beta, dout, torch.zeros_like(dskip))
    assert not torch.equal(bare[3], got[3]) and not torch.equal(bare[4], got[4])


@pytest.mark.parametrize("side,h32", [(32, False), (16, True)], ids=lambda v: str(v))
def test_upcat_gn_fp8_handoff_equals_unfused(side, h32):
    """With conv_1's delayed-scaling hand-off the forward writes e4m3(y / scale) and the amax
    partials of y instead of y: the same bytes and partials as the unfused GroupNorm's
    hand-off on the fp32 concatenation."""
    n, ca, ch = 2, 256, 256
    a, h, gamma, beta, dout, dskip = inputs(n, ca, ch, 11, side, h32)

    def hand(scale):
        return K.Fp8Handoff(torch.tensor(scale, device="cuda", dtype=torch.float32),
                            torch.zeros(4096, device="cuda", dtype=torch.int32),
                            torch.zeros(1, device="cuda", dtype=torch.int32))

    for scale in (0.004, 2.0**-70):
        h1, h2 = hand(scale), hand(scale)
        got = run(True, a, h, gamma, beta, dout, dskip, h1)
        ref = run(False, a, h, gamma, beta, dout, dskip, h2)
        assert torch.equal(h1.q.view(torch.uint8), h2.q.view(torch.uint8)), scale
        cnt = int(h1.count.item())
        assert cnt == int(h2.count.item()) == (ca + ch) // 64 * n
        assert torch.equal(h1.partials[:cnt], h2.partials[:cnt])
        for name, g_, r_ in zip(["x16", "grad a", "grad h", "dgamma", "dbeta"],
                                got[1:2] + got[3:], ref[1:2] + ref[3:]):
            assert torch.equal(g_, r_), name


def test_upcat_gn_refuses_other_shapes():
    """Sizes without the fused form: the checker says no, the entry point refuses."""
    L = dpa_mod("_lib")
    a = cl(torch.zeros((1, 64, 4, 4), dtype=torch.bfloat16))
    h = cl(torch.zeros((1, 64, 8, 8), dtype=torch.bfloat16))
    assert not G.upcat_ok(a, h, True)            # 64-pixel images
    assert not G.upcat_ok(cl(torch.zeros((1, 64, 16, 16), dtype=torch.bfloat16)),
                          cl(torch.zeros((1, 64, 32, 32), dtype=torch.float32)), True)
    assert not G.upcat_ok(cl(torch.zeros((1, 64, 8, 8), dtype=torch.float32)),
                          cl(torch.zeros((1, 64, 16, 16), dtype=torch.float32)), True)
    assert not G.upcat_ok(a, h, False)
    dummy = torch.zeros(1 << 20, device="cuda", dtype=torch.float32)
    p = dummy.data_ptr()
    for hd, side in ((0, 8), (1, 32)):  # 8x8 images; an fp32 h at 32x32
        st = L.load().dpa_upcat_gn_silu_fwd(a.data_ptr(), h.data_ptr(), hd, 1, side, side, 64,
                                            64, p, p, p, None, None, None, 0, None, p, p, None,
                                            None, 0, GROUPS, 1e-5, None)
        assert st == -4  # DPA_ERR_SHAPE
