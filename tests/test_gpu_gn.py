"""GPU parity of the fused GroupNorm(+FiLM)+SiLU forward/backward against the float64 oracle.

The reference runs GroupNorm and SiLU in float32 under autocast (diffusion/unet.py:151,
:157-159) and the FP8 conv then rounds the result to bf16 (diffusion/fp8_kernels.py:835). The
fused kernel emits that bf16 directly. Against the float64 oracle, a float32 evaluation may
land on the other side of a bf16 rounding boundary, so the forward bar is one bf16 ulp, with
almost every element bit-identical. Gradients are float32 reductions: normwise 1e-4 for the
parameter gradients and the conv tolerance (one bf16 ulp + noise) for dx.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import assert_bf16_close, dpa_mod, dropout_band, nhwc_bits, randn_bf16
from oracle import fp8_oracle as O

pytestmark = pytest.mark.gpu

GROUPS = 32


@pytest.fixture(scope="module")
def G():
    return dpa_mod("gn_silu")


def cl(t):
    return t.cuda().contiguous(memory_format=torch.channels_last)


def params(c, n, seed, film):
    g = torch.Generator().manual_seed(seed)
    gamma = 1.0 + 0.1 * torch.randn(c, generator=g)
    beta = 0.1 * torch.randn(c, generator=g)
    fs = fb = None
    if film:
        fs = 1.0 + 0.2 * torch.randn(n, c, generator=g)   # the reference's (w + 1)
        fb = 0.2 * torch.randn(n, c, generator=g)
    return gamma, beta, fs, fb


def assert_fwd_close(got_bits, ref_bits, what):
    g = O.bf16_bits_to_f32(got_bits).astype(np.float64)
    r = O.bf16_bits_to_f32(ref_bits).astype(np.float64)
    assert np.isfinite(g).all(), what
    # one bf16 ulp of the reference (at most 2^-7 |r|) plus float32 noise near zero
    bad = np.abs(g - r) > 2.0**-7 * np.abs(r) + 1e-6
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond 1 bf16 ulp"
    exact = float(np.mean(got_bits == ref_bits))
    assert exact > 0.995, f"{what}: only {exact:.4f} bit-identical"


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


CASES = [
    # (n, c, h, w, film): the reference U-Net's GroupNorm sites at reduced batch
    (2, 128, 32, 32, False),
    (2, 256, 16, 16, True),
    (2, 512, 8, 8, False),
    (3, 256, 4, 4, True),
    (2, 256, 7, 9, True),    # ragged pixel count
    (2, 128, 17, 19, True),  # chunked form with a ragged last chunk (323 = 128 + 128 + 67)
    (1, 128, 5, 3, False),
]


@pytest.mark.parametrize("n,c,h,w,film", CASES, ids=lambda v: str(v))
def test_gn_silu_fwd_bwd_vs_oracle(G, n, c, h, w, film):
    if not G.supported(c, GROUPS):
        pytest.skip(f"C={c}, G={GROUPS} outside the fused kernel's shapes")
    seed = n * 1000 + c + h
    x = randn_bf16((n, c, h, w), seed=seed, std=2.0)
    x = (x.float() + 0.5).to(torch.bfloat16)      # non-zero group means
    dout = randn_bf16((n, c, h, w), seed=seed + 1, std=1e-2)
    gamma, beta, fs, fb = params(c, n, seed + 2, film)
    fs_d = None if fs is None else fs.cuda()[:, :, None, None]
    fb_d = None if fb is None else fb.cuda()[:, :, None, None]

    out, mean, rstd = G.gn_silu_fwd(cl(x), gamma.cuda(), beta.cuda(), GROUPS, 1e-5, fs_d, fb_d)
    dx, dgamma, dbeta, dfs, dfb = G.gn_silu_bwd(
        cl(x), cl(dout), gamma.cuda(), beta.cuda(), mean, rstd, GROUPS, fs_d, fb_d)
    torch.cuda.synchronize()

    xb = nhwc_bits(x)
    npf = None if fs is None else fs.numpy()
    npb = None if fb is None else fb.numpy()
    ref = O.gn_silu_fwd(xb, gamma.numpy(), beta.numpy(), GROUPS, 1e-5, npf, npb)
    assert out.is_contiguous(memory_format=torch.channels_last) and out.dtype == torch.bfloat16
    assert_fwd_close(nhwc_bits(out.cpu()), ref, f"fwd {(n, c, h, w, film)}")

    # group statistics
    xg = O.bf16_bits_to_f32(xb).astype(np.float64).reshape(n, h * w, GROUPS, c // GROUPS)
    m_ref = xg.mean(axis=(1, 3))
    v_ref = xg.var(axis=(1, 3))
    assert rel(mean.cpu().numpy().reshape(n, GROUPS), m_ref) < 1e-5
    assert rel(rstd.cpu().numpy().reshape(n, GROUPS), 1 / np.sqrt(v_ref + 1e-5)) < 1e-5

    rdx, rdg, rdb, rdfs, rdfb = O.gn_silu_bwd(xb, nhwc_bits(dout), gamma.numpy(), beta.numpy(),
                                             GROUPS, 1e-5, npf, npb)
    assert_bf16_close(nhwc_bits(dx.cpu()), O.f32_to_bf16_bits(rdx.astype(np.float32)),
                      f"dx {(n, c, h, w, film)}")
    assert rel(dgamma.cpu().numpy(), rdg) < 1e-4
    assert rel(dbeta.cpu().numpy(), rdb) < 1e-4
    if film:
        assert rel(dfs.cpu().numpy(), rdfs) < 1e-4
        assert rel(dfb.cpu().numpy(), rdfb) < 1e-4
    else:
        assert dfs is None and dfb is None


def test_gn_silu_cfg4_full_size_vs_torch_fp32(G):
    """cfg4's norm2 site at full size ([128,256,16,16] with FiLM) through the autograd
    Function, against torch float32 GroupNorm+SiLU on the GPU."""
    n, c, h, w = 128, 256, 16, 16
    x = cl(randn_bf16((n, c, h, w), seed=0))
    gamma, beta, fs, fb = params(c, n, 3, True)
    gamma, beta = gamma.cuda().requires_grad_(), beta.cuda().requires_grad_()
    fs = fs.cuda()[:, :, None, None].requires_grad_()
    fb = fb.cuda()[:, :, None, None].requires_grad_()
    dout = cl(randn_bf16((n, c, h, w), seed=1, std=1e-2))

    xa = x.clone().requires_grad_()
    out = G.group_norm_silu(xa, gamma, beta, GROUPS, 1e-5, fs, fb)
    out.backward(dout)

    xr = x.float().clone().requires_grad_()
    gr, br = gamma.detach().clone().requires_grad_(), beta.detach().clone().requires_grad_()
    fsr, fbr = fs.detach().clone().requires_grad_(), fb.detach().clone().requires_grad_()
    ref = F.silu(fsr * F.group_norm(xr, GROUPS, gr, br, 1e-5) + fbr)
    ref.backward(dout.float())
    torch.cuda.synchronize()

    def nerr(a, b):
        a, b = a.detach().float(), b.detach().float()
        return float((a - b).norm() / b.norm())

    assert out.dtype == torch.bfloat16
    assert nerr(out, ref) < 2**-8
    assert nerr(xa.grad, xr.grad) < 1e-2
    assert xa.grad.dtype == torch.bfloat16
    for got, want in ((gamma.grad, gr.grad), (beta.grad, br.grad), (fs.grad, fsr.grad),
                      (fb.grad, fbr.grad)):
        assert got.shape == want.shape
        assert nerr(got, want) < 1e-3


@pytest.mark.parametrize("n,c,h,w", [(3, 256, 16, 16), (2, 128, 32, 32), (2, 512, 8, 8)])
def test_gn_silu_film_from_time_projection_matches_split_form(G, n, c, h, w):
    """GroupNormSiLUFilm (the kernel reads wb = [w | b] in bf16 and forms bf16(w + 1)) equals
    GroupNormSiLU on the reference's w + 1 and b (diffusion/unet.py:157-159) bit for bit:
    output, dx, dgamma, dbeta, and d(wb) = [d(w + 1) | d(b)] in bf16."""
    g = torch.Generator().manual_seed(n + c)
    x = (torch.randn((n, c, h, w), generator=g) * 2 + 0.5).to(torch.bfloat16)
    gamma, beta, _, _ = params(c, n, c + 1, False)
    wb = (0.3 * torch.randn((n, 2 * c, 1, 1), generator=g)).to(torch.bfloat16).cuda()
    dout = randn_bf16((n, c, h, w), seed=c + 7)

    xa = cl(x).requires_grad_()
    ga, ba = gamma.cuda().requires_grad_(), beta.cuda().requires_grad_()
    wba = wb.clone().requires_grad_()
    ya = G.group_norm_silu_film(xa, ga, ba, GROUPS, 1e-5, wba)
    ya.backward(cl(dout))

    xb = cl(x).requires_grad_()
    gb, bb = gamma.cuda().requires_grad_(), beta.cuda().requires_grad_()
    wbb = wb.clone().requires_grad_()
    wpart, bpart = torch.chunk(wbb, 2, dim=1)
    yb = G.group_norm_silu(xb, gb, bb, GROUPS, 1e-5, wpart + 1, bpart)
    yb.backward(cl(dout))
    torch.cuda.synchronize()
    for got, ref, what in ((ya, yb, "out"), (xa.grad, xb.grad, "dx"), (ga.grad, gb.grad, "dgamma"),
                           (ba.grad, bb.grad, "dbeta"), (wba.grad, wbb.grad, "dwb")):
        assert got.dtype == ref.dtype and got.shape == ref.shape, what
        assert torch.equal(got.detach(), ref.detach()), what


@pytest.mark.parametrize("n,c,h,w,film", [(2, 128, 40, 40, True), (1, 256, 36, 36, False)])
def test_one_launch_and_chunked_forms_agree(G, n, c, h, w, film):
    """Images above 1024 pixels (beyond the resident form) run the chunked kernels when given
    the full workspace; the one-launch kernels (no forward workspace, a backward workspace of
    only the per-image partials) compute the same quantities with another summation order."""
    L = dpa_mod("_lib")
    x = cl(randn_bf16((n, c, h, w), seed=n + c, std=2.0))
    dout = cl(randn_bf16((n, c, h, w), seed=n + c + 1, std=1e-2))
    gamma, beta, fs, fb = params(c, n, c, film)
    gamma, beta = gamma.cuda(), beta.cuda()
    fs = None if fs is None else fs.cuda().contiguous()
    fb = None if fb is None else fb.cuda().contiguous()
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    s = torch.cuda.current_stream().cuda_stream
    hw = h * w
    assert L.query("dpa_gn_silu_fwd_workspace_bytes", n, hw, c, GROUPS) > 0
    res = {}
    for form in ("chunked", "one"):
        out = torch.empty_like(x)
        mean = torch.empty(n * GROUPS, device="cuda")
        rstd = torch.empty(n * GROUPS, device="cuda")
        if form == "chunked":
            wsb = L.query("dpa_gn_silu_fwd_workspace_bytes", n, hw, c, GROUPS)
            ws = torch.empty(wsb, device="cuda", dtype=torch.uint8)
            L.call("dpa_gn_silu_fwd_ws_bf16", x.data_ptr(), gamma.data_ptr(), beta.data_ptr(),
                   p(fs), p(fb), None, out.data_ptr(), mean.data_ptr(), rstd.data_ptr(),
                   ws.data_ptr(), wsb, n, hw, c, GROUPS, 1e-5, s)
            bws = L.query("dpa_gn_silu_bwd_workspace_bytes", n, hw, c, GROUPS)
        else:
            L.call("dpa_gn_silu_fwd_bf16", x.data_ptr(), gamma.data_ptr(), beta.data_ptr(),
                   p(fs), p(fb), out.data_ptr(), mean.data_ptr(), rstd.data_ptr(), n, hw, c,
                   GROUPS, 1e-5, s)
            bws = 2 * n * c * 4
        dx = torch.empty_like(x)
        dg = torch.empty(c, device="cuda")
        db = torch.empty(c, device="cuda")
        dfs = torch.empty((n, c), device="cuda") if film else None
        dfb = torch.empty((n, c), device="cuda") if film else None
        ws = torch.empty(bws, device="cuda", dtype=torch.uint8)
        L.call("dpa_gn_silu_bwd_bf16", x.data_ptr(), dout.data_ptr(), gamma.data_ptr(),
               beta.data_ptr(), p(fs), p(fb), mean.data_ptr(), rstd.data_ptr(), dx.data_ptr(),
               dg.data_ptr(), db.data_ptr(), p(dfs), p(dfb), ws.data_ptr(), bws, n, hw, c,
               GROUPS, s)
        torch.cuda.synchronize()
        res[form] = [t.cpu() for t in (out, mean, rstd, dx, dg, db)] + (
            [dfs.cpu(), dfb.cpu()] if film else [])
    a, b = res["chunked"], res["one"]
    assert_fwd_close(nhwc_bits(a[0]), nhwc_bits(b[0]), "out")
    assert rel(a[1].numpy(), b[1].numpy()) < 1e-5 and rel(a[2].numpy(), b[2].numpy()) < 1e-5
    assert_bf16_close(nhwc_bits(a[3]), nhwc_bits(b[3]), "dx")
    for k in range(4, len(a)):
        assert rel(a[k].numpy(), b[k].numpy()) < 1e-4, k


F32_CASES = [
    # fp32 inputs (the fp32 residual stream / decoder concatenations): resident, chunked and
    # small forms; 1024 pixels without FiLM (the decoder's first GroupNorm) is resident
    (2, 128, 32, 32, False),
    (2, 512, 32, 32, False),
    (2, 128, 32, 32, True),  # 1024 pixels with FiLM: chunked
    (2, 256, 16, 16, True),
    (2, 512, 8, 8, False),
    (3, 256, 4, 4, True),
    (2, 128, 17, 19, True),  # chunked, ragged last chunk
]


@pytest.mark.parametrize("n,c,h,w,film", F32_CASES, ids=lambda v: str(v))
def test_gn_silu_fp32_input_vs_oracle(G, n, c, h, w, film):
    """An fp32 x is normalised as it is (autocast's float32 GroupNorm, diffusion/unet.py:151,
    :157) and dx comes back in fp32: forward within one bf16 ulp of the float64 oracle on the
    fp32 values, dx normwise 2e-5 of the oracle's float64 gradient."""
    seed = n * 1000 + c + h + 7
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((n, c, h, w), generator=g) * 2.0 + 0.5     # fp32, not bf16-representable
    dout = randn_bf16((n, c, h, w), seed=seed + 1, std=1e-2)
    gamma, beta, fs, fb = params(c, n, seed + 2, film)
    fs_d = None if fs is None else fs.cuda()[:, :, None, None]
    fb_d = None if fb is None else fb.cuda()[:, :, None, None]
    xd = cl(x)
    assert G.f32_input_ok(xd)
    out, mean, rstd = G.gn_silu_fwd(xd, gamma.cuda(), beta.cuda(), GROUPS, 1e-5, fs_d, fb_d)
    dx, dgamma, dbeta, dfs, dfb = G.gn_silu_bwd(
        xd, cl(dout), gamma.cuda(), beta.cuda(), mean, rstd, GROUPS, fs_d, fb_d)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and dx.dtype == torch.float32
    x_nhwc = x.permute(0, 2, 3, 1).contiguous().numpy()
    npf = None if fs is None else fs.numpy()
    npb = None if fb is None else fb.numpy()
    ref = O.gn_silu_fwd(x_nhwc, gamma.numpy(), beta.numpy(), GROUPS, 1e-5, npf, npb)
    assert_fwd_close(nhwc_bits(out.cpu()), ref, f"fp32 fwd {(n, c, h, w, film)}")
    # the bf16-rounded input would miss: normalising bf16(x) differs from the oracle here
    ref_b = O.gn_silu_fwd(nhwc_bits(x.to(torch.bfloat16)), gamma.numpy(), beta.numpy(), GROUPS,
                          1e-5, npf, npb)
    assert np.mean(ref_b != ref) > 0.05
    rdx, rdg, rdb, rdfs, rdfb = O.gn_silu_bwd(x_nhwc, nhwc_bits(dout), gamma.numpy(),
                                             beta.numpy(), GROUPS, 1e-5, npf, npb)
    got = dx.permute(0, 2, 3, 1).contiguous().cpu().numpy()
    assert rel(got, rdx) < 2e-5, rel(got, rdx)
    assert rel(dgamma.cpu().numpy(), rdg) < 1e-4
    assert rel(dbeta.cpu().numpy(), rdb) < 1e-4
    if film:
        assert rel(dfs.cpu().numpy(), rdfs) < 1e-4
        assert rel(dfb.cpu().numpy(), rdfb) < 1e-4


def test_gn_silu_fp32_autograd_and_fallback(G):
    """Through the autograd Functions: an fp32 input keeps an fp32 gradient, equal to the
    direct calls; a size outside the fp32 forms (96 x 96 = 9216 pixels) is cast to bf16 first,
    as before; the time-projection FiLM form takes fp32 x too."""
    n, c, groups = 2, 256, GROUPS
    g = torch.Generator().manual_seed(11)
    gamma, beta = (1.0 + 0.1 * torch.randn(c, generator=g)).cuda(), (0.1 * torch.randn(c, generator=g)).cuda()
    for h in (16, 96):
        x = cl(torch.randn((n, c, h, h), generator=g) * 1.5)
        xr = x.clone().requires_grad_(True)
        y = G.group_norm_silu(xr, gamma, beta, groups, 1e-5)
        dout = cl(torch.randn((n, c, h, h), generator=g) * 1e-2).to(torch.bfloat16)
        y.backward(dout)
        assert xr.grad.dtype == torch.float32
        if h == 16:
            assert G.f32_input_ok(x)
            out, mean, rstd = G.gn_silu_fwd(x, gamma, beta, groups, 1e-5)
            dx = G.gn_silu_bwd(x, dout, gamma, beta, mean, rstd, groups)[0]
        else:
            assert not G.f32_input_ok(x)
            xb = x.to(torch.bfloat16)
            out, mean, rstd = G.gn_silu_fwd(xb, gamma, beta, groups, 1e-5)
            dx = G.gn_silu_bwd(xb, dout, gamma, beta, mean, rstd, groups)[0].float()
        torch.cuda.synchronize()
        assert torch.equal(y, out), h
        assert torch.equal(xr.grad, dx), h
    # FiLM read from the bf16 time projection, fp32 x: equals the split form on the same x
    h = 16
    x = cl(torch.randn((n, c, h, h), generator=g))
    wb = (torch.randn((n, 2 * c, 1, 1), generator=g) * 0.2).cuda().to(torch.bfloat16)
    xr = x.clone().requires_grad_(True)
    y = G.group_norm_silu_film(xr, gamma, beta, groups, 1e-5, wb)
    w, b = torch.chunk(wb, 2, dim=1)
    x2 = x.clone().requires_grad_(True)
    y2 = G.group_norm_silu(x2, gamma, beta, groups, 1e-5, (w + 1).float(), b.float())
    dout = cl(torch.randn((n, c, h, h), generator=g) * 1e-2).to(torch.bfloat16)
    y.backward(dout)
    y2.backward(dout)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    assert xr.grad.dtype == torch.float32 and torch.equal(xr.grad, x2.grad)


DROP_CASES = [
    # (n, c, h, w, x fp32): chunked (bf16 and fp32 x) and small-image forms
    (2, 128, 32, 32, True),
    (3, 256, 16, 16, False),
    (2, 512, 8, 8, True),
    (4, 256, 4, 4, False),
]


@pytest.mark.parametrize("n,c,h,w,x32", DROP_CASES, ids=lambda v: str(v))
def test_gn_silu_film_dropout_vs_oracle(G, n, c, h, w, x32):
    """The dropout of diffusion/unet.py:160 fused into GroupNormSiLUFilm: the mask is the
    oracle's splitmix64 mask of the seed the op draws (reproduced from the same torch CUDA
    generator state), kept values are scaled by RN32(1 / RN32(1 - p)) in fp32 before the bf16
    rounding; the backward recomputes the mask. Forward within one bf16 ulp of the float64
    oracle, exact zeros off the mask, keep rate within 5 sigma of 1 - p; gradients against
    the oracle's masked backward."""
    p = 0.2
    seed = n * 977 + c + h
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((n, c, h, w), generator=g) * 2.0 + 0.5
    if not x32:
        x = x.to(torch.bfloat16)
    gamma, beta, _, _ = params(c, n, seed + 2, False)
    wb = (0.3 * torch.randn((n, 2 * c, 1, 1), generator=g)).to(torch.bfloat16)
    dout = randn_bf16((n, c, h, w), seed=seed + 1, std=1e-2)

    torch.cuda.manual_seed(seed)
    drop_seed = int(G.new_dropout_seed("cuda").item())
    torch.cuda.manual_seed(seed)
    xd = cl(x).requires_grad_()
    gd, bd = gamma.cuda().requires_grad_(), beta.cuda().requires_grad_()
    wbd = wb.cuda().requires_grad_()
    y = G.group_norm_silu_film(xd, gd, bd, GROUPS, 1e-5, wbd, p)
    y.backward(cl(dout))
    torch.cuda.synchronize()

    x_nhwc = (x.float() if x32 else x).permute(0, 2, 3, 1).contiguous()
    x_in = x_nhwc.numpy() if x32 else nhwc_bits(x)
    wb32 = wb.float().reshape(n, 2 * c)
    fs = (wb32[:, :c].to(torch.bfloat16).float() + 1).to(torch.bfloat16).float().numpy()
    fb = wb32[:, c:].numpy()
    keep = O.dropout_keep(drop_seed, n * h * w * c, p)
    rate = keep.mean()
    assert abs(rate - (1 - p)) < 5 * np.sqrt(p * (1 - p) / keep.size), rate
    ref = O.gn_silu_fwd(x_in, gamma.numpy(), beta.numpy(), GROUPS, 1e-5, fs, fb, drop=(drop_seed, p))
    got = nhwc_bits(y.detach().cpu())
    assert (got.reshape(-1)[~keep] == 0).all()
    assert_fwd_close(got, ref, f"dropout fwd {(n, c, h, w, x32)}")
    rdx, rdg, rdb, rdfs, rdfb = O.gn_silu_bwd(x_in, nhwc_bits(dout), gamma.numpy(), beta.numpy(),
                                             GROUPS, 1e-5, fs, fb, drop=(drop_seed, p))
    # without the mask the gradient would be far off
    rdx0 = O.gn_silu_bwd(x_in, nhwc_bits(dout), gamma.numpy(), beta.numpy(), GROUPS, 1e-5, fs, fb)[0]
    assert rel(rdx0, rdx) > 0.1
    got_dx = xd.grad.float().permute(0, 2, 3, 1).contiguous().cpu().numpy()
    assert xd.grad.dtype == x.dtype
    assert rel(got_dx, rdx) < (2e-5 if x32 else 4e-3), rel(got_dx, rdx)
    assert rel(gd.grad.cpu().numpy(), rdg) < 1e-4
    assert rel(bd.grad.cpu().numpy(), rdb) < 1e-4
    dwb = wbd.grad.float().reshape(n, 2 * c).cpu().numpy()
    assert rel(dwb[:, :c], rdfs) < 4e-3
    assert rel(dwb[:, c:], rdfb) < 4e-3


@pytest.mark.parametrize("n,c,h,w,x32", [(1, 256, 16, 16, False), (1, 256, 8, 8, True)],
                         ids=lambda v: str(v))
def test_gn_silu_film_dropout_threshold_band(G, n, c, h, w, x32):
    """The keep threshold is floor(fp32(p) * 2^16). With p = 13107 / 2^16 - 2^-40 (fp32 value
    13107 / 2^16) a hash quarter of 13106 = floor(p * 2^16) must be dropped: the seed is built
    (by inverting splitmix64) so that element 0's quarter is that value. The kernel's whole
    mask, forward and backward, equals the oracle's."""
    p, seed, _ = dropout_band()
    g = torch.Generator().manual_seed(9)
    x = torch.randn((n, c, h, w), generator=g) + 0.5
    if not x32:
        x = x.to(torch.bfloat16)
    gamma, beta, _, _ = params(c, n, 10, False)
    wb = (0.3 * torch.randn((n, 2 * c, 1, 1), generator=g)).to(torch.bfloat16)
    G.DROPOUT_SEEDS.seeds = torch.tensor([seed], device="cuda", dtype=torch.int64)
    G.DROPOUT_SEEDS.next = 0
    try:
        xd = cl(x).requires_grad_()
        y = G.group_norm_silu_film(xd, gamma.cuda(), beta.cuda(), GROUPS, 1e-5, wb.cuda(), p)
        assert G.DROPOUT_SEEDS.next == 1  # the op took the planted seed
    finally:
        G.DROPOUT_SEEDS.clear()
    y.backward(torch.ones_like(y))
    torch.cuda.synchronize()
    keep = O.dropout_keep(seed, n * h * w * c, p)
    assert not keep[0] and keep[1]
    got = nhwc_bits(y.detach().cpu()).reshape(-1)
    undropped = G.group_norm_silu_film(cl(x), gamma.cuda(), beta.cuda(), GROUPS, 1e-5,
                                       wb.cuda(), 0.0)
    ub = nhwc_bits(undropped.cpu()).reshape(-1)
    assert ub[0] & 0x7FFF != 0  # element 0 is nonzero before dropout, zero after
    assert got[0] & 0x7FFF == 0
    assert np.array_equal((got & 0x7FFF) == 0, (~keep) | ((ub & 0x7FFF) == 0))
    gx = xd.grad.float().permute(0, 2, 3, 1).contiguous().reshape(-1).cpu().numpy()
    assert np.isfinite(gx).all()


def test_gn_silu_film_dropout_zero_p_and_fresh_masks(G):
    """p = 0 gives the undropped op bit for bit; two calls draw two seeds (different masks);
    a size without a dropout form (96 x 96) is refused rather than silently undropped."""
    n, c, h, w = 2, 256, 16, 16
    g = torch.Generator().manual_seed(5)
    x = cl((torch.randn((n, c, h, w), generator=g) + 0.5).to(torch.bfloat16))
    gamma, beta, _, _ = params(c, n, 6, False)
    wb = (0.3 * torch.randn((n, 2 * c, 1, 1), generator=g)).to(torch.bfloat16).cuda()
    a = G.group_norm_silu_film(x, gamma.cuda(), beta.cuda(), GROUPS, 1e-5, wb, 0.0)
    b = G.group_norm_silu_film(x, gamma.cuda(), beta.cuda(), GROUPS, 1e-5, wb)
    assert torch.equal(a, b)
    d1 = G.group_norm_silu_film(x, gamma.cuda(), beta.cuda(), GROUPS, 1e-5, wb, 0.5)
    d2 = G.group_norm_silu_film(x, gamma.cuda(), beta.cuda(), GROUPS, 1e-5, wb, 0.5)
    z1, z2 = (d1 == 0) & (a != 0), (d2 == 0) & (a != 0)
    assert 0.45 < z1.float().mean().item() < 0.55
    assert not torch.equal(z1, z2)
    x96 = cl(torch.randn((n, c, 96, 96), generator=g).to(torch.bfloat16))
    with pytest.raises(ValueError):  # 9216 pixels: no form with fused dropout
        G.group_norm_silu_film(x96, gamma.cuda(), beta.cuda(), GROUPS, 1e-5, wb, 0.5)


@pytest.mark.parametrize("n,c,h,w,x32", [(2, 128, 32, 32, True), (3, 256, 16, 16, False),
                                         (2, 512, 8, 8, True), (4, 256, 4, 4, False),
                                         (2, 128, 12, 12, True), (1, 128, 96, 96, True)],
                         ids=lambda v: str(v))
def test_gn_silu_tee_accumulates_skip_gradient(G, n, c, h, w, x32):
    """GroupNormSiLUTee returns (silu(GroupNorm(x)), x); its backward adds the second output's
    gradient into dx in the kernel. x's gradient equals autograd's own accumulation over the
    unfused pair (GroupNormSiLU on x and x used again) bit for bit, in fp32 and bf16; 96 x 96
    (no fp32 form: x is cast to bf16) takes the separate add."""
    seed = n + c + h + 31
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((n, c, h, w), generator=g) * 2.0 + 0.5
    if not x32:
        x = x.to(torch.bfloat16)
    gamma, beta, _, _ = params(c, n, seed + 2, False)
    g1 = cl(randn_bf16((n, c, h, w), seed=seed + 1, std=1e-2))
    g2 = cl(torch.randn((n, c, h, w), generator=g).to(x.dtype))
    xa = cl(x).requires_grad_()
    ga, ba = gamma.cuda().requires_grad_(), beta.cuda().requires_grad_()
    ya, ra = G.group_norm_silu_tee(xa, ga, ba, GROUPS, 1e-5)
    torch.autograd.backward([ya, ra], [g1, g2])
    xb = cl(x).requires_grad_()
    gb, bb = gamma.cuda().requires_grad_(), beta.cuda().requires_grad_()
    yb = G.group_norm_silu(xb, gb, bb, GROUPS, 1e-5)
    torch.autograd.backward([yb, xb * 1], [g1, g2])
    torch.cuda.synchronize()
    assert torch.equal(ya, yb) and torch.equal(ra, xb)
    assert xa.grad.dtype == x.dtype
    assert torch.equal(xa.grad, xb.grad)
    assert torch.equal(ga.grad, gb.grad) and torch.equal(ba.grad, bb.grad)


@pytest.mark.parametrize("n,c,h,w,x32", [(2, 128, 32, 32, True), (2, 512, 8, 8, True),
                                         (3, 256, 16, 16, False), (2, 128, 12, 12, True)],
                         ids=lambda v: str(v))
def test_gn_silu_tee_bf16_skip_copy(G, n, c, h, w, x32):
    """With skip_bf16 the tee's second output is x.to(bfloat16) (written by the GroupNorm kernel
    for an fp32 x) and its bf16 gradient is accumulated into x's gradient as autograd does for
    the unfused pair (GroupNormSiLU on x, x.to(bfloat16) for the skip): outputs and all
    gradients bit-identical."""
    seed = n + c + h + 57
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((n, c, h, w), generator=g) * 2.0 + 0.5
    if not x32:
        x = x.to(torch.bfloat16)
    gamma, beta, _, _ = params(c, n, seed + 2, False)
    g1 = cl(randn_bf16((n, c, h, w), seed=seed + 1, std=1e-2))
    g2 = cl(randn_bf16((n, c, h, w), seed=seed + 3, std=1e-1))
    xa = cl(x).requires_grad_()
    ga, ba = gamma.cuda().requires_grad_(), beta.cuda().requires_grad_()
    ya, ra = G.group_norm_silu_tee(xa, ga, ba, GROUPS, 1e-5, True)
    torch.autograd.backward([ya, ra], [g1, g2])
    xb = cl(x).requires_grad_()
    gb, bb = gamma.cuda().requires_grad_(), beta.cuda().requires_grad_()
    yb = G.group_norm_silu(xb, gb, bb, GROUPS, 1e-5)
    rb = xb.to(torch.bfloat16)
    torch.autograd.backward([yb, rb], [g1, g2])
    torch.cuda.synchronize()
    assert ra.dtype == torch.bfloat16
    assert torch.equal(ya, yb) and torch.equal(ra, rb)
    assert xa.grad.dtype == x.dtype
    assert torch.equal(xa.grad, xb.grad)
    assert torch.equal(ga.grad, gb.grad) and torch.equal(ba.grad, bb.grad)
