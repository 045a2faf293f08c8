"""GPU parity of the fused bf16 LayerNorm (dpa_layernorm_*, layer_norm.LayerNormBF16) against a
float64 torch reference: the attention block's nn.LayerNorm (diffusion/unet.py:174, :187) run
in fp32 by autocast and rounded to bf16 by the qkv projection. Forward within one bf16 ulp
(almost all bit-identical), statistics to 1e-5, dx to the conv tolerance, dgamma/dbeta 1e-4.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import assert_bf16_close, bits, dpa_mod

pytestmark = pytest.mark.gpu

LN = dpa_mod("layer_norm")


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


@pytest.mark.parametrize("rows,c", [(512, 256), (37, 256), (300, 64), (129, 128), (64, 512),
                                    (33, 1024), (128 * 64, 256)])
def test_layernorm_fwd_bwd_vs_float64(rows, c):
    g = torch.Generator().manual_seed(rows + c)
    x = (torch.randn((rows, c), generator=g) * 2 + 0.7).to(torch.bfloat16)
    gamma = 1 + 0.2 * torch.randn(c, generator=g)
    beta = 0.1 * torch.randn(c, generator=g)
    dy = (torch.randn((rows, c), generator=g) * 1e-2).to(torch.bfloat16)

    xd = x.cuda().requires_grad_()
    gd, bd = gamma.cuda().requires_grad_(), beta.cuda().requires_grad_()
    y = LN.LayerNormBF16.apply(xd, gd, bd, 1e-5)
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16 and xd.grad.dtype == torch.bfloat16

    xr = x.double().requires_grad_()
    gr, br = gamma.double().requires_grad_(), beta.double().requires_grad_()
    yr = F.layer_norm(xr, (c,), gr, br, 1e-5)
    yr.backward(dy.double())

    yb = bits(y.detach().cpu())
    ref = bits(yr.detach().float().to(torch.bfloat16))
    got = y.detach().cpu().double().numpy()
    want = yr.detach().double().numpy()
    assert np.all(np.abs(got - want) <= 2.0**-7 * np.abs(want) + 1e-6), "forward beyond 1 bf16 ulp"
    assert np.mean(yb == ref) > 0.99
    assert_bf16_close(bits(xd.grad.cpu()), bits(xr.grad.float().to(torch.bfloat16)), f"dx {rows}x{c}")
    assert rel(gd.grad.cpu().numpy(), gr.grad.numpy()) < 1e-4
    assert rel(bd.grad.cpu().numpy(), br.grad.numpy()) < 1e-4


def test_layernorm_on_token_view_matches_module():
    """On the [B, H*W, C] token view of a channels-last activation (the attention block's
    input), against nn.LayerNorm in fp32 on the GPU rounded to bf16."""
    torch.manual_seed(0)
    x = (torch.randn((8, 256, 16, 16), device="cuda") + 0.3).to(torch.bfloat16)
    x = x.contiguous(memory_format=torch.channels_last)
    norm = torch.nn.LayerNorm(256).cuda()
    with torch.no_grad():
        norm.weight.mul_(1.5)
        norm.bias.add_(0.2)
    seq = x.permute(0, 2, 3, 1).reshape(8, 256, 256)
    y = LN.layer_norm_bf16(seq, norm)
    ref = norm(seq.float()).to(torch.bfloat16)
    torch.cuda.synchronize()
    assert y.shape == ref.shape
    frac = float((y == ref).float().mean())
    assert frac > 0.99, frac
    assert float((y.float() - ref.float()).abs().max()) <= 2**-7 * float(ref.float().abs().max())


@pytest.mark.parametrize("rows,c", [(512, 256), (37, 256), (300, 64), (129, 128), (33, 1024),
                                    (64 * 16, 256)])
def test_layernorm_fp32_tokens_vs_float64(rows, c):
    """fp32 tokens (the fp32 residual stream of the lower levels) are normalised as they are,
    as autocast's float32 nn.LayerNorm does: forward within one bf16 ulp of the float64
    reference on the fp32 values (and away from the bf16-rounded input's result), dx in fp32
    normwise 2e-5, dgamma/dbeta 1e-4."""
    g = torch.Generator().manual_seed(rows + c + 3)
    x = torch.randn((rows, c), generator=g) * 2 + 0.7
    gamma = 1 + 0.2 * torch.randn(c, generator=g)
    beta = 0.1 * torch.randn(c, generator=g)
    dy = (torch.randn((rows, c), generator=g) * 1e-2).to(torch.bfloat16)
    xd = x.cuda().requires_grad_()
    gd, bd = gamma.cuda().requires_grad_(), beta.cuda().requires_grad_()
    y = LN.LayerNormBF16.apply(xd, gd, bd, 1e-5)
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16 and xd.grad.dtype == torch.float32
    xr = x.double().requires_grad_()
    gr, br = gamma.double().requires_grad_(), beta.double().requires_grad_()
    yr = F.layer_norm(xr, (c,), gr, br, 1e-5)
    yr.backward(dy.double())
    got = y.detach().cpu().double().numpy()
    want = yr.detach().numpy()
    assert np.all(np.abs(got - want) <= 2.0**-7 * np.abs(want) + 1e-6), "forward beyond 1 bf16 ulp"
    assert np.mean(bits(y.detach().cpu()) == bits(yr.detach().float().to(torch.bfloat16))) > 0.99
    yb16 = F.layer_norm(x.to(torch.bfloat16).double(), (c,), gamma.double(), beta.double(), 1e-5)
    assert np.mean(bits(yb16.float().to(torch.bfloat16)) != bits(yr.detach().float().to(torch.bfloat16))) > 0.02
    assert rel(xd.grad.cpu().numpy(), xr.grad.numpy()) < 2e-5
    assert rel(gd.grad.cpu().numpy(), gr.grad.numpy()) < 1e-4
    assert rel(bd.grad.cpu().numpy(), br.grad.numpy()) < 1e-4


@pytest.mark.parametrize("dtype,c,hw", [(torch.bfloat16, 256, 16), (torch.float32, 256, 8),
                                        (torch.float32, 256, 4), (torch.bfloat16, 128, 16)])
def test_attention_block_skip_gradient_add_in_layernorm(dtype, c, hw):
    """The attention block with its input's skip gradient added inside the LayerNorm backward
    (LayerNormTee, dpa_layernorm_bwd_ex_add) against the same block with autograd's separate
    add: output, input gradient and every parameter gradient bit for bit, bf16 and fp32
    block inputs (the fp32 residual stream of the lower levels)."""
    U = dpa_mod("unet")
    cfg = U.cfg5_config(p_drop=0.0)
    torch.manual_seed(0)
    blk = U.CHWAttention(cfg, c).cuda()
    with torch.no_grad():                      # a non-zero out projection
        blk.out.weight.normal_(0, 0.05)
    g = torch.Generator().manual_seed(1)
    x0 = torch.randn((8, c, hw, hw), generator=g).cuda().to(dtype)
    x0 = x0.contiguous(memory_format=torch.channels_last)
    gy = torch.randn((8, c, hw, hw), generator=g).cuda().to(dtype)
    gy = gy.contiguous(memory_format=torch.channels_last)
    L = dpa_mod("_lib")
    real_call, calls = L.call, []

    def counting(name, *args):
        calls.append(name)
        return real_call(name, *args)

    res = {}
    for tee in (True, False):
        blk.ln_tee = tee
        calls.clear()
        for p in blk.parameters():
            p.grad = None
        x = x0.clone().requires_grad_()
        L.call = counting
        try:
            with torch.autocast("cuda", dtype=torch.bfloat16):
                y = blk(x)
            y.backward(gy)
            torch.cuda.synchronize()
        finally:
            L.call = real_call
        assert calls.count("dpa_layernorm_bwd_ex_add") == (1 if tee else 0), calls
        res[tee] = (y.detach(), x.grad, [p.grad.clone() for p in blk.parameters()])
    blk.ln_tee = True
    (ya, gxa, pa), (yb, gxb, pb) = res[True], res[False]
    assert torch.equal(ya, yb)
    assert gxa.dtype == gxb.dtype == dtype
    assert torch.equal(gxa, gxb)
    for a, b in zip(pa, pb):
        assert torch.equal(a, b)
