"""The HIP self-attention kernels (dpa_attention_fwd_bf16 / _bwd_bf16) against float32 attention
on the same bf16 q, k, v, and against the reference's own op, torch's
F.scaled_dot_product_attention in bf16 (diffusion/unet.py:196), whose error the kernels must not
exceed by more than a small margin.

Tolerances (normwise, ||ours - fp32|| / ||fp32||): output 1e-2, gradients 2e-2, and at most
1.5x the bf16 SDPA's own error plus 2e-3. The base-2 log-sum-exp the forward saves is checked
against float64 to 1e-5 relative. Shapes: the U-Net's token grids (L = 256, 64, 16 at 4 heads of
64, batch 128 for the 16x16 grid), padded lengths (L = 48, 144: the masked-key paths) and
peaked softmaxes (scores scaled x4).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import dpa_mod

pytestmark = pytest.mark.gpu

A = dpa_mod("attention")
U = dpa_mod("unet")
T = dpa_mod("trainer")


def _qkv(b, l, heads, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((b, l, 3 * 64 * heads), generator=g) * scale
    return x.to(torch.bfloat16).cuda()


def _split(qkv, heads):
    """qkv [B, L, 3C] -> q, k, v [B, heads, L, 64] (float32 copies)."""
    b, l, c3 = qkv.shape
    c = c3 // 3
    q, k, v = torch.chunk(qkv.float(), 3, dim=-1)
    return [t.reshape(b, l, heads, 64).transpose(1, 2).contiguous() for t in (q, k, v)]


def _ref_fp32(qkv, heads, dout):
    """float32 attention on the bf16 values: output [B, L, C] and d(qkv) [B, L, 3C]."""
    x = qkv.float().detach().requires_grad_()
    b, l, c3 = x.shape
    q, k, v = torch.chunk(x, 3, dim=-1)
    q, k, v = [t.reshape(b, l, heads, 64).transpose(1, 2) for t in (q, k, v)]
    s = torch.matmul(q.contiguous(), k.transpose(-1, -2).contiguous()) / 8.0
    p = torch.softmax(s, dim=-1)
    o = torch.matmul(p, v.contiguous())
    o = o.transpose(1, 2).reshape(b, l, c3 // 3)
    o.backward(dout.float())
    return o.detach(), x.grad.detach(), s.detach()


def _ref_sdpa_bf16(qkv, heads, dout):
    """torch's fused bf16 SDPA (the reference's op) with the reference's rearranges."""
    x = qkv.detach().clone().requires_grad_()
    b, l, c3 = x.shape
    q, k, v = torch.chunk(x, 3, dim=-1)
    q, k, v = [t.reshape(b, l, heads, 64).transpose(1, 2) for t in (q, k, v)]
    with U._fused_sdpa():
        o = F.scaled_dot_product_attention(q, k, v)
    o = o.transpose(1, 2).reshape(b, l, c3 // 3)
    o.backward(dout)
    return o.detach(), x.grad.detach()


def _rel(a, b):
    return float((a.float() - b.float()).norm() / b.float().norm())


def _run(qkv, heads, dout):
    x = qkv.detach().clone().requires_grad_()
    o = A.self_attention_qkv(x, heads)
    o.backward(dout)
    torch.cuda.synchronize()
    return o.detach(), x.grad.detach()


CASES = [  # (batch, L, heads, score scale)
    (128, 256, 4, 1.0),   # 16x16 grid, cfg5 batch
    (16, 64, 4, 1.0),     # 8x8 grid
    (32, 16, 4, 1.0),     # 4x4 grid (padded to 32 inside)
    (4, 48, 2, 1.0),      # padded to 64: masked keys and queries
    (2, 144, 4, 1.0),     # padded to 256
    (8, 256, 4, 2.0),     # peaked softmax (scores x4)
    (8, 64, 1, 2.0),
]


@pytest.mark.parametrize("b,l,heads,scale", CASES)
def test_attention_vs_fp32_and_sdpa(b, l, heads, scale):
    print(f"attention b={b} L={l} heads={heads} scale={scale}", flush=True)
    qkv = _qkv(b, l, heads, seed=l + heads, scale=scale)
    g = torch.Generator().manual_seed(99)
    dout = (torch.randn((b, l, 64 * heads), generator=g)).to(torch.bfloat16).cuda()
    o, dqkv = _run(qkv, heads, dout)
    ro, rd, _ = _ref_fp32(qkv, heads, dout)
    so, sd = _ref_sdpa_bf16(qkv, heads, dout)
    assert o.dtype == torch.bfloat16 and o.shape == (b, l, 64 * heads)
    assert dqkv.dtype == torch.bfloat16 and dqkv.shape == qkv.shape
    assert torch.isfinite(o.float()).all() and torch.isfinite(dqkv.float()).all()
    e_o, s_o = _rel(o, ro), _rel(so, ro)
    c = 64 * heads
    errs = []
    for name, sl in (("dq", slice(0, c)), ("dk", slice(c, 2 * c)), ("dv", slice(2 * c, 3 * c))):
        errs.append((name, _rel(dqkv[..., sl], rd[..., sl]), _rel(sd[..., sl], rd[..., sl])))
    print(f"  out {e_o:.2e} (sdpa {s_o:.2e}); " +
          ", ".join(f"{n} {e:.2e} (sdpa {s:.2e})" for n, e, s in errs), flush=True)
    assert e_o <= 1e-2 and e_o <= 1.5 * s_o + 2e-3
    for name, e, s in errs:
        assert e <= 2e-2 and e <= 1.5 * s + 2e-3, name


def test_attention_lse_vs_float64():
    """The forward's saved log-sum-exp: log2 sum_k 2^(s_k log2(e) / 8) per (image, head, query)."""
    b, l, heads = 4, 256, 4
    qkv = _qkv(b, l, heads, seed=5, scale=2.0)
    out = torch.empty((b, l, 64 * heads), device="cuda", dtype=torch.bfloat16)
    lse = torch.empty((b * heads, l), device="cuda", dtype=torch.float32)
    dpa_mod("_lib").call("dpa_attention_fwd_bf16", qkv.data_ptr(), out.data_ptr(), lse.data_ptr(),
                         b, l, 64 * heads, heads, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    q, k, _ = _split(qkv, heads)
    s = (q.double() @ k.double().transpose(-1, -2)) / 8.0            # [B, H, L, L]
    ref = torch.logsumexp(s, dim=-1) / math.log(2.0)                  # natural -> base 2
    ref = ref.reshape(b * heads, l)
    err = ((lse.double() - ref).abs() / ref.abs().clamp_min(1.0)).max().item()
    assert err <= 1e-5, err


def test_attention_deterministic():
    """No atomics: two runs give identical bits (forward and all three gradients)."""
    b, l, heads = 32, 256, 4
    qkv = _qkv(b, l, heads, seed=3)
    dout = torch.randn((b, l, 64 * heads), generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).cuda()
    o1, d1 = _run(qkv, heads, dout)
    o2, d2 = _run(qkv, heads, dout)
    assert torch.equal(o1, o2) and torch.equal(d1, d2)


def test_attention_uniform_keys():
    """Identical keys: the softmax is uniform, so the output is the mean of the values and
    dq vanishes (every score moves together; what remains is the bf16 rounding of ds)."""
    b, l, heads = 2, 64, 4
    qkv = _qkv(b, l, heads, seed=11)
    c = 64 * heads
    qkv[:, :, c:2 * c] = qkv[:, :1, c:2 * c]      # one key row repeated
    dout = torch.randn((b, l, c), generator=torch.Generator().manual_seed(12)).to(torch.bfloat16).cuda()
    o, d = _run(qkv, heads, dout)
    vmean = qkv[:, :, 2 * c:].float().mean(dim=1, keepdim=True).expand(b, l, c)
    assert _rel(o, vmean) <= 4e-3
    assert float(d[..., :c].float().abs().max()) <= 1e-2 * float(d[..., 2 * c:].float().abs().max())


class _Fp32Attention:
    """Attention in float32 from the (bf16) q, k, v: the model-level reference."""

    @staticmethod
    def apply(q, k, v):
        s = torch.matmul(q.float(), k.float().transpose(1, 2).contiguous()) / math.sqrt(q.shape[-1])
        return torch.matmul(torch.softmax(s, dim=-1), v.float())


def _unet_grads(monkeypatch, cfg, mode, calls):
    """loss and parameter gradients of one cfg5 forward+backward (batch 16, autocast bf16) with
    the attention run by mode: "hip" (the HIP kernels), "sdpa" (torch's fused bf16 SDPA, the
    reference's op) or "fp32" (float32 attention on the same bf16 q, k, v)."""
    monkeypatch.setattr(U, "_HIP_SDPA", mode == "hip")
    monkeypatch.setattr(U, "_GPU_SDPA", mode != "fp32")
    monkeypatch.setattr(U, "_Attention", _Fp32Attention if mode == "fp32" else RealAttention)
    st = T.TrainState(cfg, batch=16, seed=0, fixed_noise=True)
    # the attention out projections, the residual blocks' second convs and the output conv
    # start at zero (diffusion/unet.py:146, :178-179), which would hide the attention from the
    # loss and from every gradient upstream of it: random values instead
    gw = torch.Generator().manual_seed(21)
    with torch.no_grad():
        for _, prm in sorted(st.model.named_parameters()):
            if prm.dim() > 1 and not bool(prm.any()):
                w = torch.randn(prm.shape, generator=gw) * (0.5 / math.sqrt(prm[0].numel()))
                prm.copy_(w.to(prm.device, prm.dtype))
    g = torch.Generator().manual_seed(4)
    st.set_batch((torch.rand((16, 3, 32, 32), generator=g) * 2 - 1).cuda(),
                 torch.randint(0, 1000, (16,), generator=g).cuda(),
                 torch.randn((16, 3, 32, 32), generator=g).cuda())
    calls["n"] = 0
    st.model.train()
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        loss = st.ddpm.forward_batch(st.static_batch, st.static_t, st.static_eps)
    loss.backward()
    torch.cuda.synchronize()
    return (float(loss.detach()), calls["n"],
            {n: p.grad.detach().clone() for n, p in st.model.named_parameters() if p.grad is not None})


RealAttention = U._Attention


@pytest.mark.parametrize("fp8", [False, True])
def test_unet_hip_attention_vs_torch_sdpa(monkeypatch, fp8):
    """A cfg5 U-Net forward+backward through the HIP attention, through torch's fused bf16
    SDPA (the reference's op) and through float32 attention: against the float32 run, the HIP
    run's loss and every parameter gradient are no further off than the SDPA run's (1.5x its
    normwise distance plus 1e-3 of the gradient's norm), and the losses of the two bf16
    kernels agree to 1e-3. bf16 convs and linears, and the cfg5 FP8 ones (whose e4m3 casts
    turn last-bit differences of the attention into e4m3 steps, 2^-3, in both runs alike).
    The HIP kernels ran in all 12 attention blocks."""
    monkeypatch.setattr(torch.backends.cudnn, "deterministic", True)
    calls = {"n": 0}
    real = A.SelfAttentionQKV.apply

    def counting(*a):
        calls["n"] += 1
        return real(*a)

    monkeypatch.setattr(A.SelfAttentionQKV, "apply", counting)
    cfg = (U.cfg5_config(p_drop=0.0) if fp8 else
           U.cfg5_config(p_drop=0.0, fp8_convs_enabled=False, fp8_all_convs=False, fp8_linears=False))
    lh, nh, gh = _unet_grads(monkeypatch, cfg, "hip", calls)
    ls, ns, gs = _unet_grads(monkeypatch, cfg, "sdpa", calls)
    lf, nf, gf = _unet_grads(monkeypatch, cfg, "fp32", calls)
    print(f"fp8={fp8}: loss hip {lh} sdpa {ls} fp32 {lf}; HIP attention calls {nh} / {ns} / {nf}",
          flush=True)
    assert nh == 12 and ns == 0 and nf == 0
    assert np.isfinite(lh) and lh == pytest.approx(ls, rel=1e-3)
    # the scalar loss is one noisy sample of the attention's rounding: |ls - lf| has read
    # 6e-5 and 8e-6 for models that differ only in the output conv's fp32 summation order,
    # with |lh - lf| 1.6e-4 and 1.5e-4 (all 1.4e-4 relative or less, against bf16's 3.9e-3)
    assert abs(lh - lf) <= 1.5 * abs(ls - lf) + 3e-4 * abs(lf)
    assert gh.keys() == gs.keys() == gf.keys() and len(gh) > 0
    # per parameter: bf16 model 1.5x the SDPA distance + 1e-3 of the norm; the FP8 model's
    # e4m3 steps make single small tensors noisy (3x + 1e-2), so it is also held to 1.5x over
    # all gradients together
    k, floor = (1.5, 1e-3) if not fp8 else (3.0, 1e-2)
    ratios, th, ts, tf = [], 0.0, 0.0, 0.0
    for name in gh:
        ref = float(gf[name].float().norm())
        dh = float((gh[name] - gf[name]).float().norm())
        ds = float((gs[name] - gf[name]).float().norm())
        th, ts, tf = th + dh * dh, ts + ds * ds, tf + ref * ref
        ratios.append(dh / max(ds, 1e-12))
        assert dh <= k * ds + floor * ref + 1e-7, (name, dh, ds, ref)
    th, ts, tf = math.sqrt(th), math.sqrt(ts), math.sqrt(tf)
    print(f"HIP / SDPA distance to the float32 run: median {np.median(ratios):.2f}, "
          f"max {max(ratios):.2f}; all gradients {th / tf:.2e} / {ts / tf:.2e}", flush=True)
    assert th <= 1.5 * ts + 1e-4 * tf
