"""Producer-side amax for the current-scaling FP8 GEMMs: the LayerNorm forward (qkv projection
input), the self-attention forward (out projection input) and backward (qkv projection output
gradient), the residual join's backward (the out projection's, a 1x1 skip conv's or a
current-scaling conv's dy) and the GroupNorm writing the bf16 copy of an fp32 x (the 1x1 skip
conv's input) leave per-workgroup maxima of what they wrote, and the GEMM runs only the cast
(diffusion/fp8_kernels.py:559-601 with the amax pass :54-64 moved into the producer).

Each producer's record is checked against the standalone two-pass quantization of the same
tensor (identical e4m3 bytes and scale), records are refused for a tensor changed after it was
written, and whole cfg5 U-Net training steps with the records equal the same steps without
them, bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import dpa_mod

pytestmark = pytest.mark.gpu

K = dpa_mod("fp8_kernels")
LN = dpa_mod("layer_norm")
A = dpa_mod("attention")
U = dpa_mod("unet")
T = dpa_mod("trainer")


def same_quant(t: torch.Tensor):
    """(from the producer's record, standalone) for t viewed as rows, both (q bytes, scale)."""
    t2 = t.reshape(-1, t.shape[-1])
    got = K.quantize_fp8_from_producer(t2, t)
    assert got is not None, "the producer left no usable record"
    ref = K.quantize_fp8_tensor(t2)
    torch.cuda.synchronize()
    assert got[1].item() == ref[1].item() or (np.isnan(got[1].item()) and np.isnan(ref[1].item()))
    assert torch.equal(got[0].view(torch.uint8), ref[0].view(torch.uint8))


@pytest.mark.parametrize("shape,dtype", [((128, 256, 256), torch.bfloat16),
                                         ((128, 64, 256), torch.float32),
                                         ((7, 16, 512), torch.bfloat16),
                                         ((3, 5, 64), torch.bfloat16)], ids=str)
def test_layernorm_record_matches_standalone(shape, dtype):
    g = torch.Generator().manual_seed(sum(shape))
    x = (torch.randn(shape, generator=g) * 3 + 1).to(dtype).cuda()
    norm = torch.nn.LayerNorm(shape[-1]).cuda()
    with torch.no_grad():
        norm.weight.copy_(1 + 0.5 * torch.randn(shape[-1], generator=g))
        norm.bias.copy_(0.2 * torch.randn(shape[-1], generator=g))
    out = LN.layer_norm_bf16(x, norm)
    same_quant(out)


@pytest.mark.parametrize("b,l,heads", [(128, 256, 4), (16, 64, 4), (8, 16, 8), (4, 48, 2)], ids=str)
def test_attention_records_match_standalone(b, l, heads):
    """Forward output and backward dqkv (captured where the qkv projection would receive it)."""
    c = 64 * heads
    g = torch.Generator().manual_seed(b + l + heads)
    qkv = torch.randn((b, l, 3 * c), generator=g).to(torch.bfloat16).cuda().requires_grad_()
    seen = {}

    class Catch(torch.autograd.Function):
        @staticmethod
        def forward(ctx, t):
            return t.view_as(t)

        @staticmethod
        def backward(ctx, grad):
            seen["dqkv"] = grad
            return grad

    out = A.self_attention_qkv(Catch.apply(qkv), heads)
    same_quant(out)
    dout = (torch.randn((b, l, c), generator=g) * 1e-2).to(torch.bfloat16).cuda()
    out.backward(dout)
    same_quant(seen["dqkv"])


def same_quant_4d(t: torch.Tensor):
    """same_quant for a channels-last 4-D tensor (the convs' operands), through the record."""
    got = K.quantize_fp8_from_producer(t, t)
    assert got is not None, "the producer left no usable record"
    ref = K.quantize_fp8(t)
    torch.cuda.synchronize()
    assert got[1].item() == ref[1].item()
    assert torch.equal(got[0].view(torch.uint8), ref[0].view(torch.uint8))


R = dpa_mod("residual")
G = dpa_mod("gn_silu")


class _Catch(torch.autograd.Function):
    """Identity whose backward records the gradient object it receives (what the next FP8
    op's backward would receive: a leaf's .grad is a detached copy without the record)."""

    @staticmethod
    def forward(ctx, t, seen, key):
        ctx.seen, ctx.key = seen, key
        return t.view_as(t)

    @staticmethod
    def backward(ctx, grad):
        ctx.seen[ctx.key] = grad
        return grad, None, None


def catch(t, seen, key):
    return _Catch.apply(t, seen, key)


def cl(t):
    return t.cuda().contiguous(memory_format=torch.channels_last)


@pytest.mark.parametrize("dtype,shape", [(torch.bfloat16, (4, 256, 16, 16)),
                                         (torch.float32, (8, 256, 8, 8)),
                                         (torch.float32, (128, 256, 16, 16)),
                                         (torch.bfloat16, (3, 128, 5, 8))], ids=str)
def test_join_backward_records_match_standalone(dtype, shape):
    """The residual join's backward (diffusion/unet.py:161, :203) leaves the maxima of the bf16
    gradient it writes -- the dy of the attention out-projection or of a current-scaling conv
    feeding the join -- for its fp32 (fp32 stream) and bf16 forms; the gradients themselves
    equal the plain backward's bit for bit."""
    g = torch.Generator().manual_seed(sum(shape) + 3)
    a0 = cl((torch.randn(shape, generator=g) * 2).to(dtype))
    b0 = cl(torch.randn(shape, generator=g).to(torch.bfloat16))
    gy = cl((torch.randn(shape, generator=g) * 3e-2).to(dtype))
    grads = {}
    for flag in (True, False):
        K.PRODUCER_AMAX = flag
        try:
            a, b = a0.clone().requires_grad_(), b0.clone().requires_grad_()
            seen = {}
            R.residual_join(catch(a, seen, "a"), catch(b, seen, "b")).backward(gy)
        finally:
            K.PRODUCER_AMAX = True
        grads[flag] = (seen["a"], seen["b"])
    assert torch.equal(grads[True][0], grads[False][0])
    assert torch.equal(grads[True][1], grads[False][1])
    same_quant_4d(grads[True][1])


def test_handoff_join_records_the_skip_gradient():
    """With conv_2's dy handed off (delayed scaling), the join's bf16 a-gradient -- the 1x1
    skip conv's dy -- holds the same bf16 values the hand-off cast, and carries its maxima."""
    shape = (4, 256, 16, 16)
    g = torch.Generator().manual_seed(11)
    a = cl(torch.randn(shape, generator=g).to(torch.bfloat16)).requires_grad_()
    b = cl(torch.randn(shape, generator=g).to(torch.bfloat16)).requires_grad_()
    gy = cl((torch.randn(shape, generator=g) * 3e-2).to(torch.bfloat16))
    hand = K.Fp8Handoff(torch.tensor(1e-4, device="cuda"), torch.zeros(16384, device="cuda",
                                                                      dtype=torch.int32),
                        torch.zeros(1, device="cuda", dtype=torch.int32))
    seen = {}
    R.residual_join(catch(a, seen, "a"), b, hand).backward(gy)
    same_quant_4d(seen["a"])


@pytest.mark.parametrize("n,c,h,w,hand", [(2, 256, 16, 16, False), (2, 512, 8, 8, True),
                                          (1, 128, 40, 40, False), (2, 128, 32, 32, True)],
                         ids=str)
def test_groupnorm_skip_copy_records_match_standalone(n, c, h, w, hand):
    """The GroupNorm (resident form, and the chunked form at 1600 pixels) writing the bf16
    copy of an fp32 x for the 1x1 skip conv (diffusion/unet.py:137-139) leaves its maxima;
    with and without the conv input's hand-off."""
    g = torch.Generator().manual_seed(n * c + h)
    x = cl(torch.randn((n, c, h, w), generator=g) * 3 + 0.5)
    gamma = (1 + 0.1 * torch.randn(c, generator=g)).cuda()
    beta = (0.1 * torch.randn(c, generator=g)).cuda()
    hd = None
    if hand:
        hd = K.Fp8Handoff(torch.tensor(0.01, device="cuda"),
                          torch.zeros(16384, device="cuda", dtype=torch.int32),
                          torch.zeros(1, device="cuda", dtype=torch.int32))
    _, x16 = G.group_norm_silu_tee(x, gamma, beta, 32, 1e-5, True, hd)
    assert x16.dtype == torch.bfloat16
    assert torch.equal(x16, x.to(torch.bfloat16))
    same_quant_4d(x16)


def test_record_refused_after_an_in_place_change():
    x = torch.randn((64, 256), device="cuda").to(torch.bfloat16)
    norm = torch.nn.LayerNorm(256).cuda()
    out = LN.layer_norm_bf16(x, norm)
    assert K.quantize_fp8_from_producer(out, out) is not None
    out.mul_(2.0)  # the recorded maxima no longer describe it
    assert K.quantize_fp8_from_producer(out, out) is None
    assert K.quantize_fp8_from_producer(out.clone(), out) is None  # another buffer


def _state():
    cfg = U.cfg5_config(p_drop=0.2)
    st = T.TrainState(cfg, batch=4, seed=0, fixed_noise=True)
    g = torch.Generator().manual_seed(4)
    images = torch.rand((4, 3, 32, 32), generator=g) * 2 - 1
    t = torch.randint(0, 1000, (4,), generator=g)
    eps = torch.randn((4, 3, 32, 32), generator=g)
    st.set_batch(images.cuda(), t.cuda(), eps.cuda())
    return st


def test_cfg5_steps_with_records_equal_steps_without(monkeypatch):
    """Three eager cfg5 training steps with the producer records and three without, from the
    same state and random stream: identical losses, parameters, gradients and buffers, and
    three fewer standalone quantizations per attention block in each step (LayerNorm out,
    attention out, dqkv)."""
    monkeypatch.setattr(torch.backends.cudnn, "deterministic", True)
    calls = {"n": 0}
    real = K.quantize_fp8_tensor

    def counting(*a, **kw):
        calls["n"] += 1
        return real(*a, **kw)

    monkeypatch.setattr(K, "quantize_fp8_tensor", counting)
    monkeypatch.setattr(K, "quantize_fp8", counting)
    runs = {}
    for flag in (True, False):
        monkeypatch.setattr(K, "PRODUCER_AMAX", flag)
        st = _state()
        losses, counts = [], []
        for i in range(3):
            torch.cuda.manual_seed(100 + i)
            calls["n"] = 0
            st.loss_acc.zero_()
            st.eager_step()
            torch.cuda.synchronize()
            losses.append(float(st.loss_acc))
            counts.append(calls["n"])
        if st.model._wprep is not None:
            st.model._wprep.flush()
        torch.cuda.synchronize()
        runs[flag] = (st, losses, counts)
    n_attn = sum(isinstance(m, U.CHWAttention) for m in runs[True][0].model.modules())
    print(f"attention blocks {n_attn}; standalone quantizations per step: "
          f"with records {runs[True][2]}, without {runs[False][2]}", flush=True)
    assert runs[True][1] == runs[False][1]
    # per attention block: LayerNorm out, attention out, dqkv and the out projection's dy from
    # the join; plus the 1x1 skip convs' inputs and dy and the joins feeding current-scaling
    # convs
    assert runs[False][2][-1] - runs[True][2][-1] >= 4 * n_attn
    a, b = runs[True][0], runs[False][0]
    for (na, pa), pb in zip(a.model.named_parameters(), b.model.parameters()):
        assert torch.equal(pa, pb), na
        assert (pa.grad is None) == (pb.grad is None), na
        assert pa.grad is None or torch.equal(pa.grad, pb.grad), na
    for (na, ba), bb in zip(a.model.named_buffers(), b.model.buffers()):
        assert torch.equal(ba, bb), na
