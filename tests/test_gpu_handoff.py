"""Producer-fused quantization for the delayed-scaling FP8 convs: the GroupNorm+SiLU(+FiLM,
+dropout) forward writing the conv input as e4m3, the FiLM GroupNorm backward writing the
upstream conv's dy as e4m3, and the residual join's backward writing conv_2's dy as e4m3
(diffusion/unet.py:151, :157-161 feeding diffusion/fp8_kernels.py:856, :885-893).

Each is checked against the unfused pair it replaces -- the bf16 producer, then the
standalone deferred cast with the same window scale -- for identical e4m3 bytes, identical
amax (the window record's input) and identical other outputs; then a whole cfg5 U-Net
training step with the hand-offs against the same step without them, bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import dpa_mod

pytestmark = pytest.mark.gpu

GROUPS = 32
K = dpa_mod("fp8_kernels")
G = dpa_mod("gn_silu")
R = dpa_mod("residual")
U = dpa_mod("unet")
T = dpa_mod("trainer")


def cl(t):
    return t.cuda().contiguous(memory_format=torch.channels_last)


def hand(scale: float, cap: int = 16384) -> "K.Fp8Handoff":
    return K.Fp8Handoff(torch.tensor(scale, device="cuda", dtype=torch.float32),
                        torch.zeros(cap, device="cuda", dtype=torch.int32),
                        torch.zeros(1, device="cuda", dtype=torch.int32))


def amax_bits(h) -> int:
    """max of the hand-off's partials (u32 bf16 magnitudes) -- what the window record reads."""
    n = int(h.count.item())
    assert n > 0
    return int(h.partials[:n].cpu().numpy().view(np.uint32).max())


def q_bytes(q: torch.Tensor) -> np.ndarray:
    return q.view(torch.uint8).permute(0, 2, 3, 1).contiguous().cpu().numpy() if q.ndim == 4 \
        else q.view(torch.uint8).cpu().numpy()


def scales_for(t: torch.Tensor) -> list[float]:
    """A window scale near the tensor's own, one that saturates a third of the range, and one
    below 2^-64 (the kernels' division path)."""
    amax = float(t.detach().float().abs().max())
    return [amax / 448.0 * 1.3, amax / 448.0 / 3.0, 2.0**-70]


FWD_CASES = [
    # (n, c, h, w, x fp32, film+dropout): chunked and small-image forms, both x dtypes
    (2, 128, 32, 32, True, False),
    (3, 256, 16, 16, False, True),
    (2, 512, 8, 8, True, True),
    (4, 256, 4, 4, False, False),
    (2, 128, 17, 19, False, True),     # ragged last chunk
]


@pytest.mark.parametrize("n,c,h,w,x32,film", FWD_CASES, ids=lambda v: str(v))
def test_gn_forward_casts_like_the_unfused_pair(n, c, h, w, x32, film):
    seed = n * 131 + c + h
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((n, c, h, w), generator=g) * 2.0 + 0.5
    if not x32:
        x = x.to(torch.bfloat16)
    x = cl(x)
    gamma = (1.0 + 0.1 * torch.randn(c, generator=g)).cuda()
    beta = (0.1 * torch.randn(c, generator=g)).cuda()
    wb = cl((0.3 * torch.randn((n, 2 * c, 1, 1), generator=g)).to(torch.bfloat16))
    p = 0.2 if film else 0.0

    def run(hd):
        torch.cuda.manual_seed(seed)      # the same dropout seed for both forms
        if film:
            return G.group_norm_silu_film(x, gamma, beta, GROUPS, 1e-5, wb, p, hd), None
        return G.group_norm_silu_tee(x, gamma, beta, GROUPS, 1e-5, x32, hd)

    ref, ref16 = run(None)
    for s in scales_for(ref):
        hu, hf = hand(s), hand(s)
        hu.fill_from_bf16(ref)
        out, x16 = run(hf)
        torch.cuda.synchronize()
        assert K.is_placeholder(out) and out.shape == ref.shape
        assert np.array_equal(q_bytes(hf.q), q_bytes(hu.q)), (s, (n, c, h, w))
        assert amax_bits(hf) == amax_bits(hu)
        # one partial per workgroup: one per (image, 64 channels) up to 1024 pixels (resident
        # form), one per 128-pixel chunk of those above
        nblk = (c // 64) * n * (1 if h * w <= 1024 else -(-(h * w) // 128))
        assert int(hf.count.item()) == nblk
        if ref16 is not None:
            assert torch.equal(x16.view(torch.int16), ref16.view(torch.int16))


BWD_CASES = [
    (3, 256, 16, 16, True),
    (2, 256, 8, 8, True),
    (2, 128, 32, 32, True),
    (4, 256, 4, 4, False),
]


@pytest.mark.parametrize("n,c,h,w,drop", BWD_CASES, ids=lambda v: str(v))
def test_gn_backward_casts_dx_like_the_unfused_pair(n, c, h, w, drop):
    """dx of the FiLM GroupNorm (the dy of the conv that produced x) as e4m3 with that conv's
    window scale; dgamma, dbeta and the FiLM gradient unchanged."""
    seed = n * 71 + c + w
    g = torch.Generator().manual_seed(seed)
    x = cl((torch.randn((n, c, h, w), generator=g) * 2.0 + 0.5).to(torch.bfloat16))
    gamma = (1.0 + 0.1 * torch.randn(c, generator=g)).cuda()
    beta = (0.1 * torch.randn(c, generator=g)).cuda()
    wb0 = (0.3 * torch.randn((n, 2 * c, 1, 1), generator=g)).to(torch.bfloat16)
    dout = cl((torch.randn((n, c, h, w), generator=g) * 1e-2).to(torch.bfloat16))
    p = 0.2 if drop else 0.0

    def run(hd):
        xd = x.detach().clone().requires_grad_()
        gd, bd = gamma.clone().requires_grad_(), beta.clone().requires_grad_()
        wbd = cl(wb0).requires_grad_()
        torch.cuda.manual_seed(seed)
        y = G.group_norm_silu_film(xd, gd, bd, GROUPS, 1e-5, wbd, p, None, hd)
        y.backward(dout)
        return xd.grad, gd.grad, bd.grad, wbd.grad

    ref = run(None)
    for s in scales_for(ref[0]):
        hu, hf = hand(s), hand(s)
        hu.fill_from_bf16(ref[0])
        got = run(hf)
        torch.cuda.synchronize()
        assert not got[0].any()           # autograd stores the placeholder (densified) as x.grad
        assert np.array_equal(q_bytes(hf.q), q_bytes(hu.q)), (s, (n, c, h, w))
        assert amax_bits(hf) == amax_bits(hu)
        for a, b in zip(got[1:], ref[1:]):
            assert torch.equal(a, b)


@pytest.mark.parametrize("dtype,shape", [(torch.float32, (4, 256, 16, 16)),
                                         (torch.bfloat16, (4, 128, 32, 32)),
                                         (torch.float32, (128, 128, 32, 32)),   # grid-strided
                                         (torch.bfloat16, (3, 256, 5, 7))],
                         ids=lambda v: str(v))
def test_join_backward_casts_conv_dy_like_the_unfused_pair(dtype, shape):
    g = torch.Generator().manual_seed(sum(shape))
    a0 = cl(torch.randn(shape, generator=g).to(dtype))
    b0 = cl(torch.randn(shape, generator=g).to(torch.bfloat16))
    gy = cl(torch.randn(shape, generator=g).to(dtype))

    def run(hd):
        a, b = a0.clone().requires_grad_(), b0.clone().requires_grad_()
        y = R.residual_join(a, b, hd)
        y.backward(gy)
        return y, a.grad, b.grad

    ref = run(None)
    for s in scales_for(ref[2]):
        hu, hf = hand(s), hand(s)
        hu.fill_from_bf16(ref[2])
        got = run(hf)
        torch.cuda.synchronize()
        assert not got[2].any()           # b's gradient went to the hand-off
        assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])
        assert np.array_equal(q_bytes(hf.q), q_bytes(hu.q)), (s, shape)
        assert amax_bits(hf) == amax_bits(hu)


def test_handoff_take_rejects_a_real_gradient():
    """A conv whose output gradient is not its producer's placeholder (another consumer added
    to it) is an error, not a silent use of a partial gradient."""
    h = hand(1.0)
    h.q = torch.zeros(8, device="cuda", dtype=torch.uint8)
    with pytest.raises(RuntimeError):
        h.take(torch.ones((2, 4, 2, 2), device="cuda"))
    assert h.take(K.placeholder((2, 4, 2, 2), torch.bfloat16, "cuda")) is not None
    with pytest.raises(RuntimeError):
        h.take(K.placeholder((2, 4, 2, 2), torch.bfloat16, "cuda"))   # taken once


def _state(handoff: bool):
    cfg = U.cfg5_config(p_drop=0.2)
    st = T.TrainState(cfg, batch=4, seed=0, fixed_noise=True)
    for m in st.model.modules():
        if isinstance(m, U.ResidualBlock):
            m.fp8_handoff = handoff
    g = torch.Generator().manual_seed(4)
    images = torch.rand((4, 3, 32, 32), generator=g) * 2 - 1
    t = torch.randint(0, 1000, (4,), generator=g)
    eps = torch.randn((4, 3, 32, 32), generator=g)
    st.set_batch(images.cuda(), t.cuda(), eps.cuda())
    return st


def test_cfg5_steps_with_handoffs_equal_steps_without(monkeypatch):
    """Three eager cfg5 training steps (delayed scaling, dropout 0.2, prepared weights) with the
    producer hand-offs against the same steps with the standalone casts: identical losses,
    parameters, gradients and window buffers, bit for bit -- and no standalone delayed cast
    left in the hand-off steps (the first step records the FP8 layers and casts per call)."""
    # the comparison is bitwise, so every other kernel must be deterministic: the attention
    # in its dense form (the fused SDPA backward accumulates dq with atomics) and MIOpen's
    # bf16 convs (conv_in / the output conv) restricted to deterministic solutions
    monkeypatch.setattr(U, "_GPU_SDPA", False)
    monkeypatch.setattr(torch.backends.cudnn, "deterministic", True)
    calls = {"n": 0}
    real = K.quantize_fp8_delayed_deferred

    def counting(*a, **kw):
        calls["n"] += 1
        return real(*a, **kw)

    monkeypatch.setattr(K, "quantize_fp8_delayed_deferred", counting)
    a, b = _state(True), _state(False)
    per_step = {}
    for name, st in (("fused", a), ("unfused", b)):
        losses = []
        for i in range(3):
            torch.cuda.manual_seed(100 + i)
            calls["n"] = 0
            st.loss_acc.zero_()
            st.eager_step()
            torch.cuda.synchronize()
            losses.append(float(st.loss_acc))
            per_step[(name, i)] = calls["n"]
        if st.model._wprep is not None:
            st.model._wprep.flush()
        torch.cuda.synchronize()
        per_step[name] = losses
    print(f"standalone delayed casts per step: {per_step}", flush=True)
    assert per_step["fused"] == per_step["unfused"], per_step
    assert per_step[("unfused", 2)] == 86            # x and dy of the 43 delayed convs
    assert per_step[("fused", 2)] == 0
    for (na, pa), pb in zip(a.model.named_parameters(), b.model.parameters()):
        assert torch.equal(pa, pb), (na, float((pa - pb).abs().max()))
        assert (pa.grad is None) == (pb.grad is None), na
        assert pa.grad is None or torch.equal(pa.grad, pb.grad), na
    for (na, ba), bb in zip(a.model.named_buffers(), b.model.buffers()):
        assert torch.equal(ba, bb), na
