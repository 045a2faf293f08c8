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


# ---------------------------------------------------------------------------------------
# The hand-offs against the oracle: the bytes a producer writes equal the oracle's cast of the
# oracle's bf16 value (diffusion/fp8_kernels.py:69-87 with the window scale, :835 / :856 /
# :885-893 for where the bf16 value comes from), not only the same build's unfused pair.
# ---------------------------------------------------------------------------------------
from oracle import fp8_oracle as O  # noqa: E402


def _oracle_film(wb: torch.Tensor, c: int):
    """(bf16(bf16(w) + 1), b) of the FiLM projection [w | b], as the kernel and the reference's
    autocast chunk / add form them (diffusion/unet.py:157-158)."""
    wb32 = wb.detach().float().cpu().reshape(wb.shape[0], 2 * c)
    fs = (wb32[:, :c].to(torch.bfloat16).float() + 1).to(torch.bfloat16).float().numpy()
    return fs, wb32[:, c:].numpy()


def _nhwc_in(x: torch.Tensor) -> np.ndarray:
    """x as the oracle takes it: NHWC bf16 bits, or NHWC fp32 values."""
    t = x.detach().cpu().permute(0, 2, 3, 1).contiguous()
    return t.numpy() if t.dtype == torch.float32 else t.view(torch.int16).numpy().view(np.uint16)


def _bf16_nhwc(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.bfloat16).cpu().permute(0, 2, 3, 1).contiguous() \
        .view(torch.int16).numpy().view(np.uint16)


def _check_vs_oracle(hf, unfused_bits, oracle_bits, scale, what, min_exact=0.995):
    """The hand-off's e4m3 bytes equal the oracle's cast of the oracle's bf16 value wherever
    that bf16 value is the one the unfused kernel writes (elsewhere the bf16 values differ by
    a float32-vs-float64 rounding, within the producer's own tolerance), and on at least
    ``min_exact`` of all elements; its amax equals the oracle's amax of the bf16 values."""
    s = np.float32(scale)
    want = O.cast_e4m3(oracle_bits, s)
    got = q_bytes(hf.q).reshape(want.shape)
    same16 = unfused_bits == oracle_bits
    assert np.array_equal(got[same16], want[same16]), \
        (what, int((got[same16] != want[same16]).sum()))
    frac = float(np.mean(got == want))
    assert frac >= min_exact, (what, frac, float(np.mean(same16)))
    mag_o = oracle_bits & np.uint16(0x7FFF)
    mag_u = unfused_bits & np.uint16(0x7FFF)
    a_o, a_h = int(mag_o.max()), amax_bits(hf)
    assert a_h == int(mag_u.max()), what
    # one bf16 ulp at most; exactly the oracle's when the two agree on every element near
    # the maximum
    assert abs(a_h - a_o) <= 1, (what, a_h, a_o)
    near = mag_o.astype(np.int64) >= a_o - 1
    if np.array_equal(mag_u[near], mag_o[near]):
        assert a_h == a_o, (what, a_h, a_o)
    return frac


ORACLE_FWD_CASES = [
    # (n, c, h, w, x fp32, film + dropout): resident (<= 1024 pixels) and chunked forms
    (2, 128, 32, 32, False, False),    # GN1 (tee) at the first level, bf16 x
    (2, 128, 32, 32, True, True),      # GN2 with FiLM + dropout, fp32 x
    (3, 256, 16, 16, True, False),
    (3, 256, 16, 16, False, True),
    (2, 512, 8, 8, False, True),
    (4, 256, 4, 4, True, True),
    (1, 128, 40, 40, False, True),     # chunked form (1600 pixels)
    (1, 128, 48, 40, True, False),     # chunked form, fp32 x
]


@pytest.mark.parametrize("n,c,h,w,x32,film", ORACLE_FWD_CASES, ids=lambda v: str(v))
def test_gn_forward_handoff_vs_oracle(n, c, h, w, x32, film):
    """GN1 (tee, diffusion/unet.py:151) and GN2 (FiLM + dropout, :157-160) writing their
    conv's e4m3 input: bytes against oracle.cast_e4m3(oracle.gn_silu_fwd(...), window scale),
    amax against the oracle's amax of the same bf16 values."""
    seed = n * 313 + c + h + w
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((n, c, h, w), generator=g) * 2.0 + 0.5
    if not x32:
        x = x.to(torch.bfloat16)
    x = cl(x)
    gamma = (1.0 + 0.1 * torch.randn(c, generator=g)).cuda()
    beta = (0.1 * torch.randn(c, generator=g)).cuda()
    wb = cl((0.3 * torch.randn((n, 2 * c, 1, 1), generator=g)).to(torch.bfloat16))
    p = 0.2 if film else 0.0
    drop_seed = seed * 7919 + 11

    def run(hd):
        if film:
            G.DROPOUT_SEEDS.seeds = torch.tensor([drop_seed], device="cuda", dtype=torch.int64)
            G.DROPOUT_SEEDS.next = 0
            try:
                out = G.group_norm_silu_film(x, gamma, beta, GROUPS, 1e-5, wb, p, hd)
                assert G.DROPOUT_SEEDS.next == 1      # the op took the planted seed
            finally:
                G.DROPOUT_SEEDS.clear()
            return out
        return G.group_norm_silu_tee(x, gamma, beta, GROUPS, 1e-5, x32, hd)[0]

    unfused = _bf16_nhwc(run(None))
    fs = fb = None
    if film:
        fs, fb = _oracle_film(wb, c)
    ref = O.gn_silu_fwd(_nhwc_in(x), gamma.cpu().numpy(), beta.cpu().numpy(), GROUPS, 1e-5,
                        fs, fb, drop=(drop_seed, p) if film else None)
    amax = float(O.bf16_bits_to_f32(np.array([np.max(ref & np.uint16(0x7FFF))], np.uint16))[0])
    for s in (amax / 448.0 * 1.3, amax / 448.0 / 3.0, 2.0**-70):
        hf = hand(s)
        out = run(hf)
        torch.cuda.synchronize()
        assert K.is_placeholder(out)
        frac = _check_vs_oracle(hf, unfused, ref, s, (n, c, h, w, x32, film, s))
        print(f"fwd {(n, c, h, w, x32, film)} scale {s:.3e}: e4m3 = oracle on {frac:.5f}",
              flush=True)


ORACLE_BWD_CASES = [
    # (n, c, h, w, dropout): the FiLM GroupNorm backward writing conv_1's e4m3 dy
    (3, 256, 16, 16, True),
    (2, 128, 32, 32, True),
    (2, 512, 8, 8, False),
    (4, 256, 4, 4, True),
    (1, 128, 40, 40, True),            # chunked form
]


@pytest.mark.parametrize("n,c,h,w,drop", ORACLE_BWD_CASES, ids=lambda v: str(v))
def test_gn_backward_handoff_vs_oracle(n, c, h, w, drop):
    """The FiLM GroupNorm's dx (conv_1's output gradient, diffusion/unet.py:157-160 feeding
    diffusion/fp8_kernels.py:885-893) as e4m3 with conv_1's dy window scale: bytes against
    oracle.cast_e4m3(bf16(fp32(oracle.gn_silu_bwd(...).dx)), scale), amax against the
    oracle's."""
    seed = n * 577 + c + h
    g = torch.Generator().manual_seed(seed)
    x = cl((torch.randn((n, c, h, w), generator=g) * 2.0 + 0.5).to(torch.bfloat16))
    gamma = (1.0 + 0.1 * torch.randn(c, generator=g)).cuda()
    beta = (0.1 * torch.randn(c, generator=g)).cuda()
    wb0 = (0.3 * torch.randn((n, 2 * c, 1, 1), generator=g)).to(torch.bfloat16)
    dout = cl((torch.randn((n, c, h, w), generator=g) * 1e-2).to(torch.bfloat16))
    p = 0.2 if drop else 0.0
    drop_seed = seed * 104729 + 3

    def run(hd):
        xd = x.detach().clone().requires_grad_()
        G.DROPOUT_SEEDS.seeds = torch.tensor([drop_seed], device="cuda", dtype=torch.int64)
        G.DROPOUT_SEEDS.next = 0
        try:
            y = G.group_norm_silu_film(xd, gamma, beta, GROUPS, 1e-5, cl(wb0), p, None, hd)
        finally:
            G.DROPOUT_SEEDS.clear()
        y.backward(dout)
        return xd.grad

    unfused = _bf16_nhwc(run(None))
    fs, fb = _oracle_film(wb0, c)
    rdx = O.gn_silu_bwd(_nhwc_in(x), _nhwc_in(dout), gamma.cpu().numpy(), beta.cpu().numpy(),
                        GROUPS, 1e-5, fs, fb, drop=(drop_seed, p) if drop else None)[0]
    ref = O.f32_to_bf16_bits(rdx.astype(np.float32))
    amax = float(O.bf16_bits_to_f32(np.array([np.max(ref & np.uint16(0x7FFF))], np.uint16))[0])
    for s in (amax / 448.0 * 1.3, amax / 448.0 / 3.0, 2.0**-70):
        hf = hand(s)
        got = run(hf)
        torch.cuda.synchronize()
        assert not got.any()
        frac = _check_vs_oracle(hf, unfused, ref, s, (n, c, h, w, drop, s))
        print(f"bwd {(n, c, h, w, drop)} scale {s:.3e}: e4m3 = oracle on {frac:.5f}", flush=True)


@pytest.mark.parametrize("dtype,shape", [(torch.float32, (4, 256, 16, 16)),
                                         (torch.bfloat16, (4, 128, 32, 32)),
                                         (torch.float32, (128, 128, 32, 32)),
                                         (torch.bfloat16, (3, 256, 5, 7))],
                         ids=lambda v: str(v))
def test_join_backward_handoff_vs_oracle(dtype, shape):
    """The residual join's backward writing conv_2's dy (diffusion/unet.py:161 feeding
    diffusion/fp8_kernels.py:885-893): b's gradient is bf16(RN32(f32(g) * RN32(1/sqrt 2))), an
    exact oracle, so every e4m3 byte and the amax equal the oracle's."""
    g = torch.Generator().manual_seed(sum(shape) + 5)
    a0 = cl(torch.randn(shape, generator=g).to(dtype))
    b0 = cl(torch.randn(shape, generator=g).to(torch.bfloat16))
    gy = cl((torch.randn(shape, generator=g) * 3e-2).to(dtype))
    g32 = gy.detach().float().cpu().permute(0, 2, 3, 1).contiguous().numpy()
    inv = np.float32(np.float32(1.0) / np.float32(np.sqrt(2.0)))
    ref = O.f32_to_bf16_bits((g32 * inv).astype(np.float32))
    amax = float(O.amax_bf16(ref))
    for s in (amax / 448.0 * 1.3, amax / 448.0 / 3.0, 2.0**-70):
        hf = hand(s)
        a, b = a0.clone().requires_grad_(), b0.clone().requires_grad_()
        R.residual_join(a, b, hf).backward(gy)
        torch.cuda.synchronize()
        want = O.cast_e4m3(ref, np.float32(s))
        assert np.array_equal(q_bytes(hf.q).reshape(want.shape), want), (shape, s)
        assert amax_bits(hf) == int(np.max(ref & np.uint16(0x7FFF)))


def _nhwc16(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.bfloat16).permute(0, 2, 3, 1).contiguous().cpu() \
        .view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("hist,warm", [(1024, 3), (16, 20)], ids=["window1024", "window16"])
def test_cfg5_handoffs_per_site_vs_oracle(monkeypatch, hist, warm):
    """Every delayed conv of a cfg5 training step (batch 16, dropout 0.1), hand-offs on: the
    e4m3 input and dy each conv received equal oracle.cast_e4m3 of the bf16 tensor the
    unfused producer writes in the same step from the same state, at the scale
    max(window) of that conv's own windows as the state before the step holds them
    (diffusion/unet.py:69-73, fp8_kernels.py:845-856, :881-893); the window records the step
    leaves equal the oracle's scale of those bf16 tensors at the right slots (acts and weights
    at window_pos, dy one slot ahead, position advanced by one). Run once from the state after
    the reference's 3 warm-up steps with its 1024-slot windows, and once with 16-slot windows
    after 20 steps (every slot live, positions wrapped)."""
    cfg = U.cfg5_config(p_drop=0.1, fp8_amax_history=hist)
    batch = 16
    st = T.TrainState(cfg, batch=batch, seed=0, fixed_noise=True)
    g = torch.Generator().manual_seed(4)
    images = torch.rand((batch, 3, 32, 32), generator=g) * 2 - 1
    t = torch.randint(0, 1000, (batch,), generator=g)
    eps = torch.randn((batch, 3, 32, 32), generator=g)
    st.set_batch(images.cuda(), t.cuda(), eps.cuda())
    for i in range(warm):
        torch.cuda.manual_seed(1000 + i)
        st.eager_step()
    wp = st.model._wprep
    wp.flush()
    torch.cuda.synchronize()
    state0 = {k: v.clone() for k, v in st.model.state_dict().items()}
    mods = dict(st.model.named_modules())
    # the delayed convs that ran: their weight windows hold the warm-up steps' records
    delayed = [n for n, m in mods.items() if isinstance(m, U.Conv2dFP8)
               and hasattr(m, "window_pos") and float(m.amax_window_weights.abs().max()) > 0]

    def one_pass(handoff: bool):
        """forward + backward of the step (no optimizer update) from state0; returns what each
        delayed conv received and the windows after the step."""
        st.model.load_state_dict(state0)
        monkeypatch.setattr(U.ResidualBlock, "fp8_handoff", handoff)
        got: dict[str, dict] = {n: {} for n in delayed}
        hooks, dyh_owner = [], {}
        for n in delayed:
            def pre(mod, args, n=n):
                if handoff:
                    assert len(args) == 3 and args[1] is not None and args[2] is not None, n
                    got[n]["xq"] = args[1]
                    dyh_owner[id(args[2])] = n
                else:
                    assert len(args) == 1, n
                    got[n]["x16"] = args[0].detach().clone()

            def post(mod, args, out, n=n):
                if not handoff:
                    out.register_hook(lambda gr, n=n: got[n].__setitem__("dy16", gr.detach().clone()))

            hooks += [mods[n].register_forward_pre_hook(pre), mods[n].register_forward_hook(post)]
        real_take = K.Fp8Handoff.take

        def take(self, grad):
            q = real_take(self, grad)
            if id(self) in dyh_owner:
                got[dyh_owner[id(self)]]["dyq"] = q
            return q

        monkeypatch.setattr(K.Fp8Handoff, "take", take)
        try:
            torch.cuda.manual_seed(77)                # the same dropout seeds in both passes
            st.optimizer.zero_grad(set_to_none=True)
            with torch.autocast("cuda", dtype=torch.bfloat16):
                loss = st.ddpm.forward_batch(st.static_batch, st.static_t, st.static_eps)
            loss.backward()
            wp.flush()
            torch.cuda.synchronize()
        finally:
            for h in hooks:
                h.remove()
            monkeypatch.setattr(K.Fp8Handoff, "take", real_take)
        wins = {n: tuple(getattr(mods[n], w).clone() for w in
                         ("amax_window_acts", "amax_window_weights", "amax_window_dy", "window_pos"))
                for n in delayed}
        return float(loss.detach()), got, wins

    loss_u, unfused, wins_u = one_pass(False)
    loss_f, fused, wins_f = one_pass(True)
    assert loss_u == loss_f
    assert len(delayed) == 43, len(delayed)
    for n in delayed:
        u, f = unfused[n], fused[n]
        assert {"xq", "dyq"} <= set(f), (n, set(f))
        pre = f"{n}."
        acts0, w0, dy0, pos0 = (state0[pre + k] for k in
                                ("amax_window_acts", "amax_window_weights", "amax_window_dy",
                                 "window_pos"))
        xs_h = np.float32(acts0.max().item())
        dys_h = np.float32(dy0.max().item())
        x16, dy16 = _nhwc16(u["x16"]), _nhwc16(u["dy16"])
        want_x = O.cast_e4m3(x16, xs_h)
        want_dy = O.cast_e4m3(dy16, dys_h)
        got_x = f["xq"].view(torch.uint8).permute(0, 2, 3, 1).contiguous().cpu().numpy()
        got_dy = f["dyq"].view(torch.uint8).permute(0, 2, 3, 1).contiguous().cpu().numpy()
        assert np.array_equal(got_x, want_x), (n, int((got_x != want_x).sum()))
        assert np.array_equal(got_dy, want_dy), (n, int((got_dy != want_dy).sum()))
        # the window records of the step
        p = int(pos0)
        p1 = (p + 1) % hist
        acts, wts, dyw, pos = wins_f[n]
        for a, b in zip(wins_f[n], wins_u[n]):
            assert torch.equal(a, b), n
        assert int(pos) == p1, n
        assert np.float32(acts[p].item()) == O.scale_from_amax(O.amax_bf16(x16)), n
        assert np.float32(dyw[p1].item()) == O.scale_from_amax(O.amax_bf16(dy16)), n
        wq16 = _nhwc16(mods[n].conv.weight.detach())
        assert np.float32(wts[p].item()) == O.scale_from_amax(O.amax_bf16(wq16)), n
        # every other slot unchanged
        keep = torch.ones(hist, dtype=torch.bool)
        keep[p] = False
        assert torch.equal(acts.cpu()[keep], acts0.cpu()[keep]), n
        assert torch.equal(wts.cpu()[keep], w0.cpu()[keep]), n
        keep = torch.ones(hist, dtype=torch.bool)
        keep[p1] = False
        assert torch.equal(dyw.cpu()[keep], dy0.cpu()[keep]), n
    nz = sum(int((fused[n]["dyq"].view(torch.uint8) & 0x7F).count_nonzero()) for n in delayed)
    print(f"window {hist}: {len(delayed)} convs, loss {loss_f:.5f}, nonzero dy bytes {nz}",
          flush=True)
