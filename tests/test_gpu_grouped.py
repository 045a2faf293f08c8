"""Grouped FP8 linears over one shared input -- the FiLM projections of the U-Net's residual
blocks (diffusion/unet.py:101-104, :135) in one launch per direction: the quantized bytes and
scales of every layer against the per-tensor quantization, the forward, the weight gradients
and the summed input gradient against the exact oracle on the operands the op quantized, and a
cfg5 U-Net step with the grouped projections against the per-layer ones.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import assert_bf16_close, bits, dpa_mod, kaiming_uniform_bf16, randn_bf16
from oracle import fp8_oracle as O

pytestmark = pytest.mark.gpu

K = dpa_mod("fp8_kernels")
GR = dpa_mod("grouped")
U = dpa_mod("unet")
T = dpa_mod("trainer")

NS = [256, 512, 512, 256, 512, 384]


def _u8(t):
    return t.view(torch.uint8).cpu().numpy()


def test_grouped_quantize_equals_per_tensor():
    srcs = [(randn_bf16((128, n), seed=i).float() * (10.0 ** (i - 3))).to(torch.bfloat16).cuda()
            for i, n in enumerate(NS)]
    srcs[2].zero_()                                     # amax 0: scale 1
    q, qt, sc = GR.grouped_quantize(srcs)
    torch.cuda.synchronize()
    off = 0
    for i, s in enumerate(srcs):
        rq, rs = K.quantize_fp8_tensor(s)
        n = s.shape[1]
        assert np.array_equal(_u8(q)[:, off:off + n], _u8(rq)), i
        assert np.array_equal(_u8(qt)[off:off + n, :], _u8(rq).T), i
        assert float(sc[i]) == float(rs), i
        oq, os_ = O.quantize_fp8(bits(s.cpu()))
        assert np.array_equal(_u8(rq), oq) and np.float32(float(rs)) == os_
        off += n


@pytest.mark.parametrize("m", [128, 256])
def test_grouped_linear_vs_oracle(m):
    """y_i, dw_i and dx of the grouped op against the oracle GEMMs on the bytes it quantized
    (x once, each dy_i with its own scale; the weights prepared per layer)."""
    k = 512
    x = randn_bf16((m, k), seed=10).cuda().requires_grad_()
    params = [kaiming_uniform_bf16((n, k), seed=20 + i).float().cuda().requires_grad_()
              for i, n in enumerate(NS)]
    layers = []
    for w in params:
        wq, ws = K.quantize_fp8_tensor(w.detach().to(torch.bfloat16))
        wqt = wq.view(torch.uint8).t().contiguous().view(K.FP8_DTYPE)
        layers.append((wq, wqt, ws.reshape(1)))
    ys = GR.grouped_linear_fp8(x, layers, params)
    dys = [randn_bf16((m, n), seed=40 + i, std=1e-2).cuda() for i, n in enumerate(NS)]
    torch.autograd.backward(ys, dys)
    torch.cuda.synchronize()

    xq, xs = O.quantize_fp8(bits(x.detach().cpu()))
    dx_ref = np.zeros((m, k), np.float64)
    for i, (w, (wq, _, ws), y, dy) in enumerate(zip(params, layers, ys, dys)):
        wqb, wsf = _u8(wq), np.float32(float(ws))
        assert_bf16_close(bits(y.detach().cpu()), O.gemm(xq, wqb, xs, wsf), f"fwd {i}")
        dyq, dys_ = O.quantize_fp8(bits(dy.cpu()))
        assert_bf16_close(bits(w.grad.to(torch.bfloat16).cpu()),
                          O.gemm(np.ascontiguousarray(dyq.T), np.ascontiguousarray(xq.T), dys_, xs),
                          f"dw {i}")
        assert w.grad.dtype == torch.float32
        # the fp32 grad holds bf16 values
        assert torch.equal(w.grad, w.grad.to(torch.bfloat16).float())
        s = np.float32(dys_ * wsf)
        dx_ref += (O.e4m3_to_f32(dyq).astype(np.float64) @ O.e4m3_to_f32(wqb).astype(np.float64)) * s
    ref_bits = O.f32_to_bf16_bits(dx_ref.astype(np.float32))
    assert x.grad.dtype == torch.bfloat16
    assert_bf16_close(bits(x.grad.cpu()), ref_bits, "dx (sum over layers)")


def test_unet_grouped_films_match_per_layer():
    """A cfg5 U-Net training step (batch 128, prepared weights) with the 22 FiLM projections as
    one grouped op against the same step with them per layer: the grouped op runs once per
    forward, the losses agree to 1e-3 and every parameter to the graph test's bounds."""
    calls = {"n": 0}
    real = GR.GroupedLinearFP8.apply

    def counting(*a):
        calls["n"] += 1
        return real(*a)

    GR.GroupedLinearFP8.apply = counting
    try:
        states = []
        for grouped in (True, False):
            st = T.TrainState(U.cfg5_config(p_drop=0.0), batch=128, seed=0, fixed_noise=True)
            st.model.group_films = grouped
            g = torch.Generator().manual_seed(4)
            st.set_batch((torch.rand((128, 3, 32, 32), generator=g) * 2 - 1).cuda(),
                         torch.randint(0, 1000, (128,), generator=g).cuda(),
                         torch.randn((128, 3, 32, 32), generator=g).cuda())
            losses = []
            calls["n"] = 0
            for i in range(3):
                torch.cuda.manual_seed(7 + i)
                st.loss_acc.zero_()
                st.eager_step()
                losses.append(float(st.loss_acc))
            torch.cuda.synchronize()
            states.append((st, losses, calls["n"]))
    finally:
        GR.GroupedLinearFP8.apply = real
    (a, la, na), (b, lb, nb) = states
    print(f"losses grouped {la} per-layer {lb}; grouped calls {na} / {nb}", flush=True)
    assert na == 2 and nb == 0          # steps 2 and 3 (the first step records the FP8 layers)
    for x, y in zip(la, lb):
        assert np.isfinite(x) and x == pytest.approx(y, rel=1e-3)
    for (name, p), q in zip(a.model.named_parameters(), b.model.parameters()):
        d = float((p.detach() - q.detach()).float().norm())
        bound = 1e-4 * float(q.detach().float().norm()) + 1e-5 * np.sqrt(q.numel())
        assert d <= bound, (name, d, bound)
