"""GPU tests of the grouped FP8 weight preparation (weight_prep.WeightPrep and the
dpa_weight_prep_* / dpa_window_max_grouped_f32 entries): every FP8 layer type with its weight
prepared for the step gives the same bytes as the per-call path (the reference's per-layer
quantization, diffusion/unet.py:69-91 and fp8_kernels.py:822-913): outputs, input gradients,
fp32 weight gradients (autograd's cast of the bf16 gradient), amax windows and positions, over
steps that wrap the window (the prepared path writes a step's x / dy window records at the
start of the next step, or at flush()); and the prepared e4m3 weights and transposes equal the
per-layer quantization and weight transpose.
"""
from __future__ import annotations

import math

import pytest
import torch

from conftest import dpa_mod, randn_bf16

pytestmark = pytest.mark.gpu

K = dpa_mod("fp8_kernels")
U = dpa_mod("unet")
T = dpa_mod("trainer")
WP = dpa_mod("weight_prep")


def _pair(make):
    torch.manual_seed(3)
    a = make().cuda().to(memory_format=torch.channels_last)
    b = make().cuda().to(memory_format=torch.channels_last)
    b.load_state_dict(a.state_dict())
    return a, b


def _weight(m):
    return m.conv.weight if hasattr(m, "conv") else m.weight


LAYERS = {
    # registry shape, delayed scaling (window of 3 so the steps wrap it)
    "conv3x3_delayed": (lambda: U.Conv2dFP8(128, 128, True, "delayed", amax_history=3,
                                            fp8_all_convs=True), (2, 128, 32, 32)),
    # 8x8 with 128 -> 256 channels: outside the registry, current scaling (general path)
    "conv3x3_current": (lambda: U.Conv2dFP8(128, 256, True, "delayed", amax_history=3,
                                            fp8_all_convs=True), (2, 128, 8, 8)),
    "conv1x1": (lambda: U.Conv1x1FP8(256, 128, True), (2, 256, 16, 16)),
    "linear": (lambda: U.LinearFP8(512, 256, bias=False, fp8=True), (128, 512)),
}


@pytest.mark.parametrize("kind", list(LAYERS))
def test_prepared_layer_matches_per_call_path(kind):
    make, xshape = LAYERS[kind]
    a, b = _pair(make)
    plan = None
    for step in range(5):
        x = randn_bf16(xshape, seed=10 + step, std=0.5 + step)
        gy = None
        outs = []
        for mod in (a, b):
            xd = x.cuda()
            if xd.ndim == 4:
                xd = xd.contiguous(memory_format=torch.channels_last)
            xd.requires_grad_()
            _weight(mod).grad = None
            if mod is a and plan is not None:
                plan.run()
                plan.active = True
            with torch.autocast("cuda", dtype=torch.bfloat16):
                y = mod(xd)
            if mod is a and plan is not None:
                plan.active = False
            if gy is None:
                gy = (randn_bf16(tuple(y.shape), seed=20 + step, std=1e-2 * (step + 1)).cuda()
                      .to(y.dtype))
                if y.ndim == 4:
                    gy = gy.contiguous(memory_format=torch.channels_last)
            y.backward(gy)
            outs.append((y.detach(), xd.grad, _weight(mod).grad.clone()))
        if plan is not None:
            plan.flush()                             # the step's deferred window records
        torch.cuda.synchronize()
        if plan is None:
            assert a._fp8_mode is not None, kind     # recorded on the first GPU call
            plan = WP.WeightPrep([a])
            assert a._fp8_prepared is not None
        else:
            assert outs[0][2].dtype == torch.float32
        for name in ("amax_window_acts", "amax_window_weights", "amax_window_dy", "window_pos"):
            if hasattr(a, name):
                assert torch.equal(getattr(a, name), getattr(b, name)), (kind, step, name)
        for what, ta, tb in zip(("y", "dx", "dw"), *outs):
            assert ta.dtype == tb.dtype and ta.shape == tb.shape, (kind, step, what)
            assert torch.equal(ta, tb), (kind, step, what)


def test_prepared_bytes_equal_per_layer_quantization():
    """Several weights in one plan (blocks of different tensors in one launch): q equals
    quantize_fp8 of the bf16 weight, qt equals weight_transpose_fp8, scales match."""
    mods = [U.Conv1x1FP8(256, 128, True), U.Conv1x1FP8(512, 256, True),
            U.LinearFP8(512, 1024, bias=False, fp8=True), U.LinearFP8(128, 512, bias=False, fp8=True)]
    torch.manual_seed(0)
    for m in mods:
        m.cuda().to(memory_format=torch.channels_last)
        with torch.no_grad():
            _weight(m).mul_(torch.linspace(0.5, 3.0, _weight(m).numel(), device="cuda")
                            .reshape(_weight(m).shape))
        m._fp8_mode = "linear" if isinstance(m, U.LinearFP8) else "current"
    plan = WP.WeightPrep(mods)
    plan.run()
    torch.cuda.synchronize()
    for m in mods:
        w = _weight(m)
        wb = w.to(torch.bfloat16)       # autocast's cast; keeps the channels-last layout
        q_ref, s_ref = K.quantize_fp8_tensor(wb)
        pw = m._fp8_prepared
        assert torch.equal(pw.q.view(torch.uint8), q_ref.view(torch.uint8))
        assert float(pw.scale) == float(s_ref)
        q4 = pw.q if w.ndim == 4 else pw.q[:, :, None, None]
        qt_ref = K.weight_transpose_fp8(q4)
        assert torch.equal(pw.qt.view(torch.uint8).flatten(), qt_ref.view(torch.uint8).flatten())


def test_unet_steps_with_and_without_weight_prep():
    """Full U-Net (delayed scaling, all convs and linears FP8) with the same dropout masks:
    eager training steps with the grouped preparation (from the second step on) give the
    per-call path's loss, parameters, amax windows and positions bit for bit. The bf16 input
    and output convs (MIOpen) are excluded: their weight gradients are not bit-reproducible
    from run to run, so they get a tolerance, and the check stops before their differences
    reach the activations (two steps)."""
    def state(prep):
        st = T.TrainState(U.cfg5_config(), batch=4, seed=0, fixed_noise=True)
        st.model.weight_prep_enabled = prep
        g = torch.Generator().manual_seed(4)
        st.set_batch((torch.rand((4, 3, 32, 32), generator=g) * 2 - 1).cuda(),
                     torch.randint(0, 1000, (4,), generator=g).cuda(),
                     torch.randn((4, 3, 32, 32), generator=g).cuda())
        return st

    bf16_convs = ("conv_in.weight", "out.2.weight")
    a, b = state(True), state(False)
    for i in range(2):
        a.loss_acc.zero_()
        b.loss_acc.zero_()
        for st in (a, b):
            torch.manual_seed(100 + i)
            st.eager_step()
        if a.model._wprep is not None:
            a.model._wprep.flush()                   # the step's deferred window records
        torch.cuda.synchronize()
        la, lb = float(a.loss_acc), float(b.loss_acc)
        assert math.isfinite(la) and la == lb, (i, la, lb)
        for (name, p), q in zip(a.model.named_parameters(), b.model.parameters()):
            if name in bf16_convs:
                torch.testing.assert_close(p, q, rtol=1e-3, atol=1e-6, msg=f"step {i}: {name}")
            else:
                assert torch.equal(p, q), (i, name)
        for (name, buf), q in zip(a.model.named_buffers(), b.model.buffers()):
            assert torch.equal(buf, q), (i, name)
    assert a.model._wprep is not None and a.model._wprep.count > 50
    assert b.model._wprep is None


def test_tensor_prep_bf16_weights_equal_quantize_and_transpose():
    """TensorPrep on bf16 weights (cfg2's weight is bf16): q == quantize_fp8(w), the same
    scale, qt == weight_transpose_fp8(q); 3x3, 1x1 and 2-D weights in one plan, ragged
    tiles (Cout 192 is three 64-row tiles), two runs after an in-place weight update."""
    g = torch.Generator().manual_seed(7)
    ws = [(torch.randn((128, 128, 3, 3), generator=g) * 0.05).to(torch.bfloat16),
          (torch.randn((192, 256, 1, 1), generator=g) * 3.0).to(torch.bfloat16),
          (torch.randn((768, 256), generator=g)).to(torch.bfloat16)]
    ws = [w.cuda().contiguous(memory_format=torch.channels_last) if w.ndim == 4 else w.cuda()
          for w in ws]
    tp = WP.TensorPrep(ws)
    for rnd in range(2):
        if rnd:
            for w in ws:
                w.mul_(1.5)
        tp.run()
        torch.cuda.synchronize()
        for i, w in enumerate(ws):
            q_ref, s_ref = K.quantize_fp8_tensor(w)
            assert torch.equal(tp.q[i].view(torch.uint8), q_ref.view(torch.uint8)), (rnd, i)
            assert float(tp.scale(i)) == float(s_ref), (rnd, i)
            q4 = tp.q[i] if w.ndim == 4 else tp.q[i][:, :, None, None]
            qt_ref = K.weight_transpose_fp8(q4)
            assert torch.equal(tp.qt[i].view(torch.uint8).flatten(),
                               qt_ref.view(torch.uint8).flatten()), (rnd, i)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_tensor_prep_fragment_layouts_equal_quantize_and_frag(dtype):
    """TensorPrep with frag=True (DPA_WP_FRAG): q and qt are the halo-patch kernel's forward
    and data-gradient fragment layouts of quantize_fp8(bf16(w)), byte for byte, beside an
    OHWI entry in the same plan; the scale is quantize_fp8's."""
    g = torch.Generator().manual_seed(11)
    ws = [(torch.randn((256, 128, 3, 3), generator=g) * 0.05).to(dtype),
          (torch.randn((128, 256, 3, 3), generator=g) * 2.0).to(dtype),
          (torch.randn((128, 128, 3, 3), generator=g)).to(dtype)]
    ws = [w.cuda().contiguous(memory_format=torch.channels_last) for w in ws]
    tp = WP.TensorPrep(ws, frag=[True, True, False])
    tp.run()
    torch.cuda.synchronize()
    for i, w in enumerate(ws):
        q_ref, s_ref = K.quantize_fp8_tensor(w.to(torch.bfloat16))
        assert float(tp.scale(i)) == float(s_ref), i
        if i < 2:
            wf, wt = K.weight_frag_fp8(q_ref)
            torch.cuda.synchronize()
            assert tp.q[i].dtype == torch.uint8 and torch.equal(tp.q[i], wf), i
            assert torch.equal(tp.qt[i], wt), i
        else:
            assert torch.equal(tp.q[i].view(torch.uint8), q_ref.view(torch.uint8))


@pytest.mark.parametrize("case", ["cfg2", "ragged", "small", "unaligned"])
def test_quantize_with_weight_prep_equals_the_two_calls(case):
    """dpa_quantize_fp8_bf16_with_weight_prep (TensorPrep.run_with_quantize): x's e4m3 bytes
    and scale equal quantize_fp8(x), and the prepared weights (fragment layout, OHWI, 2-D, bf16
    and fp32) equal run()'s, byte for byte. cfg2's x (the combined launches), a length with a
    ragged tail of 5, and the fallbacks to the two calls (x of one workgroup, x not 16-B
    aligned); two rounds, the second after the weights and x change in place."""
    g = torch.Generator().manual_seed(13)
    ws = [(torch.randn((128, 128, 3, 3), generator=g) * 0.05).to(torch.bfloat16),
          (torch.randn((256, 128, 1, 1), generator=g) * 3.0),
          (torch.randn((768, 256), generator=g)).to(torch.bfloat16)]
    ws = [w.cuda().contiguous(memory_format=torch.channels_last) if w.ndim == 4 else w.cuda()
          for w in ws]
    frag = [True, False, False]
    n = {"cfg2": 128 * 128 * 32 * 32, "ragged": 3 * 1000 * 1000 + 5, "small": 4000,
         "unaligned": 1 << 20}[case]
    base = randn_bf16((n + 1,), seed=17, std=2.0).cuda()
    x = base[1:] if case == "unaligned" else base[:n]
    if case == "cfg2":
        x = x.view(128, 32, 32, 128).permute(0, 3, 1, 2)  # NCHW view, channels-last memory
    fused, sep = WP.TensorPrep(ws, frag=frag), WP.TensorPrep(ws, frag=frag)
    for rnd in range(2):
        if rnd:
            for w in ws:
                w.mul_(1.25)
            x.mul_(-3.0)
        qx, sx = fused.run_with_quantize(x)
        qr, sr = K.quantize_fp8_tensor(x)
        sep.run()
        torch.cuda.synchronize()
        assert float(sx) == float(sr), (case, rnd)
        assert qx.shape == qr.shape and qx.stride() == qr.stride(), (case, rnd)
        assert torch.equal(qx.view(torch.uint8), qr.view(torch.uint8)), (case, rnd)
        assert torch.equal(fused.scales, sep.scales), (case, rnd)
        for i in range(len(ws)):
            assert torch.equal(fused.q[i].view(torch.uint8), sep.q[i].view(torch.uint8)), (rnd, i)
            assert torch.equal(fused.qt[i].view(torch.uint8), sep.qt[i].view(torch.uint8)), (rnd, i)
