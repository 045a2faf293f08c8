"""GPU tests of the module level: the FP8 linear with both gradients, the delayed-scaling
Conv2dFP8 module against the oracle's state machine, a ResidualBlock (cfg4) against the
fake-quant emulation, and the graph-captured U-Net training step against eager steps.
"""
from __future__ import annotations

import copy
import math
import types

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import assert_bf16_close, bits, dpa_mod, kaiming_uniform_bf16, nhwc_bits, randn_bf16
from fakequant import emulate_on_gpu
from oracle import fp8_oracle as O

pytestmark = pytest.mark.gpu

K = dpa_mod("fp8_kernels")
U = dpa_mod("unet")
T = dpa_mod("trainer")
G = dpa_mod("gn_silu")


def f32(t):
    return np.float32(t.item())


def nerr(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def test_linear_fp8_forward_and_gradients_vs_oracle():
    """LinearFP8Function at cfg1's feature sizes (256 -> 768) with ragged rows: y, dx, dw
    against the exact oracle on the operands the function quantized."""
    m, k, n = 1000, 256, 768
    x = randn_bf16((m, k), seed=0).cuda().requires_grad_()
    w = kaiming_uniform_bf16((n, k), seed=1).float().cuda().requires_grad_()
    dy = randn_bf16((m, n), seed=2, std=1e-2).cuda()
    y = K.LinearFP8Function.apply(x, w, None)
    y.backward(dy)
    torch.cuda.synchronize()
    xq, xs = O.quantize_fp8(bits(x.detach().cpu()))
    wq, ws = O.quantize_fp8(bits(w.detach().to(torch.bfloat16).cpu()))
    dyq, dys = O.quantize_fp8(bits(dy.cpu()))
    assert y.dtype == torch.bfloat16 and x.grad.dtype == torch.bfloat16 and w.grad.dtype == torch.float32
    assert_bf16_close(bits(y.detach().cpu()), O.gemm(xq, wq, xs, ws), "linear fwd")
    assert_bf16_close(bits(x.grad.cpu()), O.gemm(dyq, np.ascontiguousarray(wq.T), dys, ws), "linear dx")
    assert_bf16_close(bits(w.grad.to(torch.bfloat16).cpu()),
                      O.gemm(np.ascontiguousarray(dyq.T), np.ascontiguousarray(xq.T), dys, xs),
                      "linear dw")


def test_conv_module_delayed_scaling_vs_oracle():
    """Conv2dFP8 in delayed mode (diffusion/unet.py:69-91): after each fwd+bwd the three
    windows and window_pos equal the oracle's state machine bit for bit, and from the second
    step on y, dx, dw match the oracle conv run with the historical scales."""
    torch.manual_seed(0)
    mod = U.Conv2dFP8(128, 128, True, "delayed", amax_history=4).cuda()
    st = O.DelayedScaling(history=4)
    wb = bits(mod.conv.weight.detach().to(torch.bfloat16).permute(0, 2, 3, 1).contiguous().cpu())
    for step in range(6):
        x = randn_bf16((2, 128, 32, 32), seed=10 + step, std=0.5 + step)
        dy = randn_bf16((2, 128, 32, 32), seed=20 + step, std=1e-2 * (step + 1))
        xd = x.cuda().contiguous(memory_format=torch.channels_last).requires_grad_()
        mod.conv.weight.grad = None
        y = mod(xd)
        y.backward(dy.cuda().contiguous(memory_format=torch.channels_last))
        torch.cuda.synchronize()
        xq, wq, xs_h, ws_h, _, _ = st.forward(nhwc_bits(x), wb)
        dyq, dys_h, _ = st.backward(nhwc_bits(dy))
        np.testing.assert_array_equal(mod.amax_window_acts.cpu().numpy(), st.win_acts)
        np.testing.assert_array_equal(mod.amax_window_weights.cpu().numpy(), st.win_weights)
        np.testing.assert_array_equal(mod.amax_window_dy.cpu().numpy(), st.win_dy)
        assert int(mod.window_pos) == st.pos
        if step == 0:
            continue            # empty history: scale 0, outside the reference's contract
        assert_bf16_close(nhwc_bits(y.detach().cpu()), O.conv2d_fwd(xq, wq, xs_h, ws_h), f"y {step}")
        assert_bf16_close(nhwc_bits(xd.grad.cpu()), O.conv2d_dgrad(dyq, wq, dys_h, ws_h, (32, 32)),
                          f"dx {step}")
        dw = mod.conv.weight.grad.to(torch.bfloat16).permute(0, 2, 3, 1).contiguous().cpu()
        assert_bf16_close(bits(dw), O.conv2d_wgrad(xq, dyq, xs_h, dys_h), f"dw {step}")


def test_conv_module_fused_window_update_matches_op_by_op():
    """The delayed-scaling module with its window bookkeeping fused into the quantization
    launches equals the reference's op-by-op form (torch.max, scatter_, add_, remainder_)
    bit for bit: windows, position, y, dx and dw over steps that wrap the window."""
    torch.manual_seed(1)
    a = U.Conv2dFP8(128, 128, True, "delayed", amax_history=3).cuda()
    b = U.Conv2dFP8(128, 128, True, "delayed", amax_history=3).cuda()
    b.load_state_dict(a.state_dict())
    b.fused_window_update = False
    for step in range(5):
        x = randn_bf16((2, 128, 32, 32), seed=30 + step, std=0.5 + step)
        dy = randn_bf16((2, 128, 32, 32), seed=40 + step, std=1e-2 * (step + 1))
        outs = []
        for mod in (a, b):
            xd = x.cuda().contiguous(memory_format=torch.channels_last).requires_grad_()
            mod.conv.weight.grad = None
            y = mod(xd)
            y.backward(dy.cuda().contiguous(memory_format=torch.channels_last))
            outs.append((y.detach(), xd.grad, mod.conv.weight.grad.clone()))
        torch.cuda.synchronize()
        for name in ("amax_window_acts", "amax_window_weights", "amax_window_dy", "window_pos"):
            assert torch.equal(getattr(a, name), getattr(b, name)), (step, name)
        for ta, tb in zip(*outs):
            assert torch.equal(ta, tb), step


def _cfg(**kw):
    base = dict(fp8_scaling_type="current", p_drop=0.0)
    base.update(kw)
    return U.cfg5_config(**base)


class _OracleDropout(torch.nn.Module):
    """The fused dropout's law written from the oracle: keep mask oracle.dropout_keep(seed, n,
    p) over the NHWC element order, kept values scaled by oracle.dropout_scale(p) in fp32
    (dropout on autocast's fp32 SiLU output, diffusion/unet.py:160)."""

    def __init__(self, seed: int, p: float):
        super().__init__()
        self.seed, self.p, self.calls = seed, p, 0

    def forward(self, h: torch.Tensor) -> torch.Tensor:
        self.calls += 1
        n, c, hh, ww = h.shape
        keep = O.dropout_keep(self.seed, h.numel(), self.p).reshape(n, hh, ww, c)
        keep = torch.from_numpy(keep).to(h.device).permute(0, 3, 1, 2)
        scale = torch.tensor(float(O.dropout_scale(self.p)), dtype=torch.float32, device=h.device)
        return torch.where(keep, h.float() * scale, torch.zeros((), device=h.device))


def _sinusoid(t: torch.Tensor, dim: int) -> torch.Tensor:
    """The U-Net's sinusoidal timestep embedding (diffusion/unet.py:346-351) at ``dim``."""
    half = dim // 2
    freqs = torch.exp(-torch.arange(half, dtype=torch.float32) * (math.log(10000.0) / half))
    emb = t[:, None].float() * freqs[None]
    return torch.cat([emb.sin(), emb.cos()], dim=1)


@pytest.mark.parametrize("cin,cout,hw,batch", [(256, 256, 16, 128), (128, 256, 32, 32)],
                         ids=lambda v: str(v))
def test_resblock_cfg4_vs_fakequant_emulation(cin, cout, hw, batch):
    """cfg4's block at its stated size (GN+SiLU -> FP8 3x3 -> FiLM from the projected 512-d
    sinusoidal embedding of t ~ U{0..999} -> GN+SiLU -> dropout 0.1 -> FP8 3x3 -> residual
    / sqrt 2; 16x16, 256 channels, batch 128), plus a 128 -> 256 block at 32x32 with the FP8
    1x1 skip at batch 32: output and every gradient against the GPU fake-quant emulation
    (torch e4m3 casts, exact fp64 products, float32 GroupNorm + FiLM + SiLU) whose dropout is
    the oracle's mask of the seed the fused kernel took."""
    p = 0.1
    torch.manual_seed(cin + batch)
    blk = U.ResidualBlock(_cfg(), cin, cout, p_drop=p).cuda().to(memory_format=torch.channels_last)
    torch.nn.init.kaiming_uniform_(blk.conv_2.conv.weight, a=math.sqrt(5))   # not the zero init
    with torch.no_grad():
        blk.norm1.weight.uniform_(0.5, 1.5)
        blk.norm2.bias.uniform_(-0.2, 0.2)
    blk.train()
    em = emulate_on_gpu(copy.deepcopy(blk))
    drop_seed = 0x5DEECE66D + batch
    em.dropout = _OracleDropout(drop_seed, p)
    x = randn_bf16((batch, cin, hw, hw), seed=1)
    g = torch.Generator().manual_seed(3)
    t_steps = torch.randint(0, 1000, (batch,), generator=g)
    temb = _sinusoid(t_steps, 512).to(torch.bfloat16)
    dout = randn_bf16((batch, cout, hw, hw), seed=3, std=1e-2).cuda() \
        .contiguous(memory_format=torch.channels_last)

    outs = {}
    for name, mod in (("hip", blk), ("emu", em)):
        xg = x.cuda().contiguous(memory_format=torch.channels_last).requires_grad_()
        tg = temb.cuda().requires_grad_()
        G = dpa_mod("gn_silu")
        G.DROPOUT_SEEDS.seeds = torch.tensor([drop_seed], device="cuda", dtype=torch.int64)
        G.DROPOUT_SEEDS.next = 0
        try:
            with torch.autocast("cuda", dtype=torch.bfloat16):
                out = mod(xg, tg)
            if name == "hip":
                assert G.DROPOUT_SEEDS.next == 1      # the fused dropout took the planted seed
        finally:
            G.DROPOUT_SEEDS.clear()
        out.backward(dout)
        outs[name] = (out.detach(), xg.grad, tg.grad,
                      {n: q.grad for n, q in mod.named_parameters()})
    torch.cuda.synchronize()
    assert em.dropout.calls == 1
    (out, dx, dt, pg), (ref, rdx, rdt, rpg) = outs["hip"], outs["emu"]
    assert out.dtype == torch.bfloat16 and ref.dtype == torch.bfloat16
    errs = {"out": nerr(out, ref), "dx": nerr(dx, rdx), "dt": nerr(dt, rdt)}
    errs.update({n: nerr(pg[n], rpg[n]) for n in pg})
    print(f"cfg4 block {(cin, cout, hw, batch)}: " +
          " ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    assert errs["out"] < 1e-2, errs
    assert errs["dx"] < 2e-2 and errs["dt"] < 2e-2, errs
    for n in pg:
        assert pg[n] is not None, n
        assert errs[n] < 3e-2, (n, errs[n])


def _state(batch, seed=0, **kw):
    st = T.TrainState(_cfg(**kw), batch=batch, seed=seed, fixed_noise=True)
    g = torch.Generator().manual_seed(4)
    images = torch.rand((batch, 3, 32, 32), generator=g) * 2 - 1
    t = torch.randint(0, 1000, (batch,), generator=g)
    eps = torch.randn((batch, 3, 32, 32), generator=g)
    st.set_batch(images.cuda(), t.cuda(), eps.cuda())
    return st


def test_graph_captured_step_matches_eager_steps():
    """prepare_cuda_graph (train.py:104-149) on the full U-Net with delayed scaling: each
    replay gives the loss and parameters of an eager step from the same state, with eager
    work and synchronisation between replays."""
    a = _state(4, fp8_scaling_type="delayed")
    b = _state(4, fp8_scaling_type="delayed")
    a.capture(warmup=3)                           # 3 eager warm-up steps, then capture
    for _ in range(3):
        b.eager_step()
    torch.cuda.synchronize()
    b.loss_acc.zero_()
    a.loss_acc.zero_()
    for i in range(3):
        a.replay()
        torch.cuda.synchronize()
        b.eager_step()
        torch.cuda.synchronize()
        la, lb = float(a.loss_acc), float(b.loss_acc)
        assert math.isfinite(la) and la == pytest.approx(lb, rel=1e-5), (i, la, lb)
        for (name, p), q in zip(a.model.named_parameters(), b.model.parameters()):
            # per tensor, normwise, with an absolute floor of 1e-5 per element (5 % of one
            # AdamW step at lr 2e-4): the bf16 input/output convs (MIOpen) are not
            # bit-reproducible, and AdamW turns that gradient noise into relative differences
            # of small-gradient elements, all of them in the zero-initialised projections
            d = float((p.detach() - q.detach()).float().norm())
            bound = 1e-4 * float(q.detach().float().norm()) + 1e-5 * math.sqrt(q.numel())
            assert d <= bound, (i, name, d, bound)
    for (name, p), q in zip(a.ema_ddpm.model.model.named_parameters(), b.ema_ddpm.model.model.parameters()):
        d = float((p.detach() - q.detach()).float().norm())
        bound = 1e-4 * float(q.detach().float().norm()) + 1e-5 * math.sqrt(q.numel())
        assert d <= bound, ("ema", name, d, bound)
    for (name, buf), q in zip(a.model.named_buffers(), b.model.buffers()):
        if buf.dtype == torch.long:                  # window positions: exact
            assert torch.equal(buf, q), name
        else:
            # amax windows: scales of bf16 amaxes. The MIOpen convs' gradient noise reaches the
            # dy maxima of the deepest blocks: measured 0 on one box and up to 1.4e-2 relative
            # on another (down_stages.3 conv_2 dy windows after six steps), so 2^-5
            torch.testing.assert_close(buf, q, rtol=2**-5, atol=0, msg=name)


def _nonzero_init(model: torch.nn.Module) -> torch.nn.Module:
    """Kaiming-uniform weights for the zero-initialised projections (each block's conv_2,
    the attention output projections, the output conv), so every path carries signal."""
    with torch.no_grad():
        for p in model.parameters():
            if p.dim() > 1 and not p.any():
                torch.nn.init.kaiming_uniform_(p, a=math.sqrt(5))
    return model


def _fp8_site_active(m, x) -> bool:
    if isinstance(m, U.Conv2dFP8):
        return m.conv_fp8(x, m.conv.weight) or m.conv_fp8_general(x, m.conv.weight)
    if isinstance(m, U.Conv1x1FP8):
        return m.fp8 and m.in_channels % 128 == 0 and m.out_channels % 128 == 0
    return m.fp8 and K.linear_fp8_supported(m.in_features, m.out_features)


def test_unet_fused_gradient_sums_equal_autograd():
    """The skip-gradient sums fused into kernels (the encoder activations' two gradients
    inside the downsampling's backward, the attention block input's inside the LayerNorm
    backward) and the 32x32 and 16x16 decoder stages' upsample-and-concatenate read by their
    first GroupNorm change no bit of the U-Net's gradients: cfg5's model at batch 2 (current
    scaling, dropout off), forward + backward under autocast with the fused forms and with
    autograd's own accumulation on the formed concatenation."""
    torch.manual_seed(5)
    model = _nonzero_init(U.UNet(_cfg())).to(memory_format=torch.channels_last).cuda()
    g = torch.Generator().manual_seed(6)
    x = (torch.rand((2, 3, 32, 32), generator=g) * 2 - 1).cuda().contiguous(
        memory_format=torch.channels_last)
    t = torch.randint(0, 1000, (2,), generator=g).cuda()
    gy = torch.randn((2, 3, 32, 32), generator=g).cuda().contiguous(
        memory_format=torch.channels_last)
    grads = []
    calls = []
    orig = G.UpcatGroupNormSiLUTee.apply

    def counted(*args):
        calls.append(1)
        return orig(*args)

    G.UpcatGroupNormSiLUTee.apply = counted  # counts the fused calls; removed again below
    try:
        _fused_vs_autograd_grads(model, x, t, gy, grads)
    finally:
        del G.UpcatGroupNormSiLUTee.apply
    assert len(calls) == 2  # the fused pass took the fused concatenation at 32x32 and 16x16
    assert grads[0].keys() == grads[1].keys() and len(grads[0]) > 100
    for n in grads[0]:
        assert torch.equal(grads[0][n], grads[1][n]), n


def _fused_vs_autograd_grads(model, x, t, gy, grads):
    for fused in (True, False):
        model.down_tee = fused
        model.upcat_gn = fused
        for m in model.modules():
            if isinstance(m, U.CHWAttention):
                m.ln_tee = fused
        model.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = model(x, t)
        y.float().backward(gy)
        grads.append({n: p.grad.clone() for n, p in model.named_parameters() if p.grad is not None})
    torch.cuda.synchronize()


def test_unet_forward_backward_vs_fakequant_emulation():
    """cfg5's U-Net (current scaling, dropout off) at batch 2, one forward+backward under
    autocast: every FP8 site (registry and general 3x3 convs, 1x1 skips, linears) is checked
    inside the model, teacher-forced: the output it computed from the x it received, and the
    dx / dw its backward produced from the dy it received, against the fake-quant emulation of
    that site on the same x and dy (tests/fakequant.py: torch e4m3 casts, exact fp64 products,
    the reference's epilogue) -- normwise 1e-2, outputs >= 95 % bit-identical. The whole
    model's loss is checked against the emulated model's (fakequant.emulate_on_gpu, same
    weights and inputs) within 1e-2 relative (train.py:104-149 around
    diffusion/unet.py:245-388).

    The epsilon prediction is not compared elementwise: an e4m3 cast turns a one-ulp
    difference at one site into rounding flips (steps of 2^-4 relative) at the next, so two
    correct FP8 implementations drift to the quantization noise level within a few layers
    (measured: 15 % normwise at the output, with the loss equal to 1e-4)."""
    from fakequant import GpuFakeQuantConv, GpuFakeQuantLinear

    torch.manual_seed(3)
    model = _nonzero_init(U.UNet(_cfg())).to(memory_format=torch.channels_last).cuda()
    em = emulate_on_gpu(copy.deepcopy(model))
    g = torch.Generator().manual_seed(4)
    x0 = torch.rand((2, 3, 32, 32), generator=g) * 2 - 1
    t = torch.randint(0, 1000, (2,), generator=g).cuda()
    eps = torch.randn((2, 3, 32, 32), generator=g).cuda()
    ab = dpa_mod("ddpm").make_schedule(1000, "linear")[1].cuda()[t].float()[:, None, None, None]
    xt = (ab.sqrt() * x0.cuda() + (1 - ab).sqrt() * eps).contiguous(memory_format=torch.channels_last)

    rec, hooks = {}, []
    for n, m in model.named_modules():
        if isinstance(m, (U.Conv2dFP8, U.Conv1x1FP8, U.LinearFP8)):
            hooks.append(m.register_forward_hook(
                lambda mod, i, o, n=n: rec.__setitem__(n, {"x": i[0].detach().clone(),
                                                           "y": o.detach().clone()})))
            hooks.append(m.register_full_backward_hook(
                lambda mod, gi, go, n=n: rec[n].update(
                    dy=go[0].detach().clone(),
                    dx=None if gi[0] is None else gi[0].detach().clone())))
    losses = {}
    for name, m in (("hip", model), ("emu", em)):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss = F.mse_loss(m(xt, t), eps)
        loss.backward()
        losses[name] = float(loss)
        for h in hooks:
            h.remove()
        hooks = []
    torch.cuda.synchronize()
    print(f"unet batch 2: loss {losses['hip']:.6f} vs emulation {losses['emu']:.6f}", flush=True)
    assert math.isfinite(losses["hip"]) and losses["hip"] == pytest.approx(losses["emu"], rel=1e-2)

    mods = dict(model.named_modules())
    checked, worst = 0, []
    for n, r in rec.items():
        m = mods[n]
        if not _fp8_site_active(m, r["x"]):
            continue
        x = r["x"].clone().requires_grad_(r["dx"] is not None)
        if isinstance(m, U.LinearFP8):
            w = m.weight.detach().clone().requires_grad_()
            y = GpuFakeQuantLinear.apply(x, w)
        else:
            w = (m.conv.weight if isinstance(m, U.Conv2dFP8) else m.weight).detach().clone()
            w = w.requires_grad_()
            y = GpuFakeQuantConv.apply(x, w, 1, 1 if isinstance(m, U.Conv2dFP8) else 0)
        y.backward(r["dy"])
        wg = (m.conv.weight if isinstance(m, U.Conv2dFP8) else m.weight).grad
        errs = {"y": nerr(r["y"], y), "dw": nerr(wg, w.grad)}
        if r["dx"] is not None:             # the time embedding's input needs no gradient
            errs["dx"] = nerr(r["dx"], x.grad)
        same = float((r["y"].view(torch.int16) == y.detach().view(torch.int16)).float().mean())
        worst.append((max(errs.values()), n, errs, same, tuple(r["x"].shape), r["x"].dtype))
        checked += 1
    worst.sort(key=lambda v: -v[0])
    for e, n, errs, same, shp, dt in worst[:12]:
        print(f"  {n} {shp} {dt}: " + " ".join(f"{k} {v:.2e}" for k, v in errs.items())
              + f" bit-identical y {same:.4f}", flush=True)
    print(f"{checked} FP8 sites", flush=True)
    # 44 3x3 convs, 5 1x1 skips, 22 FiLM projections, 24 attention projections, 2 time-MLP linears
    assert checked == 97, checked
    for e, n, errs, same, _, _ in worst:
        assert e < 1e-2, (n, errs)
        assert same >= 0.95, (n, same)


def test_graph_captured_cfg5_step_at_batch_128():
    """One graph-captured step of the timed configuration (cfg5: delayed scaling, 1024-slot
    windows, dropout 0.2, batch 128) against an eager step from the same state and the same
    random stream (the dropout seeds are drawn inside the step): finite and equal losses,
    parameters within the batch-4 test's bounds, every delayed layer's window position
    advanced by one and its new window entries written."""
    kw = dict(fp8_scaling_type="delayed", p_drop=0.2)
    a = _state(128, **kw)
    b = _state(128, **kw)
    torch.cuda.manual_seed(11)
    a.capture(warmup=3)
    torch.cuda.manual_seed(11)
    for _ in range(3):
        b.eager_step()
    for st in (a, b):
        if st.model._wprep is not None:
            st.model._wprep.flush()        # window records lag one step until flushed
    torch.cuda.synchronize()
    a.loss_acc.zero_()
    b.loss_acc.zero_()
    # the 43 registry convs run delayed scaling; the one other 3x3 conv runs current scaling
    pos0 = {n: int(v) for n, v in a.model.named_buffers() if n.endswith("window_pos") and int(v)}
    assert len(pos0) == 43 and all(v == 3 for v in pos0.values()), pos0
    assert pos0 == {n: int(v) for n, v in b.model.named_buffers()
                    if n.endswith("window_pos") and int(v)}
    torch.cuda.manual_seed(12)
    a.replay()
    torch.cuda.synchronize()
    torch.cuda.manual_seed(12)
    b.eager_step()
    torch.cuda.synchronize()
    for st in (a, b):
        if st.model._wprep is not None:
            st.model._wprep.flush()        # the deferred window records of the step
    torch.cuda.synchronize()
    la, lb = float(a.loss_acc), float(b.loss_acc)
    print(f"cfg5 batch 128: replay loss {la:.6f}, eager loss {lb:.6f}", flush=True)
    assert math.isfinite(la) and la == pytest.approx(lb, rel=1e-4), (la, lb)
    for (name, p), q in zip(a.model.named_parameters(), b.model.parameters()):
        d = float((p.detach() - q.detach()).float().norm())
        bound = 1e-4 * float(q.detach().float().norm()) + 1e-5 * math.sqrt(q.numel())
        assert d <= bound, (name, d, bound)
    bufs_a = dict(a.model.named_buffers())
    for name, p0 in pos0.items():
        assert int(bufs_a[name]) == (p0 + 1) % 1024, name
        mod = name[: -len("window_pos")]
        for w in ("amax_window_acts", "amax_window_weights"):
            assert float(bufs_a[mod + w][p0]) > 0, (mod + w, p0)   # this step's x / w scales
        assert float(bufs_a[mod + "amax_window_dy"][(p0 + 1) % 1024]) > 0, mod  # its dy scale
    for (name, buf), q in zip(a.model.named_buffers(), b.model.buffers()):
        if buf.dtype == torch.long:
            assert torch.equal(buf, q), name
        else:
            torch.testing.assert_close(buf, q, rtol=2**-5, atol=0, msg=name)


def _loss_curve(st, images, t_all, eps_all, batch, eager=False):
    """Per-step losses of a TrainState over the given timesteps and noise (images cycled)."""
    steps = t_all.shape[0]
    st.set_batch(images[:batch], t_all[0], eps_all[0])
    if eager:
        for _ in range(3):
            st.eager_step()
    else:
        st.capture(warmup=3)
    losses = torch.zeros(steps, device="cuda")
    for i in range(steps):
        j = (i * batch) % images.shape[0]
        st.set_batch(images[j:j + batch], t_all[i], eps_all[i])
        st.loss_acc.zero_()
        if eager:
            st.eager_step()
        else:
            st.replay()
        losses[i].copy_(st.loss_acc)
    return losses.cpu().numpy()


def _conv_by_matmul(x: torch.Tensor, w: torch.Tensor, pad: int) -> torch.Tensor:
    """bf16 conv (stride 1) as unfold + one 2-D GEMM, channels-last result."""
    b, c, h, wd = x.shape
    o, _, k, _ = w.shape
    cols = F.unfold(x, k, padding=pad).transpose(1, 2).reshape(b * h * wd, c * k * k)
    y = F.linear(cols, w.reshape(o, c * k * k))
    return y.reshape(b, h, wd, o).permute(0, 3, 1, 2)


def _bf16_reference(model: torch.nn.Module) -> torch.nn.Module:
    """The same U-Net with every FP8 site in plain bf16 autocast arithmetic: 3x3 and 1x1
    convs as unfold + GEMM, the linears as nn.Linear."""
    for m in model.modules():
        if isinstance(m, U.Conv2dFP8):
            m.forward = types.MethodType(lambda self, x: _conv_by_matmul(x, self.conv.weight, 1), m)
        elif isinstance(m, U.Conv1x1FP8):
            m.forward = types.MethodType(lambda self, x: _conv_by_matmul(x, self.weight, 0), m)
        elif isinstance(m, U.LinearFP8):
            m.fp8 = False
    return model


def _smooth_images(n: int, seed: int) -> torch.Tensor:
    """Synthetic images in [-1, 1] with spatial structure: bilinear upsampling of random 4x4
    colour fields (something a denoiser can learn, unlike i.i.d. pixels)."""
    g = torch.Generator().manual_seed(seed)
    low = torch.rand((n, 3, 4, 4), generator=g) * 2 - 1
    return F.interpolate(low, size=(32, 32), mode="bilinear", align_corners=False).clamp(-1, 1)


def _seeded_loss_curve(name, steps, batch, window, seed):
    """Window means of the losses of `steps` graph-replayed training steps of the cfg5-shaped
    model (name: fp8-current, fp8-delayed-h16, fp8-delayed or bf16) on the smooth images, with
    the timesteps and noise of data seed `seed`."""
    images = _smooth_images(64, seed=4).cuda()
    gen = torch.Generator(device="cuda").manual_seed(seed)
    t_all = torch.randint(0, 1000, (steps, batch), device="cuda", generator=gen)
    eps_all = torch.randn((steps, batch, 3, 32, 32), device="cuda", generator=gen)
    scaling = "current" if name == "fp8-current" else "delayed"
    hist = 16 if name.endswith("h16") else 1024
    st = T.TrainState(_cfg(fp8_scaling_type=scaling, fp8_amax_history=hist), batch=batch,
                      seed=0, fixed_noise=True)
    if name == "bf16":
        _bf16_reference(st.model)
    curve = _loss_curve(st, images, t_all, eps_all, batch).reshape(-1, window).mean(axis=1)
    print(f"loss curve {name} (data seed {seed}): window means "
          + " ".join(f"{m:.4f}" for m in curve), flush=True)
    assert np.isfinite(curve).all(), name
    del st
    return curve


def test_unet_loss_tracks_bf16_over_training():
    """The FP8 U-Net (graph-captured) against the same model in bf16: same initialisation,
    same images, timesteps and noise at every step, 1000 steps at batch 16, losses averaged
    over windows of 100 steps.

    * current scaling tracks bf16, compared on curves averaged over three data seeds (the
      timesteps and noise): every window within 15 %, windows 2-10 within 8 % on average. One
      1000-step trajectory moves with any rounding change (measured per seed: 3-6 % across
      revisions of the model's rounding, and once 20 %: data seed 7 after the image-channel
      convs moved from MIOpen to the HIP kernels, while seeds 8 and 9 stayed within 5 % with
      either conv), so a single trajectory is not the bar;
    * delayed scaling with a 16-slot window stays closer to bf16 than with 1024 slots in every
      window after the first (data seed 7; measured: ~13 % above bf16);
    * delayed scaling with the reference's 1024-slot window (diffusion/unet.py:25) learns
      but trails: the loss falls ~10x in the first 100 steps, and the maximum over the
      window keeps the large early scales for the whole run, so small values lose their
      mantissa bits in e4m3. The torch emulation of the same recipe trails the same way
      (test_unet_delayed_loss_tracks_recipe_emulation).
    """
    steps, batch, window = 1000, 16, 100
    seeds = (7, 8, 9)
    per_seed = {name: [_seeded_loss_curve(name, steps, batch, window, sd) for sd in seeds]
                for name in ("fp8-current", "bf16")}
    curves = {name: np.mean(v, axis=0) for name, v in per_seed.items()}
    for name in ("fp8-delayed-h16", "fp8-delayed"):
        curves[name] = _seeded_loss_curve(name, steps, batch, window, seeds[0])
    bf = curves["bf16"]
    assert bf[-1] < 0.2 * bf[0]
    rel = {k: np.abs(v - bf) / bf for k, v in curves.items()}
    assert rel["fp8-current"].max() <= 0.15, rel["fp8-current"]
    assert rel["fp8-current"][1:].mean() <= 0.08, rel["fp8-current"]
    # the window length is what separates delayed from current scaling (data seed 7 alone)
    bf7 = per_seed["bf16"][0]
    rel7 = {k: np.abs(curves[k] - bf7) / bf7 for k in ("fp8-delayed-h16", "fp8-delayed")}
    assert (rel7["fp8-delayed-h16"][1:] < rel7["fp8-delayed"][1:]).all(), rel7
    assert rel7["fp8-delayed-h16"][1:].mean() <= 0.2, rel7["fp8-delayed-h16"]
    assert curves["fp8-delayed"][-1] < 0.5 * curves["fp8-delayed"][0]


def test_unet_delayed_loss_tracks_recipe_emulation():
    """The timed configuration's scaling (delayed, 1024-slot windows) over 1000 steps at batch
    16: the HIP model's loss curve (graph replays) against the torch emulation of the same
    recipe (fakequant.emulate_on_gpu: the window state machine of diffusion/unet.py:69-91 and
    diffusion/fp8_kernels.py:845-889 on the module buffers, torch e4m3 casts, exact fp64
    products, torch's clip_grad_norm_ + fused AdamW + EMA), from the same initial weights with
    the same images, timesteps and noise. The emulation runs eager steps: replays of a graph
    holding torch's multi-block reductions (its amax) are unreliable on these GPUs.

    The delayed trajectory is chaotic: two emulations that differ only in optimizer rounding
    (torch's tail, the fused tail) differed by 15-25 % per 100-step window (measured), repeated
    HIP runs by up to 24 %, and an emulation run has spiked to 2.4x its neighbours for one
    window (0.117 at window 7, measured). So the mean over windows 2-10 of the HIP curve must
    lie within [0.6, 1.6]x the emulation's, and every window within [1/3, 3]x. The recipe
    itself trails current scaling over a run this short (the window maximum keeps the first
    steps' large scales for all 1000 steps): windows 6-10 of both curves are >= 2x the
    current-scaling HIP curve (measured ~3.3x)."""
    steps, batch, window = 1000, 16, 100
    images = _smooth_images(64, seed=4).cuda()
    gen = torch.Generator(device="cuda").manual_seed(7)
    t_all = torch.randint(0, 1000, (steps, batch), device="cuda", generator=gen)
    eps_all = torch.randn((steps, batch, 3, 32, 32), device="cuda", generator=gen)
    curves = {}
    for name in ("fp8-current", "fp8-delayed", "emu-delayed"):
        scaling = "current" if name == "fp8-current" else "delayed"
        emu = name.startswith("emu")
        st = T.TrainState(_cfg(fp8_scaling_type=scaling, fp8_amax_history=1024), batch=batch,
                          seed=0, fixed_noise=True, fused_tail=not emu)
        if emu:
            emulate_on_gpu(st.model)
            for m in st.model.modules():       # GroupNorm+SiLU stay the fused kernel
                if hasattr(m, "fused"):
                    m.fused = True
        losses = _loss_curve(st, images, t_all, eps_all, batch, eager=emu)
        curves[name] = losses.reshape(-1, window).mean(axis=1)
        print(f"loss curve {name}: window means " + " ".join(f"{m:.4f}" for m in curves[name]),
              flush=True)
        assert np.isfinite(curves[name]).all(), name
        del st
    hip, emu, cur = curves["fp8-delayed"], curves["emu-delayed"], curves["fp8-current"]
    ratio = hip[1:] / emu[1:]
    assert 0.6 < hip[1:].mean() / emu[1:].mean() < 1.6, (hip, emu)
    assert ((ratio > 1 / 3) & (ratio < 3)).all(), ratio
    assert hip[5:].mean() >= 2 * cur[5:].mean() and emu[5:].mean() >= 2 * cur[5:].mean(), curves


def test_unet_delayed_steps_teacher_forced_vs_recipe_emulation(monkeypatch):
    """20 training steps of the HIP U-Net in the timed configuration's scaling (delayed,
    1024-slot windows, producer hand-offs on, prepared weights, fused optimizer tail) after the
    3 warm-up steps of train.py:117-128. Before each step the torch emulation of the recipe
    (fakequant.emulate_on_gpu: the window state machine of diffusion/unet.py:69-91 and
    diffusion/fp8_kernels.py:845-889 on the module buffers, torch e4m3 casts of bf16 tensors,
    exact fp64 products) is loaded with the HIP model's parameters, windows and positions and
    runs the same batch. Every delayed conv operand of the HIP steps comes from a hand-off (no
    standalone delayed cast). Bars:

    * each step's loss within 1e-3 relative (measured <= 7e-5);
    * the whole gradient within 2e-2 normwise on the median step (measured ~1e-3);
    * window records: positions and written slots identical, weight scales bit-exact,
      activation scales within 2^-4 relative (the amax of activations that carry the
      forward's accumulated rounding differences: measured up to 5 %).

    Individual steps' gradients are not bounded: with 1024 slots the first step leaves 1.0 in
    every dy window (the output conv is zero-initialised, diffusion/unet.py:346, so every dy of
    that step is 0 and its scale 1, fp8_kernels.py:101), the window maximum keeps it for 1024
    steps, every dy casts at scale 1.0 and only a few elements survive the e4m3 underflow, so
    at some steps the weight gradients are a handful of rounding decisions that any second
    implementation makes differently (measured 0.06-0.9 at 5 of 20 steps, ~1e-3 at the
    others). The hand-off bytes and records themselves are pinned per conv against the
    oracle by test_gpu_handoff.test_cfg5_handoffs_per_site_vs_oracle.

    Teacher forcing keeps the comparison tight: run freely, the trajectory diverges from any
    second valid implementation within a few steps (measured: the same emulation with fp32
    instead of fp64 accumulation -- the reference's tl.dot accumulates in fp32 -- drifts
    2.5e-3 from the fp64 one by step 11 and 7e-3 by step 20)."""
    monkeypatch.setattr(torch.backends.cudnn, "deterministic", True)   # MIOpen bf16 convs
    D = dpa_mod("ddpm")
    calls = {"n": 0}
    real = K.quantize_fp8_delayed_deferred

    def counting(*a, **kw):
        calls["n"] += 1
        return real(*a, **kw)

    monkeypatch.setattr(K, "quantize_fp8_delayed_deferred", counting)
    steps, batch, warm, hist = 20, 16, 3, 1024
    cfg = _cfg(fp8_scaling_type="delayed", fp8_amax_history=hist)
    images = _smooth_images(64, seed=4).cuda()
    gen = torch.Generator(device="cuda").manual_seed(7)
    t_all = torch.randint(0, 1000, (steps + warm, batch), device="cuda", generator=gen)
    eps_all = torch.randn((steps + warm, batch, 3, 32, 32), device="cuda", generator=gen)
    st = T.TrainState(cfg, batch=batch, seed=0, fixed_noise=True)
    assert getattr(st.optimizer, "fuses_clip_and_ema", False)
    emu = emulate_on_gpu(U.UNet(cfg).cuda().to(memory_format=torch.channels_last))
    for m in emu.modules():                    # GroupNorm+SiLU stay the fused kernel
        if hasattr(m, "fused"):
            m.fused = True
    ddpm_e = D.DiffusionWrapper(emu, schedule_type="linear", max_t=1000, in_dim=32, device="cuda")
    wins = ("amax_window_acts", "amax_window_weights", "amax_window_dy")
    delayed = [n for n, m in st.model.named_modules()
               if isinstance(m, U.Conv2dFP8) and getattr(m, "scaling_type", "") == "delayed"
               and hasattr(m, "window_pos")]
    assert len(delayed) >= 40
    rel_loss, gerr, werr = [], [], dict.fromkeys(wins, 0.0)
    for i in range(warm + steps):
        j = (i * batch) % images.shape[0]
        st.set_batch(images[j:j + batch], t_all[i], eps_all[i])
        if i < warm:
            st.eager_step()
            continue
        st.model._wprep.flush()                # the deferred window records of the last step
        torch.cuda.synchronize()
        emu.load_state_dict(st.model.state_dict())
        emu.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss_e = ddpm_e.forward_batch(st.static_batch, st.static_t, st.static_eps)
        loss_e.backward()
        # the HIP step: trainer._one_step with the gradients read before the update
        calls["n"] = 0
        st.optimizer.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss_h = st.ddpm.forward_batch(st.static_batch, st.static_t, st.static_eps)
        loss_h.backward()
        assert calls["n"] == 0, (i, calls["n"])          # every delayed operand handed off
        grads = {n: p.grad.detach().float().clone() for n, p in st.model.named_parameters()
                 if p.grad is not None}
        st.optimizer.step()
        st.model._wprep.flush()
        torch.cuda.synchronize()
        rel_loss.append(abs(float(loss_h.detach()) / float(loss_e.detach()) - 1.0))
        ge = dict(emu.named_parameters())
        assert set(grads) == {n for n, q in ge.items() if q.grad is not None}, i
        den = sum(float(ge[n].grad.float().norm() ** 2) for n in grads) ** 0.5
        num = sum(float((grads[n] - ge[n].grad.float()).norm() ** 2) for n in grads) ** 0.5
        gerr.append(num / den)
        hm, em_ = dict(st.model.named_modules()), dict(emu.named_modules())
        for n in delayed:
            a, b = hm[n], em_[n]
            assert torch.equal(a.window_pos, b.window_pos), (i, n)
            for w in wins:
                wa, wb_ = getattr(a, w), getattr(b, w)
                assert torch.equal(wa == 0, wb_ == 0), (i, n, w)        # the same slots
                r = float(((wa - wb_).abs() / wb_.abs().clamp_min(1e-30)).max())
                werr[w] = max(werr[w], r)
    print("teacher-forced loss rel " + " ".join(f"{v:.1e}" for v in rel_loss), flush=True)
    print("teacher-forced grad rel " + " ".join(f"{v:.1e}" for v in gerr), flush=True)
    print(f"teacher-forced window rel {werr}", flush=True)
    assert max(rel_loss) <= 1e-3, rel_loss
    assert float(np.median(gerr)) <= 2e-2, gerr
    assert werr["amax_window_weights"] == 0.0, werr
    assert werr["amax_window_acts"] <= 2**-4, werr
