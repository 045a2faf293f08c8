"""CPU checks of the model harness: module tree and parameter names of the reference U-Net,
the FP8 gate, the DDPM schedule, the EMA update and the delayed-scaling state machine of the
oracle (scripted sequences written out by hand from diffusion/unet.py:69-91 and
diffusion/fp8_kernels.py:845-889)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import dpa_mod
from oracle import fp8_oracle as O

U = dpa_mod("unet")
D = dpa_mod("ddpm")
K = dpa_mod("fp8_kernels")


def reference_train_config(**kw):
    """extra/profile_cuda_graph.py:121-133 (and train.py:220-233): attention at 16 and 8."""
    return U.cfg5_config(**kw)


def _analytic_param_count(ch=128, temb=512, attn_res=(16, 8)):
    """Parameters of the reference U-Net counted from its structure (diffusion/unet.py)."""
    def block(ci, co):
        return 9 * ci * co + 9 * co * co + 2 * ci + 2 * co + temb * 2 * co + (ci * co if ci != co else 0)

    def attn(c):
        return 3 * c * c + c * c + 2 * c

    def stage(ci, hid, co, att, nb):
        io = [(ci, hid)] + [(hid, hid)] * (nb - 2) + [(hid, co)]
        return sum(block(a, b) + (attn(b) if att else 0) for a, b in io)

    c1, c2 = ch, 2 * ch
    n = 3 * c1 * 9 + ch * temb + temb * temb + 2 * c1 + c1 * 3 * 9
    n += stage(c1, c1, c2, 32 in attn_res, 2) + stage(c2, c2, c2, 16 in attn_res, 2)
    n += stage(c2, c2, c2, 8 in attn_res, 2) + stage(c2, c2, c2, False, 2)      # down + mid-down
    n += stage(c2, c2, c2, True, 2)                                             # mid
    n += stage(2 * c2, c2, c2, False, 3) + stage(2 * c2, c2, c2, 8 in attn_res, 3)
    n += stage(2 * c2, c2, c2, 16 in attn_res, 3) + stage(2 * c2, c1, c1, 32 in attn_res, 3)
    return n


def test_parameter_count_matches_reference_model():
    m = U.UNet(reference_train_config())
    n = sum(p.numel() for p in m.parameters())
    assert n == _analytic_param_count() == 33_573_888, n     # the 33.57 M of the reference
    m16 = U.UNet(reference_train_config(attn_resolutions=[16]))
    assert sum(p.numel() for p in m16.parameters()) == _analytic_param_count(attn_res=(16,))


def test_state_dict_names_follow_reference():
    sd = U.UNet(reference_train_config()).state_dict()
    for key in [
        "conv_in.weight", "time_embed.0.weight", "time_embed.2.weight",
        "down_stages.0.blocks.0.conv_1.conv.weight", "down_stages.0.blocks.0.conv_1.window_pos",
        "down_stages.0.blocks.0.conv_1.amax_window_acts", "down_stages.0.blocks.0.conv_1.amax_window_dy",
        "down_stages.0.blocks.0.conv_2.amax_window_weights", "down_stages.0.blocks.1.skip_connection.weight",
        "down_stages.0.blocks.0.norm1.weight", "down_stages.0.blocks.0.norm2.bias",
        "down_stages.0.blocks.0.t_embed_wb.mlp.weight", "down_stages.1.attns.0.qkv.weight",
        "down_stages.1.attns.1.out.weight", "down_stages.1.attns.0.norm.weight", "mid.attns.0.qkv.weight",
        "up_stages.3.blocks.2.conv_2.conv.weight", "out.0.weight", "out.0.bias", "out.2.weight",
    ]:
        assert key in sd, key
    assert "freqs" not in sd  # non-persistent buffer
    assert sd["down_stages.0.blocks.0.conv_1.window_pos"].dtype == torch.long
    assert sd["down_stages.0.blocks.0.conv_1.amax_window_acts"].shape == (1024,)


def _fp8_conv_shapes(model, res=32):
    """(Cin, Cout, H, W) at every Conv2dFP8 site, from a shape-only trace on the meta device."""
    shapes = []

    def hook(mod, inp, out):
        x = inp[0]
        shapes.append((x.shape[1], mod.conv.weight.shape[0], x.shape[2], x.shape[3]))

    for m in model.modules():
        if isinstance(m, U.Conv2dFP8):
            m.register_forward_hook(hook)
    cfg = model.config
    with torch.no_grad():
        model(torch.zeros(1, cfg.in_channels, res, res), torch.zeros(1, dtype=torch.long))
    return shapes


def test_fp8_gate_covers_43_of_44_convs():
    """With the reference's registry gate, 43 of the 44 3x3 convs run in FP8; the first conv
    of the innermost up stage (512 -> 256 at 4x4) is not in the registry."""
    model = U.UNet(reference_train_config(fp8_convs_enabled=False, fused_gn_silu=False))
    shapes = _fp8_conv_shapes(model)
    assert len(shapes) == 44
    in_registry = [s for s in shapes if s in K.SUPPORTED_UNET_SHAPES]
    assert len(in_registry) == 43
    assert [s for s in shapes if s not in K.SUPPORTED_UNET_SHAPES] == [(512, 256, 4, 4)]
    # every site is a multiple of 128 channels, so fp8_all_convs covers all 44
    assert all(c % 128 == 0 and o % 128 == 0 for c, o, _, _ in shapes)


def test_cpu_forward_backward_without_fp8_is_zero_at_init():
    """The output conv is zero-initialised (diffusion/unet.py:380-382): eps_pred == 0 at init,
    so the loss is mean(eps^2). Runs the torch path (FP8 off) on the CPU."""
    torch.manual_seed(0)
    cfg = reference_train_config(fp8_convs_enabled=False, fp8_linears=False, p_drop=0.0)
    model = U.UNet(cfg).to(memory_format=torch.channels_last)
    ddpm = D.DiffusionWrapper(model, "linear", 1000, 32, device="cpu")
    x = torch.rand(2, 3, 32, 32) * 2 - 1
    eps = torch.randn(2, 3, 32, 32)
    t = torch.tensor([5, 900])
    loss = ddpm.forward_batch(x, t, eps)
    assert float(loss.detach()) == pytest.approx(float((eps * eps).mean()), rel=1e-6)
    loss.backward()
    g = model.out[2].weight.grad
    assert g is not None and g.abs().sum() > 0


def test_linear_schedule():
    alphas, alpha_bars, betas, q_vars, p_vars = D.make_schedule(1000, "linear")
    assert betas[0].item() == pytest.approx(1e-4) and betas[-1].item() == pytest.approx(0.02)
    b64 = np.linspace(1e-4, 0.02, 1000)
    np.testing.assert_allclose(alpha_bars.numpy(), np.cumprod(1 - b64), rtol=1e-6)
    assert q_vars.shape == p_vars.shape == (1000,)
    # posterior variance beta_t (1 - abar_{t-1}) / (1 - abar_t) at t = 10
    ab = np.cumprod(1 - b64)
    assert q_vars[10].item() == pytest.approx(b64[10] * (1 - ab[9]) / (1 - ab[10]), rel=1e-6)
    assert p_vars[0].item() == pytest.approx(q_vars[0].item())
    _, ab_cos, b_cos, _, _ = D.make_schedule(1000, "cosine")
    assert 0 < b_cos.min() and b_cos.max() <= 0.999


def test_noise_batch_closed_form():
    ddpm = D.DiffusionWrapper(torch.nn.Identity(), "linear", 1000, 32, device="cpu")
    x = torch.rand(3, 3, 4, 4)
    eps = torch.randn(3, 3, 4, 4)
    t = torch.tensor([0, 499, 999])
    xt, x0, e, tt = ddpm.noise_batch(x, t, eps)
    ab = ddpm.alpha_bars[t][:, None, None, None]
    torch.testing.assert_close(xt, ab.sqrt() * x + (1 - ab).sqrt() * eps)
    assert x0 is x and e is eps and tt is t


def test_ema_update_skips_integer_buffers():
    m = torch.nn.Module()
    m.w = torch.nn.Parameter(torch.full((4,), 2.0))
    m.register_buffer("pos", torch.tensor(7, dtype=torch.long))
    ema = D.EWMAWrapper(m, beta=0.75)
    with torch.no_grad():
        m.w.fill_(6.0)
        m.pos.fill_(9)
    ema.update(m)
    torch.testing.assert_close(ema.model.w.data, torch.full((4,), 0.75 * 2 + 0.25 * 6))
    assert int(ema.model.pos) == 9


def _bf16_tensor_bits(values):
    return O.f32_to_bf16_bits(np.asarray(values, dtype=np.float32))


def test_delayed_scaling_state_machine_scripted():
    """Window of 3 slots. Step i feeds x with amax a_i, w with amax b_i, dy with amax d_i.
    Forward reads max(window) for x/w/dy, writes the current x/w scales at pos and advances;
    backward writes the dy scale at the advanced pos (one slot ahead)."""
    st = O.DelayedScaling(history=3)
    a = [448.0, 896.0, 224.0, 112.0]
    b = [4.48, 0.448, 44.8, 4.48]
    d = [0.0448, 0.448, 0.00448, 4.48]
    seen = []
    for i in range(4):
        xq, wq, xs_h, ws_h, xs_c, ws_c = st.forward(_bf16_tensor_bits([a[i], -1.0]),
                                                   _bf16_tensor_bits([b[i], 0.0]))
        dyq, dys_h, dys_c = st.backward(_bf16_tensor_bits([d[i]]))
        seen.append((float(xs_h), float(ws_h), float(dys_h), st.pos,
                     st.win_acts.copy(), st.win_weights.copy(), st.win_dy.copy()))
        assert float(xs_c) == O.scale_from_amax(np.float32(O.bf16_bits_to_f32(_bf16_tensor_bits([a[i]]))[0]))
        assert float(dys_c) == O.scale_from_amax(np.float32(O.bf16_bits_to_f32(_bf16_tensor_bits([d[i]]))[0]))

    s = lambda v: float(O.scale_from_amax(np.float32(O.bf16_bits_to_f32(_bf16_tensor_bits([v]))[0])))  # noqa: E731
    # step 0: all windows zero -> historical scales 0 (out of contract for casting)
    assert seen[0][:4] == (0.0, 0.0, 0.0, 1)
    np.testing.assert_array_equal(seen[0][4], [s(a[0]), 0, 0])
    np.testing.assert_array_equal(seen[0][6], [0, s(d[0]), 0])          # dy one slot ahead
    # step 1: history maxima come from step 0
    assert seen[1][:4] == (s(a[0]), s(b[0]), s(d[0]), 2)
    np.testing.assert_array_equal(seen[1][4], [s(a[0]), s(a[1]), 0])
    np.testing.assert_array_equal(seen[1][6], [0, s(d[0]), s(d[1])])
    # step 2: pos wraps to 0, so dy overwrites slot 0
    assert seen[2][:4] == (s(a[1]), s(b[0]), s(d[1]), 0)
    np.testing.assert_array_equal(seen[2][6], [s(d[2]), s(d[0]), s(d[1])])
    # step 3: x/w write slot 0 (wrapped), dy writes slot 1, evicting d[0]
    assert seen[3][3] == 1
    np.testing.assert_array_equal(seen[3][4], [s(a[3]), s(a[1]), s(a[2])])
    np.testing.assert_array_equal(seen[3][5], [s(b[3]), s(b[1]), s(b[2])])
    np.testing.assert_array_equal(seen[3][6], [s(d[2]), s(d[3]), s(d[1])])
    assert seen[3][0] == max(s(a[0]), s(a[1]), s(a[2]))


def test_resblock_math_on_cpu():
    """ResidualBlock arithmetic on the torch path: (skip(x) + conv_2(...)) / sqrt(2); with the
    zero-initialised conv_2 the block is skip(x) / sqrt(2)."""
    cfg = reference_train_config(fp8_convs_enabled=False, fp8_linears=False, p_drop=0.0)
    blk = U.ResidualBlock(cfg, 128, 256)
    x = torch.randn(2, 128, 8, 8)
    t = torch.randn(2, 512)
    out = blk(x, t)
    torch.testing.assert_close(out, blk.skip_connection(x) / math.sqrt(2.0))


def test_checkpoint_round_trip_in_reference_format(tmp_path):
    """train.py:85-91 format: {"model_state_dict", "step", "config"} via torch.save. Every
    entry, FP8 amax windows and window positions included, survives the round trip bit for
    bit; the file loads with weights_only=True; a checkpoint of a torch.compile'd model
    (keys prefixed "_orig_mod.", config with the reference's fields and hparams.* entries)
    loads into a model built from its config; a missing key fails under strict loading."""
    from importlib import import_module

    T = import_module("diffusion-profiled_amd.trainer")
    torch.manual_seed(0)
    m = U.UNet(reference_train_config())
    g = torch.Generator().manual_seed(3)
    for name, buf in m.named_buffers():
        if name.endswith("window_pos"):
            buf.fill_(int(torch.randint(0, 1024, (1,), generator=g)))
        elif "amax_window" in name:
            buf.copy_(torch.rand(buf.shape, generator=g))
    config = m.config.as_dict()
    config.update({"hparams.max_t": 1000, "hparams.batch_size": 128})
    path = tmp_path / "checkpoint_linear.pt"
    T.save_checkpoint(m, 1234, config, str(path))
    raw = torch.load(path, weights_only=True)
    assert set(raw) == set(T.CHECKPOINT_KEYS)
    m2, step, cfg2 = T.load_checkpoint(path)
    assert step == 1234 and cfg2 == config
    sd, sd2 = m.state_dict(), m2.state_dict()
    assert list(sd) == list(sd2)
    for k in sd:
        assert sd[k].dtype == sd2[k].dtype and torch.equal(sd[k], sd2[k]), k

    ref_fields = {"in_channels", "base_hidden", "scales", "n_heads", "p_drop", "attn_resolutions",
                  "in_resolution", "n_resblocks", "fp8_convs_enabled", "fp8_scaling_type",
                  "fp8_amax_history"}  # diffusion/unet.py:13-25
    ref_cfg = {k: v for k, v in config.items() if k in ref_fields or k.startswith("hparams.")}
    compiled = {"_orig_mod." + k: v for k, v in sd.items()}
    torch.save({"model_state_dict": compiled, "step": 7, "config": ref_cfg}, tmp_path / "c.pt")
    m3, step3, _ = T.load_checkpoint(tmp_path / "c.pt")
    assert step3 == 7
    for k, v in m3.state_dict().items():
        assert torch.equal(v, sd[k]), k

    broken = dict(sd)
    broken.pop("down_stages.0.blocks.0.conv_1.window_pos")
    torch.save({"model_state_dict": broken, "step": 1, "config": config}, tmp_path / "b.pt")
    with pytest.raises(RuntimeError):
        T.load_checkpoint(tmp_path / "b.pt")
    torch.save({"step": 1}, tmp_path / "n.pt")
    with pytest.raises(KeyError):
        T.load_checkpoint(tmp_path / "n.pt")


def test_mse_loss_hip_refuses_mismatched_operands():
    """The HIP loss reads pred.numel() elements of each operand: a target of another shape
    (which F.mse_loss would broadcast) or on another device is refused before any launch."""
    D = dpa_mod("ddpm")
    pred = torch.zeros((2, 3, 4, 4))
    with pytest.raises(ValueError):
        D.mse_loss_hip(pred, torch.zeros((1, 3, 4, 4)))
    with pytest.raises(ValueError):
        D.mse_loss_hip(pred, torch.zeros((2, 3, 4, 4), device="meta"))
