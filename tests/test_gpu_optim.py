"""GPU tests of the fused optimizer tail (optim.FusedAdamWEMA, dpa_adamw_ema_step) against
torch's clip_grad_norm_ + AdamW(fused) + the EWMAWrapper foreach EMA of the reference step
(train.py:104-149, :253, :256): parameters, moments, EMA copies and the float/int
buffers over several steps, including clipping, an unused parameter (grad None) and, on odd
steps, a conv weight gradient in NCHW layout beside its channels-last parameter."""
from __future__ import annotations

import copy

import pytest
import torch

from conftest import dpa_mod

pytestmark = pytest.mark.gpu

OPT = dpa_mod("optim")


class _Net(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.conv = torch.nn.Conv2d(128, 64, 3, bias=False)
        self.lin = torch.nn.Linear(300, 70)          # odd sizes: vector tails
        self.norm = torch.nn.GroupNorm(8, 64)
        self.unused = torch.nn.Parameter(torch.randn(37))
        self.register_buffer("win", torch.rand(16))
        self.register_buffer("pos", torch.zeros((), dtype=torch.long))


@pytest.mark.parametrize("max_norm", [1.0, 1e3])
def test_fused_tail_matches_torch(max_norm):
    torch.manual_seed(0)
    net = _Net().cuda().to(memory_format=torch.channels_last)
    ema = copy.deepcopy(net)
    ref, ref_ema = copy.deepcopy(net), copy.deepcopy(net)
    fused = OPT.FusedAdamWEMA(net, ema, lr=2e-3, max_norm=max_norm, ema_beta=0.99)
    topt = torch.optim.AdamW(ref.parameters(), lr=2e-3, fused=True)
    beta = 0.99
    g = torch.Generator(device="cuda").manual_seed(1)
    for step in range(4):
        for (name, p), q in zip(net.named_parameters(), ref.parameters()):
            if name == "unused":
                p.grad, q.grad = None, None
                continue
            gr = torch.randn(p.shape, generator=g, device="cuda") * (3.0 if step == 1 else 0.05)
            cl = gr.ndim == 4 and step % 2 == 0
            p.grad = gr.clone().contiguous(memory_format=torch.channels_last) if cl else gr.clone()
            # torch's fused AdamW needs the parameter's layout; the fused tail takes either
            q.grad = gr.clone().contiguous(memory_format=torch.channels_last) if gr.ndim == 4 \
                else gr.clone()
        with torch.no_grad():
            net.win.mul_(1.1)
            ref.win.mul_(1.1)
            net.pos.add_(1)
            ref.pos.add_(1)
        fused.step()
        torch.nn.utils.clip_grad_norm_(ref.parameters(), max_norm=max_norm)
        topt.step()
        with torch.no_grad():
            e_sd, s_sd = ref_ema.state_dict(), ref.state_dict()
            fl = [k for k, v in e_sd.items() if v.is_floating_point()]
            torch._foreach_mul_([e_sd[k] for k in fl], beta)
            torch._foreach_add_([e_sd[k] for k in fl], [s_sd[k] for k in fl], alpha=1 - beta)
            for k, v in e_sd.items():
                if not v.is_floating_point():
                    v.copy_(s_sd[k])
        torch.cuda.synchronize()
        for (name, p), q in zip(net.named_parameters(), ref.parameters()):
            torch.testing.assert_close(p, q, rtol=2e-6, atol=1e-7, msg=f"step {step} {name}")
        for (k, v) in ema.state_dict().items():
            torch.testing.assert_close(v, ref_ema.state_dict()[k], rtol=2e-6, atol=1e-7,
                                       msg=f"step {step} ema {k}")
    st = topt.state[ref.lin.weight]
    torch.testing.assert_close(fused.exp_avg[1 + 1], st["exp_avg"], rtol=1e-5, atol=1e-9)
    assert float(fused.step_t) == 4.0
