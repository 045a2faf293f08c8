"""The drop-in under torch.compile: the reference compiles the model that calls its FP8 ops
(train.py:252) and shapes its launches for it (diffusion/fp8_kernels.py:47-51). Here the
reference-named ops are torch.library custom ops (ops.py) with fake implementations, so
Dynamo keeps every FP8 launch inside the graph.

* Each reference-form FP8 site (``triton_conv2d_fp8`` in current and delayed mode -- the
  delayed one with the module's window state machine, diffusion/unet.py:69-91 --, the FP8
  linear, the stride-2 and 1x1 convs) compiles with ``fullgraph=True`` (any graph break is an
  error) under aot_eager and Inductor, and two compiled forward+backward calls equal two eager
  calls bit for bit: outputs, input and weight gradients, window buffers.
* The cfg5 U-Net compiled with aot_eager (its other HIP kernels -- GroupNorm, attention,
  residual joins -- are ctypes calls that Dynamo runs between graphs) equals the eager model
  bit for bit over two training steps, and no graph break falls inside the FP8 ops.
"""
from __future__ import annotations

import copy
import os

import pytest
import torch
import torch._dynamo

from conftest import dpa_mod

pytestmark = pytest.mark.gpu

K = dpa_mod("fp8_kernels")
U = dpa_mod("unet")

FP8_FILES = ("fp8_kernels.py", "ops.py")


def cl(t):
    return t.cuda().contiguous(memory_format=torch.channels_last)


class CurrentConv(torch.nn.Module):
    """diffusion/unet.py:65-67: the registry conv in current scaling."""

    def __init__(self, cin=128, cout=128):
        super().__init__()
        self.w = torch.nn.Parameter(cl(torch.randn(cout, cin, 3, 3) / 34.0))

    def forward(self, x):
        return K.triton_conv2d_fp8(x, self.w)


class DelayedConv(torch.nn.Module):
    """diffusion/unet.py:69-91: the registry conv in delayed scaling, the reference's op-by-op
    window state machine around triton_conv2d_fp8(..., do_delayed=True)."""

    def __init__(self):
        super().__init__()
        self.c = U.Conv2dFP8(128, 128, True, "delayed", 16)
        self.c.fused_window_update = False
        self.c.cuda().to(memory_format=torch.channels_last)
        with torch.no_grad():
            self.c.amax_window_acts.fill_(0.01)
            self.c.amax_window_weights.fill_(1e-4)
            self.c.amax_window_dy.fill_(1e-5)

    def forward(self, x):
        return self.c(x)


class Linear(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.w = torch.nn.Parameter(torch.randn(768, 256, device="cuda") / 16.0)

    def forward(self, x):
        return K.LinearFP8Function.apply(x, self.w, None)


class GeneralConv(torch.nn.Module):
    def __init__(self, k, stride, cin=256, cout=256):
        super().__init__()
        self.k, self.stride = k, stride
        self.w = torch.nn.Parameter(cl(torch.randn(cout, cin, k, k) / 48.0))

    def forward(self, x):
        return K.conv2d_fp8(x, self.w, self.stride, 1 if self.k == 3 else 0)


CASES = {
    "current": (CurrentConv, (4, 128, 32, 32)),
    "delayed": (DelayedConv, (4, 128, 32, 32)),
    "linear": (Linear, (2, 256, 256)),
    "stride2": (lambda: GeneralConv(3, 2), (4, 256, 16, 16)),
    "1x1": (lambda: GeneralConv(1, 1, 128, 256), (4, 128, 32, 32)),
}


def _run(mod, x0, iters=2):
    for _ in range(iters):
        for p in mod.parameters():
            p.grad = None
        x = x0.clone().requires_grad_()
        y = mod(x)
        y.float().square().sum().backward()
    torch.cuda.synchronize()
    return (y.detach(), x.grad, [p.grad for p in mod.parameters()],
            [b.clone() for b in mod.buffers()])


@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
@pytest.mark.parametrize("case", list(CASES))
def test_fp8_site_compiles_without_graph_break(case, backend):
    ctor, shape = CASES[case]
    torch.manual_seed(0)
    m = ctor()
    x0 = torch.randn(shape).to(torch.bfloat16)
    x0 = cl(x0) if x0.ndim == 4 else x0.cuda()
    torch._dynamo.reset()
    ex = torch._dynamo.explain(copy.deepcopy(m))(x0)
    assert ex.graph_break_count == 0 and ex.graph_count == 1, ex.break_reasons
    torch._dynamo.reset()
    eager, compiled = copy.deepcopy(m), copy.deepcopy(m)
    comp = torch.compile(compiled, backend=backend, fullgraph=True)
    ya, ga, pa, ba = _run(eager, x0)
    yb, gb, pb, bb = _run(comp, x0)
    assert torch.equal(ya, yb), case
    assert torch.equal(ga, gb), case
    for a, b in zip(pa, pb):
        assert torch.equal(a, b), case
    for a, b in zip(ba, bb):
        assert torch.equal(a, b), case


def test_ops_are_registered_with_fakes():
    """Every op of the torch.ops.dpa_fp8 namespace the reference-named functions call passes
    torch.library's checks on small inputs: the fake implementation's outputs (shapes,
    dtypes, strides) equal the real ones, and autograd is registered where it is needed."""
    ops = dpa_mod("ops")
    g = torch.Generator().manual_seed(3)
    x = cl(torch.randn((2, 128, 16, 16), generator=g).to(torch.bfloat16))
    w = cl(torch.randn((256, 128, 3, 3), generator=g) / 34.0)
    xq, xs = ops.quantize(x)
    wq, ws = ops.quantize(w.to(torch.bfloat16))
    y = ops.conv_fwd(xq, wq, xs, ws, 1, 1)
    dyq, dys = ops.quantize(y)
    checks = [
        (torch.ops.dpa_fp8.quantize.default, (x,)),
        (torch.ops.dpa_fp8.quantize_delayed.default, (x, xs)),
        (torch.ops.dpa_fp8.conv_fwd.default, (xq, wq, xs, ws, 1, 1)),
        (torch.ops.dpa_fp8.conv_fwd.default, (xq, wq, xs, ws, 2, 1)),
        (torch.ops.dpa_fp8.conv_dgrad.default, (dyq, wq, dys, ws, 16, 16, 1, 1)),
        (torch.ops.dpa_fp8.conv_wgrad.default, (xq, dyq, xs, dys, 3, 1, 1, 0, False)),
        (torch.ops.dpa_fp8.conv_wgrad.default, (xq, dyq, xs, dys, 3, 1, 1, 0, True)),
        (torch.ops.dpa_fp8.conv2d_fp8.default, (x.float().requires_grad_(), w, 1, 1)),
    ]
    a = torch.randn((256, 128), generator=g).to(torch.bfloat16).cuda()
    b = torch.randn((384, 128), generator=g).to(torch.bfloat16).cuda()
    aq, as_ = ops.quantize(a)
    bq, bs = ops.quantize(b)
    cq, cs = ops.quantize(torch.randn((256, 384), generator=g).to(torch.bfloat16).cuda())
    checks += [
        (torch.ops.dpa_fp8.gemm.default, (aq, bq, as_, bs, None)),
        (torch.ops.dpa_fp8.gemm_dgrad.default, (cq, bq, cs, bs)),
        (torch.ops.dpa_fp8.gemm_wgrad.default, (aq, cq, as_, cs, False)),
        (torch.ops.dpa_fp8.linear_fp8.default, (a.float().requires_grad_(), b.float())),
    ]
    for op, args in checks:
        # (test_schema is left out: it compares e4m3 tensors with arithmetic torch does not
        # implement for float8)
        torch.library.opcheck(op, args, test_utils=("test_faketensor",
                                                     "test_autograd_registration"))


def test_unet_compiled_equals_eager_without_breaks_in_fp8_ops(monkeypatch):
    """The cfg5 U-Net (delayed scaling, every conv and linear of 128-multiple channels in FP8,
    dropout 0.2) at batch 2 under torch.compile(backend="aot_eager") against the same model
    eager, two training steps each (forward, backward, optimizer step): losses, every
    parameter gradient, every parameter and every window buffer equal bit for bit. The eager
    model runs the build's fused window update; the compiled one the reference's op-by-op
    window state machine around the custom ops -- the same values. torch._dynamo.explain's
    graph breaks all lie outside the FP8 ops (at the GroupNorm, attention and elementwise HIP
    kernels, which are ctypes calls)."""
    # the comparison is bitwise: MIOpen's bf16 input and output convs restricted to
    # deterministic solutions
    monkeypatch.setattr(torch.backends.cudnn, "deterministic", True)
    cfg = U.cfg5_config()
    torch.manual_seed(0)
    base = U.UNet(cfg).cuda().to(memory_format=torch.channels_last)
    with torch.no_grad():              # windows as after calibration; non-zero output conv
        for m in base.modules():
            if isinstance(m, U.Conv2dFP8) and hasattr(m, "window_pos"):
                m.amax_window_acts.fill_(0.02)
                m.amax_window_weights.fill_(2e-4)
                m.amax_window_dy.fill_(1e-6)
        torch.nn.init.normal_(base.out[-1].weight, std=1e-3)
    g = torch.Generator().manual_seed(4)
    x0 = cl(torch.rand((2, 3, 32, 32), generator=g) * 2 - 1)
    t0 = torch.randint(0, 1000, (2,), generator=g).cuda()
    target = cl(torch.randn((2, 3, 32, 32), generator=g))

    def step(model, fwd, opt, seed):
        opt.zero_grad(set_to_none=True)
        torch.cuda.manual_seed(seed)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out = fwd(x0, t0)
            loss = torch.nn.functional.mse_loss(out.float(), target)
        loss.backward()
        grads = {n: p.grad.clone() for n, p in model.named_parameters() if p.grad is not None}
        opt.step()
        return float(loss.detach()), grads

    ex_model = copy.deepcopy(base)
    torch._dynamo.reset()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        ex = torch._dynamo.explain(ex_model)(x0, t0)
    inside = []
    for br in ex.break_reasons:
        frames = [f.filename for f in (br.user_stack or [])]
        if any(os.path.basename(f) in FP8_FILES for f in frames):
            inside.append((br.reason, frames[-3:]))
    print(f"U-Net under Dynamo: {ex.graph_count} graphs, {ex.graph_break_count} breaks, "
          f"{len(inside)} inside the FP8 ops", flush=True)
    assert not inside, inside[:3]
    torch._dynamo.reset()

    eager, compiled = copy.deepcopy(base), copy.deepcopy(base)
    runs = {}
    for name, model in (("eager", eager), ("compiled", compiled)):
        fwd = torch.compile(model, backend="aot_eager") if name == "compiled" else model
        opt = torch.optim.AdamW(model.parameters(), lr=2e-4)
        runs[name] = [step(model, fwd, opt, 100 + i) for i in range(2)]
        torch.cuda.synchronize()
    for i, ((la, ga), (lb, gb)) in enumerate(zip(runs["eager"], runs["compiled"])):
        assert la == lb, (i, la, lb)
        assert ga.keys() == gb.keys()
        for n in ga:
            assert torch.equal(ga[n], gb[n]), (i, n)
    for (n, a), b in zip(eager.named_parameters(), compiled.parameters()):
        assert torch.equal(a, b), n
    for (n, a), b in zip(eager.named_buffers(), compiled.buffers()):
        assert torch.equal(a, b), n
