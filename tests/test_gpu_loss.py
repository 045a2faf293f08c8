"""The DDPM training loss (diffusion/ddpm.py:209-215, F.mse_loss under autocast) on the HIP
library's deterministic reduction (dpa_mse_loss_f32): the value against a float64 sum of the
same fp32 operands, the gradient bit for bit against torch's mse_loss backward, repeated runs
bit-identical, and a captured graph of the loss replayed correctly with other GPU work before
each replay (the case where torch's own multi-block reduction, which records a memset,
returned 0 inside the training step's graph)."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import dpa_mod

pytestmark = pytest.mark.gpu

D = dpa_mod("ddpm")


@pytest.mark.parametrize("shape,dtype", [((128, 3, 32, 32), torch.bfloat16),
                                         ((128, 3, 32, 32), torch.float32),
                                         ((3, 5, 7), torch.float32),
                                         ((100,), torch.bfloat16),
                                         ((257, 1031), torch.float32)], ids=str)
def test_mse_loss_value_and_gradient(shape, dtype):
    g = torch.Generator().manual_seed(len(shape) + shape[0])
    pred = torch.randn(shape, generator=g).to(dtype).cuda()
    tgt = torch.randn(shape, generator=g).cuda()
    if len(shape) == 4:
        pred = pred.contiguous(memory_format=torch.channels_last)
        tgt = tgt.contiguous(memory_format=torch.channels_last)
    p1 = pred.clone().requires_grad_()
    loss = D.mse_loss_hip(p1, tgt)
    gr = torch.randn((), generator=g).cuda()
    loss.backward(gr)
    p2 = pred.clone().requires_grad_()
    ref = F.mse_loss(p2.float(), tgt)
    ref.backward(gr)
    torch.cuda.synchronize()
    exact = ((pred.double() - tgt.double()) ** 2).mean().item()
    assert loss.dtype == torch.float32 and loss.shape == ()
    assert abs(loss.item() - exact) <= 1e-6 * exact, (loss.item(), exact)
    assert p1.grad.dtype == dtype and torch.equal(p1.grad, p2.grad)
    again = D.mse_loss_hip(pred, tgt)
    assert torch.equal(again, loss.detach())


def test_mse_loss_in_a_replayed_graph():
    x = torch.randn((128, 3, 32, 32), device="cuda").to(torch.bfloat16)
    y = torch.randn((128, 3, 32, 32), device="cuda")
    acc = torch.zeros((), device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            acc.add_(D.mse_loss_hip(x, y))
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        acc.add_(D.mse_loss_hip(x, y))
    ref = ((x.double() - y.double()) ** 2).mean().item()
    for i in range(4):
        z = torch.randn(1 << 20, device="cuda")
        z.sum()                                  # other work before the replay
        acc.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert abs(acc.item() - ref) <= 1e-6 * ref, (i, acc.item(), ref)
