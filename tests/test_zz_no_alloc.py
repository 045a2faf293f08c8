"""The allocation-free quantize entry point (dpa_quantize_fp8_bf16_noalloc) against the
workspace entry point it mirrors (dpa_quantize_fp8_bf16) and the oracle, through the C ABI.

Two calls in a row on the one device array, the second on a smaller tensor (fewer amax
partials: the stale partials of the first call must not be read), then the single-workgroup
and unaligned forms. Bytes and scale bit-exact."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from conftest import bits, dpa_mod, kaiming_uniform_bf16, randn_bf16
from oracle import fp8_oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    L = dpa_mod("_lib")
    return L.load(build_if_missing=False)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def run_workspace(lib, x: torch.Tensor):
    n = x.numel()
    q = torch.empty(n, dtype=torch.uint8, device=x.device)
    s = torch.empty((), dtype=torch.float32, device=x.device)
    wsb = lib.dpa_quant_workspace_bytes(n)
    ws = torch.empty(wsb, dtype=torch.uint8, device=x.device)
    st = lib.dpa_quantize_fp8_bf16(ctypes.c_void_p(x.data_ptr()), n, ctypes.c_void_p(q.data_ptr()),
                                   ctypes.c_void_p(s.data_ptr()), ctypes.c_void_p(ws.data_ptr()),
                                   wsb, ctypes.c_void_p(_stream()))
    assert st == 0, st
    return q, s


def run_noalloc(lib, x: torch.Tensor, q: torch.Tensor, s: torch.Tensor):
    st = lib.dpa_quantize_fp8_bf16_noalloc(ctypes.c_void_p(x.data_ptr()), x.numel(),
                                           ctypes.c_void_p(q.data_ptr()),
                                           ctypes.c_void_p(s.data_ptr()),
                                           ctypes.c_void_p(_stream()))
    assert st == 0, st


def check(lib, x: torch.Tensor, what: str):
    print(f"noalloc quantize: {what} n={x.numel()}", flush=True)
    q_ref, s_ref = run_workspace(lib, x)
    q = torch.full_like(q_ref, 0x55)
    s = torch.full_like(s_ref, -1.0)
    run_noalloc(lib, x, q, s)
    torch.cuda.synchronize()
    assert s.item() == s_ref.item(), (what, s.item(), s_ref.item())
    assert torch.equal(q, q_ref), what
    qo, so = O.quantize_fp8(bits(x.cpu()).reshape(-1))
    assert np.float32(s.item()) == so
    np.testing.assert_array_equal(q.cpu().numpy(), qo)


def test_noalloc_matches_workspace_entry_two_calls(lib):
    """cfg2 activation (256 amax partials), then a smaller tensor with a much larger
    magnitude in its last element (its own partials give a different scale), then the
    cfg2 weight: each call bit-identical to the workspace entry point."""
    big = randn_bf16((128, 128, 32, 32), seed=0).cuda().reshape(-1)
    check(lib, big, "cfg2 x")
    small = randn_bf16((3 * 65536 + 5,), seed=3, std=1e-2).cuda()
    small[-1] = 7.0
    check(lib, small, "smaller tensor, amax in its last element")
    w = kaiming_uniform_bf16((128, 128, 3, 3), seed=1).cuda().reshape(-1)
    check(lib, w, "cfg2 weight")


def test_noalloc_small_unaligned_and_zero(lib):
    """The single-workgroup form (tiny n), an unaligned view (scalar form) and an all-zero
    tensor (scale 1.0, all bytes 0)."""
    check(lib, randn_bf16((1000,), seed=4).cuda(), "tiny")
    base = randn_bf16((100003,), seed=5).cuda()
    check(lib, base[3:], "unaligned view")
    check(lib, torch.zeros(70000, dtype=torch.bfloat16, device="cuda"), "zeros")
