"""GPU parity of the amax/scale/e4m3 cast against the oracle — bit-exact, through the C ABI.

Covers the configs' tensors at full size, ragged and unaligned sizes, special values, the
zero tensor, delayed scaling, every reachable scale for the current-scaling finalize, and
the whole (bf16 x, scale) domain (65536 x 32639 pairs) against tests/golden/cast_digests.npz.
"""
from __future__ import annotations

import math

import os

import numpy as np
import pytest
import torch

from conftest import bits, dpa_mod, kaiming_uniform_bf16, randn_bf16
from oracle import fp8_oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "cast_digests.npz")


@pytest.fixture(scope="module")
def K():
    return dpa_mod("fp8_kernels")


@pytest.fixture(scope="module")
def L():
    lib = dpa_mod("_lib")
    lib.load(build_if_missing=False)
    return lib


def check_current(K, x_cpu: torch.Tensor):
    xb = bits(x_cpu)
    q_ref, s_ref = O.quantize_fp8(xb)
    q, s = K.quantize_fp8_tensor(x_cpu.cuda())
    torch.cuda.synchronize()
    assert q.dtype == torch.float8_e4m3fn and q.shape == x_cpu.shape
    assert s.dtype == torch.float32 and s.ndim == 0
    assert np.float32(s.item()) == s_ref, (s.item(), s_ref)
    np.testing.assert_array_equal(bits(q), q_ref)


def test_cfg2_activation_full_size(K):
    check_current(K, randn_bf16((128, 128, 32, 32), seed=0))


def test_cfg2_weight_and_cfg1_tensors(K):
    check_current(K, kaiming_uniform_bf16((128, 128, 3, 3), seed=1))
    check_current(K, randn_bf16((32768, 256), seed=0))
    check_current(K, kaiming_uniform_bf16((768, 256), seed=1))
    check_current(K, randn_bf16((128, 128, 32, 32), seed=2, std=1e-2))  # grad_out scale


@pytest.mark.parametrize("n", [1, 7, 8, 15, 16, 17, 255, 4095, 4097, 8191, 8193, 16384, 16385,
                               65537, 1 << 20 | 3])
@pytest.mark.parametrize("peak", ["none", "first", "last"])
def test_ragged_sizes(K, n, peak):
    """n-element tensors on both sides of the single-workgroup limit (16384 elements) and of
    the 8-element vector groups; the maximum |x| planted in the first or the last element
    (the vector tail) must reach the scale."""
    x = randn_bf16((n,), seed=n)
    assert x.shape == (n,)
    if peak == "first":
        x[0] = -40.0
    elif peak == "last":
        x[-1] = 40.0
    check_current(K, x)
    if peak != "none":
        q, s = K.quantize_fp8_tensor(x.cuda())
        assert np.float32(s.item()) == np.float32(40.0) / np.float32(448.0)


def test_unaligned_view(K):
    base = randn_bf16((10001,), seed=5).cuda()
    view = base[3:]  # data pointer 6 bytes past an allocation boundary
    xb = bits(view.cpu())
    q_ref, s_ref = O.quantize_fp8(xb)
    q, s = K.quantize_fp8_tensor(view)
    assert np.float32(s.item()) == s_ref
    np.testing.assert_array_equal(bits(q), q_ref)


def test_channels_last_preserves_layout(K):
    x = randn_bf16((4, 128, 8, 8), seed=6).cuda().contiguous(memory_format=torch.channels_last)
    q, s = K.quantize_fp8(x)
    assert q.is_contiguous(memory_format=torch.channels_last)
    q_ref, s_ref = O.quantize_fp8(bits(x.permute(0, 2, 3, 1).cpu()))
    np.testing.assert_array_equal(bits(q.permute(0, 2, 3, 1).cpu()), q_ref)


def test_zero_tensor_and_zero_weight(K):
    q, s = K.quantize_fp8(torch.zeros((128, 128, 3, 3), dtype=torch.bfloat16, device="cuda"))
    assert s.item() == 1.0 and not bits(q).any()


def test_special_values(K):
    vals = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x007F, 0x0080, 0x7F7F, 0xFF7F, 0x3F80,
                     0xBF80, 0x4040, 0x3C00, 0x0400], dtype=np.uint16)
    rng = np.random.default_rng(7)
    x = np.concatenate([vals, rng.integers(0, 0x7F80, 5000).astype(np.uint16)])
    t = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
    check_current(K, t)
    # a tensor of bf16 denormals only: the scale is itself an fp32 denormal
    check_current(K, torch.from_numpy(np.arange(1, 128, dtype=np.int16)).view(torch.bfloat16))


def test_delayed(K):
    x = randn_bf16((128, 128, 32, 32), seed=0)
    xb = bits(x)
    for prev in (np.float32(0.0123), np.float32(1.0), O.scale_from_amax(O.amax_bf16(xb))):
        q_ref, s_ref = O.quantize_fp8_delayed(xb, prev)
        q, s = K.quantize_fp8_delayed(x.cuda(), torch.tensor(prev, device="cuda"))
        assert np.float32(s.item()) == s_ref
        np.testing.assert_array_equal(bits(q), q_ref)


@pytest.mark.parametrize("n", [3000, 128 * 32 * 32 * 16])   # single-launch and two-pass paths
def test_delayed_window_update(K, n):
    """quantize_fp8_delayed_window: the same bytes and scale as quantize_fp8_delayed, plus
    window[pos] = scale and pos advancing modulo the window length (diffusion/unet.py:86-91)."""
    x = randn_bf16((n,), seed=n)
    prev = torch.tensor(np.float32(0.02), device="cuda")
    q0, s0 = K.quantize_fp8_tensor(x.cuda(), prev)
    win = torch.full((4,), -1.0, device="cuda")
    pos = torch.tensor(2, dtype=torch.long, device="cuda")
    q1, s1 = K.quantize_fp8_delayed_window(x.cuda(), prev, win, pos, advance=False)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(q1), bits(q0))
    assert s1.item() == s0.item()
    assert win.cpu().tolist() == [-1.0, -1.0, s0.item(), -1.0] and int(pos) == 2
    for expect_pos in (3, 0, 1, 2):                              # advance, wrapping at 4
        K.quantize_fp8_delayed_window(x.cuda(), prev, win, pos, advance=True)
        torch.cuda.synchronize()
        assert int(pos) == expect_pos
    assert win.cpu().tolist() == [s0.item()] * 4
    # window maxima of three windows in one launch, as torch.max
    w3 = [torch.rand(1024, device="cuda") for _ in range(3)]
    w3[1][17] = 0.0
    m = K.window_max3(*w3)
    torch.cuda.synchronize()
    assert m.cpu().tolist() == [float(w.max()) for w in w3]
    w3[2][5] = float("nan")
    assert math.isnan(K.window_max3(*w3)[2].item())


def test_every_reachable_scale_current(L):
    """Current scaling's finalize for each positive finite bf16 magnitude a: the tensor
    [a/2, -a] must give scale RN32(a/448)."""
    mags = np.arange(1, 0x7F80, dtype=np.uint16)
    ref = (O.bf16_bits_to_f32(mags) / O.FP8_MAX).astype(np.float32)
    half = O.f32_to_bf16_bits((O.bf16_bits_to_f32(mags) / 2).astype(np.float32))
    data = np.stack([half, mags | 0x8000], axis=1).astype(np.uint16)
    xd = torch.from_numpy(data.view(np.int16)).view(torch.bfloat16).cuda()
    q = torch.empty((mags.size, 2), dtype=torch.uint8, device="cuda")
    sc = torch.empty(mags.size, dtype=torch.float32, device="cuda")
    ws = torch.empty(4096, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    fn = L.load().dpa_quantize_fp8_bf16
    for i in range(mags.size):
        st = fn(xd[i].data_ptr(), 2, q[i].data_ptr(), sc[i:i + 1].data_ptr(), ws.data_ptr(), 4096, stream)
        assert st == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(sc.cpu().numpy(), ref)
    assert (q[:, 1].cpu().numpy() == 0xFE).all()  # -a / (a/448) clamps to -448 exactly


def _mix64(n: int) -> torch.Tensor:
    x = np.arange(n, dtype=np.uint64)
    z = x + np.uint64(0x9E3779B97F4A7C15)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    mix = (z ^ (z >> np.uint64(31))) | np.uint64(1)
    return torch.from_numpy(mix.view(np.int64))


def test_exhaustive_cast_domain_vs_golden(L):
    """All 65536 bf16 inputs x all 32639 reachable scales through dpa_quantize_fp8_delayed_bf16
    (which casts with a given scale); per-scale digests must equal the C oracle's."""
    d = np.load(GOLDEN, allow_pickle=False)
    scales, golden = d["scales"], d["digests"].view(np.int64)
    x = torch.from_numpy(np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.int16)).view(torch.bfloat16).cuda()
    mix = _mix64(65536).cuda()
    # the GPU digest arithmetic reproduces the golden digest on oracle bytes
    xb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    for i in (0, scales.size // 2):
        qo = torch.from_numpy(O.cast_e4m3(xb, scales[i])).cuda()
        assert int(((qo.to(torch.int64) + 1) * mix).sum()) == int(golden[i])
    s_dev = torch.from_numpy(scales).cuda()
    chunk = 512
    q = torch.empty((chunk, 65536), dtype=torch.uint8, device="cuda")
    cur = torch.empty((), dtype=torch.float32, device="cuda")
    ws = torch.empty(4096, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    fn = L.load().dpa_quantize_fp8_delayed_bf16
    got = np.empty(scales.size, dtype=np.int64)
    for c0 in range(0, scales.size, chunk):
        c1 = min(c0 + chunk, scales.size)
        for i in range(c0, c1):
            st = fn(x.data_ptr(), 65536, s_dev[i:i + 1].data_ptr(), q[i - c0].data_ptr(),
                    cur.data_ptr(), ws.data_ptr(), 4096, stream)
            assert st == 0
        got[c0:c1] = ((q[: c1 - c0].to(torch.int64) + 1) * mix).sum(dim=1).cpu().numpy()
    bad = np.nonzero(got != golden)[0]
    if bad.size:
        # name the first failing scale and the inputs it disagrees on
        i = int(bad[0])
        st = fn(x.data_ptr(), 65536, s_dev[i:i + 1].data_ptr(), q[0].data_ptr(), cur.data_ptr(),
                ws.data_ptr(), 4096, stream)
        qg = q[0].cpu().numpy()
        qo = O.cast_e4m3(xb, scales[i])
        diff = np.nonzero(qg != qo)[0][:8]
        pytest.fail(f"{bad.size} scales differ; first scale {scales[i]!r}: x bits "
                    f"{[hex(v) for v in diff]} gpu {[hex(qg[v]) for v in diff]} oracle {[hex(qo[v]) for v in diff]}")


def test_exhaustive_cast_domain_multiblock_path(L):
    """The same domain through the multi-workgroup cast kernel: the 65536 bf16 inputs tiled
    5 times (past the single-workgroup size limit), every 16th reachable scale; the first and
    last copies must both give the golden digest."""
    d = np.load(GOLDEN, allow_pickle=False)
    scales, golden = d["scales"][::16], d["digests"].view(np.int64)[::16]
    base = torch.from_numpy(np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.int16))
    x = base.repeat(5).view(torch.bfloat16).cuda()
    assert x.numel() > (1 << 18)
    mix = _mix64(65536).cuda()
    s_dev = torch.from_numpy(scales).cuda()
    q = torch.empty(x.numel(), dtype=torch.uint8, device="cuda")
    cur = torch.empty((), dtype=torch.float32, device="cuda")
    ws = torch.empty(4096, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    fn = L.load().dpa_quantize_fp8_delayed_bf16
    first = torch.empty(scales.size, dtype=torch.int64, device="cuda")
    last = torch.empty(scales.size, dtype=torch.int64, device="cuda")
    for i in range(scales.size):
        st = fn(x.data_ptr(), x.numel(), s_dev[i:i + 1].data_ptr(), q.data_ptr(), cur.data_ptr(),
                ws.data_ptr(), 4096, stream)
        assert st == 0
        first[i] = ((q[:65536].to(torch.int64) + 1) * mix).sum()
        last[i] = ((q[-65536:].to(torch.int64) + 1) * mix).sum()
    np.testing.assert_array_equal(first.cpu().numpy(), golden)
    np.testing.assert_array_equal(last.cpu().numpy(), golden)
