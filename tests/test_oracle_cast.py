"""Pins the oracle's scale and e4m3 cast (CPU only).

- C packer vs torch's float8_e4m3fn conversion on every fp32 bit pattern in [-464, 464];
- numpy packer vs the C packer (boundaries + random) and the known answers;
- numpy cast vs C cast on the full bf16 domain for sampled scales;
- the committed exhaustive-domain digests (tests/golden/cast_digests.npz) vs the C oracle;
- planted mistakes in a copy of the oracle are caught by these pins.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import c_oracle
import conftest
from oracle import fp8_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "cast_digests.npz")

KNOWN = [  # (value, e4m3 byte): RNE ties, subnormals, the 464 tie to even
    (1.0625, 0x38), (1.1875, 0x3A), (2.0**-10, 0x00), (3 * 2.0**-11, 0x01), (464.0, 0x7E),
    (448.0, 0x7E), (-448.0, 0xFE), (2.0**-6, 0x08), (2.0**-9, 0x01), (-0.0, 0x80), (0.0, 0x00),
    (1.0, 0x38), (240.0, 0x77), (0.875 * 2.0**-6, 0x07),
]


def torch_e4m3(v: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


@pytest.mark.parametrize("v,e", KNOWN)
def test_known_answers(v, e):
    lib = c_oracle()
    assert lib.oracle_e4m3_rne(v) == e
    assert int(O.f32_to_e4m3_rne(np.array([v], np.float32))[0]) == e
    assert int(torch_e4m3(np.array([v]))[0]) == e


def test_c_packer_exhaustive_vs_torch():
    """Every fp32 bit pattern with |v| <= 464 (both signs): C packer == torch conversion."""
    lib = c_oracle()
    chunk = 1 << 24
    hi_lim = 0x43E80001
    buf = np.empty(chunk, dtype=np.uint8)
    bad = 0
    for lo in range(0, hi_lim, chunk):
        hi = min(lo + chunk, hi_lim)
        n = hi - lo
        lib.oracle_e4m3_rne_range(lo, hi, buf.ctypes.data)
        f = torch.from_numpy(np.arange(lo, hi, dtype=np.uint32).view(np.float32))
        bad += int((f.to(torch.float8_e4m3fn).view(torch.uint8).numpy() != buf[:n]).sum())
        bad += int(((-f).to(torch.float8_e4m3fn).view(torch.uint8).numpy() != (buf[:n] | 0x80)).sum())
    assert bad == 0


def _boundary_values() -> np.ndarray:
    """All e4m3 values and all midpoints between neighbours, each +-1 and +-2 fp32 ulps."""
    pos = np.unique(O.e4m3_to_f32(np.arange(0, 0x7F, dtype=np.uint8)))
    mids = ((pos[1:].astype(np.float64) + pos[:-1]) / 2).astype(np.float32)
    base = np.concatenate([pos, mids, np.array([464.0, 460.0, 470.0], np.float32)])
    u = base.view(np.uint32).astype(np.int64)
    vals = np.concatenate([u + d for d in (-2, -1, 0, 1, 2)])
    vals = vals[(vals >= 0) & (vals < 0x7F800000)].astype(np.uint32).view(np.float32)
    return np.concatenate([vals, -vals])


def test_numpy_packer_vs_torch_boundaries_and_random():
    rng = np.random.default_rng(0)
    rand = rng.integers(0, 0x43E80001, size=1 << 21, dtype=np.int64).astype(np.uint32).view(np.float32)
    vals = np.concatenate([_boundary_values(), rand, -rand])
    np.testing.assert_array_equal(O.f32_to_e4m3_rne(vals), torch_e4m3(vals))


def test_numpy_cast_vs_c_cast_full_bf16_domain():
    lib = c_oracle()
    x = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    scales = O.reachable_scales()
    rng = np.random.default_rng(1)
    pick = np.concatenate([scales[:8], scales[-8:], rng.choice(scales, 48, replace=False),
                           np.array([1.0], np.float32)])
    out = np.empty(65536, dtype=np.uint8)
    for s in pick:
        lib.oracle_cast(x.ctypes.data, x.size, float(s), out.ctypes.data)
        np.testing.assert_array_equal(O.cast_e4m3(x, s), out, err_msg=f"scale {s!r}")


def test_scale_rule():
    assert O.scale_from_amax(np.float32(0.0)) == np.float32(1.0)
    assert O.scale_from_amax(np.float32(448.0)) == np.float32(1.0)
    a = np.float32(3.140625)
    assert O.scale_from_amax(a) == np.float32(a / np.float32(448.0))
    # amax is exact over bf16 magnitudes, independent of order and sign
    xb = np.array([0x3F80, 0xC040, 0x0001, 0x8000], dtype=np.uint16)  # 1, -3, tiny, -0
    assert O.amax_bf16(xb) == np.float32(3.0)
    assert O.amax_bf16(xb[::-1]) == np.float32(3.0)
    # the zero-initialised conv_2 weight (diffusion/unet.py:146): scale 1, all bytes 0
    q, s = O.quantize_fp8(np.zeros(1152, dtype=np.uint16))
    assert s == np.float32(1.0) and not q.any()
    # quantizing the amax element itself hits exactly +-448
    q, s = O.quantize_fp8(np.array([0x4040, 0xC040, 0x3F80], dtype=np.uint16))  # 3, -3, 1
    assert q[0] == 0x7E and q[1] == 0xFE


def test_reachable_scales():
    s = O.reachable_scales()
    assert s.dtype == np.float32 and np.all(np.diff(s) > 0)
    assert np.float32(1.0) in s
    assert s.size == 32639


def test_golden_digests_match_c_oracle():
    """The committed fixture equals what the C oracle computes (random 256 scales)."""
    d = np.load(GOLDEN, allow_pickle=False)
    scales, digests = d["scales"], d["digests"]
    np.testing.assert_array_equal(scales, O.reachable_scales())
    rng = np.random.default_rng(2)
    idx = np.concatenate([[0, scales.size - 1], rng.choice(scales.size, 254, replace=False)])
    lib = c_oracle()
    sub = np.ascontiguousarray(scales[idx])
    out = np.zeros(idx.size, dtype=np.uint64)
    lib.oracle_cast_digests(sub.ctypes.data, sub.size, out.ctypes.data, os.cpu_count() or 1)
    np.testing.assert_array_equal(out, digests[idx])


def digest_numpy(q: np.ndarray) -> np.uint64:
    """Same digest as oracle/fp8_cast.c, in numpy (uint64 arithmetic wraps mod 2^64)."""
    x = np.arange(65536, dtype=np.uint64)
    z = x + np.uint64(0x9E3779B97F4A7C15)
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    mix = (z ^ (z >> np.uint64(31))) | np.uint64(1)
    with np.errstate(over="ignore"):
        return np.sum((q.astype(np.uint64) + np.uint64(1)) * mix, dtype=np.uint64)


def test_digest_numpy_matches_c():
    d = np.load(GOLDEN, allow_pickle=False)
    x = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    for i in (0, 1000, 20000, d["scales"].size - 1):
        s = d["scales"][i]
        assert digest_numpy(O.cast_e4m3(x, s)) == d["digests"][i]


# ---- planted mistakes: each must be caught by one of the pins above ----
def _cast_round_half_up(x_bits, scale):
    v = O.bf16_bits_to_f32(x_bits) / np.float32(scale)
    v = np.fmax(-O.FP8_MAX, np.fmin(v, O.FP8_MAX)).astype(np.float32)
    # mistake: ties away from zero instead of to even
    b = v.view(np.uint32).astype(np.uint64)
    a = b & 0x7FFFFFFF
    r = ((a + 0x80000) >> 20) - 0x3C0
    good = O.f32_to_e4m3_rne(v)
    normal = a >= 0x3C800000
    return np.where(normal, (((b >> 24) & 0x80) | r).astype(np.uint8), good)


def _cast_swapped_clamp(x_bits, scale):
    v = O.bf16_bits_to_f32(x_bits) / np.float32(scale)
    # mistake: clamp applied as min(max(...)) with the bounds swapped in sign
    v = np.fmin(np.fmax(v, -O.FP8_MAX), O.FP8_MAX * np.float32(0.999)).astype(np.float32)
    return O.f32_to_e4m3_rne(v)


def _cast_reciprocal(x_bits, scale):
    # mistake: multiply by RN(1/scale) instead of dividing
    v = O.bf16_bits_to_f32(x_bits) * np.float32(np.float32(1.0) / np.float32(scale))
    v = np.fmax(-O.FP8_MAX, np.fmin(v, O.FP8_MAX)).astype(np.float32)
    return O.f32_to_e4m3_rne(v)


@pytest.mark.parametrize("bad_cast", [_cast_round_half_up, _cast_swapped_clamp, _cast_reciprocal])
def test_planted_mistakes_are_caught(bad_cast):
    d = np.load(GOLDEN, allow_pickle=False)
    x = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    caught = False
    for i in range(0, d["scales"].size, 97):
        if digest_numpy(bad_cast(x, d["scales"][i])) != d["digests"][i]:
            caught = True
            break
    assert caught


def test_dropout_hash_known_answers_and_rate():
    """The fused dropout's hash is splitmix64: with seed 0 the state seed + idx * golden gamma
    at idx = 1, 2, 3, 4 gives the published first outputs of splitmix64 seeded with 0; the keep
    rate is 1 - p; the scale is torch's RN32(1 / RN32(1 - p))."""
    got = O.splitmix64(0, np.arange(1, 5, dtype=np.uint64))
    assert [int(v) for v in got] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4,
                                     0x06C45D188009454F, 0xF88BB8A8724C81EC]
    for p in (0.1, 0.2, 0.5):
        keep = O.dropout_keep(987654321, 1 << 18, p)
        assert abs(keep.mean() - (1 - p)) < 5 * np.sqrt(p * (1 - p) / keep.size)
    assert O.dropout_keep(7, 1000, 0.0).all()
    assert O.dropout_scale(0.2) == np.float32(1.25)
    assert O.dropout_scale(0.1) == np.float32(1.0) / np.float32(0.9)


def test_e4m3_decode_matches_torch_on_all_codes():
    """e4m3_to_f32 decodes every operand of the conv/GEMM oracle; it must equal torch's own
    float8_e4m3fn decoder on all 256 codes (subnormals k * 2^-9, both zeros, NaN at 0x7f/0xff)."""
    codes = np.arange(256, dtype=np.uint8)
    got = O.e4m3_to_f32(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan_g, nan_r = np.isnan(got), np.isnan(ref)
    assert np.array_equal(nan_g, nan_r)
    assert np.flatnonzero(nan_r).tolist() == [0x7F, 0xFF]
    assert np.array_equal(got[~nan_g].view(np.uint32), ref[~nan_r].view(np.uint32))


def test_bf16_rounding_matches_torch():
    """f32_to_bf16_bits against torch's Tensor.to(bfloat16) on > 1M fp32 values: random bit
    patterns over the whole finite range, exact ties (low half 0x8000) at both mantissa
    parities, values one ulp either side of a tie, subnormals, infinities and the largest
    finite values (which round to inf); bf16_bits_to_f32 against torch's widening."""
    rng = np.random.default_rng(11)
    u = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    u = u[(u & 0x7F800000) != 0x7F800000]  # finite
    hi = rng.integers(0, 1 << 16, size=1 << 16, dtype=np.uint32) << 16
    ties = hi | 0x8000
    near = np.concatenate([ties - 1, ties + 1])
    sub = rng.integers(1, 1 << 23, size=1 << 14, dtype=np.uint32)
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7F7FFFFF, 0xFF7FFFFF,
                        0x7F7F8000, 0x7F7F7FFF, 0x00008000, 0x00018000], dtype=np.uint32)
    allu = np.concatenate([u, ties, near, sub, sub | 0x80000000, special])
    allu = allu[(allu & 0x7FFFFFFF) <= 0x7F800000]  # NaNs have no single rounding
    f = allu.view(np.float32)
    got = O.f32_to_bf16_bits(f)
    ref = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert f.size > 1_000_000
    assert np.array_equal(got, ref)
    codes = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    wide = O.bf16_bits_to_f32(codes)
    tw = torch.from_numpy(codes.view(np.int16)).view(torch.bfloat16).float().numpy()
    fin = ~np.isnan(tw)
    assert np.array_equal(np.isnan(wide), ~fin)
    assert np.array_equal(wide[fin].view(np.uint32), tw[fin].view(np.uint32))


def test_dropout_threshold_uses_fp32_p():
    """The keep threshold is floor(fp32(p) * 2^16): for p = 13107 / 2^16 - 2^-40 that is 13107,
    one above floor(p * 2^16). A hash quarter of 13106 (built by inverting splitmix64) is
    dropped; the other three quarters of the same hash decide elements 1-3."""
    p, seed, h0 = conftest.dropout_band()
    z = int(O.splitmix64(seed, np.zeros(1, dtype=np.uint64))[0])
    assert z & 0xFFFF == h0 == 13106 and (z >> 16) & 0xFFFF == 0xFFFF and z >> 48 > 0xFF00
    keep = O.dropout_keep(seed, 5, p)
    assert not keep[0] and keep[1:4].all()
    assert O.dropout_keep(seed, 1, np.float32(p))[0] == keep[0]
    assert O.dropout_keep(seed, 1, 13106 / 65536.0)[0]  # a threshold of 13106 keeps it


def test_dropout_mask_layout():
    """Element idx reads 16-bit quarter idx % 4 of splitmix64(seed, idx // 4), low quarter
    first: the mask at p just above a quarter's value drops exactly the elements whose
    quarter is below it, checked on hashes computed here quarter by quarter."""
    seed, n = 0x1234_5678_9ABC_DEF0, 64
    z = O.splitmix64(seed, np.arange(n // 4, dtype=np.uint64))
    q = np.array([(int(z[i // 4]) >> (16 * (i % 4))) & 0xFFFF for i in range(n)])
    for t in (1, int(q[5]), int(q[6]) + 1, 32768, 65535):
        p = t / 65536.0
        assert np.array_equal(O.dropout_keep(seed, n, p), q >= t), t
    assert O.dropout_keep(seed, n, 0.0).all()
