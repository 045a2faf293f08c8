"""Shared test setup: repo root on sys.path, the ``gpu`` marker, seeded input builders."""
from __future__ import annotations

import importlib
import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PKG_NAME = "diffusion-profiled_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through the C ABI")


def dpa():
    """The product package (directory name has a hyphen, hence importlib)."""
    return importlib.import_module(PKG_NAME)


def dpa_mod(name: str):
    return importlib.import_module(f"{PKG_NAME}.{name}")


# ---- seeded inputs (CPU generator, fp32 draw, then bf16), as the bench and CPU baseline ----
def randn_bf16(shape, seed: int, std: float = 1.0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * std).to(torch.bfloat16)


def kaiming_uniform_bf16(shape, seed: int) -> torch.Tensor:
    """nn.Conv2d / nn.Linear default init: U(+-1/sqrt(fan_in)) (kaiming_uniform_(a=sqrt(5)))."""
    g = torch.Generator().manual_seed(seed)
    fan_in = int(np.prod(shape[1:]))
    bound = 1.0 / np.sqrt(fan_in)
    return (torch.rand(shape, generator=g, dtype=torch.float32) * 2 * bound - bound).to(torch.bfloat16)


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bit pattern of a CPU tensor as a numpy array (uint16 for bf16, uint8 for fp8)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype in (torch.float8_e4m3fn, torch.uint8):
        return t.view(torch.uint8).numpy()
    raise TypeError(t.dtype)


def nhwc_bits(t: torch.Tensor) -> np.ndarray:
    """NCHW-logical tensor -> NHWC bit array."""
    return bits(t.permute(0, 2, 3, 1).contiguous())


def assert_bf16_close(got_bits: np.ndarray, ref_bits: np.ndarray, what: str = "",
                      rel_norm_tol: float = 1e-2):
    """The conv/GEMM tolerance: normwise relative error <= 1e-2 (the stated contract), and
    elementwise |g - r| <= 2^-7 |r| + 2^-10 rms(r) (one bf16 ulp plus fp32 accumulation noise).
    Returns the fraction of bit-identical elements."""
    from oracle.fp8_oracle import bf16_bits_to_f32

    g = bf16_bits_to_f32(got_bits).astype(np.float64)
    r = bf16_bits_to_f32(ref_bits).astype(np.float64)
    assert g.shape == r.shape, (g.shape, r.shape)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    rms = np.sqrt(np.mean(r * r)) if r.size else 0.0
    norm_err = np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30)
    assert norm_err <= rel_norm_tol, f"{what}: normwise rel err {norm_err:.3e}"
    bound = 2.0**-7 * np.abs(r) + 2.0**-10 * rms
    bad = np.abs(g - r) > bound
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} elements beyond 1 bf16 ulp; worst "
        f"{np.max(np.abs(g - r) - bound):.3e}, norm err {norm_err:.3e}"
    )
    return float(np.mean(got_bits == ref_bits))


def _splitmix64_state_for(z: int) -> int:
    """Inverse of splitmix64's finaliser: the state whose output is z (each xorshift and odd
    multiply is a bijection on 64-bit words)."""
    m = (1 << 64) - 1
    z ^= (z >> 31) ^ (z >> 62)
    z = (z * pow(0x94D049BB133111EB, -1, 1 << 64)) & m
    z ^= (z >> 27) ^ (z >> 54)
    z = (z * pow(0xBF58476D1CE4E5B9, -1, 1 << 64)) & m
    z ^= (z >> 30) ^ (z >> 60)
    return z


def dropout_band(k: int = 13107) -> tuple[float, int, int]:
    """A drop probability p whose fp32 value is k / 2^16 while floor(p * 2^16) = k - 1, and a
    seed whose element-0 hash quarter is k - 1: element 0 is kept under the double-precision
    threshold and dropped under the fp32 one the C ABI takes; elements 1-3 (quarters 0xFFFF)
    are kept. Returns (p, seed, element-0 quarter)."""
    p = k / 65536.0 - 2.0**-40
    assert float(np.float32(p)) == k / 65536.0 and int(p * 65536.0) == k - 1
    h0 = k - 1
    for hi in range(0xFFFF, 0xFF00, -1):  # quarter 3 stays near the top; the seed fits an int64
        seed = _splitmix64_state_for((hi << 48) | (0xFFFF << 32) | (0xFFFF << 16) | h0)
        if seed < 2**62:
            return p, seed, h0
    raise AssertionError("no seed below 2^62")
