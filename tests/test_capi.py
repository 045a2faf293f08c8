"""The C-ABI library loads, exports every symbol include/dpa_fp8.h declares, and rejects bad
arguments with the documented status codes before launching anything (no GPU needed)."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from conftest import ROOT, dpa_mod

HEADER = os.path.join(ROOT, "include", "dpa_fp8.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dpa_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return dpa_mod("_lib").load()


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for name in ("dpa_quantize_fp8_bf16", "dpa_quantize_fp8_delayed_bf16", "dpa_conv2d_fwd_fp8",
                 "dpa_conv2d_dgrad_fp8", "dpa_conv2d_wgrad_fp8", "dpa_gemm_fp8",
                 "dpa_gn_silu_fwd_bf16", "dpa_gn_silu_bwd_bf16"):
        assert name in syms


def test_every_declared_symbol_is_exported(lib):
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_python_binding_covers_header():
    sigs = dpa_mod("_lib").SIGNATURES
    assert sorted(sigs) == declared_symbols()


def test_status_strings(lib):
    assert lib.dpa_abi_version() == 1
    L = dpa_mod("_lib")
    assert L.status_string(0) == "ok"
    assert "NULL" in L.status_string(-1)
    assert "shape" in L.status_string(-4)
    assert "workspace" in L.status_string(-5)


def test_precondition_errors_return_before_launch(lib):
    nul = None
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails a check first
    # NULL inputs
    assert lib.dpa_quantize_fp8_bf16(nul, 16, fake, fake, fake, 4096, nul) == -1
    assert lib.dpa_conv2d_fwd_fp8(nul, fake, fake, fake, nul, fake, 1, 8, 8, 128, 128, 3, 3, 1, 1, nul) == -1
    # bad sizes / shapes
    assert lib.dpa_quantize_fp8_bf16(fake, 0, fake, fake, fake, 4096, nul) == -2
    assert lib.dpa_conv2d_fwd_fp8(fake, fake, fake, fake, nul, fake, 1, 8, 8, 96, 128, 3, 3, 1, 1, nul) == -4
    assert lib.dpa_conv2d_fwd_fp8(fake, fake, fake, fake, nul, fake, 1, 8, 8, 128, 128, 5, 5, 1, 2, nul) == -4
    assert lib.dpa_conv2d_fwd_fp8(fake, fake, fake, fake, nul, fake, 1, 8, 8, 128, 128, 1, 1, 2, 0, nul) == -4
    assert lib.dpa_gemm_fp8(fake, fake, fake, fake, nul, fake, 16, 100, 128, nul) == -4
    assert lib.dpa_gn_silu_fwd_bf16(fake, fake, fake, nul, nul, fake, fake, fake, 1, 16, 96, 32, 1e-5, nul) == -4
    assert lib.dpa_quantize_fp8_delayed_window_bf16(fake, 16, fake, fake, fake, nul, fake, 4, 0,
                                                    fake, 4096, nul) == -1
    assert lib.dpa_quantize_fp8_delayed_window_bf16(fake, 16, fake, fake, fake, fake, fake, 0, 0,
                                                    fake, 4096, nul) == -2
    assert lib.dpa_window_max3_f32(nul, fake, fake, 4, fake, nul) == -1
    assert lib.dpa_window_max3_f32(fake, fake, fake, 0, fake, nul) == -2
    # workspace too small
    assert lib.dpa_quantize_fp8_bf16(fake, 16, fake, fake, fake, 8, nul) == -5
    assert lib.dpa_conv2d_dgrad_fp8(fake, fake, fake, fake, fake, fake, 10, 1, 8, 8, 128, 128, 3, 3, 1, 1, nul) == -5
    assert lib.dpa_conv2d_wgrad_fp8(fake, fake, fake, fake, fake, fake, 10, 2, 8, 8, 128, 128, 3, 3, 1, 1, 0, nul) == -5
    # misaligned e4m3 operand
    odd = ctypes.c_void_p(0x1001)
    assert lib.dpa_conv2d_fwd_fp8(odd, fake, fake, fake, nul, fake, 1, 8, 8, 128, 128, 3, 3, 1, 1, nul) == -3


def test_workspace_queries(lib):
    assert lib.dpa_quant_workspace_bytes(1 << 24) == 4096
    assert lib.dpa_conv2d_dgrad_workspace_bytes(128, 256, 3, 3) == 128 * 256 * 9
    ws = lib.dpa_conv2d_wgrad_workspace_bytes(128, 32, 32, 128, 128, 3, 3, 1, 1, 0)
    assert ws > 0 and ws % (128 * 128 * 9 * 4) == 0
    assert lib.dpa_conv2d_wgrad_workspace_bytes(128, 32, 32, 128, 128, 3, 3, 1, 1, 4) == 4 * 128 * 128 * 9 * 4
    assert lib.dpa_conv2d_wgrad_workspace_bytes(128, 32, 32, 100, 128, 3, 3, 1, 1, 0) == 0
