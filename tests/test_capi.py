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
    assert lib.dpa_quantize_fp8_bf16_with_weight_prep(fake, 16, fake, fake, fake, 4096, nul, 1, 1, fake, 4, nul) == -1
    # bad sizes / shapes
    assert lib.dpa_quantize_fp8_bf16(fake, 0, fake, fake, fake, 4096, nul) == -2
    assert lib.dpa_quantize_fp8_bf16_with_weight_prep(fake, 16, fake, fake, fake, 4096, fake, 0, 1, fake, 4, nul) == -2
    assert lib.dpa_quantize_fp8_bf16_with_weight_prep(fake, 16, fake, fake, fake, 4096, fake, 1, 1, fake, 0, nul) == -5
    assert lib.dpa_conv2d_fwd_fp8(fake, fake, fake, fake, nul, fake, 1, 8, 8, 96, 128, 3, 3, 1, 1, nul) == -4
    assert lib.dpa_conv2d_fwd_fp8(fake, fake, fake, fake, nul, fake, 1, 8, 8, 128, 128, 5, 5, 1, 2, nul) == -4
    assert lib.dpa_conv2d_fwd_fp8(fake, fake, fake, fake, nul, fake, 1, 8, 8, 128, 128, 1, 1, 2, 0, nul) == -4
    assert lib.dpa_gemm_fp8(fake, fake, fake, fake, nul, fake, 16, 100, 128, nul) == -4
    assert lib.dpa_gn_silu_fwd_bf16(fake, fake, fake, nul, nul, fake, fake, fake, 1, 16, 96, 32, 1e-5, nul) == -4
    assert lib.dpa_gn_silu_fwd_ws_bf16(fake, fake, fake, nul, nul, nul, fake, fake, fake, fake, 8, 2, 1024, 128, 32, 1e-5, nul) == -5
    assert lib.dpa_gn_silu_fwd_ws_bf16(fake, fake, fake, nul, nul, nul, fake, fake, fake, nul, 0, 1, 16, 96, 32, 1e-5, nul) == -4
    assert lib.dpa_gn_silu_fwd_ws_bf16(nul, fake, fake, nul, nul, nul, fake, fake, fake, nul, 0, 1, 16, 128, 32, 1e-5, nul) == -1
    # fused dropout: p outside [0, 1) and images without a dropout form (96 x 96) are refused
    assert lib.dpa_gn_silu_fwd_ex(fake, 0, fake, fake, nul, nul, fake, fake, fake, fake, nul, 0, 1, 16, 128, 32, 1e-5, fake, 1.0, nul, nul) == -2
    assert lib.dpa_gn_silu_fwd_ex(fake, 0, fake, fake, nul, nul, fake, fake, fake, fake, nul, 0, 1, 9216, 128, 32, 1e-5, fake, 0.2, nul, nul) == -4
    assert lib.dpa_gn_silu_bwd_ex(fake, 0, fake, fake, fake, nul, nul, fake, fake, fake, fake, nul, 0, fake, fake, nul, nul, fake, fake, 1 << 20, 1, 16, 128, 32, fake, -0.5, nul) == -2
    # dx_add: 16-B aligned, chunked or small-image form only; x_bf16 needs an fp32 x
    assert lib.dpa_gn_silu_fwd_ex(fake, 0, fake, fake, nul, nul, nul, fake, fake, fake, nul, 0, 1, 16, 128, 32, 1e-5, nul, 0.0, fake, nul) == -4
    assert lib.dpa_gn_silu_bwd_ex(fake, 0, fake, fake, fake, nul, nul, nul, fake, fake, fake, ctypes.c_void_p(0x1008), 0, fake, fake, nul, nul, nul, fake, 1 << 20, 1, 16, 128, 32, nul, 0.0, nul) == -3
    assert lib.dpa_gn_silu_bwd_ex(fake, 0, fake, fake, fake, nul, nul, nul, fake, fake, fake, fake, 0, fake, fake, nul, nul, nul, fake, 1 << 20, 1, 9216, 128, 32, nul, 0.0, nul) == -4
    # dx_add_dtype: BF16 or F32 only, and an fp32 dx_add only beside an fp32 x
    assert lib.dpa_gn_silu_bwd_ex(fake, 0, fake, fake, fake, nul, nul, nul, fake, fake, fake, fake, 1, fake, fake, nul, nul, nul, fake, 1 << 20, 1, 1024, 128, 32, nul, 0.0, nul) == -4
    assert lib.dpa_gn_silu_bwd_ex(fake, 1, fake, fake, fake, nul, nul, nul, fake, fake, fake, fake, 2, fake, fake, nul, nul, nul, fake, 1 << 20, 1, 1024, 128, 32, nul, 0.0, nul) == -4
    assert lib.dpa_gn_silu_bwd_ex(fake, 0, fake, fake, fake, nul, nul, nul, fake, fake, fake, fake, -1, fake, fake, nul, nul, nul, fake, 1 << 20, 1, 1024, 128, 32, nul, 0.0, nul) == -4
    assert lib.dpa_quantize_fp8_delayed_window_bf16(fake, 16, fake, fake, fake, nul, fake, 4, 0,
                                                    fake, 4096, nul) == -1
    assert lib.dpa_quantize_fp8_delayed_window_bf16(fake, 16, fake, fake, fake, fake, fake, 0, 0,
                                                    fake, 4096, nul) == -2
    assert lib.dpa_window_max3_f32(nul, fake, fake, 4, fake, nul) == -1
    assert lib.dpa_window_max3_f32(fake, fake, fake, 0, fake, nul) == -2
    # the allocation-free quantize checks its arguments before it looks up its device array
    assert lib.dpa_quantize_fp8_bf16_noalloc(nul, 16, fake, fake, nul) == -1
    assert lib.dpa_quantize_fp8_bf16_noalloc(fake, 0, fake, fake, nul) == -2
    assert lib.dpa_quantize_fp8_bf16_noalloc(fake, 16, fake, ctypes.c_void_p(0x1002), nul) == -3
    assert lib.dpa_quantize_fp8_bf16_noalloc_scratch_bytes() == lib.dpa_quant_workspace_bytes(1 << 40)
    # self-attention: NULL, batch 0, heads that do not make 64-wide heads, L outside
    # {16, 32, ..., 256}, misaligned qkv
    assert lib.dpa_attention_fwd_bf16(nul, fake, fake, 2, 64, 256, 4, nul) == -1
    assert lib.dpa_attention_fwd_bf16(fake, fake, fake, 0, 64, 256, 4, nul) == -2
    assert lib.dpa_attention_fwd_bf16(fake, fake, fake, 2, 64, 256, 2, nul) == -4
    assert lib.dpa_attention_fwd_bf16(fake, fake, fake, 2, 72, 256, 4, nul) == -4
    assert lib.dpa_attention_fwd_bf16(fake, fake, fake, 2, 272, 256, 4, nul) == -4
    assert lib.dpa_attention_fwd_bf16(ctypes.c_void_p(0x1008), fake, fake, 2, 64, 256, 4, nul) == -3
    assert lib.dpa_attention_bwd_bf16(fake, fake, nul, fake, fake, 2, 64, 256, 4, nul) == -1
    assert lib.dpa_attention_bwd_bf16(fake, fake, fake, fake, fake, 2, 8, 256, 4, nul) == -4
    assert lib.dpa_attention_bwd_bf16(fake, fake, ctypes.c_void_p(0x1008), fake, fake, 2, 64, 256, 4, nul) == -3
    # the training loss: NULL, n = 0, dtype, workspace, alignment
    assert lib.dpa_mse_loss_f32(nul, 0, fake, 16, fake, fake, 1024, nul) == -1
    assert lib.dpa_mse_loss_f32(fake, 0, fake, 0, fake, fake, 1024, nul) == -2
    assert lib.dpa_mse_loss_f32(fake, 2, fake, 16, fake, fake, 1024, nul) == -4
    assert lib.dpa_mse_loss_f32(fake, 0, fake, 16, fake, fake, 8, nul) == -5
    assert lib.dpa_mse_loss_f32(fake, 1, fake, 16, fake, ctypes.c_void_p(0x1002), 1024, nul) == -3
    # workspace too small
    assert lib.dpa_quantize_fp8_bf16(fake, 16, fake, fake, fake, 8, nul) == -5
    assert lib.dpa_conv2d_dgrad_fp8(fake, fake, fake, fake, fake, fake, 10, 1, 8, 8, 128, 128, 3, 3, 1, 1, nul) == -5
    assert lib.dpa_conv2d_wgrad_fp8(fake, fake, fake, fake, fake, fake, 10, 2, 8, 8, 128, 128, 3, 3, 1, 1, 0, nul) == -5
    assert lib.dpa_conv2d_fwd_fp8_split(fake, fake, fake, fake, nul, fake, fake, 10, 128, 4, 4, 256, 256, 3, 3, 1, 1, nul) == -5
    assert lib.dpa_conv2d_fwd_fp8_split(fake, fake, fake, fake, nul, fake, nul, 1 << 30, 128, 4, 4, 256, 256, 3, 3, 1, 1, nul) == -5
    assert lib.dpa_conv2d_dgrad_fp8_wt_split(fake, fake, fake, fake, fake, fake, 10, 128, 4, 4, 256, 256, 3, 3, 1, 1, nul) == -5
    assert lib.dpa_gemm_fp8_split(fake, fake, fake, fake, nul, fake, fake, 10, 128, 512, 1024, nul) == -5
    assert lib.dpa_conv2d_fwd_fp8_split(nul, fake, fake, fake, nul, fake, fake, 10, 128, 4, 4, 256, 256, 3, 3, 1, 1, nul) == -1
    assert lib.dpa_gemm_fp8_split(fake, fake, fake, fake, nul, fake, fake, 1 << 30, 128, 500, 1024, nul) == -4
    assert lib.dpa_conv2d_dgrad_fp8_wt_split(fake, fake, fake, fake, fake, fake, 1 << 30, 128, 4, 4, 256, 256, 5, 5, 1, 2, nul) == -4
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


def test_gn_workspace_queries(lib):
    """Chunked GroupNorm for images of 256+ pixels: (mean, M2) per (image, chunk of 128
    pixels, group) forward; per-image partials plus per-chunk channel sums backward."""
    assert lib.dpa_gn_silu_fwd_workspace_bytes(128, 1024, 128, 32) == 128 * 8 * 32 * 8
    assert lib.dpa_gn_silu_fwd_workspace_bytes(128, 64, 256, 32) == 0
    assert lib.dpa_gn_silu_fwd_workspace_bytes(2, 323, 128, 32) == 2 * 3 * 32 * 8
    assert lib.dpa_gn_silu_bwd_workspace_bytes(128, 1024, 128, 32) == 2 * 128 * 128 * 4 + 8 * 128 * 128 * 16
    assert lib.dpa_gn_silu_bwd_workspace_bytes(128, 64, 256, 32) == 2 * 128 * 256 * 4


def test_split_workspace_queries(lib):
    """Split-K plans (256 CUs; one 256 x 128 fp32 block per work item): the 4x4 / 256-channel
    U-Net conv has 16 output tiles and 18 K-steps, so it splits 3 ways (six K-steps per
    part); launches that fill the GPU, and the halo-kernel shapes, need none."""
    block = 256 * 128 * 4
    assert lib.dpa_conv2d_fwd_split_workspace_bytes(128, 32, 32, 128, 128, 3, 3, 1, 1) == 0
    assert lib.dpa_conv2d_fwd_split_workspace_bytes(128, 4, 4, 256, 256, 3, 3, 1, 1) == 3 * 16 * block
    assert lib.dpa_conv2d_dgrad_split_workspace_bytes(128, 4, 4, 256, 256, 3, 3, 1, 1) == 3 * 16 * block
    # 8x8, 512 -> 256: 64 tiles, 36 K-steps: 4 ways (256 work items = CUs)
    assert lib.dpa_conv2d_fwd_split_workspace_bytes(128, 8, 8, 512, 256, 3, 3, 1, 1) == 4 * 64 * block
    # cfg1 GEMM: 768 tiles, no split; a 128-row GEMM with K = 1024 and 512 outputs: 4 tiles,
    # 8 K-steps: 4 ways of two steps
    assert lib.dpa_gemm_split_workspace_bytes(32768, 768, 256) == 0
    assert lib.dpa_gemm_split_workspace_bytes(128, 512, 1024) == 4 * 4 * block
    # fewer than eight K-steps per tile never split; unsupported shapes report 0
    assert lib.dpa_gemm_split_workspace_bytes(128, 512, 512) == 0
    assert lib.dpa_gemm_split_workspace_bytes(128, 512, 128) == 0
    assert lib.dpa_gemm_split_workspace_bytes(128, 500, 1024) == 0
    assert lib.dpa_conv2d_fwd_split_workspace_bytes(128, 4, 4, 96, 256, 3, 3, 1, 1) == 0


def test_weight_prep_plan_on_host(lib):
    """dpa_weight_prep_plan reads the ctypes DpaWeightEntry array (layout of
    include/dpa_fp8.h) and assigns one block per tile of 64 x 64 channels of one tap, in
    order."""
    import ctypes
    WP = dpa_mod("weight_prep")
    shapes = [(128, 9, 128), (256, 1, 512), (512, 1, 128)]
    entries = (WP.DpaWeightEntry * len(shapes))()
    for e, (co, taps, ci) in zip(entries, shapes):
        e.w, e.q, e.qt, e.scale_used = 0x10000, 0x20000, 0x30000, 0x40000
        e.n, e.cout, e.taps, e.cin = co * taps * ci, co, taps, ci
    total = lib.dpa_weight_prep_plan(ctypes.addressof(entries), len(shapes))
    nblk = [-(-co // 64) * taps * -(-ci // 64) for co, taps, ci in shapes]
    assert nblk == [36, 32, 16]
    assert total == sum(nblk)
    assert [e.nblk for e in entries] == nblk
    assert [e.blk0 for e in entries] == [0, nblk[0], nblk[0] + nblk[1]]
    assert lib.dpa_weight_prep_workspace_bytes(total) == 4 * total
    entries[1].cin = 500                      # n no longer cout * taps * cin
    assert lib.dpa_weight_prep_plan(ctypes.addressof(entries), len(shapes)) == -4
    entries[1].cin = 512
    entries[2].w = 0x10004                    # fp32 weights must be 16-B aligned
    assert lib.dpa_weight_prep_plan(ctypes.addressof(entries), len(shapes)) == -3
    nul = None
    assert lib.dpa_weight_prep_run(nul, 3, total, ctypes.c_void_p(0x1000), 4 * total, nul) == -1
    assert lib.dpa_weight_prep_run(ctypes.c_void_p(0x1000), 3, total, ctypes.c_void_p(0x1000), 8, nul) == -5
    assert lib.dpa_window_max_grouped_f32(nul, 3, 1024, ctypes.c_void_p(0x1000), nul) == -1
    assert lib.dpa_conv2d_wgrad_fp8_f32(ctypes.c_void_p(0x1000), ctypes.c_void_p(0x1000), ctypes.c_void_p(0x1000),
                                        ctypes.c_void_p(0x1000), ctypes.c_void_p(0x1008), ctypes.c_void_p(0x1000),
                                        1 << 30, 2, 8, 8, 128, 128, 3, 3, 1, 1, 0, nul) == -3


def test_deferred_window_entries(lib):
    import ctypes
    WP = dpa_mod("weight_prep")
    assert ctypes.sizeof(WP.DpaDeferredWindow) == 64
    assert lib.dpa_quant_partials_count(0) == 0
    assert lib.dpa_quant_partials_count(8) == 1
    assert lib.dpa_quant_partials_count(1 << 30) == 256  # the amax pass's grid cap
    fake, nul = ctypes.c_void_p(0x1000), None
    assert lib.dpa_quantize_fp8_delayed_deferred_bf16(nul, 16, fake, fake, fake, 512, fake, nul) == -1
    assert lib.dpa_quantize_fp8_delayed_deferred_bf16(fake, 0, fake, fake, fake, 512, fake, nul) == -2
    assert lib.dpa_quantize_fp8_delayed_deferred_bf16(fake, 1 << 30, fake, fake, fake, 100, fake, nul) == -5
    assert lib.dpa_quantize_fp8_delayed_deferred_bf16(ctypes.c_void_p(0x1008), 16, fake, fake, fake, 512, fake, nul) == -3
    assert lib.dpa_delayed_windows_finalize(nul, 3, nul) == -1
    assert lib.dpa_delayed_windows_finalize(fake, 0, nul) == -2
