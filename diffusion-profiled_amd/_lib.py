"""ctypes binding of the C ABI in ``include/dpa_fp8.h`` (``lib/libdpa_fp8.so``).

Every entry point takes raw device pointers, sizes and a ``hipStream_t``; this module only
declares the signatures and turns non-zero status codes into ``RuntimeError``. There is no
fallback: if the library is missing, every op raises.
"""
from __future__ import annotations

import ctypes
import threading
from ctypes import POINTER, c_char_p, c_float, c_int, c_int64, c_void_p

import torch

from . import build as _build


@torch.compiler.disable
def current_stream(t: "torch.Tensor") -> int:
    """The hipStream_t of torch's current stream on t's device, where every launch goes (so
    launches order with torch's own kernels and graph capture records them). Dynamo never
    traces it: under torch.compile a call here ends the graph and the ctypes launch that
    follows runs eagerly. The FP8 ops call it inside torch.library custom-op bodies, which
    Dynamo does not enter."""
    return torch.cuda.current_stream(t.device).cuda_stream

c_float_p = POINTER(c_float)

# name -> (restype, argtypes); kept in the order of include/dpa_fp8.h
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "dpa_status_string": (c_char_p, [c_int]),
    "dpa_abi_version": (c_int, []),
    "dpa_quant_workspace_bytes": (c_int64, [c_int64]),
    "dpa_quantize_fp8_bf16": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_void_p]),
    "dpa_quantize_fp8_bf16_noalloc_scratch_bytes": (c_int64, []),
    "dpa_quantize_fp8_bf16_noalloc": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_void_p]),
    "dpa_quantize_fp8_delayed_bf16": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p],
    ),
    "dpa_quantize_fp8_delayed_window_bf16": (
        c_int,
        [c_void_p, c_int64] + [c_void_p] * 5 + [c_int64, c_int, c_void_p, c_int64, c_void_p],
    ),
    "dpa_window_max3_f32": (c_int, [c_void_p] * 3 + [c_int64, c_void_p, c_void_p]),
    "dpa_conv2d_fwd_fp8": (
        c_int,
        [c_void_p] * 6 + [c_int] * 9 + [c_void_p],
    ),
    "dpa_conv2d_dgrad_workspace_bytes": (c_int64, [c_int] * 4),
    "dpa_conv2d_dgrad_fp8": (
        c_int,
        [c_void_p] * 6 + [c_int64] + [c_int] * 9 + [c_void_p],
    ),
    "dpa_conv2d_dgrad_fp8_wt": (
        c_int,
        [c_void_p] * 5 + [c_int] * 9 + [c_void_p],
    ),
    "dpa_weight_transpose_fp8": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p]),
    "dpa_weight_frag_bytes": (c_int64, [c_int] * 4),
    "dpa_weight_frag_fp8": (c_int, [c_void_p] * 3 + [c_int] * 4 + [c_void_p]),
    "dpa_conv2d_fwd_fp8_wf": (c_int, [c_void_p] * 6 + [c_int] * 5 + [c_void_p]),
    "dpa_conv2d_dgrad_fp8_wf": (c_int, [c_void_p] * 5 + [c_int] * 5 + [c_void_p]),
    "dpa_conv2d_wgrad_workspace_bytes": (c_int64, [c_int] * 10),
    "dpa_conv2d_wgrad_fp8": (
        c_int,
        [c_void_p] * 6 + [c_int64] + [c_int] * 10 + [c_void_p],
    ),
    "dpa_gemm_fp8": (c_int, [c_void_p] * 6 + [c_int] * 3 + [c_void_p]),
    "dpa_quant_partials_count": (c_int, [c_int64]),
    "dpa_quantize_fp8_delayed_deferred_bf16": (
        c_int,
        [c_void_p, c_int64] + [c_void_p] * 3 + [c_int, c_void_p, c_void_p],
    ),
    "dpa_delayed_windows_finalize": (c_int, [c_void_p, c_int, c_void_p]),
    "dpa_weight_prep_plan": (c_int, [c_void_p, c_int]),
    "dpa_weight_prep_workspace_bytes": (c_int64, [c_int]),
    "dpa_weight_prep_run": (c_int, [c_void_p, c_int, c_int, c_void_p, c_int64, c_void_p]),
    "dpa_quantize_fp8_bf16_with_weight_prep": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int, c_int, c_void_p, c_int64, c_void_p]),
    "dpa_window_max_grouped_f32": (c_int, [c_void_p, c_int, c_int64, c_void_p, c_void_p]),
    "dpa_conv2d_wgrad_fp8_f32": (
        c_int,
        [c_void_p] * 6 + [c_int64] + [c_int] * 10 + [c_void_p],
    ),
    "dpa_conv2d_fwd_split_workspace_bytes": (c_int64, [c_int] * 9),
    "dpa_conv2d_fwd_fp8_split": (
        c_int,
        [c_void_p] * 7 + [c_int64] + [c_int] * 9 + [c_void_p],
    ),
    "dpa_conv2d_dgrad_split_workspace_bytes": (c_int64, [c_int] * 9),
    "dpa_conv2d_dgrad_fp8_wt_split": (
        c_int,
        [c_void_p] * 6 + [c_int64] + [c_int] * 9 + [c_void_p],
    ),
    "dpa_gemm_split_workspace_bytes": (c_int64, [c_int] * 3),
    "dpa_gemm_fp8_split": (c_int, [c_void_p] * 7 + [c_int64] + [c_int] * 3 + [c_void_p]),
    "dpa_gn_silu_fwd_bf16": (
        c_int,
        [c_void_p] * 8 + [c_int] * 4 + [c_float, c_void_p],
    ),
    "dpa_layernorm_fwd_bf16": (
        c_int,
        [c_void_p] * 6 + [c_int64, c_int, c_float, c_void_p],
    ),
    "dpa_layernorm_bwd_workspace_bytes": (c_int64, [c_int64, c_int]),
    "dpa_layernorm_bwd_bf16": (
        c_int,
        [c_void_p] * 9 + [c_int64, c_int64, c_int, c_void_p],
    ),
    "dpa_layernorm_fwd_ex": (c_int, [c_void_p, c_int] + [c_void_p] * 5 + [c_int64, c_int, c_float, c_void_p]),
    "dpa_layernorm_bwd_ex": (c_int, [c_void_p, c_int] + [c_void_p] * 8 + [c_int64, c_int64, c_int, c_void_p]),
    "dpa_layernorm_bwd_ex_add": (
        c_int, [c_void_p, c_int] + [c_void_p] * 9 + [c_int64, c_int64, c_int, c_void_p],
    ),
    "dpa_attention_fwd_bf16": (c_int, [c_void_p] * 3 + [c_int] * 4 + [c_void_p]),
    "dpa_attention_bwd_bf16": (c_int, [c_void_p] * 5 + [c_int] * 4 + [c_void_p]),
    "dpa_attention_fwd_amax": (c_int, [c_void_p] * 3 + [c_int] * 4 + [c_void_p, c_void_p]),
    "dpa_attention_bwd_amax": (c_int, [c_void_p] * 5 + [c_int] * 4 + [c_void_p, c_void_p]),
    "dpa_layernorm_fwd_partials": (c_int, [c_int64, c_int]),
    "dpa_layernorm_fwd_amax": (c_int, [c_void_p, c_int] + [c_void_p] * 5 + [c_int64, c_int, c_float, c_void_p, c_void_p]),
    "dpa_quantize_fp8_bf16_from_partials": (c_int, [c_void_p, c_int64, c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
    "dpa_residual_scale_bf16": (c_int, [c_void_p] * 3 + [c_int64, c_float, c_void_p]),
    "dpa_residual_scale_f32": (c_int, [c_void_p] * 3 + [c_int64, c_float, c_void_p]),
    "dpa_residual_scale_bwd_f32": (c_int, [c_void_p] * 3 + [c_int64, c_float, c_void_p]),
    "dpa_upsample_concat_f32": (c_int, [c_void_p, c_int, c_void_p, c_int, c_void_p] + [c_int] * 6 + [c_void_p]),
    "dpa_upsample_concat_bwd_f32": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_int] + [c_int] * 6 + [c_void_p]),
    "dpa_upcat_gn_silu_fwd": (c_int, [c_void_p, c_void_p] + [c_int] * 6
                              + [c_void_p] * 6 + [c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                                  c_void_p, c_int, c_int, c_float, c_void_p]),
    "dpa_upcat_gn_silu_bwd": (c_int, [c_void_p, c_void_p] + [c_int] * 6 + [c_void_p] * 11
                              + [c_int64, c_int, c_void_p]),
    "dpa_downsample2_f32": (c_int, [c_void_p, c_int, c_void_p] + [c_int] * 4 + [c_void_p]),
    "dpa_downsample2_bwd_f32": (c_int, [c_void_p, c_void_p, c_int] + [c_int] * 4 + [c_void_p]),
    "dpa_downsample2_bwd_add_f32": (c_int, [c_void_p] * 3 + [c_int] * 5 + [c_void_p]),
    "dpa_mse_loss_workspace_bytes": (c_int64, []),
    "dpa_mse_loss_f32": (c_int, [c_void_p, c_int, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p]),
    "dpa_adamw_ema_workspace_bytes": (c_int64, [c_void_p, c_int]),
    "dpa_adamw_ema_step": (
        c_int,
        [c_void_p, c_int, c_void_p] + [c_float] * 7 + [c_void_p, c_int64, c_void_p],
    ),
    "dpa_gn_silu_fwd_workspace_bytes": (c_int64, [c_int] * 4),
    "dpa_gn_silu_fwd_ws_bf16": (
        c_int,
        [c_void_p] * 10 + [c_int64] + [c_int] * 4 + [c_float, c_void_p],
    ),
    "dpa_gn_silu_bwd_workspace_bytes": (c_int64, [c_int] * 4),
    "dpa_gn_silu_bwd_bf16": (
        c_int,
        [c_void_p] * 14 + [c_int64] + [c_int] * 4 + [c_void_p],
    ),
    "dpa_gn_silu_film_fwd_bf16": (
        c_int,
        [c_void_p] * 7 + [c_int] * 4 + [c_float, c_void_p],
    ),
    "dpa_gn_silu_film_bwd_bf16": (
        c_int,
        [c_void_p] * 12 + [c_int64] + [c_int] * 4 + [c_void_p],
    ),
    "dpa_gn_silu_fwd_ex": (
        c_int,
        [c_void_p, c_int] + [c_void_p] * 9 + [c_int64] + [c_int] * 4
        + [c_float, c_void_p, c_float, c_void_p, c_void_p],
    ),
    "dpa_gn_silu_bwd_ex": (
        c_int,
        [c_void_p, c_int] + [c_void_p] * 10 + [c_int] + [c_void_p] * 6 + [c_int64] + [c_int] * 4
        + [c_void_p, c_float, c_void_p],
    ),
    "dpa_gn_silu_fp8_partials": (c_int, [c_int] * 4),
    "dpa_gn_silu_fwd_fp8": (
        c_int,
        [c_void_p, c_int] + [c_void_p] * 8 + [c_int] + [c_void_p] * 4 + [c_int64] + [c_int] * 4
        + [c_float, c_void_p, c_float, c_void_p, c_void_p],
    ),
    "dpa_gn_silu_fwd_ex_amax": (
        c_int,
        [c_void_p, c_int] + [c_void_p] * 9 + [c_int64] + [c_int] * 4
        + [c_float, c_void_p, c_float, c_void_p, c_void_p, c_int, c_void_p],
    ),
    "dpa_gn_silu_fwd_fp8_amax": (
        c_int,
        [c_void_p, c_int] + [c_void_p] * 8 + [c_int] + [c_void_p] * 4 + [c_int64] + [c_int] * 4
        + [c_float, c_void_p, c_float, c_void_p, c_void_p, c_int, c_void_p],
    ),
    "dpa_gn_silu_bwd_fp8": (
        c_int,
        [c_void_p] * 12 + [c_int] + [c_void_p] * 7 + [c_int64] + [c_int] * 4
        + [c_void_p, c_float, c_void_p],
    ),
    "dpa_grouped_quantize_fp8_bf16": (c_int, [c_void_p, c_void_p, c_int, c_int] + [c_void_p] * 4),
    "dpa_grouped_linear_fwd_fp8": (c_int, [c_void_p] * 6 + [c_int] * 3 + [c_void_p]),
    "dpa_grouped_linear_wgrad_fp8_f32": (c_int, [c_void_p] * 6 + [c_int] * 3 + [c_void_p]),
    "dpa_grouped_linear_dgrad_workspace_bytes": (c_int64, [c_int] * 3),
    "dpa_grouped_linear_dgrad_fp8": (
        c_int, [c_void_p] * 6 + [c_int] * 3 + [c_void_p, c_int64, c_void_p],
    ),
    "dpa_residual_scale_fp8_partials": (c_int, [c_int64]),
    "dpa_residual_scale_bwd_fp8": (
        c_int, [c_void_p, c_int] + [c_void_p] * 4 + [c_int, c_void_p, c_int64, c_float, c_void_p],
    ),
    "dpa_residual_scale_bwd_amax": (
        c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int, c_int64, c_float, c_void_p],
    ),
    "dpa_conv3x3_thin_fwd": (
        c_int, [c_void_p, c_int, c_void_p, c_int] + [c_int] * 4 + [c_void_p] + [c_int] * 5 + [c_void_p],
    ),
    "dpa_conv3x3_thin_dgrad": (
        c_int, [c_void_p, c_void_p, c_int] + [c_int] * 4 + [c_void_p] + [c_int] * 5 + [c_void_p],
    ),
    "dpa_conv3x3_thin_wgrad_workspace_bytes": (c_int64, [c_int] * 5),
    "dpa_conv3x3_thin_wgrad": (
        c_int, [c_void_p, c_int, c_void_p, c_void_p] + [c_int] * 5 + [c_void_p, c_int64, c_void_p],
    ),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def library_path():
    return _build.LIB_PATH


def load(build_if_missing: bool = True) -> ctypes.CDLL:
    """Load (once) and return the library. Builds it only when no built library exists."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = _build.LIB_PATH
        if not path.exists():
            if not build_if_missing:
                raise RuntimeError(f"FP8 HIP library not built: {path}")
            _build.build_library()
        lib = ctypes.CDLL(str(path))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def status_string(status: int) -> str:
    return load().dpa_status_string(status).decode()


def check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what} failed: {status_string(status)} (status {status})")


def call(name: str, *args) -> None:
    """Call an entry point that returns a status code; raise on failure."""
    check(getattr(load(), name)(*args), name)


def query(name: str, *args) -> int:
    """Call an entry point that returns a size."""
    return int(getattr(load(), name)(*args))
