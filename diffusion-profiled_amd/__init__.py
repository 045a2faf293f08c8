"""MI355X-native (gfx950) FP8 conv/GEMM path for the fattorib/diffusion-profiled U-Net.

Import with ``importlib.import_module("diffusion-profiled_amd")`` (the directory name has a
hyphen). The kernels live in ``lib/libdpa_fp8.so`` (C ABI: ``include/dpa_fp8.h``), built
from ``csrc/*.hip`` by ``build.build_library()``.
"""
from . import _lib, attention, build, fp8_kernels, gn_silu  # noqa: F401
from . import ddpm, unet, trainer  # noqa: F401
from .fp8_kernels import (  # noqa: F401
    FP8_DTYPE,
    FP8_MAX_E4M3,
    SUPPORTED_UNET_SHAPES,
    Conv2dFP8Specialized,
    conv2d_bwd_input_fp8,
    conv2d_bwd_input_fp8_prequantized,
    conv2d_bwd_weight_fp8,
    conv2d_bwd_weight_fp8_prequantized,
    conv2d_fp8,
    conv2d_fwd_fp8,
    conv2d_fwd_fp8_prequantized,
    hip_conv2d_fp8,
    LinearFP8Function,
    linear_fp8,
    linear_fp8_autograd,
    quantize_fp8,
    quantize_fp8_delayed,
    triton_conv2d_fp8,
)
