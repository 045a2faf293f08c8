"""FP8 conv/GEMM operators on the gfx950 HIP library — drop-in for the reference's
``diffusion/fp8_kernels.py`` (fattorib/diffusion-profiled).

Same public names, argument meanings, return values and error behaviour as the reference
(AssertionError for the launch-time checks, KeyError for shapes missing from the registry,
NotImplementedError for a non-channels-last weight gradient). The Triton kernels are replaced
by C-ABI calls into ``lib/libdpa_fp8.so``; every output and workspace is a fresh tensor from
torch's caching allocator and every launch goes on torch's current stream, so the ops are
safe inside ``torch.cuda.graph`` capture. There is no CPU or PyTorch fallback.

Beyond the reference (no reference kernel exists for these; same FP8 recipe):
``quantize_fp8_tensor`` (any rank), ``conv2d_fp8_*_general`` (stride 2 and 1x1),
``linear_fp8`` / ``LinearFP8Function`` and ``DW_SPLIT_K`` defaults tuned for 256 CUs.
"""
from __future__ import annotations

from typing import Any, cast

import torch
from torch.amp.autocast_mode import custom_bwd, custom_fwd

from . import _lib

# diffusion/fp8_kernels.py:11-12
FP8_DTYPE = torch.float8_e4m3fn
FP8_MAX_E4M3 = torch.finfo(torch.float8_e4m3fn).max

# (input channels, output channels, input height, input width); diffusion/fp8_kernels.py:17-27
SUPPORTED_UNET_SHAPES = (
    (128, 128, 32, 32),
    (128, 256, 32, 32),
    (256, 256, 16, 16),
    (512, 256, 16, 16),
    (256, 256, 8, 8),
    (512, 256, 8, 8),
    (512, 128, 32, 32),
    (256, 256, 32, 32),
    (256, 256, 4, 4),
)

# Split-K for the weight gradient per registry shape. The reference's table
# (diffusion/fp8_kernels.py:129-139) was tuned for 46 SMs; None lets the library choose one
# round of workgroups over the MI355X's 256 CUs. The KeyError for unknown shapes is kept.
DW_CONFIG_BY_SHAPE: dict[tuple[int, int, int, int], int | None] = {
    shape: None for shape in SUPPORTED_UNET_SHAPES
}


def _stream(t: torch.Tensor) -> int:
    return _lib.current_stream(t)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# --------------------------------------------------------------------------------------
# checks (diffusion/fp8_kernels.py:471-515, :667-668)
# --------------------------------------------------------------------------------------
def torch_checks_conv(a: torch.Tensor, b: torch.Tensor, dtype: torch.dtype) -> None:
    assert a.ndim == b.ndim == 4
    assert a.is_cuda and b.is_cuda and a.device == b.device
    assert a.is_contiguous() or a.is_contiguous(memory_format=torch.channels_last)
    assert b.is_contiguous() or b.is_contiguous(memory_format=torch.channels_last)


def fwd_shapes(x: torch.Tensor, weight: torch.Tensor, dtype: torch.dtype) -> tuple[int, int, int, int, int]:
    torch_checks_conv(x, weight, dtype)
    batch, cin, height, width = x.shape
    cout, weight_cin, kh, kw = weight.shape
    assert (weight_cin, kh, kw) == (cin, 3, 3)
    assert (cin, cout, height, width) in SUPPORTED_UNET_SHAPES, f"{(cin, cout, height, width)=}"
    return batch, cin, cout, height, width


def xgrad_shapes(dy: torch.Tensor, weight: torch.Tensor, dtype: torch.dtype) -> tuple[int, int, int, int, int]:
    torch_checks_conv(dy, weight, dtype)
    batch, cout, height, width = dy.shape
    weight_cout, cin, kh, kw = weight.shape
    assert (weight_cout, kh, kw) == (cout, 3, 3)
    assert (cin, cout, height, width) in SUPPORTED_UNET_SHAPES
    return batch, cin, cout, height, width


def wgrad_shapes(x: torch.Tensor, dy: torch.Tensor, dtype: torch.dtype) -> tuple[int, int, int, int, int]:
    torch_checks_conv(x, dy, dtype)
    batch, cin, height, width = x.shape
    dy_batch, cout, dy_height, dy_width = dy.shape
    assert (dy_batch, dy_height, dy_width) == (batch, height, width)
    assert (cin, cout, height, width) in SUPPORTED_UNET_SHAPES
    return batch, cin, cout, height, width


def torch_checks_scale(scale: torch.Tensor, device: torch.device) -> None:
    assert scale.device == device and scale.dtype == torch.float32 and scale.numel() == 1


def _nhwc(t: torch.Tensor) -> torch.Tensor:
    """Channels-last dense view of a 4-D tensor (copies only if the layout differs).

    The reference kernels index C with unit stride without checking it, so a contiguous
    (NCHW) FP8 operand silently produced garbage there; here it is converted instead."""
    if t.is_contiguous(memory_format=torch.channels_last):
        return t
    return t.contiguous(memory_format=torch.channels_last)


# --------------------------------------------------------------------------------------
# quantization (diffusion/fp8_kernels.py:518-601)
# --------------------------------------------------------------------------------------
def _workspace(nbytes: int, device: torch.device) -> torch.Tensor | None:
    """Device scratch of ``nbytes`` (None for 0), 16-B aligned as the caching allocator's are."""
    return torch.empty(nbytes, device=device, dtype=torch.uint8) if nbytes > 0 else None


def _dense(t: torch.Tensor) -> bool:
    return t.is_contiguous() or (t.ndim == 4 and t.is_contiguous(memory_format=torch.channels_last))


def _quantize_impl(tensor: torch.Tensor, prev_scale: torch.Tensor | None) -> tuple[torch.Tensor, torch.Tensor]:
    if not _dense(tensor):
        tensor = tensor.contiguous()
    n = tensor.numel()
    quantized = torch.empty_like(tensor, dtype=FP8_DTYPE, memory_format=torch.preserve_format)
    scale = torch.empty((), device=tensor.device, dtype=torch.float32)
    ws_bytes = _lib.query("dpa_quant_workspace_bytes", n)
    workspace = torch.empty(ws_bytes, device=tensor.device, dtype=torch.uint8)
    if prev_scale is None:
        _lib.call(
            "dpa_quantize_fp8_bf16",
            tensor.data_ptr(), n, quantized.data_ptr(), scale.data_ptr(),
            workspace.data_ptr(), ws_bytes, _stream(tensor),
        )
    else:
        torch_checks_scale(prev_scale, tensor.device)
        _lib.call(
            "dpa_quantize_fp8_delayed_bf16",
            tensor.data_ptr(), n, prev_scale.data_ptr(), quantized.data_ptr(), scale.data_ptr(),
            workspace.data_ptr(), ws_bytes, _stream(tensor),
        )
    return quantized, scale


def quantize_fp8_delayed_window(tensor: torch.Tensor, prev_scale: torch.Tensor,
                                window: torch.Tensor, window_pos: torch.Tensor,
                                advance: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """``quantize_fp8_delayed`` plus the module's amax-window update in the same launches:
    ``window[window_pos] = cur_scale`` and, if ``advance``, ``window_pos = (window_pos + 1) %
    len(window)`` (diffusion/unet.py:82-91, fp8_kernels.py:888-889)."""
    assert tensor.dtype == torch.bfloat16 and tensor.is_cuda, f"{tensor.dtype} {tensor.is_cuda}"
    torch_checks_scale(prev_scale, tensor.device)
    assert window.dtype == torch.float32 and window.is_cuda and window.is_contiguous()
    assert window_pos.dtype == torch.long and window_pos.is_cuda and window_pos.numel() == 1
    if not _dense(tensor):
        tensor = tensor.contiguous()
    n = tensor.numel()
    quantized = torch.empty_like(tensor, dtype=FP8_DTYPE, memory_format=torch.preserve_format)
    scale = torch.empty((), device=tensor.device, dtype=torch.float32)
    ws_bytes = _lib.query("dpa_quant_workspace_bytes", n)
    workspace = torch.empty(ws_bytes, device=tensor.device, dtype=torch.uint8)
    _lib.call(
        "dpa_quantize_fp8_delayed_window_bf16",
        tensor.data_ptr(), n, prev_scale.data_ptr(), quantized.data_ptr(), scale.data_ptr(),
        window.data_ptr(), window_pos.data_ptr(), window.numel(), 1 if advance else 0,
        workspace.data_ptr(), ws_bytes, _stream(tensor),
    )
    return quantized, scale


# Producer-side amax for current scaling: a kernel that writes a bf16 tensor the FP8 GEMM
# quantizes next (the attention LayerNorm, the self-attention forward and backward) can leave
# its per-workgroup maxima of |t| beside it; the GEMM then runs only the cast
# (dpa_quantize_fp8_bf16_from_partials) instead of the amax pass and the cast
# (diffusion/fp8_kernels.py:559-601). Same bytes and scale: the maxima are of the very bf16
# values written. False sends every site through quantize_fp8_tensor.
PRODUCER_AMAX = True


def mark_amax_partials(t: torch.Tensor, partials: torch.Tensor, count: int) -> torch.Tensor:
    """Record on t (bf16, dense -- contiguous or channels-last -- and just written) the int32
    buffer holding ``count`` per-workgroup maxima of |t| (bf16 magnitude bits) that its
    producer left."""
    t._dpa_amax = (partials, int(count), t.data_ptr(), t._version, t.numel())
    return t


def quantize_fp8_from_producer(x2: torch.Tensor, src: torch.Tensor):
    """``quantize_fp8_tensor(x2)`` from the maxima recorded on ``src`` when x2 is src's data
    unchanged (same address, element count and version), else None."""
    rec = getattr(src, "_dpa_amax", None)
    if rec is None and src._base is not None:   # a view autograd made of the recorded tensor
        rec = getattr(src._base, "_dpa_amax", None)
    if rec is None or not PRODUCER_AMAX:
        return None
    partials, count, ptr, version, numel = rec
    if (x2.dtype != torch.bfloat16 or not _dense(x2) or x2.data_ptr() != ptr
            or x2._version != version or x2.numel() != numel):
        return None
    q = torch.empty_like(x2, dtype=FP8_DTYPE, memory_format=torch.preserve_format)
    scale = torch.empty((), device=x2.device, dtype=torch.float32)
    _lib.call("dpa_quantize_fp8_bf16_from_partials", x2.data_ptr(), x2.numel(),
              partials.data_ptr(), count, q.data_ptr(), scale.data_ptr(), _stream(x2))
    return q, scale


def quantize_fp8_delayed_deferred(tensor: torch.Tensor, prev_scale: torch.Tensor,
                                  partials: torch.Tensor, count: torch.Tensor) -> torch.Tensor:
    """``quantize_fp8_delayed``'s cast (scale ``prev_scale``) leaving the block maxima of this
    tensor and their count in persistent buffers for a later ``dpa_delayed_windows_finalize``
    (the window record of the step, written at the start of the next one)."""
    assert tensor.dtype == torch.bfloat16 and tensor.is_cuda
    if not _dense(tensor):
        tensor = tensor.contiguous()
    quantized = torch.empty_like(tensor, dtype=FP8_DTYPE, memory_format=torch.preserve_format)
    _lib.call(
        "dpa_quantize_fp8_delayed_deferred_bf16",
        tensor.data_ptr(), tensor.numel(), prev_scale.data_ptr(), quantized.data_ptr(),
        partials.data_ptr(), partials.numel(), count.data_ptr(), _stream(tensor),
    )
    return quantized


_ZEROS: dict[tuple, torch.Tensor] = {}


def placeholder(shape, dtype: torch.dtype, device) -> torch.Tensor:
    """A tensor of the given shape that holds no data (one shared zero element, all strides
    0): what autograd carries where a producer handed the e4m3 operand to its FP8 conv
    directly. No launch after the first per device and dtype."""
    key = (torch.device(device), dtype)
    z = _ZEROS.get(key)
    if z is None:
        z = _ZEROS[key] = torch.zeros((), dtype=dtype, device=device)
    return z.expand(shape)


def is_placeholder(t: torch.Tensor) -> bool:
    return t.numel() > 1 and all(s == 0 for s in t.stride())


class Fp8Handoff:
    """The e4m3 operand of a delayed-scaling FP8 conv written by the kernel that produces it
    (diffusion/unet.py:151, :157-161 feeding diffusion/fp8_kernels.py:856, :885-893): cast
    with the conv's window scale, its block maxima left in the conv's deferred-window buffers,
    which is what ``quantize_fp8_delayed_deferred`` does in a pass of its own.

    For a gradient the producer's backward sets ``q`` and gives autograd a ``placeholder`` for
    the bf16 gradient; the conv's backward ``take``s ``q``. The placeholder reaches the conv
    unchanged only when the conv's output has no other consumer, which ``take`` checks."""

    __slots__ = ("scale", "partials", "count", "q")

    def __init__(self, scale: torch.Tensor, partials: torch.Tensor, count: torch.Tensor):
        self.scale, self.partials, self.count = scale, partials, count
        self.q: torch.Tensor | None = None

    def fill_from_bf16(self, t: torch.Tensor) -> None:
        """The unfused form: cast a bf16 tensor the producer had to write."""
        t = t.to(torch.bfloat16).contiguous(memory_format=torch.channels_last)
        self.q = quantize_fp8_delayed_deferred(t, self.scale, self.partials, self.count)

    def take(self, grad: torch.Tensor) -> torch.Tensor:
        if self.q is None or not is_placeholder(grad):
            raise RuntimeError("FP8 hand-off: the conv's output gradient did not come from its "
                               "producer alone (another consumer or no fused producer backward)")
        q, self.q = self.q, None
        return q


def window_max3(w0: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor) -> torch.Tensor:
    """``torch.stack([w0.max(), w1.max(), w2.max()])`` for three equal-length fp32 windows in
    one launch (diffusion/unet.py:72-73, fp8_kernels.py:849)."""
    for w in (w0, w1, w2):
        assert w.dtype == torch.float32 and w.is_cuda and w.is_contiguous() and w.numel() == w0.numel()
    out = torch.empty(3, device=w0.device, dtype=torch.float32)
    _lib.call("dpa_window_max3_f32", w0.data_ptr(), w1.data_ptr(), w2.data_ptr(), w0.numel(),
              out.data_ptr(), _stream(w0))
    return out


def quantize_fp8_delayed(tensor: torch.Tensor, prev_scale: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Tensorwise quantization from bfloat16 to fp8 with delay: cast with ``prev_scale`` and
    return the scale of the current amax (diffusion/fp8_kernels.py:518-556)."""
    assert tensor.dtype == torch.bfloat16 and tensor.is_cuda and tensor.ndim == 4, (
        f"{tensor.dtype} {tensor.is_cuda} {tensor.ndim}"
    )
    torch_checks_scale(prev_scale, tensor.device)
    return _ops.quantize_delayed(tensor, prev_scale)


def quantize_fp8(tensor: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Current-scaling quantization (diffusion/fp8_kernels.py:559-601)."""
    assert tensor.dtype == torch.bfloat16 and tensor.is_cuda and tensor.ndim == 4, (
        f"{tensor.dtype} {tensor.is_cuda} {tensor.ndim}"
    )
    return _ops.quantize(tensor)


def quantize_fp8_tensor(tensor: torch.Tensor, prev_scale: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """``quantize_fp8`` / ``quantize_fp8_delayed`` for a bf16 tensor of any rank."""
    assert tensor.dtype == torch.bfloat16 and tensor.is_cuda, f"{tensor.dtype} {tensor.is_cuda}"
    if prev_scale is None:
        return _ops.quantize(tensor)
    torch_checks_scale(prev_scale, tensor.device)
    return _ops.quantize_delayed(tensor, prev_scale)


# --------------------------------------------------------------------------------------
# convolution (diffusion/fp8_kernels.py:604-819), general form first
# --------------------------------------------------------------------------------------
def _out_hw(h: int, w: int, k: int, stride: int, pad: int) -> tuple[int, int]:
    return (h + 2 * pad - k) // stride + 1, (w + 2 * pad - k) // stride + 1


def conv2d_fp8_fwd_general(
    x: torch.Tensor,
    weight: torch.Tensor,
    x_scale: torch.Tensor,
    weight_scale: torch.Tensor,
    stride: int = 1,
    padding: int = 1,
    bias: torch.Tensor | None = None,
    split: bool = True,
) -> torch.Tensor:
    """FP8 conv forward for 3x3 (pad 1, stride 1|2) and 1x1 (pad 0, stride 1); NCHW-logical,
    channels-last bf16 output. ``bias`` (fp32 [Cout]) is added after dequantization.
    ``split`` lets the library split the reduction of launches too small to fill the GPU
    (fp32 partial sums in a workspace); False runs the single-pass kernel only."""
    assert x.dtype == FP8_DTYPE and weight.dtype == FP8_DTYPE
    torch_checks_scale(x_scale, x.device)
    torch_checks_scale(weight_scale, x.device)
    x = _nhwc(x)
    weight = _nhwc(weight)
    batch, cin, height, width = x.shape
    cout, wcin, kh, kw = weight.shape
    assert wcin == cin and kh == kw
    oh, ow = _out_hw(height, width, kh, stride, padding)
    y = torch.empty((batch, cout, oh, ow), device=x.device, dtype=torch.bfloat16,
                    memory_format=torch.channels_last)
    if bias is not None:
        assert bias.dtype == torch.float32 and bias.numel() == cout and bias.is_contiguous()
    geom = (batch, height, width, cin, cout, kh, kw, stride, padding)
    if split:
        ws_bytes = _lib.query("dpa_conv2d_fwd_split_workspace_bytes", *geom)
        workspace = _workspace(ws_bytes, x.device)
        _lib.call(
            "dpa_conv2d_fwd_fp8_split",
            x.data_ptr(), weight.data_ptr(), x_scale.data_ptr(), weight_scale.data_ptr(),
            _ptr(bias), y.data_ptr(), _ptr(workspace), ws_bytes, *geom, _stream(x),
        )
        return y
    _lib.call(
        "dpa_conv2d_fwd_fp8",
        x.data_ptr(), weight.data_ptr(), x_scale.data_ptr(), weight_scale.data_ptr(),
        _ptr(bias), y.data_ptr(), *geom, _stream(x),
    )
    return y


def conv2d_fp8_dgrad_general(
    dy: torch.Tensor,
    weight: torch.Tensor,
    dy_scale: torch.Tensor,
    weight_scale: torch.Tensor,
    input_hw: tuple[int, int],
    stride: int = 1,
    padding: int = 1,
    weight_t: torch.Tensor | None = None,
    split: bool = True,
) -> torch.Tensor:
    """FP8 data gradient; ``input_hw`` is the forward input's (H, W). ``weight_t`` may carry
    the weight already transposed to [Cin][R][S][Cout] bytes. ``split`` as in
    conv2d_fp8_fwd_general (False: the single-pass kernel only)."""
    assert dy.dtype == FP8_DTYPE and weight.dtype == FP8_DTYPE
    torch_checks_scale(dy_scale, dy.device)
    torch_checks_scale(weight_scale, dy.device)
    dy = _nhwc(dy)
    weight = _nhwc(weight)
    batch, cout, _, _ = dy.shape
    wcout, cin, kh, kw = weight.shape
    assert wcout == cout and kh == kw
    height, width = input_hw
    dx = torch.empty((batch, cin, height, width), device=dy.device, dtype=torch.bfloat16,
                     memory_format=torch.channels_last)
    geom = (batch, height, width, cin, cout, kh, kw, stride, padding)
    if split:
        if weight_t is None:
            weight_t = weight_transpose_fp8(weight)
        assert weight_t.numel() == weight.numel() and weight_t.is_contiguous()
        ws_bytes = _lib.query("dpa_conv2d_dgrad_split_workspace_bytes", *geom)
        workspace = _workspace(ws_bytes, dy.device)
        _lib.call(
            "dpa_conv2d_dgrad_fp8_wt_split",
            dy.data_ptr(), weight_t.data_ptr(), dy_scale.data_ptr(), weight_scale.data_ptr(),
            dx.data_ptr(), _ptr(workspace), ws_bytes, *geom, _stream(dy),
        )
    elif weight_t is None:
        ws_bytes = _lib.query("dpa_conv2d_dgrad_workspace_bytes", cin, cout, kh, kw)
        workspace = torch.empty(ws_bytes, device=dy.device, dtype=torch.uint8)
        _lib.call(
            "dpa_conv2d_dgrad_fp8",
            dy.data_ptr(), weight.data_ptr(), dy_scale.data_ptr(), weight_scale.data_ptr(),
            dx.data_ptr(), workspace.data_ptr(), ws_bytes, batch, height, width, cin, cout,
            kh, kw, stride, padding, _stream(dy),
        )
    else:
        assert weight_t.numel() == weight.numel() and weight_t.is_contiguous()
        _lib.call(
            "dpa_conv2d_dgrad_fp8_wt",
            dy.data_ptr(), weight_t.data_ptr(), dy_scale.data_ptr(), weight_scale.data_ptr(),
            dx.data_ptr(), batch, height, width, cin, cout, kh, kw, stride, padding, _stream(dy),
        )
    return dx


def hconv_shape(batch: int, cin: int, cout: int, height: int, width: int, k: int = 3,
                stride: int = 1, padding: int = 1) -> bool:
    """Shapes of the halo-patch conv kernel (3x3, stride 1, pad 1, images 16 or 32 pixels
    wide with whole 256-pixel row groups, channels multiples of 128): the only shapes the
    fragment-layout weight entries (dpa_conv2d_*_fp8_wf) accept."""
    return (k == 3 and stride == 1 and padding == 1 and width in (16, 32)
            and height % (256 // width) == 0 and cin % 128 == 0 and cout % 128 == 0
            and batch * height * width * max(cin, cout) < 2**31)


def weight_frag_fp8(weight: torch.Tensor, forward: bool = True, dgrad: bool = True):
    """The fragment-native layouts of an OHWI e4m3 weight for the halo-patch conv: (forward,
    data gradient), flat uint8 tensors (either None when not asked for)."""
    assert weight.dtype == FP8_DTYPE
    weight = _nhwc(weight)
    cout, cin, kh, kw = weight.shape
    n = weight.numel()
    wf = torch.empty(n, device=weight.device, dtype=torch.uint8) if forward else None
    wt = torch.empty(n, device=weight.device, dtype=torch.uint8) if dgrad else None
    _lib.call("dpa_weight_frag_fp8", weight.data_ptr(), _ptr(wf), _ptr(wt), cout, kh, kw, cin,
              _stream(weight))
    return wf, wt


def conv2d_fp8_fwd_wf(x: torch.Tensor, wf: torch.Tensor, x_scale: torch.Tensor,
                      weight_scale: torch.Tensor, cout: int,
                      bias: torch.Tensor | None = None) -> torch.Tensor:
    """The 3x3 / stride-1 / pad-1 forward with the weight in its fragment layout
    (weight_frag_fp8): the same values as conv2d_fp8_fwd_general."""
    assert x.dtype == FP8_DTYPE and wf.dtype == torch.uint8 and wf.is_contiguous()
    x = _nhwc(x)
    batch, cin, height, width = x.shape
    assert wf.numel() == cout * 9 * cin and hconv_shape(batch, cin, cout, height, width)
    y = torch.empty((batch, cout, height, width), device=x.device, dtype=torch.bfloat16,
                    memory_format=torch.channels_last)
    _lib.call("dpa_conv2d_fwd_fp8_wf", x.data_ptr(), wf.data_ptr(), x_scale.data_ptr(),
              weight_scale.data_ptr(), _ptr(bias), y.data_ptr(), batch, height, width, cin, cout,
              _stream(x))
    return y


def conv2d_fp8_dgrad_wf(dy: torch.Tensor, wf_dgrad: torch.Tensor, dy_scale: torch.Tensor,
                        weight_scale: torch.Tensor, cin: int) -> torch.Tensor:
    """The 3x3 / stride-1 / pad-1 data gradient with the weight in its data-gradient fragment
    layout (weight_frag_fp8): the same values as conv2d_fp8_dgrad_general."""
    assert dy.dtype == FP8_DTYPE and wf_dgrad.dtype == torch.uint8 and wf_dgrad.is_contiguous()
    dy = _nhwc(dy)
    batch, cout, height, width = dy.shape
    assert wf_dgrad.numel() == cout * 9 * cin and hconv_shape(batch, cin, cout, height, width)
    dx = torch.empty((batch, cin, height, width), device=dy.device, dtype=torch.bfloat16,
                     memory_format=torch.channels_last)
    _lib.call("dpa_conv2d_dgrad_fp8_wf", dy.data_ptr(), wf_dgrad.data_ptr(), dy_scale.data_ptr(),
              weight_scale.data_ptr(), dx.data_ptr(), batch, height, width, cin, cout, _stream(dy))
    return dx


def weight_transpose_fp8(weight: torch.Tensor) -> torch.Tensor:
    """[Cout][R][S][Cin] e4m3 bytes -> [Cin][R][S][Cout] (the data-gradient operand)."""
    assert weight.dtype == FP8_DTYPE
    weight = _nhwc(weight)
    cout, cin, kh, kw = weight.shape
    out = torch.empty((cin, kh, kw, cout), device=weight.device, dtype=FP8_DTYPE)
    _lib.call("dpa_weight_transpose_fp8", weight.data_ptr(), out.data_ptr(), cout, kh, kw, cin,
              _stream(weight))
    return out


def conv2d_fp8_wgrad_general(
    x: torch.Tensor,
    dy: torch.Tensor,
    x_scale: torch.Tensor,
    dy_scale: torch.Tensor,
    kernel_size: int = 3,
    stride: int = 1,
    padding: int = 1,
    split_k: int | None = None,
    out_f32: bool = False,
) -> torch.Tensor:
    """FP8 weight gradient -> bf16 (Cout, Cin, k, k) in channels-last memory; ``out_f32``
    gives the same values as fp32 (the gradient of a channels-last fp32 master weight)."""
    assert x.dtype == FP8_DTYPE and dy.dtype == FP8_DTYPE
    torch_checks_scale(x_scale, x.device)
    torch_checks_scale(dy_scale, x.device)
    x = _nhwc(x)
    dy = _nhwc(dy)
    batch, cin, height, width = x.shape
    _, cout, _, _ = dy.shape
    sk = 0 if split_k is None else int(split_k)
    ws_bytes = _lib.query("dpa_conv2d_wgrad_workspace_bytes", batch, height, width, cin, cout,
                          kernel_size, kernel_size, stride, padding, sk)
    if ws_bytes <= 0:
        raise RuntimeError(f"dpa_conv2d_wgrad_fp8: unsupported shape {(batch, cin, cout, height, width, kernel_size, stride)}")
    workspace = torch.empty(ws_bytes, device=x.device, dtype=torch.uint8)
    dw = torch.empty((cout, cin, kernel_size, kernel_size), device=x.device,
                     dtype=torch.float32 if out_f32 else torch.bfloat16,
                     memory_format=torch.channels_last)
    _lib.call(
        "dpa_conv2d_wgrad_fp8_f32" if out_f32 else "dpa_conv2d_wgrad_fp8",
        x.data_ptr(), dy.data_ptr(), x_scale.data_ptr(), dy_scale.data_ptr(), dw.data_ptr(),
        workspace.data_ptr(), ws_bytes, batch, height, width, cin, cout, kernel_size,
        kernel_size, stride, padding, sk, _stream(x),
    )
    return dw


# ---- reference-named entry points (3x3, stride 1, pad 1, registry shapes) ----
def conv2d_fwd_fp8_prequantized(
    x: torch.Tensor,
    weight: torch.Tensor,
    x_scale: torch.Tensor,
    weight_scale: torch.Tensor,
) -> torch.Tensor:
    """diffusion/fp8_kernels.py:604-639."""
    fwd_shapes(x, weight, FP8_DTYPE)
    torch_checks_scale(x_scale, x.device)
    torch_checks_scale(weight_scale, x.device)
    return _ops.conv_fwd(x, weight, x_scale, weight_scale, 1, 1)


def conv2d_fwd_fp8(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """diffusion/fp8_kernels.py:642-650."""
    x_fp8, x_scale = quantize_fp8(x)
    weight_fp8, weight_scale = quantize_fp8(weight)
    return conv2d_fwd_fp8_prequantized(x_fp8, weight_fp8, x_scale, weight_scale)


def conv2d_fwd_fp8_delayed(x: torch.Tensor, weight: torch.Tensor, x_scale: torch.Tensor, w_scale: torch.Tensor):
    """diffusion/fp8_kernels.py:653-664."""
    x_fp8, _ = quantize_fp8_delayed(x, x_scale)
    weight_fp8, _ = quantize_fp8_delayed(weight, w_scale)
    return conv2d_fwd_fp8_prequantized(x_fp8, weight_fp8, x_scale, w_scale)


def conv2d_bwd_input_fp8_prequantized(
    dy: torch.Tensor,
    weight: torch.Tensor,
    dy_scale: torch.Tensor,
    weight_scale: torch.Tensor,
) -> torch.Tensor:
    """diffusion/fp8_kernels.py:671-709."""
    batch, cin, cout, height, width = xgrad_shapes(dy, weight, FP8_DTYPE)
    torch_checks_scale(dy_scale, dy.device)
    torch_checks_scale(weight_scale, dy.device)
    return _ops.conv_dgrad(dy, weight, dy_scale, weight_scale, height, width, 1, 1)


def conv2d_bwd_input_fp8(dy: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """diffusion/fp8_kernels.py:712-720."""
    dy_fp8, dy_scale = quantize_fp8(dy)
    weight_fp8, weight_scale = quantize_fp8(weight)
    return conv2d_bwd_input_fp8_prequantized(dy_fp8, weight_fp8, dy_scale, weight_scale)


def conv2d_bwd_weight_fp8_prequantized(
    x: torch.Tensor,
    dy: torch.Tensor,
    x_scale: torch.Tensor,
    dy_scale: torch.Tensor,
    split_k: int | None = None,
    out_f32: bool = False,
) -> torch.Tensor:
    """diffusion/fp8_kernels.py:723-808. Returns bf16 (Cout, Cin, 3, 3), channels-last
    (``out_f32``: the same values in fp32)."""
    batch, cin, cout, height, width = wgrad_shapes(x, dy, FP8_DTYPE)
    torch_checks_scale(x_scale, x.device)
    torch_checks_scale(dy_scale, x.device)
    if split_k is None:
        split_k = DW_CONFIG_BY_SHAPE[(cin, cout, height, width)]
    if not (x.is_contiguous(memory_format=torch.channels_last)
            and dy.is_contiguous(memory_format=torch.channels_last)):
        raise NotImplementedError
    return _ops.conv_wgrad(x, dy, x_scale, dy_scale, 3, 1, 1, split_k or 0, out_f32)


def conv2d_bwd_weight_fp8(x: torch.Tensor, dy: torch.Tensor) -> torch.Tensor:
    """diffusion/fp8_kernels.py:811-819."""
    x_fp8, x_scale = quantize_fp8(x)
    dy_fp8, dy_scale = quantize_fp8(dy)
    return conv2d_bwd_weight_fp8_prequantized(x_fp8, dy_fp8, x_scale, dy_scale)


# --------------------------------------------------------------------------------------
# autograd boundary (diffusion/fp8_kernels.py:822-923)
# --------------------------------------------------------------------------------------
class Conv2dFP8Specialized(torch.autograd.Function):
    """FP8 3x3/stride-1/pad-1 conv with e4m3 saved activations; current or delayed scaling.

    Same inputs, saved tensors, outputs and in-place window update as the reference
    (diffusion/fp8_kernels.py:823-913)."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(
        ctx: Any,
        x: torch.Tensor,
        weight: torch.Tensor,
        hist_scales: tuple[torch.Tensor, torch.Tensor] | None = None,
        dy_ptrs: tuple[torch.Tensor, torch.Tensor] | None = None,
        do_delayed: bool = False,
    ) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        x = x.to(torch.bfloat16)
        # the reference relies on the model having been converted to channels-last; a
        # contiguous (OIHW) parameter is converted here instead of producing wrong results
        weight = weight.to(torch.bfloat16).contiguous(memory_format=torch.channels_last)

        assert x.is_contiguous(memory_format=torch.channels_last)

        ctx.do_delayed = do_delayed
        if do_delayed:
            assert hist_scales is not None
            assert dy_ptrs is not None
            x_scale, weight_scale = hist_scales
            x_fp8, x_scale_curr = quantize_fp8_delayed(x, x_scale)
            weight_fp8, weight_scale_curr = quantize_fp8_delayed(weight, weight_scale)

            dy_amax_window, window_pos = dy_ptrs
            dy_scale_hist = torch.max(dy_amax_window)

            ctx.dy_window = dy_amax_window
            ctx.window_pos = window_pos
            ctx.save_for_backward(x_fp8, weight_fp8, x_scale, weight_scale, dy_scale_hist)
        else:
            x_fp8, x_scale = quantize_fp8(x)
            weight_fp8, weight_scale = quantize_fp8(weight)
            ctx.save_for_backward(x_fp8, weight_fp8, x_scale, weight_scale)

        out = conv2d_fwd_fp8_prequantized(x_fp8, weight_fp8, x_scale, weight_scale)

        if do_delayed:
            ctx.mark_non_differentiable(x_scale_curr, weight_scale_curr)
            return out, x_scale_curr, weight_scale_curr
        return out

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx: Any, *grad_outputs: Any) -> Any:
        dy = cast(torch.Tensor, grad_outputs[0])
        dy = dy.contiguous(memory_format=torch.channels_last)
        if dy.dtype != torch.bfloat16:
            dy = dy.to(torch.bfloat16)

        if ctx.do_delayed:
            x_fp8, weight_fp8, x_scale, weight_scale, dy_scale = ctx.saved_tensors
            dy_fp8, dy_scale_curr = quantize_fp8_delayed(dy, dy_scale)
            window_idx = ctx.window_pos.unsqueeze(0)
            ctx.dy_window.scatter_(0, window_idx, dy_scale_curr.unsqueeze(0))
        else:
            x_fp8, weight_fp8, x_scale, weight_scale = ctx.saved_tensors
            dy_fp8, dy_scale = quantize_fp8(dy)

        assert dy_fp8.is_contiguous(memory_format=torch.channels_last)
        assert weight_fp8.is_contiguous(memory_format=torch.channels_last)
        assert x_fp8.is_contiguous(memory_format=torch.channels_last)

        dx = conv2d_bwd_input_fp8_prequantized(dy_fp8, weight_fp8, dy_scale, weight_scale)
        dw = conv2d_bwd_weight_fp8_prequantized(x_fp8, dy_fp8, x_scale, dy_scale)
        return dx, dw, None, None, None


class Conv2dFP8DelayedWindowed(torch.autograd.Function):
    """Delayed-scaling FP8 3x3 conv with the module's amax-window bookkeeping inside: the same
    arithmetic, saved tensors and window/position updates as ``Conv2dFP8.forward`` on top of
    ``Conv2dFP8Specialized`` (diffusion/unet.py:69-91, fp8_kernels.py:845-889), with the three
    window maxima in one launch and each window write riding on its quantization's finalize
    launch instead of separate torch reductions, scatters and position arithmetic."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx: Any, x: torch.Tensor, weight: torch.Tensor, win_acts: torch.Tensor,
                win_weights: torch.Tensor, win_dy: torch.Tensor,
                window_pos: torch.Tensor) -> torch.Tensor:
        x = x.to(torch.bfloat16)
        weight = weight.to(torch.bfloat16).contiguous(memory_format=torch.channels_last)
        assert x.is_contiguous(memory_format=torch.channels_last)
        hist = window_max3(win_acts, win_weights, win_dy)   # before this step's writes
        x_scale, weight_scale, dy_scale = hist[0], hist[1], hist[2]
        x_fp8, _ = quantize_fp8_delayed_window(x, x_scale, win_acts, window_pos, advance=False)
        weight_fp8, _ = quantize_fp8_delayed_window(weight, weight_scale, win_weights, window_pos,
                                                    advance=True)
        ctx.dy_window = win_dy
        ctx.window_pos = window_pos
        ctx.save_for_backward(x_fp8, weight_fp8, x_scale, weight_scale, dy_scale)
        return conv2d_fwd_fp8_prequantized(x_fp8, weight_fp8, x_scale, weight_scale)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx: Any, dy: torch.Tensor) -> Any:
        dy = dy.contiguous(memory_format=torch.channels_last)
        if dy.dtype != torch.bfloat16:
            dy = dy.to(torch.bfloat16)
        x_fp8, weight_fp8, x_scale, weight_scale, dy_scale = ctx.saved_tensors
        dy_fp8, _ = quantize_fp8_delayed_window(dy, dy_scale, ctx.dy_window, ctx.window_pos,
                                                advance=False)
        dx = conv2d_bwd_input_fp8_prequantized(dy_fp8, weight_fp8, dy_scale, weight_scale)
        dw = conv2d_bwd_weight_fp8_prequantized(x_fp8, dy_fp8, x_scale, dy_scale)
        return dx, dw, None, None, None, None


def triton_conv2d_fp8(
    x: torch.Tensor,
    weight: torch.Tensor,
    hist_scales: tuple[torch.Tensor, torch.Tensor] | None = None,
    dy_ptrs: tuple[torch.Tensor, torch.Tensor] | None = None,
    do_delayed: bool = False,
) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Reference-named entry point (diffusion/fp8_kernels.py:916-923); runs the HIP kernels."""
    return Conv2dFP8Specialized.apply(x, weight, hist_scales, dy_ptrs, do_delayed)


hip_conv2d_fp8 = triton_conv2d_fp8


# --------------------------------------------------------------------------------------
# generalised conv (stride 2, 1x1) and the FP8 linear: same recipe, no reference kernel
# --------------------------------------------------------------------------------------
class Conv2dFP8General(torch.autograd.Function):
    """Current-scaling FP8 conv for any supported (k, stride, pad); saves e4m3 x and w."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx: Any, x: torch.Tensor, weight: torch.Tensor, stride: int, padding: int) -> torch.Tensor:
        x = x.to(torch.bfloat16).contiguous(memory_format=torch.channels_last)
        weight = weight.to(torch.bfloat16).contiguous(memory_format=torch.channels_last)
        x_fp8, x_scale = quantize_fp8(x)
        w_fp8, w_scale = quantize_fp8(weight)
        ctx.save_for_backward(x_fp8, w_fp8, x_scale, w_scale)
        ctx.stride, ctx.padding = stride, padding
        ctx.input_hw = (x.shape[2], x.shape[3])
        return _ops.conv_fwd(x_fp8, w_fp8, x_scale, w_scale, stride, padding)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx: Any, dy: torch.Tensor) -> Any:
        x_fp8, w_fp8, x_scale, w_scale = ctx.saved_tensors
        dy = dy.to(torch.bfloat16).contiguous(memory_format=torch.channels_last)
        dy_fp8, dy_scale = quantize_fp8(dy)
        k = w_fp8.shape[2]
        dx = None
        if ctx.needs_input_grad[0]:
            dx = _ops.conv_dgrad(dy_fp8, w_fp8, dy_scale, w_scale, ctx.input_hw[0],
                                 ctx.input_hw[1], ctx.stride, ctx.padding)
        dw = _ops.conv_wgrad(x_fp8, dy_fp8, x_scale, dy_scale, k, ctx.stride, ctx.padding, 0,
                             False)
        return dx, dw, None, None


def conv2d_fp8(x: torch.Tensor, weight: torch.Tensor, stride: int = 1, padding: int = 1) -> torch.Tensor:
    return Conv2dFP8General.apply(x, weight, stride, padding)


def linear_fp8_prequantized(
    a: torch.Tensor,
    b: torch.Tensor,
    a_scale: torch.Tensor,
    b_scale: torch.Tensor,
    bias: torch.Tensor | None = None,
    split: bool = True,
) -> torch.Tensor:
    """c[M, N] = bf16(a[M, K] @ b[N, K]^T * a_scale * b_scale [+ bias]); e4m3 inputs.
    ``split`` as in conv2d_fp8_fwd_general."""
    assert a.dtype == FP8_DTYPE and b.dtype == FP8_DTYPE and a.is_cuda and b.is_cuda
    assert a.ndim == 2 and b.ndim == 2 and a.shape[1] == b.shape[1]
    torch_checks_scale(a_scale, a.device)
    torch_checks_scale(b_scale, a.device)
    a = a.contiguous()
    b = b.contiguous()
    m, k = a.shape
    n = b.shape[0]
    c = torch.empty((m, n), device=a.device, dtype=torch.bfloat16)
    if bias is not None:
        assert bias.dtype == torch.float32 and bias.numel() == n and bias.is_contiguous()
    if split:
        ws_bytes = _lib.query("dpa_gemm_split_workspace_bytes", m, n, k)
        workspace = _workspace(ws_bytes, a.device)
        _lib.call("dpa_gemm_fp8_split", a.data_ptr(), b.data_ptr(), a_scale.data_ptr(),
                  b_scale.data_ptr(), _ptr(bias), c.data_ptr(), _ptr(workspace), ws_bytes, m, n,
                  k, _stream(a))
        return c
    _lib.call("dpa_gemm_fp8", a.data_ptr(), b.data_ptr(), a_scale.data_ptr(), b_scale.data_ptr(),
              _ptr(bias), c.data_ptr(), m, n, k, _stream(a))
    return c


def linear_fp8(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """Forward-only FP8 linear with current scaling: bf16 x[..., K] and weight[N, K]."""
    lead = x.shape[:-1]
    x2 = x.to(torch.bfloat16).reshape(-1, x.shape[-1])
    xq, xs = quantize_fp8_tensor(x2)
    wq, wsc = quantize_fp8_tensor(weight.to(torch.bfloat16))
    y = linear_fp8_prequantized(xq, wq, xs, wsc, bias)
    return y.reshape(*lead, weight.shape[0])


def linear_fp8_dgrad_prequantized(
    dy: torch.Tensor,
    weight: torch.Tensor,
    dy_scale: torch.Tensor,
    weight_scale: torch.Tensor,
    split: bool = True,
) -> torch.Tensor:
    """dx[M, K] = bf16(dy[M, N] @ weight[N, K] * dy_scale * weight_scale); e4m3 inputs.

    Runs the 1x1 data-gradient kernel on M one-pixel images; ``split`` as in
    conv2d_fp8_fwd_general."""
    assert dy.dtype == FP8_DTYPE and weight.dtype == FP8_DTYPE and dy.ndim == weight.ndim == 2
    assert dy.shape[1] == weight.shape[0]
    torch_checks_scale(dy_scale, dy.device)
    torch_checks_scale(weight_scale, dy.device)
    dy = dy.contiguous()
    weight = weight.contiguous()
    m, n = dy.shape
    k = weight.shape[1]
    dx = torch.empty((m, k), device=dy.device, dtype=torch.bfloat16)
    if split:
        weight_t = torch.empty((k, n), device=dy.device, dtype=FP8_DTYPE)
        _lib.call("dpa_weight_transpose_fp8", weight.data_ptr(), weight_t.data_ptr(), n, 1, 1, k,
                  _stream(dy))
        geom = (m, 1, 1, k, n, 1, 1, 1, 0)
        ws_bytes = _lib.query("dpa_conv2d_dgrad_split_workspace_bytes", *geom)
        workspace = _workspace(ws_bytes, dy.device)
        _lib.call(
            "dpa_conv2d_dgrad_fp8_wt_split",
            dy.data_ptr(), weight_t.data_ptr(), dy_scale.data_ptr(), weight_scale.data_ptr(),
            dx.data_ptr(), _ptr(workspace), ws_bytes, *geom, _stream(dy),
        )
        return dx
    ws_bytes = _lib.query("dpa_conv2d_dgrad_workspace_bytes", k, n, 1, 1)
    workspace = torch.empty(ws_bytes, device=dy.device, dtype=torch.uint8)
    _lib.call(
        "dpa_conv2d_dgrad_fp8",
        dy.data_ptr(), weight.data_ptr(), dy_scale.data_ptr(), weight_scale.data_ptr(),
        dx.data_ptr(), workspace.data_ptr(), ws_bytes, m, 1, 1, k, n, 1, 1, 1, 0, _stream(dy),
    )
    return dx


def linear_fp8_wgrad_prequantized(
    x: torch.Tensor,
    dy: torch.Tensor,
    x_scale: torch.Tensor,
    dy_scale: torch.Tensor,
    out_f32: bool = False,
) -> torch.Tensor:
    """dw[N, K] = bf16(dy[M, N]^T @ x[M, K] * x_scale * dy_scale); e4m3 inputs (``out_f32``:
    the same values in fp32).

    Runs the 1x1 weight-gradient kernel on M one-pixel images."""
    assert x.dtype == FP8_DTYPE and dy.dtype == FP8_DTYPE and x.ndim == dy.ndim == 2
    assert x.shape[0] == dy.shape[0]
    torch_checks_scale(x_scale, x.device)
    torch_checks_scale(dy_scale, x.device)
    x = x.contiguous()
    dy = dy.contiguous()
    m, k = x.shape
    n = dy.shape[1]
    ws_bytes = _lib.query("dpa_conv2d_wgrad_workspace_bytes", m, 1, 1, k, n, 1, 1, 1, 0, 0)
    if ws_bytes <= 0:
        raise RuntimeError(f"dpa_conv2d_wgrad_fp8: unsupported linear shape {(m, k, n)}")
    workspace = torch.empty(ws_bytes, device=x.device, dtype=torch.uint8)
    dw = torch.empty((n, k), device=x.device, dtype=torch.float32 if out_f32 else torch.bfloat16)
    _lib.call(
        "dpa_conv2d_wgrad_fp8_f32" if out_f32 else "dpa_conv2d_wgrad_fp8",
        x.data_ptr(), dy.data_ptr(), x_scale.data_ptr(), dy_scale.data_ptr(), dw.data_ptr(),
        workspace.data_ptr(), ws_bytes, m, 1, 1, k, n, 1, 1, 1, 0, 0, _stream(x),
    )
    return dw


def linear_fp8_supported(in_features: int, out_features: int) -> bool:
    """Feature counts the FP8 GEMM and its gradients implement (multiples of 128)."""
    return in_features % 128 == 0 and out_features % 128 == 0 and in_features > 0


class LinearFP8Function(torch.autograd.Function):
    """y = x @ weight^T (+ bias) with current per-tensor e4m3 scaling of x, weight and dy.

    Same recipe as the conv (diffusion/fp8_kernels.py:822-913) applied to the U-Net's
    nn.Linear sites (diffusion/unet.py:101, :171-172, :189, :199): bf16 inputs, e4m3 saved
    operands, bf16 output and gradients (autograd casts them to the parameter dtype)."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx: Any, x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None):
        lead = x.shape[:-1]
        n, k = weight.shape
        assert x.shape[-1] == k
        x2 = x.to(torch.bfloat16).reshape(-1, k).contiguous()
        w = weight.to(torch.bfloat16).contiguous()
        xq, xs = quantize_fp8_tensor(x2)
        wq, wsc = quantize_fp8_tensor(w)
        b32 = None if bias is None else bias.detach().float().contiguous()
        y = _ops.gemm(xq, wq, xs, wsc, b32)
        ctx.save_for_backward(xq, wq, xs, wsc)
        ctx.lead = lead
        ctx.has_bias = bias is not None
        return y.reshape(*lead, n)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx: Any, dy: torch.Tensor):
        xq, wq, xs, wsc = ctx.saved_tensors
        n, k = wq.shape
        dy2 = dy.to(torch.bfloat16).reshape(-1, n).contiguous()
        dyq, dys = quantize_fp8_tensor(dy2)
        dx = dw = db = None
        if ctx.needs_input_grad[0]:
            dx = _ops.gemm_dgrad(dyq, wq, dys, wsc).reshape(*ctx.lead, k)
        if ctx.needs_input_grad[1]:
            dw = _ops.gemm_wgrad(xq, dyq, xs, dys, False)
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = dy2.float().sum(0)
        return dx, dw, db


# --------------------------------------------------------------------------------------
# layers whose weight was prepared for the step by weight_prep.WeightPrep (grouped launches):
# same arithmetic and window updates as the per-call Functions above; the weight arrives as
# e4m3 bytes, its transpose and the scale it was cast with, and the gradient of the fp32
# master weight is returned in fp32 directly
# --------------------------------------------------------------------------------------
class Conv2dFP8DelayedPrepared(torch.autograd.Function):
    """Conv2dFP8DelayedWindowed with the weight prepared: hist = the step's three window maxima
    (acts, weights, dy) taken before any of this step's window writes. The x and dy
    quantizations cast with hist[0] / hist[2] and leave their block maxima in the layer's
    persistent buffers (``parts`` = x partials, x count, dy partials, dy count); the weight
    preparation of the next step (or ``WeightPrep.flush``) writes their window records and
    advances the position, which gives the per-call path's window state.

    xq: the e4m3 input written by its producer (``Fp8Handoff``; x is then a placeholder);
    dy_handoff: an ``Fp8Handoff`` whose producer backward writes the e4m3 dy."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx: Any, x: torch.Tensor, weight: torch.Tensor, wq: torch.Tensor,
                wq_t: torch.Tensor, w_scale: torch.Tensor, hist: torch.Tensor,
                parts: tuple, xq: torch.Tensor | None = None,
                dy_handoff: Fp8Handoff | None = None) -> torch.Tensor:
        x_scale, dy_scale = hist[0], hist[2]
        if xq is not None:
            x_fp8 = xq
        else:
            x = x.to(torch.bfloat16)
            assert x.is_contiguous(memory_format=torch.channels_last)
            x_fp8 = quantize_fp8_delayed_deferred(x, x_scale, parts[0], parts[1])
        ctx.parts = parts
        ctx.dy_handoff = dy_handoff
        ctx.cin_cout = (weight.shape[1], weight.shape[0])
        ctx.save_for_backward(x_fp8, wq, wq_t, x_scale, w_scale, dy_scale)
        if wq.dtype == torch.uint8:      # fragment layouts of the halo-patch kernel
            fwd_shapes(x_fp8, weight, FP8_DTYPE)
            return conv2d_fp8_fwd_wf(x_fp8, wq, x_scale, w_scale, weight.shape[0])
        return conv2d_fwd_fp8_prequantized(x_fp8, wq, x_scale, w_scale)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx: Any, dy: torch.Tensor) -> Any:
        x_fp8, wq, wq_t, x_scale, w_scale, dy_scale = ctx.saved_tensors
        if ctx.dy_handoff is not None:
            dy_fp8 = ctx.dy_handoff.take(dy)
        else:
            dy = dy.contiguous(memory_format=torch.channels_last)
            if dy.dtype != torch.bfloat16:
                dy = dy.to(torch.bfloat16)
            dy_fp8 = quantize_fp8_delayed_deferred(dy, dy_scale, ctx.parts[2], ctx.parts[3])
        if wq.dtype == torch.uint8:
            dx = conv2d_fp8_dgrad_wf(dy_fp8, wq_t, dy_scale, w_scale, ctx.cin_cout[0])
        else:
            batch, cin, cout, height, width = xgrad_shapes(dy_fp8, wq, FP8_DTYPE)
            dx = conv2d_fp8_dgrad_general(dy_fp8, wq, dy_scale, w_scale, (height, width), 1, 1,
                                          weight_t=wq_t)
        dw = conv2d_bwd_weight_fp8_prequantized(x_fp8, dy_fp8, x_scale, dy_scale, out_f32=True)
        return dx, dw, None, None, None, None, None, None, None


class Conv2dFP8GeneralPrepared(torch.autograd.Function):
    """Conv2dFP8General (current scaling) with the weight prepared for the step."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx: Any, x: torch.Tensor, weight: torch.Tensor, wq: torch.Tensor,
                wq_t: torch.Tensor, w_scale: torch.Tensor, stride: int,
                padding: int) -> torch.Tensor:
        src = x
        x = x.to(torch.bfloat16).contiguous(memory_format=torch.channels_last)
        x_fp8, x_scale = quantize_fp8_from_producer(x, src) or quantize_fp8(x)
        ctx.save_for_backward(x_fp8, wq, wq_t, x_scale, w_scale)
        ctx.stride, ctx.padding = stride, padding
        ctx.input_hw = (x.shape[2], x.shape[3])
        ctx.k, ctx.cin = weight.shape[2], weight.shape[1]
        if wq.dtype == torch.uint8:      # fragment layouts of the halo-patch kernel
            assert stride == 1 and padding == 1 and ctx.k == 3
            return conv2d_fp8_fwd_wf(x_fp8, wq, x_scale, w_scale, weight.shape[0])
        return conv2d_fp8_fwd_general(x_fp8, wq, x_scale, w_scale, stride, padding)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx: Any, dy: torch.Tensor) -> Any:
        x_fp8, wq, wq_t, x_scale, w_scale = ctx.saved_tensors
        src = dy
        dy = dy.to(torch.bfloat16).contiguous(memory_format=torch.channels_last)
        dy_fp8, dy_scale = quantize_fp8_from_producer(dy, src) or quantize_fp8(dy)
        k = ctx.k
        dx = None
        if ctx.needs_input_grad[0]:
            if wq.dtype == torch.uint8:
                dx = conv2d_fp8_dgrad_wf(dy_fp8, wq_t, dy_scale, w_scale, ctx.cin)
            else:
                dx = conv2d_fp8_dgrad_general(dy_fp8, wq, dy_scale, w_scale, ctx.input_hw,
                                              ctx.stride, ctx.padding, weight_t=wq_t)
        dw = conv2d_fp8_wgrad_general(x_fp8, dy_fp8, x_scale, dy_scale, k, ctx.stride,
                                      ctx.padding, out_f32=True)
        return dx, dw, None, None, None, None, None


def _linear_dgrad_wt(dy: torch.Tensor, wq: torch.Tensor, wq_t: torch.Tensor, dy_scale, w_scale):
    """linear_fp8_dgrad_prequantized with the transposed weight [K][N] given."""
    m, n = dy.shape
    k = wq.shape[1]
    dx = torch.empty((m, k), device=dy.device, dtype=torch.bfloat16)
    geom = (m, 1, 1, k, n, 1, 1, 1, 0)
    ws_bytes = _lib.query("dpa_conv2d_dgrad_split_workspace_bytes", *geom)
    workspace = _workspace(ws_bytes, dy.device)
    _lib.call(
        "dpa_conv2d_dgrad_fp8_wt_split",
        dy.data_ptr(), wq_t.data_ptr(), dy_scale.data_ptr(), w_scale.data_ptr(), dx.data_ptr(),
        _ptr(workspace), ws_bytes, *geom, _stream(dy),
    )
    return dx


class LinearFP8Prepared(torch.autograd.Function):
    """LinearFP8Function with the weight prepared for the step. ``x_cache`` (a dict owned by the
    step's weight preparation, emptied at the start of every forward) shares the e4m3 copy of an
    input among the layers that read the same tensor in one forward (the 22 time-embedding
    projections all read t_emb): the same bytes and scale as quantizing it per layer."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx: Any, x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
                wq: torch.Tensor, wq_t: torch.Tensor, w_scale: torch.Tensor,
                x_cache: dict | None = None):
        lead = x.shape[:-1]
        n, k = weight.shape
        key = None
        if x_cache is not None:
            key = (x.data_ptr(), x._version, tuple(x.shape), tuple(x.stride()), x.dtype)
        hit = x_cache.get(key) if key is not None else None
        if hit is not None:
            xq, xs = hit[1], hit[2]
        else:
            x2 = x.to(torch.bfloat16).reshape(-1, k).contiguous()
            xq, xs = quantize_fp8_from_producer(x2, x) or quantize_fp8_tensor(x2)
            if key is not None:
                x_cache[key] = (x, xq, xs)      # x kept alive: its address is not reused
        b32 = None if bias is None else bias.detach().float().contiguous()
        y = linear_fp8_prequantized(xq, wq, xs, w_scale, b32)
        ctx.save_for_backward(xq, wq, wq_t, xs, w_scale)
        ctx.lead = lead
        ctx.has_bias = bias is not None
        return y.reshape(*lead, n)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx: Any, dy: torch.Tensor):
        xq, wq, wq_t, xs, wsc = ctx.saved_tensors
        n, k = wq.shape
        dy2 = dy.to(torch.bfloat16).reshape(-1, n).contiguous()
        dyq, dys = quantize_fp8_from_producer(dy2, dy) or quantize_fp8_tensor(dy2)
        dx = dw = db = None
        if ctx.needs_input_grad[0]:
            dx = _linear_dgrad_wt(dyq, wq, wq_t, dys, wsc).reshape(*ctx.lead, k)
        if ctx.needs_input_grad[1]:
            dw = linear_fp8_wgrad_prequantized(xq, dyq, xs, dys, out_f32=True)
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = dy2.float().sum(0)
        return dx, dw, db, None, None, None, None


def linear_fp8_autograd(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    return LinearFP8Function.apply(x, weight, bias)


# registers the torch.ops.dpa_fp8 custom ops the reference-named functions above call
from . import ops as _ops  # noqa: E402
