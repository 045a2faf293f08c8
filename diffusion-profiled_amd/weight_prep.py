"""Grouped FP8 weight preparation for a model's FP8 layers.

The reference quantizes each FP8 layer's weight inside the layer call (diffusion/unet.py:69-91
-> diffusion/fp8_kernels.py:822-889: autocast bf16 cast, quantize_fp8 or quantize_fp8_delayed,
window bookkeeping; the data gradient then reads the weight transposed). ``WeightPrep`` does
the same for every FP8 layer of a model in three launches at the start of each forward
(``dpa_window_max_grouped_f32`` + ``dpa_weight_prep_run``), straight from the fp32 master
weights, into persistent buffers; the layers then run the ``*Prepared`` autograd Functions of
``fp8_kernels`` and return fp32 weight gradients directly. Bytes, scales and window states are
identical to the per-call path (tests/test_gpu_weight_prep.py).

Each layer records the FP8 path it took (``_fp8_mode``: "delayed", "current" or "linear") on
its first GPU call, so a plan covers exactly the layers the model runs in FP8 at its shapes.
"""
from __future__ import annotations

import ctypes
from ctypes import c_int32, c_int64, c_void_p
from dataclasses import dataclass

import torch

from . import _lib
from .fp8_kernels import FP8_DTYPE

# amax partials per deferred window record that a producer-fused cast may leave
PRODUCER_PARTIALS = 16384


class DpaDeferredWindow(ctypes.Structure):
    """include/dpa_fp8.h ``DpaDeferredWindow``."""

    _fields_ = [
        ("x_partials", c_void_p), ("x_count", c_void_p), ("dy_partials", c_void_p),
        ("dy_count", c_void_p), ("window_acts", c_void_p), ("window_dy", c_void_p),
        ("pos", c_void_p), ("len", c_int64),
    ]


class DpaWeightEntry(ctypes.Structure):
    """include/dpa_fp8.h ``DpaWeightEntry``."""

    _fields_ = [
        ("w", c_void_p), ("q", c_void_p), ("qt", c_void_p), ("scale_used", c_void_p),
        ("cur_scale", c_void_p), ("prev_scale", c_void_p), ("window", c_void_p), ("pos", c_void_p),
        ("window_len", c_int64), ("n", c_int64), ("cout", c_int32), ("taps", c_int32),
        ("cin", c_int32), ("blk0", c_int32), ("nblk", c_int32), ("flags", c_int32),
    ]


@dataclass
class PreparedWeight:
    """The step's prepared weight of one layer (views into persistent buffers)."""

    q: torch.Tensor        # e4m3, the layer's weight shape and memory format
    qt: torch.Tensor       # e4m3 [Cin][R][S][Cout] / [K][N]
    scale: torch.Tensor    # [1] fp32: the scale q was cast with
    hist: torch.Tensor | None  # [3] fp32 window maxima (acts, weights, dy), delayed layers
    parts: tuple | None = None  # delayed layers: (x partials, x count, dy partials, dy count)
    # q / qt hold the halo-patch conv's fragment layouts (flat uint8): forward, data gradient
    frag: bool = False


def _fp8_weight(module) -> torch.Tensor:
    return module.conv.weight if hasattr(module, "conv") else module.weight


class WeightPrep:
    """Persistent buffers and the device entry table for a list of FP8 layers."""

    def __init__(self, layers: list):
        assert layers, "no FP8 layers"
        self.layers = layers
        dev = _fp8_weight(layers[0]).device
        delayed = [m for m in layers if m._fp8_mode == "delayed"]
        self.n_delayed = len(delayed)
        self.scales = torch.zeros(2 * len(layers), device=dev, dtype=torch.float32)
        self.hist = torch.zeros(max(3 * self.n_delayed, 1), device=dev, dtype=torch.float32)
        # deferred window records of the delayed layers' x / dy quantizations: room for the
        # standalone cast's partials and for those of the producers that cast for the layer
        # (one per GroupNorm workgroup: 8192 for 512 channels of 32x32 images at batch 128)
        cap = max(_lib.query("dpa_quant_partials_count", 1 << 40), PRODUCER_PARTIALS)
        self.dparts = torch.zeros((max(self.n_delayed, 1), 2, cap), device=dev, dtype=torch.int32)
        self.dcounts = torch.zeros((max(self.n_delayed, 1), 2), device=dev, dtype=torch.int32)
        deferred = (DpaDeferredWindow * max(self.n_delayed, 1))()
        window_ptrs = []
        self.window_len = 0
        entries = (DpaWeightEntry * len(layers))()
        self._keep = []
        d = 0
        for i, m in enumerate(layers):
            w = _fp8_weight(m)
            assert w.dtype == torch.float32 and w.device == dev
            frag = bool(getattr(m, "_fp8_frag", False))
            if w.ndim == 4 and frag:
                # the layer's convs run the halo-patch kernel: fragment layouts, same bytes
                cout, cin, kh, kw = w.shape
                assert w.is_contiguous(memory_format=torch.channels_last)
                q = torch.empty(w.numel(), device=dev, dtype=torch.uint8)
                qt = torch.empty(w.numel(), device=dev, dtype=torch.uint8)
                taps = kh * kw
            elif w.ndim == 4:
                cout, cin, kh, kw = w.shape
                assert w.is_contiguous(memory_format=torch.channels_last)
                q = torch.empty((cout, cin, kh, kw), device=dev, dtype=FP8_DTYPE,
                                memory_format=torch.channels_last)
                qt = torch.empty((cin, kh, kw, cout), device=dev, dtype=FP8_DTYPE)
                taps = kh * kw
            else:
                cout, cin = w.shape
                assert w.is_contiguous()
                q = torch.empty((cout, cin), device=dev, dtype=FP8_DTYPE)
                qt = torch.empty((cin, cout), device=dev, dtype=FP8_DTYPE)
                taps = 1
            e = entries[i]
            e.w, e.q, e.qt = w.data_ptr(), q.data_ptr(), qt.data_ptr()
            e.scale_used = self.scales[2 * i].data_ptr()
            e.cur_scale = self.scales[2 * i + 1].data_ptr()
            e.n, e.cout, e.taps, e.cin = w.numel(), cout, taps, cin
            e.flags = 2 if frag and w.ndim == 4 else 0        # DPA_WP_FRAG
            hist = parts = None
            if m._fp8_mode == "delayed":
                hist = self.hist[3 * d:3 * d + 3]
                e.prev_scale = hist[1].data_ptr()
                e.window = m.amax_window_weights.data_ptr()
                e.pos = m.window_pos.data_ptr()
                e.window_len = m.amax_window_weights.numel()
                for win in (m.amax_window_acts, m.amax_window_weights, m.amax_window_dy):
                    assert win.dtype == torch.float32 and win.is_contiguous()
                    if self.window_len == 0:
                        self.window_len = win.numel()
                    assert win.numel() == self.window_len, "one amax history length per model"
                    window_ptrs.append(win.data_ptr())
                parts = (self.dparts[d, 0], self.dcounts[d, 0:1], self.dparts[d, 1],
                         self.dcounts[d, 1:2])
                dw = deferred[d]
                dw.x_partials, dw.x_count = parts[0].data_ptr(), parts[1].data_ptr()
                dw.dy_partials, dw.dy_count = parts[2].data_ptr(), parts[3].data_ptr()
                dw.window_acts = m.amax_window_acts.data_ptr()
                dw.window_dy = m.amax_window_dy.data_ptr()
                dw.pos = m.window_pos.data_ptr()
                dw.len = m.amax_window_acts.numel()
                d += 1
            m._fp8_prepared = PreparedWeight(q, qt, self.scales[2 * i:2 * i + 1], hist, parts,
                                             frag and w.ndim == 4)
            m._fp8_plan = self
            self._keep += [q, qt]
        self.active = False
        self.x_cache: dict = {}     # e4m3 copies of layer inputs shared within one forward
        blocks = _lib.load().dpa_weight_prep_plan(ctypes.addressof(entries), len(layers))
        _lib.check(min(blocks, 0), "dpa_weight_prep_plan")
        self.blocks = int(blocks)
        self.count = len(layers)
        raw = bytes(entries)
        self.table = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(dev)
        self.ws_bytes = _lib.query("dpa_weight_prep_workspace_bytes", self.blocks)
        self.workspace = torch.empty(self.ws_bytes, device=dev, dtype=torch.uint8)
        self.windows = (torch.tensor(window_ptrs, dtype=torch.int64).to(dev)
                        if window_ptrs else None)
        self.deferred = torch.frombuffer(bytearray(bytes(deferred)), dtype=torch.uint8).to(dev)

    def flush(self) -> None:
        """Write the window records the delayed layers' last x / dy quantizations left pending
        (run() does this first; call it before reading or saving the windows)."""
        if self.n_delayed:
            stream = _lib.current_stream(self.table)
            _lib.call("dpa_delayed_windows_finalize", self.deferred.data_ptr(), self.n_delayed,
                      stream)

    def run(self) -> None:
        """The step's weights: the previous step's pending window records, the window maxima
        (delayed layers), then amax + cast of every weight."""
        stream = _lib.current_stream(self.table)
        self.x_cache.clear()
        self.flush()
        if self.windows is not None:
            _lib.call("dpa_window_max_grouped_f32", self.windows.data_ptr(), 3 * self.n_delayed,
                      self.window_len, self.hist.data_ptr(), stream)
        _lib.call("dpa_weight_prep_run", self.table.data_ptr(), self.count, self.blocks,
                  self.workspace.data_ptr(), self.ws_bytes, stream)

    def detach_layers(self) -> None:
        for m in self.layers:
            m._fp8_prepared = None
            m._fp8_plan = None

    @staticmethod
    def from_model(model: torch.nn.Module) -> "WeightPrep | None":
        layers = [m for m in model.modules() if getattr(m, "_fp8_mode", None) is not None]
        return WeightPrep(layers) if layers else None


class TensorPrep:
    """Current-scaling e4m3 copies of fixed weight tensors (fp32 or bf16; 4-D channels-last
    conv weights or 2-D [N][K]) with their data-gradient transposes and scales, for all of
    them in two launches: ``quantize_fp8`` of each weight plus ``weight_transpose_fp8``,
    bit-identical. Buffers are allocated once; run() refreshes them from the weights."""

    def __init__(self, weights: list, frag: list | None = None):
        """``frag[i]``: weight i feeds the halo-patch conv, so q / qt hold its forward and
        data-gradient fragment layouts (flat uint8) instead of OHWI / [Cin][R][S][Cout]."""
        assert weights
        dev = weights[0].device
        self.weights = weights
        self.frag = [bool(f) for f in (frag or [False] * len(weights))]
        self.scales = torch.zeros(len(weights), device=dev, dtype=torch.float32)
        self.q, self.qt = [], []
        entries = (DpaWeightEntry * len(weights))()
        for i, w in enumerate(weights):
            assert w.dtype in (torch.float32, torch.bfloat16) and w.device == dev
            if w.ndim == 4 and self.frag[i]:
                cout, cin, kh, kw = w.shape
                assert w.is_contiguous(memory_format=torch.channels_last)
                q = torch.empty(w.numel(), device=dev, dtype=torch.uint8)
                qt = torch.empty(w.numel(), device=dev, dtype=torch.uint8)
                taps = kh * kw
            elif w.ndim == 4:
                cout, cin, kh, kw = w.shape
                assert w.is_contiguous(memory_format=torch.channels_last)
                q = torch.empty((cout, cin, kh, kw), device=dev, dtype=FP8_DTYPE,
                                memory_format=torch.channels_last)
                qt = torch.empty((cin, kh, kw, cout), device=dev, dtype=FP8_DTYPE)
                taps = kh * kw
            else:
                cout, cin = w.shape
                assert w.is_contiguous()
                q = torch.empty((cout, cin), device=dev, dtype=FP8_DTYPE)
                qt = torch.empty((cin, cout), device=dev, dtype=FP8_DTYPE)
                taps = 1
            e = entries[i]
            e.w, e.q, e.qt = w.data_ptr(), q.data_ptr(), qt.data_ptr()
            e.scale_used = self.scales[i].data_ptr()
            e.n, e.cout, e.taps, e.cin = w.numel(), cout, taps, cin
            e.flags = ((1 if w.dtype == torch.bfloat16 else 0)                 # DPA_WP_BF16
                       | (2 if w.ndim == 4 and self.frag[i] else 0))          # DPA_WP_FRAG
            self.q.append(q)
            self.qt.append(qt)
        blocks = _lib.load().dpa_weight_prep_plan(ctypes.addressof(entries), len(weights))
        _lib.check(min(blocks, 0), "dpa_weight_prep_plan")
        self.blocks, self.count = int(blocks), len(weights)
        self.table = torch.frombuffer(bytearray(bytes(entries)), dtype=torch.uint8).to(dev)
        self.ws_bytes = _lib.query("dpa_weight_prep_workspace_bytes", self.blocks)
        self.workspace = torch.empty(self.ws_bytes, device=dev, dtype=torch.uint8)

    def scale(self, i: int) -> torch.Tensor:
        return self.scales[i]

    def run(self) -> None:
        stream = _lib.current_stream(self.table)
        _lib.call("dpa_weight_prep_run", self.table.data_ptr(), self.count, self.blocks,
                  self.workspace.data_ptr(), self.ws_bytes, stream)

    def run_with_quantize(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """run() and ``quantize_fp8(x)`` (current scaling, bf16 x) in the same two launches
        (dpa_quantize_fp8_bf16_with_weight_prep); returns x's (e4m3, scale) as quantize_fp8
        does, the weights' copies land in q / qt / scales as after run()."""
        assert x.dtype == torch.bfloat16 and x.device == self.table.device
        if not (x.is_contiguous() or (x.ndim == 4 and x.is_contiguous(
                memory_format=torch.channels_last))):
            x = x.contiguous()
        n = x.numel()
        q = torch.empty_like(x, dtype=FP8_DTYPE, memory_format=torch.preserve_format)
        scale = torch.empty((), device=x.device, dtype=torch.float32)
        ws_bytes = _lib.query("dpa_quant_workspace_bytes", n)
        ws = torch.empty(ws_bytes, device=x.device, dtype=torch.uint8)
        stream = _lib.current_stream(x)
        _lib.call("dpa_quantize_fp8_bf16_with_weight_prep", x.data_ptr(), n, q.data_ptr(),
                  scale.data_ptr(), ws.data_ptr(), ws_bytes, self.table.data_ptr(), self.count,
                  self.blocks, self.workspace.data_ptr(), self.ws_bytes, stream)
        return q, scale
