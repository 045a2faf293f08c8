"""Self-attention of the U-Net's attention block on the HIP library's dpa_attention_* kernels,
as an autograd Function over the qkv projection's output.

Replaces ``F.scaled_dot_product_attention`` with the head rearranges around it
(diffusion/unet.py:188-198): the forward takes qkv [B, L, 3C] (q, k, v = its three thirds,
head h at columns h * 64 of each) and returns [B, L, C] in the layout the out projection
reads ("b nh l hd -> b l (nh hd)"); the backward returns d(qkv) in the same [B, L, 3C] layout,
so no head transposes, chunk copies or concatenations run in either direction. Head dim 64,
L a multiple of 16 up to 256 (the 16x16, 8x8 and 4x4 token grids of the U-Net).
"""
from __future__ import annotations

from typing import Any

import torch
from torch.amp.autocast_mode import custom_bwd, custom_fwd

from . import _lib
from . import fp8_kernels as _fp8

HEAD_DIM = 64


def _stream(t: torch.Tensor) -> int:
    return _lib.current_stream(t)


def supported(seq_len: int, channels: int, heads: int) -> bool:
    return (heads > 0 and channels == HEAD_DIM * heads and seq_len % 16 == 0
            and 16 <= seq_len <= 256)


class SelfAttentionQKV(torch.autograd.Function):
    """softmax(q k^T / sqrt(64)) v per (image, head) from qkv [B, L, 3C] (bf16; other float
    dtypes are rounded to bf16 first), output bf16 [B, L, C]."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx: Any, qkv: torch.Tensor, heads: int):
        b, l, c3 = qkv.shape
        c = c3 // 3
        if not supported(l, c, heads) or c3 != 3 * c:
            raise ValueError(f"self-attention kernel: unsupported shape {tuple(qkv.shape)}, heads {heads}")
        x = qkv.to(torch.bfloat16).contiguous()
        out = torch.empty((b, l, c), device=x.device, dtype=torch.bfloat16)
        lse = torch.empty((b * heads, l), device=x.device, dtype=torch.float32)
        if _fp8.PRODUCER_AMAX:
            # one |out| maximum per (image, head) for the out projection's e4m3 cast
            part = torch.empty(b * heads, device=x.device, dtype=torch.int32)
            _lib.call("dpa_attention_fwd_amax", x.data_ptr(), out.data_ptr(), lse.data_ptr(),
                      b, l, c, heads, part.data_ptr(), _stream(x))
            _fp8.mark_amax_partials(out, part, b * heads)
        else:
            _lib.call("dpa_attention_fwd_bf16", x.data_ptr(), out.data_ptr(), lse.data_ptr(),
                      b, l, c, heads, _stream(x))
        ctx.save_for_backward(x, out, lse)
        ctx.heads = heads
        ctx.in_dtype = qkv.dtype
        return out

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx: Any, dout: torch.Tensor):
        x, out, lse = ctx.saved_tensors
        b, l, c3 = x.shape
        g = dout.to(torch.bfloat16).contiguous()
        dqkv = torch.empty_like(x)
        if _fp8.PRODUCER_AMAX and ctx.in_dtype == torch.bfloat16:
            # one |dqkv| maximum per (image, head) for the qkv projection's e4m3 cast of dy
            part = torch.empty(b * ctx.heads, device=x.device, dtype=torch.int32)
            _lib.call("dpa_attention_bwd_amax", x.data_ptr(), out.data_ptr(), g.data_ptr(),
                      lse.data_ptr(), dqkv.data_ptr(), b, l, c3 // 3, ctx.heads,
                      part.data_ptr(), _stream(x))
            return _fp8.mark_amax_partials(dqkv, part, b * ctx.heads), None
        _lib.call("dpa_attention_bwd_bf16", x.data_ptr(), out.data_ptr(), g.data_ptr(),
                  lse.data_ptr(), dqkv.data_ptr(), b, l, c3 // 3, ctx.heads, _stream(x))
        return dqkv.to(ctx.in_dtype), None


def self_attention_qkv(qkv: torch.Tensor, heads: int) -> torch.Tensor:
    return SelfAttentionQKV.apply(qkv, heads)
