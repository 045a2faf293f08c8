"""CPU checks of the fake-quant emulation's own arithmetic (tests/fakequant.py), the module-
level reference of the GPU tests: its exact im2col convolutions equal torch's float64
convolution routines, and its cast follows the reference's clamp and NaN rule."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import fakequant as FQ
from oracle import fp8_oracle as O


@pytest.mark.parametrize("n,c,h,o,k,s,p", [(2, 8, 8, 16, 3, 1, 1), (2, 8, 8, 16, 3, 2, 1),
                                           (3, 8, 6, 4, 1, 1, 0), (1, 4, 5, 4, 3, 2, 1)])
def test_im2col_convs_equal_torch_float64(n, c, h, o, k, s, p):
    g = torch.Generator().manual_seed(n * 100 + c + k + s)
    x = torch.randn(n, c, h, h, generator=g, dtype=torch.float64)
    w = torch.randn(o, c, k, k, generator=g, dtype=torch.float64)
    y = FQ._conv_fwd64(x, w, s, p)
    ref = F.conv2d(x, w, stride=s, padding=p)
    dy = torch.randn(ref.shape, generator=g, dtype=torch.float64)
    torch.testing.assert_close(y, ref, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(FQ._conv_dgrad64(dy, w, x.shape, s, p),
                               torch.nn.grad.conv2d_input(x.shape, w, dy, stride=s, padding=p),
                               rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(FQ._conv_wgrad64(x, dy, w.shape, s, p),
                               torch.nn.grad.conv2d_weight(x, w.shape, dy, stride=s, padding=p),
                               rtol=1e-12, atol=1e-12)


def test_emulated_cast_matches_oracle_and_nan_rule():
    """_cast / _scale_of on bf16 values give the oracle's e4m3 bytes and scale; an empty
    history (scale 0) maps finite x to +-448 and 0 to +448, as Triton's min/max do."""
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(4096, generator=g) * 3).to(torch.bfloat16)
    xf = x.float()
    s = FQ._scale_of(xf)
    q = FQ._cast(xf, s).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    qo, so = O.quantize_fp8(x.view(torch.int16).numpy().view(np.uint16))
    assert np.float32(s.item()) == so
    np.testing.assert_array_equal(q, qo)
    z = FQ._cast(torch.tensor([1.5, -2.0, 0.0]), torch.tensor(0.0))
    assert z.tolist() == [448.0, -448.0, 448.0]


def test_emulated_division_is_correctly_rounded_at_e4m3_ties():
    """With scale 7 * 2^-11 many bf16 inputs divide to an exact e4m3 rounding midpoint; the
    emulation's quotient must be the IEEE one so those ties round to even, as the oracle's."""
    s = torch.tensor(7.0 * 2.0**-11)
    x = (torch.arange(-2000, 2000, dtype=torch.float32) * 7.0 * 2.0**-11 / 16).to(torch.bfloat16)
    q = FQ._cast(x.float(), s).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    ref = O.f32_to_e4m3_rne(np.clip(O.bf16_bits_to_f32(x.view(torch.int16).numpy().view(np.uint16))
                                    / np.float32(s.item()), -448, 448).astype(np.float32))
    np.testing.assert_array_equal(q, ref)
