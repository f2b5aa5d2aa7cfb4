"""Pins the oracle's e4m3 codec and monotone key (CPU only).

Known answers are derived by hand from the OCP e4m3fn format (bias 7, 3
mantissa bits, max 448, no inf) and the monotone-key definition of
csrc/attention/sm70_mla_decode.cu:43-46; the two oracle encoders (torch's
cast after a clamp, and the C grid search in oracle/dsa_ref.c) are also
checked against each other over a dense sweep.
"""
import math

import numpy as np
import pytest
import torch

from oracle import cref
from oracle import dsa_oracle as O

# (value, expected byte)
ENCODE_KAT = [
    (0.0, 0x00),
    (-0.0, 0x80),
    (1.0, 0x38),          # exp 7, mant 0
    (-1.0, 0xB8),
    (1.125, 0x39),
    (1.0625, 0x38),       # tie 1.0 / 1.125 -> even mantissa (0)
    (1.1875, 0x3A),       # tie 1.125 / 1.25 -> even mantissa (2)
    (448.0, 0x7E),
    (449.0, 0x7E),        # SATFINITE
    (1e9, 0x7E),
    (-1e9, 0xFE),
    (float("inf"), 0x7E),
    (float("-inf"), 0xFE),
    (2.0 ** -6, 0x08),    # smallest normal
    (2.0 ** -9, 0x01),    # smallest denormal
    (2.0 ** -10, 0x00),   # tie 0 / 2^-9 -> even (0)
    (3 * 2.0 ** -10, 0x02),  # tie 2^-9 / 2^-8 -> even (2)
    (7 * 2.0 ** -9, 0x07),   # largest denormal
    (7.5 * 2.0 ** -9, 0x08), # tie 7*2^-9 / 2^-6 -> even (code 8)
    (240.0, 0x77),        # 1.875 * 2^7
    (0.1, 0x1D),          # 0.1 = 1.6 * 2^-4 -> mant 0.6*8 = 4.8 -> 5
]


@pytest.mark.parametrize("val,byte", ENCODE_KAT)
def test_encode_kat_torch(val, byte):
    got = int(O.e4m3_encode(torch.tensor([val], dtype=torch.float32))[0])
    assert got == byte, f"{val} -> {got:#x}, want {byte:#x}"


@pytest.mark.parametrize("val,byte", ENCODE_KAT)
def test_encode_kat_c(val, byte):
    got = int(cref.e4m3_encode(torch.tensor([val], dtype=torch.float32))[0])
    assert got == byte, f"{val} -> {got:#x}, want {byte:#x}"


def _exact_value(b: int) -> float:
    s = -1.0 if b & 0x80 else 1.0
    e, m = (b >> 3) & 15, b & 7
    return s * (math.ldexp(m, -9) if e == 0 else math.ldexp(8 + m, e - 10))


def test_decode_all_codes():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    finite = torch.tensor([(b & 0x7F) != 0x7F for b in range(256)])
    want = torch.tensor([_exact_value(b) for b in range(256)], dtype=torch.float32)
    got_t = O.e4m3_decode(codes)
    got_c = cref.e4m3_decode(codes)
    assert torch.equal(got_t[finite], want[finite])
    assert torch.equal(got_c[finite], want[finite])
    assert torch.isnan(got_t[~finite]).all() and torch.isnan(got_c[~finite]).all()


def test_encode_decode_roundtrip_all_finite():
    codes = torch.tensor([b for b in range(256) if (b & 0x7F) != 0x7F], dtype=torch.int32)
    vals = O.e4m3_decode(codes.to(torch.uint8))
    back = O.e4m3_encode(vals).to(torch.int32)
    # -0 and +0 keep their sign
    assert torch.equal(back, codes)


def test_encoders_agree_dense_sweep():
    g = torch.Generator().manual_seed(0)
    # every code's value, midpoints (ties), and values just around them
    vals = O.e4m3_decode(torch.tensor([b for b in range(128) if b != 0x7F],
                                      dtype=torch.int32).to(torch.uint8)).double()
    mids = (vals[:-1] + vals[1:]) / 2
    eps = torch.tensor([-1e-7, 0.0, 1e-7], dtype=torch.float64)
    pts = torch.cat([vals, (mids[:, None] * (1 + eps[None, :])).reshape(-1)])
    rnd = torch.randn(200000, generator=g, dtype=torch.float64) * torch.exp(
        torch.randn(200000, generator=g, dtype=torch.float64) * 3)
    x = torch.cat([pts, -pts, rnd]).to(torch.float32)
    a = O.e4m3_encode(x)
    b = cref.e4m3_encode(x)
    assert torch.equal(a, b)


def test_mono_key_kat():
    vals = torch.tensor([float("-inf"), -1.0, -0.0, 0.0, 1.0, float("inf")])
    want = [0x007FFFFF, 0x407FFFFF, 0x7FFFFFFF, 0x80000000, 0xBF800000, 0xFF800000]
    assert O.mono_key(vals).tolist() == want


def test_mono_key_is_monotone():
    g = torch.Generator().manual_seed(1)
    x = torch.cat([torch.randn(10000, generator=g) * 1e3, torch.tensor([0.0, -0.0])])
    k = O.mono_key(x).numpy()
    xs = x.numpy().astype(np.float64)
    # -0.0 == +0.0 as floats; the key orders -0 first
    order = np.lexsort((~np.signbit(xs), xs))
    assert np.all(np.diff(k[order]) >= 0)
