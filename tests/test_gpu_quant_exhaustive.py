"""Exhaustive GPU check of the e4m3 quantizer used by the indexer-K and
latent cache scatters (e4m3_quant8: reciprocal division with a Markstein
correction + the hardware RNE conversion): identical codes to IEEE division
+ the integer SATFINITE encoder for every positive finite fp16 / bf16 amax
and every fp16 / bf16 value v with |v| <= amax, both signs.  The kernel is
in tests/hip/quant_exhaustive.hip (test kit, built by build())."""
import ctypes
import os

import pytest

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "hip", "libdsa_testkit.so")


@pytest.mark.parametrize("bf16", [False, True], ids=["fp16", "bf16"])
def test_quantizer_exhaustive(dev, bf16):
    kit = ctypes.CDLL(LIB)
    bad = ctypes.c_ulonglong(0)
    first = (ctypes.c_uint32 * 2)()
    rc = kit.dsa_test_quant_exhaustive(int(bf16), ctypes.byref(bad), first)
    assert rc == 0
    assert bad.value == 0, f"{bad.value} mismatches, first amax bits {first[0]:#x} v {first[1]:#x}"
