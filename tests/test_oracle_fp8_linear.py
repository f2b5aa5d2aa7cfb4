"""Pins the oracle's fp8 weight quantizer, dequant and GEMV (CPU only).

Known answers: a block whose amax is 448 has scale 1 and encodes exactly; an
all-zero block gets the 1e-12 floor (glue.patch:1528); dequant of chosen
(byte, scale) pairs; GEMV of a weight equal to a scaled identity.
"""
import torch

from oracle import dsa_oracle as O


def test_quantize_kat_scale_one():
    w = torch.zeros(128, 256, dtype=torch.float16)
    w[0, 0] = 448.0
    w[3, 5] = -2.0
    w[0, 200] = 1.0
    q8, s = O.attn_fp8_quantize(w)
    assert s.shape == (1, 2)
    assert s[0, 0] == 1.0 and s[0, 1] == 1.0 / 448.0
    assert q8[0, 0] == 0x7E and q8[3, 5] == 0xC0  # -2.0 = 1.0 * 2^1 -> exp 8
    assert q8[0, 200] == 0x7E  # 1.0 / (1/448) = 448


def test_quantize_zero_block_floor():
    w = torch.zeros(130, 16, dtype=torch.float16)
    q8, s = O.attn_fp8_quantize(w)
    assert s.shape == (2, 1)
    assert torch.all(s == torch.tensor(1e-12, dtype=torch.float32))
    assert torch.all(q8 == 0)


def test_quantize_roundtrip_error_bound():
    g = torch.Generator().manual_seed(0)
    w = (torch.randn(300, 520, generator=g) * 0.02).to(torch.float16)
    q8, s = O.attn_fp8_quantize(w)
    deq = O.e4m3_decode(q8) * O.expand_block_scale(s, 300, 520)
    amax = O.expand_block_scale(s, 300, 520) * 448
    assert ((deq - w.float()).abs() <= amax * 2.0 ** -4 + 1e-12).all()


def test_dequant_kat():
    w = torch.tensor([[0x38, 0xB8, 0x01, 0x7E] * 4], dtype=torch.int32).to(torch.uint8)
    s = torch.tensor([[0.5]], dtype=torch.float32)
    out = O.attn_fp8_dequant(w, s)
    assert out[0, :4].tolist() == [0.5, -0.5, 2.0 ** -10, 224.0]
    # 448 * 1e-7 is not representable in fp16: RNE of the fp32 product
    s2 = torch.tensor([[1e-7]], dtype=torch.float32)
    got = O.attn_fp8_dequant(w, s2)[0, 3]
    assert got == torch.tensor(448 * 1e-7, dtype=torch.float32).to(torch.float16)


def test_gemv_scaled_identity():
    n = k = 256
    w = torch.zeros(n, k, dtype=torch.uint8)
    w[torch.arange(n), torch.arange(k)] = 0x38  # 1.0
    s = torch.tensor([[0.25, 0.0], [0.0, 2.0]], dtype=torch.float32)
    x = torch.randn(3, k).to(torch.float16)
    y = O.attn_fp8_gemv(x, w, s)
    want = x.double().clone()
    want[:, :128] *= 0.25
    want[:, 128:] *= 2.0
    assert torch.equal(y, want)
