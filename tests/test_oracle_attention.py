"""Pins the oracle's sparse MLA attention and fp8_ds_mla writer (CPU only).

Independent checks: closed forms (one key, equal scores, no valid key), the
DSA invariant sparse == dense when every context position is selected
(reference/triton_mla.py:225-233), invariance under idx order and under a
physical block permutation, and byte-level layout checks of the 656-byte
row (csrc/attention/sm70_mla_decode.cu:74-100).
"""
import math

import pytest
import torch

from oracle import dsa_oracle as O

SCALE = 576 ** -0.5


def make_cache(g, nblk=6, page=16, fp8=False):
    lat = torch.randn(nblk * page, 576, generator=g) / 4
    if fp8:
        return O.dsmla_rows(lat).view(nblk, page, 656), lat
    return lat.to(torch.float16).view(nblk, page, 576), lat


def test_single_key_closed_form():
    g = torch.Generator().manual_seed(0)
    kv, _ = make_cache(g)
    bt = torch.randperm(6, generator=g).to(torch.int32)[None]
    q = torch.randn(1, 4, 576, generator=g).to(torch.float16)
    j = 37
    idx = torch.full((1, 8), -1, dtype=torch.int32)
    idx[0, 3] = j
    o, lse = O.sparse_mla(q, kv, idx, bt, torch.tensor([50], dtype=torch.int32), SCALE)
    row = int(bt[0, j // 16]) * 16 + j % 16
    K = kv.view(-1, 576)[row].double()
    assert torch.allclose(o[0], K[:512].float().expand(4, 512))
    qs = O.scaled_q(q, SCALE)[0].double()
    assert torch.allclose(lse[0].double(), qs @ K, atol=1e-6)


def test_equal_scores_closed_form():
    g = torch.Generator().manual_seed(1)
    kv, _ = make_cache(g)
    bt = torch.arange(6, dtype=torch.int32)[None]
    q = torch.zeros(1, 2, 576, dtype=torch.float16)
    idx = torch.tensor([[5, 9, 11, -1, 70, 2]], dtype=torch.int32)  # 70 >= seq_len
    o, lse = O.sparse_mla(q, kv, idx, bt, torch.tensor([64], dtype=torch.int32), SCALE)
    V = kv.view(-1, 576)[[5, 9, 11, 2], :512].double()
    assert torch.allclose(o[0].double(), V.mean(0).expand(2, 512), atol=1e-6)
    assert torch.allclose(lse[0].double(), torch.full((2,), math.log(4.0), dtype=torch.float64))


def test_no_valid_key():
    g = torch.Generator().manual_seed(2)
    kv, _ = make_cache(g)
    bt = torch.arange(6, dtype=torch.int32)[None]
    q = torch.randn(1, 3, 576, generator=g).to(torch.float16)
    idx = torch.tensor([[-1, 40, 41]], dtype=torch.int32)
    o, lse = O.sparse_mla(q, kv, idx, bt, torch.tensor([40], dtype=torch.int32), SCALE)
    assert torch.all(o == 0) and torch.all(torch.isinf(lse)) and torch.all(lse < 0)


@pytest.mark.parametrize("fp8", [False, True])
def test_sparse_equals_dense_when_all_selected(fp8):
    g = torch.Generator().manual_seed(3)
    kv, _ = make_cache(g, fp8=fp8)
    B, H = 2, 8
    bt = torch.stack([torch.randperm(6, generator=g) for _ in range(B)]).to(torch.int32)
    seq = torch.tensor([61, 96], dtype=torch.int32)
    q = (torch.randn(B, H, 576, generator=g) / 4).to(torch.float16)
    idx = torch.full((B, 128), -1, dtype=torch.int32)
    for b in range(B):
        perm = torch.randperm(int(seq[b]), generator=g).to(torch.int32)
        idx[b, : perm.numel()] = perm
    o_s, l_s = O.sparse_mla(q, kv, idx, bt, seq, SCALE)
    o_d, l_d = O.dense_mla(q, kv, bt, seq, SCALE)
    assert torch.allclose(o_s, o_d, atol=1e-6)
    assert torch.allclose(l_s, l_d, atol=1e-6)


def test_block_permutation_invariance():
    g = torch.Generator().manual_seed(4)
    kv, _ = make_cache(g)
    q = torch.randn(1, 4, 576, generator=g).to(torch.float16)
    bt = torch.arange(6, dtype=torch.int32)[None]
    idx = torch.randint(0, 90, (1, 32), generator=g, dtype=torch.int32)
    seq = torch.tensor([90], dtype=torch.int32)
    o1, l1 = O.sparse_mla(q, kv, idx, bt, seq, SCALE)
    perm = torch.randperm(6, generator=g)
    kv2 = torch.empty_like(kv)
    kv2[perm] = kv  # logical block i now lives in physical block perm[i]
    o2, l2 = O.sparse_mla(q, kv2, idx, perm.to(torch.int32)[None], seq, SCALE)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_dsmla_row_layout():
    g = torch.Generator().manual_seed(5)
    lat = torch.randn(10, 576, generator=g)
    rows = O.dsmla_rows(lat)
    assert rows.shape == (10, 656) and rows.dtype == torch.uint8
    sc = rows[:, 512:528].contiguous().view(torch.float32)
    amax = lat[:, :512].abs().amax(1)
    assert torch.equal(sc, (amax / 448.0).unsqueeze(1).expand(10, 4))
    rope = rows[:, 528:].contiguous().view(torch.float16)
    assert torch.equal(rope, lat[:, 512:].to(torch.float16))
    deq = O.e4m3_decode(rows[:, :512].contiguous()) * sc.repeat_interleave(128, 1)
    err = (deq - lat[:, :512]).abs() / amax[:, None]
    assert err.max() <= 2.0 ** -4  # e4m3 relative step at the top binade
    # the row maximum itself is encoded as +-448
    i = lat[:, :512].abs().argmax(1)
    top = rows[torch.arange(10), i] & 0x7F
    assert torch.all(top == 0x7E)


def test_dsmla_per_tile_layout():
    lat = torch.zeros(1, 576)
    lat[0, 0] = 4.0
    lat[0, 200] = -8.0
    rows = O.dsmla_rows(lat, per_tile=True)
    sc = rows[:, 512:528].contiguous().view(torch.float32)[0]
    assert sc[0] == 4.0 / 448 and sc[1] == 8.0 / 448
    assert sc[2] == O.FLT_MIN and sc[3] == O.FLT_MIN
    assert int(rows[0, 0]) == 0x7E and int(rows[0, 200]) == 0xFE


@pytest.mark.parametrize("B,H,expect", [(32, 16, -1e30), (31, 16, -math.inf), (32, 17, -math.inf)])
def test_empty_token_lse_follows_reference_dispatch(B, H, expect):
    """An empty token's lse is -1e30 exactly when the reference's op takes its
    prefill kernel (B >= 32 and H <= 16, sm70_mla_decode.cu:2511, whose
    epilogue writes m_init + ln 1, :1789-1793), else -inf (:1175-1183)."""
    g = torch.Generator().manual_seed(9)
    kv, _ = make_cache(g)
    bt = torch.randperm(6, generator=g).to(torch.int32).expand(B, 6).contiguous()
    q = torch.randn(B, H, 576, generator=g).to(torch.float16)
    idx = torch.full((B, 4), -1, dtype=torch.int32)
    idx[1:, 0] = 5
    o, lse = O.sparse_mla(q, kv, idx, bt, torch.full((B,), 40, dtype=torch.int32), SCALE)
    assert torch.all(o[0] == 0) and torch.all(lse[0] == expect)
    assert torch.isfinite(lse[1:]).all() and (lse[1:] > -1e29).all()


# ---- dense MLA decode (sm70_mla_decode) ----

@pytest.mark.parametrize("fp16_acc", [False, True])
def test_dense_single_position_closed_form(fp16_acc):
    """seq_len = 1: o = V of position 0 (fp16 rounding of V / 1), lse = s."""
    g = torch.Generator().manual_seed(10)
    kv, _ = make_cache(g)
    bt = torch.randperm(6, generator=g).to(torch.int32)[None]
    q = torch.randn(1, 32, 576, generator=g).to(torch.float16)
    o, lse = O.mla_decode(q, kv, bt, torch.tensor([1], dtype=torch.int32), SCALE, fp16_acc)
    K = kv.view(-1, 576)[int(bt[0, 0]) * 16].double()
    assert torch.allclose(o[0].double(), K[:512].expand(32, 512), atol=1e-6)
    qs = O.scaled_q(q, SCALE)[0].double()
    assert torch.allclose(lse[0].double(), qs @ K, atol=1e-5)


@pytest.mark.parametrize("fp16_acc", [False, True])
def test_dense_unresolvable_rows_are_zero_keys(fp16_acc):
    """Every position below seq_len on a -1 block: each is a zero key with
    score 0, so o = 0 and lse = ln seq_len (the reference's zero-row read,
    sm70_mla_decode.cu:762-771); seq_len 0 gives o = 0, lse = -inf."""
    g = torch.Generator().manual_seed(11)
    kv, _ = make_cache(g)
    bt = torch.full((2, 6), -1, dtype=torch.int32)
    q = torch.randn(2, 32, 576, generator=g).to(torch.float16)
    o, lse = O.mla_decode(q, kv, bt, torch.tensor([70, 0], dtype=torch.int32), SCALE, fp16_acc)
    assert torch.all(o == 0)
    assert torch.allclose(lse[0].double(), torch.full((32,), math.log(70.0), dtype=torch.float64),
                          atol=1e-6)
    assert torch.all(torch.isinf(lse[1])) and torch.all(lse[1] < 0)


def test_dense_equals_sparse_over_all_positions():
    """With every row resolvable, dense decode is the sparse op with idx =
    0..seq_len-1 (the pinned sparse_mla), empty token included."""
    g = torch.Generator().manual_seed(12)
    kv, _ = make_cache(g, nblk=8)
    bt = torch.stack([torch.randperm(8, generator=g)[:6] for _ in range(3)]).to(torch.int32)
    q = torch.randn(3, 32, 576, generator=g).to(torch.float16)
    seq = torch.tensor([96, 33, 0], dtype=torch.int32)
    o, lse = O.mla_decode(q, kv, bt, seq, SCALE)
    idx = torch.arange(96, dtype=torch.int32).expand(3, 96).contiguous()
    ro, rl = O.sparse_mla(q, kv, idx, bt, seq, SCALE, empty_lse=float("-inf"))
    assert torch.allclose(o, ro, atol=1e-6) and torch.equal(torch.isinf(lse), torch.isinf(rl))
    fin = torch.isfinite(rl)
    assert torch.allclose(lse[fin], rl[fin], atol=1e-6)


def test_dense_fp16_accumulation_stays_near_exact():
    """The reference's fp16 running O (restated tile by tile) differs from
    the exact result by fp16 rounding only: within the attention tolerance,
    and not bit-equal (the rounding is really applied)."""
    g = torch.Generator().manual_seed(13)
    kv, _ = make_cache(g, nblk=40, page=64)
    bt = torch.randperm(40, generator=g).to(torch.int32)[None].repeat(2, 1)
    q = (torch.randn(2, 32, 576, generator=g) / 4).to(torch.float16)
    seq = torch.tensor([2500, 700], dtype=torch.int32)
    o, lse = O.mla_decode(q, kv, bt, seq, SCALE)
    o16, lse16 = O.mla_decode(q, kv, bt, seq, SCALE, fp16_acc=True)
    torch.testing.assert_close(o16, o, rtol=2e-3, atol=1e-3)
    assert (lse16 - lse).abs().max() <= 1e-4
    assert not torch.equal(o16, o)


def _e4m3_by_hand(b: int) -> float:
    """OCP e4m3fn byte -> value from the format's definition (sign, 4-bit
    exponent with bias 7, 3-bit mantissa, exponent 0 = subnormal)."""
    sign = -1.0 if b & 0x80 else 1.0
    e, m = (b >> 3) & 0xF, b & 7
    if e == 0:
        return sign * (m / 8.0) * 2.0 ** -6
    return sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def _dsmla_row_by_hand(codes, scales, rope):
    """656-byte fp8_ds_mla row assembled byte by byte: 512 e4m3 codes, the 4
    fp32 tile scales at bytes 512 + 4t (little endian), 64 fp16 RoPE values
    at bytes 528 + 2i (sm70_mla_decode.cu:74-100)."""
    import struct
    raw = bytes(codes) + struct.pack("<4f", *scales) + struct.pack("<64e", *rope)
    assert len(raw) == 656
    return torch.tensor(list(raw), dtype=torch.uint8)


def test_fp8_reader_per_tile_known_answer():
    """The fp8_ds_mla branch of latent_rows_fp16, pinned value by value on a
    row with four distinct tile scales: dim d < 512 reads
    fp16_rn(e4m3(byte d) * scale[d // 128]); dims 512..575 are the RoPE
    fp16 bits copied.  A tile-index, byte-offset or rounding mistake changes
    at least one of the 576 values."""
    import numpy as np
    rng = np.random.default_rng(7)
    codes = [int(c) for c in rng.integers(0, 256, 512)]
    codes = [c if (c & 0x7F) != 0x7F else c ^ 1 for c in codes]  # no NaN codes
    codes[0], codes[1], codes[130], codes[300] = 0x00, 0x80, 0x7E, 0x01  # +0, -0, 448, min denormal
    scales = [0.25, 3.0, 1.0 / 96.0, 5.5]
    rope = [float(np.float16(x)) for x in rng.standard_normal(64)]
    row = _dsmla_row_by_hand(codes, scales, rope)
    page = 4
    kv = torch.zeros(2, page, 656, dtype=torch.uint8)
    kv[1, 2] = row  # physical row 6
    got = O.latent_rows_fp16(kv, torch.tensor([6, -1]))
    want = [float(np.float16(_e4m3_by_hand(codes[d]) * np.float32(scales[d // 128])))
            for d in range(512)] + rope
    assert got[0].double().tolist() == want
    assert torch.all(got[1] == 0)
    # bit-level: the RoPE half of the row is copied, not converted
    assert torch.equal(got[0, 512:].view(torch.int16),
                       row[528:].view(torch.int16))
    # one selected key: o is the key's value part, lse = q_s . k summed by hand
    q = torch.tensor(rng.standard_normal((1, 2, 576)) * 0.3, dtype=torch.float16)
    bt = torch.tensor([[1, 0]], dtype=torch.int32)   # position 2 -> block 1, row 6
    idx = torch.tensor([[2, -1, -1]], dtype=torch.int32)
    o, lse = O.sparse_mla(q, kv, idx, bt, torch.tensor([4], dtype=torch.int32), SCALE)
    assert o[0].double().tolist() == [want[:512]] * 2
    s16 = float(np.float16(SCALE))
    for h in range(2):
        qs = [float(np.float16(float(q[0, h, d]) * s16)) for d in range(576)]
        dot = math.fsum(qs[d] * want[d] for d in range(576))
        assert abs(float(lse[0, h]) - dot) <= 1e-6 + 2.0 ** -23 * abs(dot)  # fp32 lse rounding


@pytest.mark.parametrize("fp8", [False, True])
def test_unresolved_row_is_zero_key_on_split_decode_shapes(fp8):
    """A selected position below seq_len whose page maps to block -1, or to a
    block past the cache, is a zero key with score 0 on the reference's
    split-decode shapes (sm70_mla_decode.cu:970-992, :1047-1053), and masked
    on its prefill-kernel shapes, B >= 32 and H <= 16 (:1617-1628, :1705).
    Closed forms: with one resolvable key of score s and n zero keys,
    o = e^s v / (e^s + n) and lse = ln(e^s + n); masked, o = v and lse = s."""
    g = torch.Generator().manual_seed(11)
    page = 8
    kv, _ = make_cache(g, nblk=3, page=page, fp8=fp8)
    n_rows = 3 * page
    bt_row = torch.tensor([2, -1, 7, 0], dtype=torch.int32)  # block 7 is past the cache
    for B, H, zero in ((1, 4, True), (32, 16, False)):
        bt = bt_row.expand(B, 4).contiguous()
        q = torch.randn(B, H, 576, generator=g).to(torch.float16)
        # position 3 -> block 2 (resolves); 9 -> block -1; 17 -> block 7 (row >= n_rows);
        # 30 -> block 0 but >= seq_len (masked either way); 33 -> page 4, past the table
        idx = torch.tensor([3, 9, 17, 30, 33], dtype=torch.int32).expand(B, 5).contiguous()
        seq = torch.full((B,), 29, dtype=torch.int32)
        o, lse = O.sparse_mla(q, kv, idx, bt, seq, SCALE)
        K = O.latent_rows_fp16(kv, torch.tensor([2 * page + 3]))[0].double()
        assert 2 * page + 3 < n_rows
        s = O.scaled_q(q, SCALE).double() @ K  # [B, H]
        if zero:
            w = torch.exp(s) / (torch.exp(s) + 2.0)
            assert torch.allclose(o.double(), w[..., None] * K[:512], atol=1e-6)
            assert torch.allclose(lse.double(), torch.log(torch.exp(s) + 2.0), atol=1e-6)
        else:
            assert torch.allclose(o.double(), K[:512].expand(B, H, 512), atol=1e-6)
            assert torch.allclose(lse.double(), s, atol=1e-6)
