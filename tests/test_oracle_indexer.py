"""Pins the oracle's indexer logits, K store and Q packing (CPU only).

Independent checks: a pure-Python loop over positions and heads on tiny
shapes (the formula of csrc/attention/sm70_mla_decode.cu:131-136 evaluated
term by term), dyadic inputs whose fp32 sums are exact, -inf / zero-row
conventions, the histogram as a bincount, and the packing of
reference/sparse_attn_indexer.py:136-145 checked element by element.
"""
import math

import torch

from oracle import dsa_oracle as O


def brute_logits(q, kflat, w, bt, seq, page, max_kv):
    B = q.shape[0]
    out = [[float("-inf")] * max_kv for _ in range(B)]
    n_rows = kflat.shape[0]
    for b in range(B):
        for p in range(min(int(seq[b]), max_kv)):
            pg = p // page
            blk = int(bt[b, pg]) if pg < bt.shape[1] else -1
            row = blk * page + p % page
            kv = kflat[row].double() if (blk >= 0 and 0 <= row < n_rows) else torch.zeros(128, dtype=torch.float64)
            tot = 0.0
            for h in range(32):
                d = float(q[b, h].double() @ kv)
                tot += max(d, 0.0) * float(w[b, h])
            out[b][p] = tot
    return torch.tensor(out, dtype=torch.float64)


def test_matches_brute_force():
    g = torch.Generator().manual_seed(0)
    page, nblk = 8, 7
    kc = torch.randn(nblk, page, 128, generator=g).to(torch.float16)
    q = torch.randn(2, 32, 128, generator=g).to(torch.float16)
    w = torch.randn(2, 32, generator=g).to(torch.float16)
    bt = torch.tensor([[3, 1, -1, 6, 0], [2, 5, 4, 0, 1]], dtype=torch.int32)
    seq = torch.tensor([37, 60], dtype=torch.int32)  # row 1 reaches past bt width
    max_kv = 64
    got, _ = O.indexer_logits(q, kc, w, bt, seq, max_kv)
    want = brute_logits(q, kc.view(-1, 128), w, bt, seq, page, max_kv)
    fin = torch.isfinite(want)
    assert torch.equal(torch.isinf(got), ~fin)
    assert torch.allclose(got[fin].double(), want[fin], rtol=1e-6, atol=1e-5)
    # page index 2 of row 0 is -1 and positions >= 40 of row 1 are beyond the
    # table: both read K = 0, i.e. score 0
    assert torch.all(got[0, 16:24] == 0)
    assert torch.all(got[1, 40:60] == 0)


def test_dyadic_inputs_are_exact():
    g = torch.Generator().manual_seed(1)
    page, nblk = 16, 4
    kc = (torch.randint(-8, 9, (nblk, page, 128), generator=g) / 8).to(torch.float16)
    q = (torch.randint(-8, 9, (3, 32, 128), generator=g) / 8).to(torch.float16)
    w = (torch.randint(-4, 5, (3, 32), generator=g) / 4).to(torch.float16)
    bt = torch.stack([torch.randperm(nblk, generator=g) for _ in range(3)]).to(torch.int32)
    seq = torch.tensor([64, 17, 1], dtype=torch.int32)
    s64, _ = O.indexer_logits(q, kc, w, bt, seq, 64, dtype=torch.float64)
    s32, _ = O.indexer_logits(q, kc, w, bt, seq, 64, dtype=torch.float32)
    assert torch.equal(s64, s32)


def test_relu_and_weight_sign():
    kc = torch.zeros(1, 4, 128, dtype=torch.float16)
    kc[0, 0, 0] = 1.0
    kc[0, 1, 0] = -1.0
    q = torch.zeros(1, 32, 128, dtype=torch.float16)
    q[0, :, 0] = 2.0
    w = torch.full((1, 32), 0.5, dtype=torch.float16)
    w[0, 1] = -1.0
    bt = torch.zeros(1, 1, dtype=torch.int32)
    s, hist = O.indexer_logits(q, kc, w, bt, torch.tensor([3], dtype=torch.int32), 4,
                               with_hist=True)
    # pos 0: relu(2)*(31*0.5 - 1) = 29; pos 1: relu(-2) = 0; pos 2: k=0 -> 0
    assert s[0].tolist()[:3] == [29.0, 0.0, 0.0]
    assert math.isinf(s[0, 3]) and s[0, 3] < 0
    bins = (O.mono_key(s[0, :3]) >> 20).tolist()
    assert int(hist.sum()) == 3 and all(int(hist[0, b]) >= 1 for b in bins)


def test_fp8_cache_path_close_to_fp16():
    g = torch.Generator().manual_seed(2)
    page, nblk = 16, 4
    k = torch.randn(nblk * page, 128, generator=g).to(torch.float16)
    kc16 = k.view(nblk, page, 128)
    kc8 = O.indexer_k_store(torch.zeros(nblk, page, 132, dtype=torch.uint8), k,
                            torch.arange(nblk * page, dtype=torch.int32))
    q = torch.randn(2, 32, 128, generator=g).to(torch.float16)
    w = (torch.randn(2, 32, generator=g) / 32 ** 0.5).to(torch.float16)
    bt = torch.arange(nblk, dtype=torch.int32).expand(2, nblk).contiguous()
    seq = torch.tensor([64, 50], dtype=torch.int32)
    a, _ = O.indexer_logits(q, kc16, w, bt, seq, 64)
    b, _ = O.indexer_logits(q, kc8, w, bt, seq, 64)
    fin = torch.isfinite(a)
    assert torch.equal(fin, torch.isfinite(b))
    scale = a[fin].abs().max()
    assert ((a[fin] - b[fin]).abs() / scale).max() < 0.05


def test_k_store_fp8_row_kat():
    k = torch.zeros(1, 128, dtype=torch.float16)
    k[0, 0] = 448.0
    k[0, 1] = -1.0
    k[0, 2] = 0.5
    rows = O.idxk_fp8_row(k)
    assert rows[0, 0] == 0x7E and rows[0, 1] == 0xB8 and rows[0, 2] == 0x30
    assert rows[0, 128:].contiguous().view(torch.float32).item() == 1.0
    zero = O.idxk_fp8_row(torch.zeros(1, 128, dtype=torch.float16))
    assert zero[0, 128:].contiguous().view(torch.float32).item() == O.FLT_MIN
    assert torch.all(zero[0, :128] == 0)


def test_k_store_skips_bad_slots():
    kc = torch.zeros(2, 4, 128, dtype=torch.float16)
    k = torch.ones(3, 128, dtype=torch.float16)
    k[1] *= 2
    k[2] *= 3
    out = O.indexer_k_store(kc, k, torch.tensor([5, -1, 8], dtype=torch.int32))
    flat = out.view(-1, 128)
    assert torch.all(flat[5] == 1) and flat.abs().sum() == 128


def test_pack_q_layout():
    g = torch.Generator().manual_seed(3)
    n = 37
    q = torch.randn(n, 32, 128, generator=g).to(torch.float16)
    qp = O.pack_indexer_q(q)
    assert qp.shape == (32, 3, 8, 16, 16)
    for (h, t, kt, r, c) in [(0, 0, 0, 0, 0), (5, 1, 3, 7, 9), (31, 2, 7, 4, 15), (2, 2, 1, 15, 3)]:
        tok = 16 * t + r
        want = q[tok, h, 16 * kt + c] if tok < n else 0.0
        assert float(qp[h, t, kt, r, c]) == float(want)
    assert torch.equal(O.unpack_indexer_q(qp, n), q)


def test_packed_uses_each_tiles_first_row():
    """The packed kernel gathers a 32-query tile's keys with the table row of
    the tile's first query (sm70_mla_decode.cu:556, :566): rows 0-31 use
    bt[0], rows 32-63 bt[32], rows 64-69 bt[64]; the other rows' tables are
    never read."""
    g = torch.Generator().manual_seed(5)
    page, nblk, B, max_kv = 8, 9, 70, 48
    kc = torch.randn(nblk, page, 128, generator=g).to(torch.float16)
    q = torch.randn(B, 32, 128, generator=g).to(torch.float16)
    w = torch.randn(B, 32, generator=g).to(torch.float16)
    bt = torch.stack([torch.randperm(nblk, generator=g)[:6] for _ in range(B)]).to(torch.int32)
    seq = torch.randint(1, max_kv + 1, (B,), generator=g).to(torch.int32)
    got = O.indexer_logits_packed(O.pack_indexer_q(q), kc, w, bt, seq, max_kv)
    first = torch.tensor([0] * 32 + [32] * 32 + [64] * 6)
    want = brute_logits(q, kc.view(-1, 128), w, bt[first], seq, page, max_kv)
    fin = torch.isfinite(want)
    assert torch.equal(torch.isinf(got), ~fin)
    assert torch.allclose(got[fin].double(), want[fin], rtol=1e-6, atol=1e-5)
    per_row, _ = O.indexer_logits(q, kc, w, bt, seq, max_kv)
    assert not torch.equal(per_row[1:32], got[1:32])  # the distinction is visible


def test_packed_fp8_keys_round_to_fp16_first():
    """Known answer: a key byte 0x39 (e4m3 1.125) with scale 1 + 2^-12.  The
    decode kernel multiplies the fp32 dot by the scale: 1.125 * (1 + 2^-12);
    the packed kernel rounds the dequantised key to fp16 first
    (sm70_mla_decode.cu:561-580): fp16_rn(1.12527...) = 1.125."""
    page = 4
    row = torch.zeros(132, dtype=torch.uint8)
    row[0] = 0x39
    row[128:132] = torch.tensor([1 + 2 ** -12], dtype=torch.float32).view(torch.uint8)
    assert float(O.e4m3_decode(row[:1])) == 1.125
    kc = row[None].repeat(page, 1).view(1, page, 132)
    q = torch.zeros(1, 32, 128, dtype=torch.float16)
    q[0, 0, 0] = 1
    w = torch.zeros(1, 32, dtype=torch.float16)
    w[0, 0] = 1
    bt = torch.zeros(1, 1, dtype=torch.int32)
    seq = torch.tensor([page], dtype=torch.int32)
    packed = O.indexer_logits_packed(O.pack_indexer_q(q), kc, w, bt, seq, page)
    dec, _ = O.indexer_logits(q, kc, w, bt, seq, page)
    assert torch.all(packed == 1.125)
    assert torch.all(dec == torch.tensor(1.125 * (1 + 2 ** -12), dtype=torch.float32))
