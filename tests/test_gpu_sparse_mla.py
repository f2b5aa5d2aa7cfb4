"""GPU parity: sparse MLA attention (decode split/merge configuration and the
64-head prefill configuration), fp16 and fp8_ds_mla caches.

Tolerances: o within 2e-3 relative / 1e-3 absolute
(fp16), lse within 1e-4 absolute, against the fp64 oracle on the same
seeded inputs."""
import math

import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu

SCALE = 576 ** -0.5
RTOL, ATOL, LSE_ATOL = 2e-3, 1e-3, 1e-4


def make(seed, B, H, nblk, page, fp8, topk, seqs, invalid_frac=0.0, shared_bt=False):
    g = torch.Generator().manual_seed(seed)
    lat = torch.randn(nblk * page, 576, generator=g) / 24.0
    kv = (O.dsmla_rows(lat).view(nblk, page, 656) if fp8
          else lat.to(torch.float16).view(nblk, page, 576))
    mb = max((max(seqs) + page - 1) // page, 1)
    if shared_bt:
        bt = torch.randperm(nblk, generator=g)[:mb].expand(B, mb).to(torch.int32).contiguous()
    else:
        bt = torch.stack([torch.randperm(nblk, generator=g)[:mb] for _ in range(B)]).to(torch.int32)
    seq = torch.tensor(seqs, dtype=torch.int32)
    q = (torch.randn(B, H, 576, generator=g) / 24.0 * 6).to(torch.float16)
    idx = torch.full((B, topk), -1, dtype=torch.int32)
    for b in range(B):
        L = int(seq[b])
        n = min(L, topk)
        if n > 0:
            sel = torch.randperm(L, generator=g)[:n].sort().values
            idx[b, :n] = sel.to(torch.int32)
    if invalid_frac:
        m = torch.rand(B, topk, generator=g) < invalid_frac
        idx[m] = -1
        idx[torch.rand(B, topk, generator=g) < invalid_frac] = 10 ** 8  # >= seq_len
    return q, kv, idx, bt, seq


def run(ops, dev, q, kv, idx, bt, seq):
    B, H = q.shape[:2]
    o = torch.full((B, H, 512), float("nan"), dtype=torch.float16, device=dev)
    lse = torch.full((B, H), float("nan"), device=dev)
    ops.sm70_sparse_mla_decode(o, lse, q.to(dev), kv.to(dev), idx.to(dev), bt.to(dev),
                               seq.to(dev), SCALE)
    return o.float().cpu(), lse.cpu()


def check(o, lse, ro, rl):
    assert torch.equal(torch.isinf(lse), torch.isinf(rl))
    fin = torch.isfinite(rl)
    assert (lse[fin] - rl[fin]).abs().max().item() <= LSE_ATOL if fin.any() else True
    torch.testing.assert_close(o, ro, rtol=RTOL, atol=ATOL)


DECODE = [
    # seed, B, H, nblk, page, fp8, topk, seqs
    (0, 1, 64, 40, 64, False, 2048, [2500]),
    (1, 4, 64, 40, 64, True, 2048, [2500, 2048, 700, 1]),
    (2, 2, 16, 30, 64, True, 512, [1900, 30]),
    (3, 3, 8, 20, 16, False, 256, [300, 200, 17]),   # partial head tile
    (4, 4, 64, 60, 64, True, 2048, [3800, 3800, 3800, 3800]),
    (5, 1, 128, 40, 64, False, 1024, [2400]),         # two 64-head groups
    (6, 2, 16, 30, 48, True, 512, [1400, 500]),      # page size not a power of two
    # fp8 split decode with the merge numbered onto each token's XCDs: 8 / B
    # XCDs per token (B = 1: 8, B = 8: 1), and B = 3, which takes plain order
    (7, 1, 64, 40, 64, True, 2048, [2500]),
    (8, 8, 16, 40, 64, True, 512, [2000, 1500, 700, 512, 90, 2400, 1, 1800]),
    (9, 1, 16, 30, 64, True, 1024, [1500]),
    (11, 3, 64, 40, 64, True, 2048, [2500, 2100, 900]),
]


@pytest.mark.parametrize("case", DECODE, ids=[f"d{c[0]}" for c in DECODE])
def test_decode(ops, dev, case):
    seed, B, H, nblk, page, fp8, topk, seqs = case
    q, kv, idx, bt, seq = make(seed, B, H, nblk, page, fp8, topk, seqs)
    o, lse = run(ops, dev, q, kv, idx, bt, seq)
    ro, rl = O.sparse_mla(q, kv, idx, bt, seq, SCALE)
    check(o, lse, ro, rl)


def test_decode_invalid_entries(ops, dev):
    q, kv, idx, bt, seq = make(10, 3, 64, 40, 64, True, 2048, [2500, 1000, 2048],
                               invalid_frac=0.3)
    idx[2] = -1  # a token with no valid key: o = 0, lse = -inf
    o, lse = run(ops, dev, q, kv, idx, bt, seq)
    ro, rl = O.sparse_mla(q, kv, idx, bt, seq, SCALE)
    check(o, lse, ro, rl)
    assert torch.all(o[2] == 0) and torch.all(torch.isinf(lse[2]))


UNRESOLVED = [
    # B, H, fp8, topk: kernel path -> rule for a position below seq_len on a bad block
    (4, 64, True, 2048),    # fp8 split decode (LDS-DMA kernel): zero key
    (2, 64, False, 1024),   # fp16 split decode (register-staged kernel): zero key
    (16, 64, True, 2048),   # fp8 pipelined kernel with 16 key splits: zero key
    (16, 64, False, 2048),  # fp16 pipelined kernel with 16 key splits: zero key
    (300, 64, True, 256),   # fp8 prefill configuration: zero key (64 heads)
    (300, 64, False, 256),  # fp16 prefill configuration: zero key
    (40, 16, True, 256),    # B >= 32, H <= 16 (the reference's prefill kernel): masked
    (300, 16, False, 256),  # same rule in the prefill configuration: masked
]


def make_unresolved(seed, B, H, fp8, topk, nblk=40, page=64, seq_len=2500):
    """Half of every token's selected positions lie on pages whose table
    entry is -1 or names a block past the cache (pages 3 and 7), the other
    half on good pages; latent values are O(1) so that the zero-key and
    masking rules give clearly different outputs."""
    g = torch.Generator().manual_seed(seed)
    lat = torch.randn(nblk * page, 576, generator=g)
    kv = (O.dsmla_rows(lat).view(nblk, page, 656) if fp8
          else lat.to(torch.float16).view(nblk, page, 576))
    mb = (seq_len + page - 1) // page
    bt = torch.stack([torch.randperm(nblk, generator=g)[:mb] for _ in range(B)]).to(torch.int32)
    bt[:, 3] = -1
    bt[:, 7] = nblk + 5
    bad = torch.cat([torch.arange(3 * page, 4 * page), torch.arange(7 * page, 8 * page)])
    good = torch.tensor([p for p in range(seq_len) if p // page not in (3, 7)])
    idx = torch.empty(B, topk, dtype=torch.int32)
    for b in range(B):
        nb = min(topk // 2, bad.numel())
        sel = torch.cat([bad[torch.randperm(bad.numel(), generator=g)[:nb]],
                         good[torch.randperm(good.numel(), generator=g)[:topk - nb]]])
        idx[b] = sel.sort().values.to(torch.int32)
    q = (torch.randn(B, H, 576, generator=g) * 0.05).to(torch.float16)
    seq = torch.full((B,), seq_len, dtype=torch.int32)
    return q, kv, idx, bt, seq


@pytest.mark.parametrize("case", UNRESOLVED, ids=[f"B{c[0]}H{c[1]}{'fp8' if c[2] else 'fp16'}"
                                                 for c in UNRESOLVED])
def test_unresolved_rows_follow_reference_dispatch(ops, dev, case):
    """Selected positions below seq_len whose block-table entry is -1 or
    names a block past the cache: zero keys with score 0 on the reference's
    split-decode shapes, masked on its prefill-kernel shapes (B >= 32 and
    H <= 16), as the oracle states.  The other rule's answer is checked to
    be far outside the tolerance, so the test separates the two."""
    B, H, fp8, topk = case
    q, kv, idx, bt, seq = make_unresolved(70 + B + H, B, H, fp8, topk)
    o, lse = run(ops, dev, q, kv, idx, bt, seq)
    ro, rl = O.sparse_mla(q, kv, idx, bt, seq, SCALE)
    check(o, lse, ro, rl)
    zero = not (B >= 32 and H <= 16)
    _, alt_lse = O.sparse_mla(q[:2], kv, idx[:2], bt[:2], seq[:2], SCALE, zero_unresolved=not zero)
    assert (lse[:2] - alt_lse).abs().min().item() > 100 * LSE_ATOL


@pytest.mark.parametrize("B,H,expect", [(40, 16, -1e30), (300, 16, -1e30), (40, 64, -math.inf),
                                         (31, 16, -math.inf)])
def test_empty_token_lse_convention(ops, dev, B, H, expect):
    """A token with no valid key gets o = 0 and the reference's lse: -1e30
    where the reference runs its prefill kernel (B >= 32, H <= 16), -inf on
    its split-decode path."""
    seqs = [90 + (i % 7) for i in range(B)]
    q, kv, idx, bt, seq = make(30 + B + H, B, H, 12, 16, True, 64, seqs)
    idx[3] = -1
    o, lse = run(ops, dev, q, kv, idx, bt, seq)
    ro, rl = O.sparse_mla(q, kv, idx, bt, seq, SCALE)
    check(o, lse, ro, rl)
    assert torch.all(o[3] == 0)
    assert torch.all(lse[3] == expect) and torch.all(rl[3] == expect)


@pytest.mark.parametrize("fp8", [True, False], ids=["fp8", "fp16"])
def test_prefill_config(ops, dev, fp8):
    """B >= 256 tokens takes the 64-head prefill configuration."""
    B = 300
    seqs = [1800 + 3 * i for i in range(B)]
    q, kv, idx, bt, seq = make(20, B, 64, 60, 64, fp8, 2048, seqs, shared_bt=True)
    o, lse = run(ops, dev, q, kv, idx, bt, seq)
    ro, rl = O.sparse_mla(q, kv, idx, bt, seq, SCALE)
    check(o, lse, ro, rl)


@pytest.mark.parametrize("fp8", [True, False], ids=["fp8", "fp16"])
def test_prefill_config_segments_partial_heads(ops, dev, fp8):
    """Prefill configuration with a partial second 64-head group (H = 80),
    top-k past one 2048-key segment, and invalid / out-of-range entries."""
    B = 128
    seqs = [2600 + 5 * i for i in range(B)]
    q, kv, idx, bt, seq = make(22, B, 80, 60, 64, fp8, 2304, seqs, invalid_frac=0.05,
                               shared_bt=True)
    o, lse = run(ops, dev, q, kv, idx, bt, seq)
    ro, rl = O.sparse_mla(q, kv, idx, bt, seq, SCALE)
    check(o, lse, ro, rl)


PIPE_SPLIT = [
    # seed, B, H, fp8, topk, seqs: batches of 8..255 tokens at > 32 heads run the
    # 64-head pipelined kernels with round(256 / (B * ceil(H / 64))) key splits
    # (at least two 32-key tiles each), then the merge
    (40, 16, 64, True, 2048, [3000 - 37 * i for i in range(15)] + [1]),   # 16 splits
    (41, 16, 64, False, 2048, [3000 - 37 * i for i in range(15)] + [100]),
    (42, 10, 80, True, 2304, [2900 - 11 * i for i in range(10)]),  # 13 splits, last one empty
    (43, 10, 80, False, 2304, [2900 - 11 * i for i in range(10)]),
    (44, 64, 64, True, 1024, [1500 + 7 * i for i in range(64)]),   # 4 splits
    (45, 8, 64, False, 200, [150, 200, 260, 20, 199, 201, 64, 3]),  # 32 -> 4 splits, short lists
]


@pytest.mark.parametrize("case", PIPE_SPLIT, ids=[f"B{c[1]}H{c[2]}{'fp8' if c[3] else 'fp16'}"
                                                  for c in PIPE_SPLIT])
def test_decode_pipelined_key_split(ops, dev, case):
    """The pipelined kernels with a key split and the merge, against the
    oracle: ragged top-k lists (-1 padding, splits with no valid key, one
    split past the list's end), a partial second 64-head group, invalid
    entries, and one token with no valid key (o = 0, lse = -inf)."""
    seed, B, H, fp8, topk, seqs = case
    q, kv, idx, bt, seq = make(seed, B, H, 60, 64, fp8, topk, seqs, invalid_frac=0.03)
    idx[B // 2] = -1
    o, lse = run(ops, dev, q, kv, idx, bt, seq)
    ro, rl = O.sparse_mla(q, kv, idx, bt, seq, SCALE)
    check(o, lse, ro, rl)
    assert torch.all(o[B // 2] == 0) and torch.all(torch.isinf(lse[B // 2]))


PREFILL_SEG = [
    # seed, B, H, topk, page, seqs: the fp8 prefill configuration (B * ceil(H / 64) >=
    # 256, one key split)
    # lists longer than one 2048-key segment, so one workgroup runs its tile
    # pipeline twice (the second segment 5 and 2 tiles long)
    (50, 256, 64, 2200, 64, [2600 - 3 * i for i in range(256)]),
    (51, 260, 32, 2100, 64, [2500 - (i % 7) * 60 for i in range(260)]),  # 32 of 64 heads
    # short lists: two tiles, the second ragged; tokens with fewer keys than the list
    (52, 256, 64, 40, 64, [1 + (i * 7) % 90 for i in range(256)]),
    # two 64-head groups per token, a page size that is not a power of two
    (53, 200, 128, 96, 48, [50 + (i * 13) % 700 for i in range(200)]),
    # workgroups of 4-5 consecutive tokens (one tile stream across them)
    (54, 1100, 64, 96, 64, [30 + (i * 37) % 900 for i in range(1100)]),
    # one tile per token: every tile starts and ends a token
    (55, 700, 64, 20, 16, [1 + (i * 11) % 300 for i in range(700)]),
]


@pytest.mark.parametrize("case", PREFILL_SEG, ids=[f"B{c[1]}H{c[2]}k{c[3]}" for c in PREFILL_SEG])
def test_prefill_two_segments(ops, dev, case):
    """fp8 prefill configuration, against the oracle: more than 2048 keys per
    token, short ragged lists, two head groups, ragged pages, invalid
    entries."""
    seed, B, H, topk, page, seqs = case
    q, kv, idx, bt, seq = make(seed, B, H, 60, page, True, topk, seqs, invalid_frac=0.03)
    o, lse = run(ops, dev, q, kv, idx, bt, seq)
    ro, rl = O.sparse_mla(q, kv, idx, bt, seq, SCALE)
    check(o, lse, ro, rl)


def test_prefill_equals_decode_config(ops, dev):
    """Split-count / configuration invariance: the first rows of a 256-token
    batch (prefill configuration) equal the same rows run alone (decode
    configuration with splits and merge) within rounding."""
    B = 256
    q, kv, idx, bt, seq = make(21, B, 64, 40, 64, False, 2048, [2300] * B, shared_bt=True)
    o_all, l_all = run(ops, dev, q, kv, idx, bt, seq)
    o_4, l_4 = run(ops, dev, q[:4], kv, idx[:4], bt[:4], seq[:4])
    torch.testing.assert_close(o_all[:4], o_4, rtol=RTOL, atol=ATOL)
    assert (l_all[:4] - l_4).abs().max() <= LSE_ATOL


def test_closed_forms(ops, dev):
    g = torch.Generator().manual_seed(30)
    nblk, page = 8, 64
    lat = torch.randn(nblk * page, 576, generator=g) / 24.0
    kv = lat.to(torch.float16).view(nblk, page, 576)
    bt = torch.arange(nblk, dtype=torch.int32)[None].repeat(2, 1)
    seq = torch.tensor([500, 500], dtype=torch.int32)
    q = torch.randn(2, 64, 576, generator=g).to(torch.float16)
    idx = torch.full((2, 2048), -1, dtype=torch.int32)
    idx[0, 1000] = 123          # single key: o = V, lse = s
    q[1] = 0                    # equal scores: o = mean V, lse = ln n
    idx[1, :10] = torch.arange(10, 20, dtype=torch.int32)
    o, lse = run(ops, dev, q, kv, idx, bt, seq)
    V = kv.view(-1, 576).float()
    torch.testing.assert_close(o[0], V[123, :512].expand(64, 512), rtol=1e-3, atol=1e-3)
    qs = O.scaled_q(q[:1], SCALE)[0].float()
    assert (lse[0] - qs @ V[123]).abs().max() <= LSE_ATOL
    torch.testing.assert_close(o[1], V[10:20, :512].mean(0).expand(64, 512), rtol=1e-3, atol=1e-3)
    assert (lse[1] - math.log(10)).abs().max() <= LSE_ATOL


def test_sparse_equals_dense_below_topk(ops, dev):
    """DSA invariant (reference/triton_mla.py:225-233): with seq_len <= topk
    every position is selected and sparse attention equals dense attention."""
    q, kv, idx, bt, seq = make(31, 2, 64, 40, 64, True, 2048, [1500, 2048])
    o, lse = run(ops, dev, q, kv, idx, bt, seq)
    ro, rl = O.dense_mla(q, kv, bt, seq, SCALE)
    check(o, lse, ro, rl)


def test_c3_full_size(ops, pkg, dev):
    """Config C3: B=4, 180k context, 64 heads, topk 2048, fp8_ds_mla cache of
    11,520 pages; the oracle runs on just the selected rows."""
    d = pkg.synthetic.decode_inputs(device=dev)
    B, H = d["q"].shape[:2]
    o = torch.empty(B, H, 512, dtype=torch.float16, device=dev)
    lse = torch.empty(B, H, device=dev)
    ops.sm70_sparse_mla_decode(o, lse, d["q"], d["kv"], d["idx"], d["bt"], d["seq"], d["scale"])
    # compact cache with only the selected rows, in idx order
    page = d["kv"].shape[1]
    pos = d["idx"].long()
    rows = d["bt"].long().gather(1, pos // page) * page + pos % page
    sel = d["kv"].view(-1, 656)[rows.reshape(-1)].cpu()
    n = sel.shape[0]
    kv_c = sel.view(n // 64, 64, 656)
    topk = pos.shape[1]
    idx_c = torch.arange(B * topk, dtype=torch.int32).view(B, topk)
    bt_c = torch.arange(n // 64, dtype=torch.int32)[None].repeat(B, 1)
    seq_c = torch.full((B,), n, dtype=torch.int32)
    ro, rl = O.sparse_mla(d["q"].cpu(), kv_c, idx_c, bt_c, seq_c, d["scale"])
    check(o.float().cpu(), lse.cpu(), ro, rl)
