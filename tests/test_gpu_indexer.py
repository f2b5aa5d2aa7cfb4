"""GPU parity: indexer logits (decode and packed prefill) and the fused
histogram.  Dyadic inputs make every fp32 partial sum exact, so those cases
are bit-exact against the oracle; random inputs are compared within fp32
reassociation tolerance; the histogram is bit-exact given the kernel's own
scores."""
import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def make_case(seed, B, nblk, page, fp8, dyadic, max_kv, seq):
    g = torch.Generator().manual_seed(seed)
    if dyadic:
        k = (torch.randint(-8, 9, (nblk * page, 128), generator=g) / 8).to(torch.float16)
        q = (torch.randint(-8, 9, (B, 32, 128), generator=g) / 8).to(torch.float16)
        w = (torch.randint(-4, 5, (B, 32), generator=g) / 4).to(torch.float16)
    else:
        k = torch.randn(nblk * page, 128, generator=g).to(torch.float16)
        q = torch.randn(B, 32, 128, generator=g).to(torch.float16)
        w = (torch.randn(B, 32, generator=g) / 32 ** 0.5).to(torch.float16)
    if fp8:
        kc = O.indexer_k_store(torch.zeros(nblk, page, 132, dtype=torch.uint8), k,
                               torch.arange(nblk * page, dtype=torch.int32))
    else:
        kc = k.view(nblk, page, 128)
    mb = (max_kv + page - 1) // page
    bt = torch.stack([torch.randperm(nblk, generator=g)[:mb] for _ in range(B)]).to(torch.int32)
    seq = torch.tensor(seq, dtype=torch.int32)
    return q, kc, w, bt, seq


CASES = [
    # seed, B, nblk, page, fp8, dyadic, max_kv, seq_lens
    (0, 1, 40, 64, False, True, 2048, [2048]),
    (1, 3, 40, 64, False, True, 2500, [2500, 1, 1700]),
    (2, 4, 70, 16, False, False, 1100, [1100, 900, 1024, 0]),
    (3, 2, 40, 64, True, True, 2048, [2000, 2048]),
    (4, 2, 40, 64, True, False, 2560, [2560, 77]),
    (5, 9, 20, 64, False, False, 1280, [1280] * 9),   # B >= 8 (reference WMMA branch)
    # fp8 rows in 16-row pages (the staged 16-key spans) and in 8-row pages
    # (per-key loads)
    (6, 2, 130, 16, True, False, 2048, [2048, 1500]),
    (7, 2, 300, 8, True, False, 2400, [2400, 1999]),
]


@pytest.mark.parametrize("case", CASES, ids=[f"seed{c[0]}" for c in CASES])
def test_logits_and_hist(ops, dev, case):
    seed, B, nblk, page, fp8, dyadic, max_kv, seq = case
    q, kc, w, bt, seq = make_case(seed, B, nblk, page, fp8, dyadic, max_kv, seq)
    score = torch.full((B, max_kv), 7.0, device=dev)
    hist = torch.zeros(B, 4096, dtype=torch.int32, device=dev)
    ops.sm70_indexer_logits(score, q.to(dev), kc.to(dev), w.to(dev), bt.to(dev), seq.to(dev), hist)
    got = score.cpu()
    want, _ = O.indexer_logits(q, kc, w, bt, seq, max_kv)
    assert torch.equal(torch.isinf(got), torch.isinf(want))
    fin = torch.isfinite(want)
    if dyadic and not fp8:
        assert torch.equal(got[fin], want[fin])
    else:
        tol = 1e-5 * want[fin].abs().max().item() + 1e-6
        assert (got[fin] - want[fin]).abs().max().item() <= tol
    # histogram == bincount of the kernel's own scores over p < seq_len
    for b in range(B):
        L = min(int(seq[b]), max_kv)
        ref = torch.bincount((O.mono_key(got[b, :L]) >> 20).long(), minlength=4096)
        assert torch.equal(hist[b].cpu().long(), ref)


@pytest.mark.parametrize("offset", [0, 1], ids=["aligned", "word-offset"])
def test_hist_flush_alignment(ops, dev, offset):
    """The histogram flush adds two adjacent bins per 64-bit atomic when the
    hist rows are 8-byte aligned, one bin per atomic otherwise (a hist view
    one int32 into its buffer); both give the exact bincount."""
    q, kc, w, bt, seq = make_case(12, 4, 140, 64, False, False, 8192, [8192, 8000, 5000, 8191])
    buf = torch.full((4 * 4096 + offset,), 0, dtype=torch.int32, device=dev)
    hist = buf[offset:].view(4, 4096)
    assert (hist.data_ptr() % 8 == 0) == (offset == 0)
    score = torch.empty(4, 8192, device=dev)
    ops.sm70_indexer_logits(score, q.to(dev), kc.to(dev), w.to(dev), bt.to(dev), seq.to(dev), hist)
    got = score.cpu()
    for b in range(4):
        ref = torch.bincount((O.mono_key(got[b, :int(seq[b])]) >> 20).long(), minlength=4096)
        assert torch.equal(hist[b].cpu().long(), ref)
    assert int(hist.sum()) == int(seq.sum())


@pytest.mark.parametrize("fp8", [False, True], ids=["fp16", "fp8"])
def test_unmapped_pages_in_full_workgroups(ops, dev, fp8):
    """Block-table entries that are -1 or point past the cache, inside
    workgroups that lie wholly in the row (the branch-free path) and in the
    row's last one: those positions score 0 below seq_len, -inf above."""
    q, kc, w, bt, _ = make_case(11, 3, 60, 64, fp8, True, 3500, [3500] * 3)
    bt[0, 3] = -1            # positions 192..255 of row 0
    bt[1, 20] = 60 + 5       # past the 60-page cache: positions 1280..1343 of row 1
    bt[2, 54] = -1           # in the row's last (partial) workgroup
    seq = torch.tensor([3500, 3000, 3490], dtype=torch.int32)
    score = torch.full((3, 3500), 7.0, device=dev)
    hist = torch.zeros(3, 4096, dtype=torch.int32, device=dev)
    ops.sm70_indexer_logits(score, q.to(dev), kc.to(dev), w.to(dev), bt.to(dev), seq.to(dev), hist)
    got = score.cpu()
    want, _ = O.indexer_logits(q, kc, w, bt, seq, 3500)
    assert torch.equal(got[0, 192:256], torch.zeros(64)) and torch.equal(got[1, 1280:1344], torch.zeros(64))
    assert torch.equal(torch.isinf(got), torch.isinf(want))
    fin = torch.isfinite(want)
    if fp8:
        tol = 1e-5 * want[fin].abs().max().item() + 1e-6
        assert (got[fin] - want[fin]).abs().max().item() <= tol
    else:
        assert torch.equal(got[fin], want[fin])
    for b in range(3):  # histogram == bincount of the kernel's own scores over p < seq_len
        ref = torch.bincount((O.mono_key(got[b, :int(seq[b])]) >> 20).long(), minlength=4096)
        assert torch.equal(hist[b].cpu().long(), ref)


@pytest.mark.parametrize("page", [64, 16])
def test_fp8_span_and_per_key_loads_agree(ops, dev, page):
    """fp8 rows in a launch of >= 512 workgroups: workgroups inside the row
    stage each 16-key block's 16 consecutive rows (2112 bytes) through LDS
    when the cache is 16-byte aligned; a cache view 4 bytes into its buffer
    takes the per-key loads (pinned against the oracle by the cases above).
    Same scores and histogram bit for bit, unmapped pages included."""
    B, max_kv = 4, 131072  # 4 x 128 workgroups
    nblk = max_kv // page + 5
    q, kc, w, bt, _ = make_case(13 + page, B, nblk, page, True, False, max_kv, [max_kv] * B)
    bt[0, 5] = -1
    bt[2, 100] = nblk + 7
    seq = torch.tensor([131072, 131000, 70000, 1000], dtype=torch.int32)
    buf = torch.zeros(kc.numel() + 16, dtype=torch.uint8, device=dev)
    outs = []
    for off in (0, 4):
        kv = buf[off:off + kc.numel()].view(nblk, page, 132)
        kv.copy_(kc.to(dev))
        assert (kv.data_ptr() % 16 == 0) == (off == 0)
        score = torch.empty(B, max_kv, device=dev)
        hist = torch.zeros(B, 4096, dtype=torch.int32, device=dev)
        ops.sm70_indexer_logits(score, q.to(dev), kv, w.to(dev), bt.to(dev), seq.to(dev), hist)
        outs.append((score.cpu(), hist.cpu()))
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])
    got = outs[0][0]
    assert torch.equal(got[0, 5 * page:6 * page], torch.zeros(page))
    assert torch.equal(got[2, 100 * page:101 * page], torch.zeros(page))
    for b in range(B):
        L = int(seq[b])
        assert torch.isfinite(got[b, :L]).all() and torch.isinf(got[b, L:]).all()
        ref = torch.bincount((O.mono_key(got[b, :L]) >> 20).long(), minlength=4096)
        assert torch.equal(outs[0][1][b].long(), ref)


def test_duplicate_keys_score_identically(ops, dev):
    g = torch.Generator().manual_seed(11)
    page, nblk = 64, 32
    k = torch.randn(nblk * page, 128, generator=g).to(torch.float16)
    perm = torch.randperm(nblk * page, generator=g)
    src, dst = perm[:300], perm[300:600]  # disjoint: every copy is exact
    k[dst] = k[src]
    q = torch.randn(1, 32, 128, generator=g).to(torch.float16)
    w = torch.randn(1, 32, generator=g).to(torch.float16)
    bt = torch.arange(nblk, dtype=torch.int32)[None]
    seq = torch.tensor([nblk * page], dtype=torch.int32)
    score = torch.empty(1, nblk * page, device=dev)
    ops.sm70_indexer_logits(score, q.to(dev), k.view(nblk, page, 128).to(dev), w.to(dev),
                            bt.to(dev), seq.to(dev), None)
    s = score.cpu()[0]
    assert torch.equal(s[dst], s[src])


PACKED = [
    # seed, B, nblk, page, fp8, dyadic, max_kv, causal
    (0, 16, 20, 64, False, True, 1024, True),
    (1, 37, 20, 64, False, True, 1280, True),
    (2, 130, 40, 64, False, False, 2560, True),
    (3, 64, 20, 64, True, False, 1024, False),
    (4, 5, 10, 16, False, False, 160, True),
]


@pytest.mark.parametrize("case", PACKED, ids=[f"p{c[0]}" for c in PACKED])
def test_packed_logits(ops, dev, case):
    seed, B, nblk, page, fp8, dyadic, max_kv, causal = case
    base = max_kv - B
    seq = [base + i + 1 for i in range(B)] if causal else [max_kv] * B
    q, kc, w, bt1, seq = make_case(seed, 1, nblk, page, fp8, dyadic, max_kv, seq[:1])
    g = torch.Generator().manual_seed(seed + 100)
    if dyadic:
        q = (torch.randint(-8, 9, (B, 32, 128), generator=g) / 8).to(torch.float16)
        w = (torch.randint(-4, 5, (B, 32), generator=g) / 4).to(torch.float16)
    else:
        q = torch.randn(B, 32, 128, generator=g).to(torch.float16)
        w = (torch.randn(B, 32, generator=g) / 32 ** 0.5).to(torch.float16)
    seqs = torch.tensor([base + i + 1 for i in range(B)] if causal else [max_kv] * B,
                        dtype=torch.int32)
    bt = bt1.expand(B, bt1.shape[1]).contiguous()  # one request row, expanded
    qp = O.pack_indexer_q(q)
    score = torch.full((B, max_kv), 7.0, device=dev)
    ops.sm70_indexer_logits_packed(score, qp.to(dev), kc.to(dev), w.to(dev), bt.to(dev),
                                   seqs.to(dev))
    got = score.cpu()
    want = O.indexer_logits_packed(qp, kc, w, bt, seqs, max_kv)
    assert torch.equal(torch.isinf(got), torch.isinf(want))
    fin = torch.isfinite(want)
    if dyadic:
        assert torch.equal(got[fin], want[fin])
    else:
        tol = 1e-5 * want[fin].abs().max().item() + 1e-6
        assert (got[fin] - want[fin]).abs().max().item() <= tol


def test_packed_matches_decode_kernel_on_dyadic(ops, dev):
    """Both kernels compute exactly the same scores on exact inputs."""
    B, nblk, page, max_kv = 24, 20, 64, 1280
    q, kc, w, bt1, _ = make_case(21, 1, nblk, page, False, True, max_kv, [max_kv])
    g = torch.Generator().manual_seed(22)
    q = (torch.randint(-8, 9, (B, 32, 128), generator=g) / 8).to(torch.float16)
    w = (torch.randint(-4, 5, (B, 32), generator=g) / 4).to(torch.float16)
    bt = bt1.expand(B, bt1.shape[1]).contiguous().to(dev)
    seq = torch.arange(max_kv - B + 1, max_kv + 1, dtype=torch.int32, device=dev)
    a = torch.empty(B, max_kv, device=dev)
    b = torch.empty(B, max_kv, device=dev)
    ops.sm70_indexer_logits(a, q.to(dev), kc.to(dev), w.to(dev), bt, seq, None)
    ops.sm70_indexer_logits_packed(b, O.pack_indexer_q(q).to(dev), kc.to(dev), w.to(dev), bt, seq)
    assert torch.equal(a, b)


# Launch shapes of the packed kernel's tile split (full tiles are 64 queries
# x 256 keys; W = tiles per launch): all full (W = 200); more than one round
# (W = 260, 280 with a partial last query tile, and fp8 keys), which takes
# the four-wave 32-query kernel, its last round as 16-query quarter tiles when
# that round holds at most 256 of its workgroups (W = 260, 280, 384; W = 400
# keeps a full last round); launches of at most 64 tiles as 16-query pieces
# with the 32 heads split over two wave groups, and of 65-128 tiles as half
# tiles.
SPLIT = [
    # seed, B, max_kv, fp8
    (31, 128, 256 * 100, False),
    (32, 128, 256 * 130, False),
    (33, 100, 256 * 140, False),
    (34, 128, 256 * 130, True),
    # more full tiles: the four-wave 32-query kernel as well
    (35, 128, 256 * 200, False),
    (36, 100, 256 * 200, True),      # a partial 32-query tile
    (37, 1000, 256 * 24, False),
    # <= 64 full tiles: head-split 16-query pieces, one per CU
    (38, 128, 256 * 30, False),
    (39, 37, 256 * 20, False),       # a partial 16-query tile
    (40, 64, 256 * 50, True),
    (43, 20, 256 * 3, False),        # two pieces per key tile, the second partial
    # 65-128 full tiles: every tile as two halves
    (41, 128, 256 * 50, False),
    (42, 96, 256 * 40, True),        # fp8 keys, a partial query tile
]


@pytest.mark.parametrize("case", SPLIT, ids=[f"B{c[1]}_kv{c[2]}_{'fp8' if c[3] else 'f16'}"
                                             for c in SPLIT])
def test_packed_tile_split(ops, dev, case):
    """Dyadic inputs: the packed kernel equals the decode kernel bit for bit
    (fp16 keys) on every row, and the oracle on sampled rows, whatever mix of
    full and half tiles the launch uses."""
    seed, B, max_kv, fp8 = case
    page = 64
    nblk = max_kv // page + 3
    q, kc, w, bt1, _ = make_case(seed, 1, nblk, page, fp8, True, max_kv, [max_kv])
    g = torch.Generator().manual_seed(seed + 7)
    q = (torch.randint(-8, 9, (B, 32, 128), generator=g) / 8).to(torch.float16)
    w = (torch.randint(-4, 5, (B, 32), generator=g) / 4).to(torch.float16)
    bt = bt1.expand(B, bt1.shape[1]).contiguous()
    seq = torch.arange(max_kv - B + 1, max_kv + 1, dtype=torch.int32)
    b = torch.full((B, max_kv), 7.0, device=dev)
    ops.sm70_indexer_logits_packed(b, O.pack_indexer_q(q).to(dev), kc.to(dev), w.to(dev),
                                   bt.to(dev), seq.to(dev))
    got = b.cpu()
    rows = sorted({r for r in (0, 15, 16, 31, 32, 63, 64, B - 1) if r < B})
    if fp8:
        flat = kc.view(-1, 132)
        k16 = (O.e4m3_decode(flat[:, :128].contiguous()) *
               flat[:, 128:].contiguous().view(torch.float32)).to(torch.float16)
        kc_ref = k16.view(nblk, page, 128)
    else:
        kc_ref = kc
        a = torch.full((B, max_kv), 7.0, device=dev)
        ops.sm70_indexer_logits(a, q.to(dev), kc.to(dev), w.to(dev), bt.to(dev), seq.to(dev),
                                None)
        assert torch.equal(a.cpu(), got)
    want, _ = O.indexer_logits(q[rows], kc_ref, w[rows], bt[rows], seq[rows], max_kv)
    sub = got[rows]
    assert torch.equal(torch.isinf(sub), torch.isinf(want))
    fin = torch.isfinite(want)
    if fp8:
        tol = 1e-5 * want[fin].abs().max().item() + 1e-6
        assert (sub[fin] - want[fin]).abs().max().item() <= tol
    else:
        assert torch.equal(sub[fin], want[fin])


def test_decode_c2_full_size(ops, pkg, dev):
    """Config C2 (B=4, 64k keys, ~1% duplicated keys) against an fp32 torch
    computation on the GPU (gather + matmul + relu*w), then top-k bit-exact
    against the C oracle on the kernel's own scores."""
    from oracle import cref

    d = pkg.synthetic.indexer_decode_inputs(device=dev)
    B, max_kv = 4, d["max_kv"]
    score = torch.empty(B, max_kv, device=dev)
    hist = torch.zeros(B, 4096, dtype=torch.int32, device=dev)
    ops.sm70_indexer_logits(score, d["q"], d["kc"], d["w"], d["bt"], d["seq"], hist)
    page = 64
    pos = torch.arange(max_kv, device=dev)
    rows = (d["bt"].long()[:, pos // page] * page + pos % page)  # [B, max_kv]
    K = d["k"].float()[rows]  # [B, max_kv, 128]
    dots = torch.bmm(d["q"].float(), K.transpose(1, 2).contiguous())  # [B, 32, max_kv]
    ref = (torch.relu(dots) * d["w"].float()[:, :, None]).sum(1)
    err = (score - ref).abs().max().item()
    assert err <= 1e-5 * ref.abs().max().item(), err
    idx = torch.empty(B, 2048, dtype=torch.int32, device=dev)
    ops.sm70_decode_topk(idx, score, d["seq"], hist, 2048)
    want = cref.topk_rows(score.cpu(), d["seq"].cpu(), 2048)
    assert torch.equal(idx.cpu(), want)
