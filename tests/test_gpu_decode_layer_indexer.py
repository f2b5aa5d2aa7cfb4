"""GPU check of the fused decode-layer indexer launch
(mi355_dsa_decode_layer_indexer: the latent and indexer-K cache writes and
the indexer logits with the level-1 histogram in one launch) and of the
layer's top-k phase (mi355_dsa_decode_layer_topk: the top-k, leaving the
histogram zero, with q_latent run in its select launch).  Everything must equal,
bit for bit, the separate calls they replace: the cache writes
(concat_and_cache_mla, sm70_indexer_k_store), q_latent, sm70_indexer_logits
with a zeroed histogram, then sm70_decode_topk -- including the rows whose
new key is read in the same launch that writes it (the last position of
every row, and in speculative rows the earlier tokens of the request), a
skipped slot, and the histogram left zero on every top-k path.  The separate
calls are pinned against the oracle by their own tests."""
import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu

PAGE = 64
TOPK = 2048

CASES = [
    # B tokens, next_n, fp8 latent cache, fp8 indexer-K cache, context lengths of the requests
    (4, 1, True, False, [5000, 4100, 3000, 6100]),
    (4, 1, True, True, [5000, 4100, 3000, 6100]),
    (4, 2, False, False, [5000, 2600]),           # speculative rows read each other's keys
    (20, 1, True, True, [900 + 301 * r for r in range(20)]),  # short rows: select's early path
    (3, 1, False, True, [2000, 1500, 64]),        # max_kv = top-k: the whole-row kernel path
    # 20 x 27 = 540 logits workgroups: fp8 index keys staged as 16-row spans
    (20, 1, False, True, [26000 + 37 * r for r in range(20)]),
]


def _case(pkg, dev, case, seed):
    B, n, fp8, ik_fp8, lens = case
    m = pkg.dsa_layer
    ops = pkg._sm70_ops
    R = B // n
    g = torch.Generator().manual_seed(seed)
    H, P = 16, 128
    mb = (max(lens) + PAGE - 1) // PAGE
    nblk = R * mb + 3
    if fp8:
        lat = torch.randn(nblk * PAGE, 576, generator=g) / 24.0
        lat0 = O.dsmla_rows(lat).view(nblk, PAGE, 656).to(dev)
    else:  # drawn on the device: the large case's cache has 535k rows
        gd = torch.Generator(device=dev).manual_seed(seed)
        lat0 = (torch.randn(nblk * PAGE, 576, generator=gd, device=dev) / 24.0).to(
            torch.float16).view(nblk, PAGE, 576)
    keys = torch.randn(nblk * PAGE, 128, generator=g).to(torch.float16).to(dev)
    if ik_fp8:  # a quantised cache, written row by row with the store op
        ik0 = torch.zeros(nblk, PAGE, 132, dtype=torch.uint8, device=dev)
        ops.sm70_indexer_k_store(ik0, keys, torch.arange(nblk * PAGE, dtype=torch.int32,
                                                         device=dev))
    else:
        ik0 = keys.view(nblk, PAGE, 128).clone()
    perm = torch.randperm(nblk, generator=g)
    bt = torch.stack([perm[r * mb:(r + 1) * mb] for r in range(R)]).to(torch.int32)
    w = m.DsaLayerWeights(
        (torch.randn(H, P, 512, generator=g) / P ** 0.5).to(torch.float16).to(dev),
        (torch.randn(H, 512, 128, generator=g) / 24).to(torch.float16).to(dev), 0.05)
    q = (torch.randn(B, H, P + 64, generator=g) / 4).to(torch.float16).to(dev)
    idx_q = (torch.randn(B, 32, 128, generator=g) / 4).to(torch.float16).to(dev)
    idx_w = (torch.randn(B, 32, generator=g) / 6).to(torch.float16).to(dev)
    kv_c = (torch.randn(B, 512, generator=g) / 24).to(torch.float16).to(dev)
    k_pe = (torch.randn(B, 64, generator=g) / 24).to(torch.float16).to(dev)
    idx_k = torch.randn(B, 128, generator=g).to(torch.float16).to(dev)
    # token j of request r sits at position lens[r] - n + j of its request
    pos = [lens[r] - n + j for r in range(R) for j in range(n)]
    bt_tok = bt.repeat_interleave(n, dim=0)
    slot = torch.tensor([int(bt_tok[i][p // PAGE]) * PAGE + p % PAGE for i, p in enumerate(pos)],
                        dtype=torch.int32)
    if B > 4:
        slot[1] = -1  # skipped: row 1 reads its stale cache row in both paths
    sl = torch.tensor([p + 1 for p in pos], dtype=torch.int32)
    return (m, ops, w, lat0, ik0, q, idx_q, idx_w, kv_c, k_pe, idx_k, bt_tok.to(dev),
            sl.to(dev), slot.to(dev))


@pytest.mark.parametrize("case", CASES, ids=[f"B{c[0]}n{c[1]}-{'fp8' if c[2] else 'f16'}lat-"
                                             f"{'fp8' if c[3] else 'f16'}idx" for c in CASES])
def test_indexer_step_equals_separate_calls(pkg, dev, case):
    (m, ops, w, lat0, ik0, q, idx_q, idx_w, kv_c, k_pe, idx_k, bt, sl,
     slot) = _case(pkg, dev, case, seed=sum(case[4]) + case[0])
    B = q.shape[0]
    max_kv = bt.shape[1] * PAGE
    # separate calls
    L1 = m.DsaLayer(w, lat0.clone(), ik0.clone())
    L1.store(kv_c, k_pe, idx_k, slot)
    ql1 = m.q_latent(q, w)
    score1 = torch.empty(B, max_kv, device=dev)
    hist1 = torch.zeros(B, 4096, dtype=torch.int32, device=dev)
    ops.sm70_indexer_logits(score1, idx_q, L1.idx_k_cache, idx_w, bt, sl, hist1)
    idx1 = torch.empty(B, TOPK, dtype=torch.int32, device=dev)
    ops.sm70_decode_topk(idx1, score1, sl, hist1.clone(), TOPK)
    # fused, twice in a row (the second step sees the histogram the first left)
    L2 = m.DsaLayer(w, lat0.clone(), ik0.clone())
    assert L2._fusable(q, kv_c, k_pe, idx_k, slot) and L2._indexer_fusable(q, idx_q, idx_w)
    for _ in range(2):
        ql2, idx2 = L2._indexer_step(q, idx_q, idx_w, bt, sl, kv_c, k_pe, idx_k, slot)
        torch.cuda.synchronize()
        assert torch.equal(ql1.view(torch.int16), ql2.view(torch.int16))
        assert torch.equal(L1.latent_cache.view(torch.uint8), L2.latent_cache.view(torch.uint8))
        assert torch.equal(L1.idx_k_cache.view(torch.uint8), L2.idx_k_cache.view(torch.uint8))
        assert torch.equal(score1.view(torch.int32), L2.last_score.view(torch.int32))
        assert torch.equal(idx1, idx2)
        assert not L2._zero_hist(B, dev).any()


def test_indexer_step_histogram(pkg, lib, dev):
    """The fused launch's histogram (before the top-k consumes it) equals the
    standalone logits launch's."""
    import ctypes
    case = CASES[1]
    (m, ops, w, lat0, ik0, q, idx_q, idx_w, kv_c, k_pe, idx_k, bt, sl,
     slot) = _case(pkg, dev, case, seed=7)
    B = q.shape[0]
    max_kv = bt.shape[1] * PAGE
    L1 = m.DsaLayer(w, lat0.clone(), ik0.clone())
    L1.store(kv_c, k_pe, idx_k, slot)
    score1 = torch.empty(B, max_kv, device=dev)
    hist1 = torch.zeros(B, 4096, dtype=torch.int32, device=dev)
    ops.sm70_indexer_logits(score1, idx_q, L1.idx_k_cache, idx_w, bt, sl, hist1)
    lat, ikc = lat0.clone(), ik0.clone()
    score2 = torch.empty(B, max_kv, device=dev)
    hist2 = torch.zeros(B, 4096, dtype=torch.int32, device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    rc = lib.mi355_dsa_decode_layer_indexer(
        B, P(lat), 1, lat.numel() // 656, P(kv_c), kv_c.stride(0), P(k_pe), k_pe.stride(0), 0,
        P(slot), 0, P(ikc), 1, ikc.numel() // 132, P(idx_k), P(slot), P(score2), B, max_kv,
        P(idx_q), P(idx_w), PAGE, P(bt), bt.shape[1], P(sl), P(hist2),
        ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    assert rc == 0, lib.mi355_dsa_last_error()
    torch.cuda.synchronize()
    assert torch.equal(hist1, hist2)
    assert torch.equal(score1.view(torch.int32), score2.view(torch.int32))
    assert torch.equal(L1.idx_k_cache, ikc) and torch.equal(L1.latent_cache, lat)


def test_indexer_step_rejects_too_many_tokens(pkg, lib):
    """More than 64 new tokens are refused before any launch."""
    import ctypes
    one = ctypes.c_void_p(256)
    rc = lib.mi355_dsa_decode_layer_indexer(
        65, one, 1, 64 * 10, one, 512, one, 64, 0, one, 0, one, 0, 640, one, one, one, 65, 1024,
        one, one, 64, one, 16, one, one, None)
    assert rc != 0
    assert b"at most 64" in lib.mi355_dsa_last_error()


def test_layer_decode_graph_replays(pkg, dev):
    """DsaLayer.decode captured in a HIP graph and replayed, with eager work
    and synchronisations between replays: every replay gives the eager step's
    out and top-k rows bit for bit, and leaves the layer's histogram zero
    (the state the next replay's logits launch adds into)."""
    case = (4, 1, True, False, [5000, 4100, 3000, 6100])
    (m, ops, w, lat0, ik0, q, idx_q, idx_w, kv_c, k_pe, idx_k, bt, sl,
     slot) = _case(pkg, dev, case, seed=11)
    B = q.shape[0]
    L = m.DsaLayer(w, lat0.clone(), ik0.clone())
    args = (q, idx_q, idx_w, bt, sl, kv_c, k_pe, idx_k, slot)
    want = L.decode(*args).clone()
    want_idx = L.last_idx.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    res = {}
    with torch.cuda.stream(s):
        L.decode(*args)  # warm-up outside the capture
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            res["out"] = L.decode(*args)
            res["idx"] = L.last_idx
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(3):
        res["out"].fill_(0)
        res["idx"].fill_(-7)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(res["out"].view(torch.int16), want.view(torch.int16))
        assert torch.equal(res["idx"], want_idx)
        assert not L._zero_hist(B, dev).any()
