"""GPU check of the fused decode-layer prologue (mi355_dsa_decode_layer_prologue):
its four outputs -- q_latent, the latent-cache rows, the indexer-K rows and
the cleared histogram -- must equal, bit for bit, those of the four separate
calls it replaces (mi355_dsa_head_proj, concat_and_cache_mla,
sm70_indexer_k_store, a zero fill), across cache formats, input dtypes, slot
widths, skipped slots and token counts that span several workgroups of each
piece.  The separate ops are pinned against the oracle by their own tests."""
import pytest
import torch

pytestmark = pytest.mark.gpu

PAGE = 64

CASES = [
    # T, H, P, latent cache, kv dtype, indexer cache, slot dtype
    (4, 64, 128, "fp8_ds_mla", torch.float16, "fp16", torch.int32),
    (4, 64, 128, "fp8_ds_mla", torch.bfloat16, "fp8", torch.int64),
    (37, 16, 128, "auto", torch.float16, "fp16", torch.int64),
    (37, 16, 256, "fp8_ds_mla", torch.float16, "fp8", torch.int32),
    (20, 32, 512, "auto", torch.float16, "fp8", torch.int32),
]


@pytest.mark.parametrize("case", CASES, ids=[f"T{c[0]}H{c[1]}P{c[2]}-{c[3]}-{c[5]}"
                                             for c in CASES])
def test_prologue_equals_separate_calls(pkg, lib, dev, case):
    T, H, P, kv_dtype, in_dtype, ik_kind, slot_dtype = case
    m = pkg.dsa_layer
    ops = pkg._sm70_ops
    g = torch.Generator(device=dev)
    g.manual_seed(T * 7 + H + P)
    nblk = 9
    fp8 = kv_dtype == "fp8_ds_mla"
    lat0 = (torch.randint(0, 256, (nblk, PAGE, 656), generator=g, device=dev, dtype=torch.uint8)
            if fp8 else torch.randn(nblk, PAGE, 576, generator=g, device=dev).to(torch.float16))
    ik0 = (torch.randint(0, 256, (nblk, PAGE, 132), generator=g, device=dev, dtype=torch.uint8)
           if ik_kind == "fp8" else
           torch.randn(nblk, PAGE, 128, generator=g, device=dev).to(torch.float16))
    w = m.DsaLayerWeights(
        (torch.randn(H, P, 512, generator=g, device=dev) / P ** 0.5).to(torch.float16),
        (torch.randn(H, 512, 128, generator=g, device=dev) / 24).to(torch.float16), 0.05)
    q = (torch.randn(T, H, P + 64, generator=g, device=dev) / 4).to(torch.float16)
    kv_c = (torch.randn(T + 3, 512, generator=g, device=dev) * 3).to(in_dtype)[:T]
    k_pe = (torch.randn(T, 64, generator=g, device=dev)).to(in_dtype)
    idx_k = torch.randn(T, 128, generator=g, device=dev).to(torch.float16)
    slot = torch.randperm(nblk * PAGE, generator=g, device=dev)[:T]
    slot[1] = -1                  # skipped
    slot[T - 1] = nblk * PAGE + 5  # past the cache: skipped
    slot = slot.to(slot_dtype)

    # separate calls
    L1 = m.DsaLayer(w, lat0.clone(), ik0.clone())
    L1.store(kv_c, k_pe, idx_k, slot)
    ql1 = m.q_latent(q, w)
    # fused
    L2 = m.DsaLayer(w, lat0.clone(), ik0.clone())
    assert L2._fusable(q, kv_c, k_pe, idx_k, slot)
    ql2, hist = L2._prologue(q, kv_c, k_pe, idx_k, slot)
    torch.cuda.synchronize()
    assert torch.equal(ql1.view(torch.int16), ql2.view(torch.int16))
    assert torch.equal(L1.latent_cache.view(torch.uint8), L2.latent_cache.view(torch.uint8))
    assert torch.equal(L1.idx_k_cache.view(torch.uint8), L2.idx_k_cache.view(torch.uint8))
    assert hist.shape == (T, 4096) and not hist.any()
    # the written rows really changed (the skipped slots did not)
    assert not torch.equal(L2.latent_cache.view(torch.uint8), lat0.view(torch.uint8))


def test_prologue_clears_a_dirty_histogram_in_a_graph(pkg, dev):
    """Replayed from a HIP graph with the histogram dirtied between replays:
    every replay clears it and writes the same q_latent."""
    m = pkg.dsa_layer
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    H, P, T = 64, 128, 4
    w = m.DsaLayerWeights(
        (torch.randn(H, P, 512, generator=g, device=dev) / P ** 0.5).to(torch.float16),
        (torch.randn(H, 512, 128, generator=g, device=dev) / 24).to(torch.float16), 0.05)
    L = m.DsaLayer(w, torch.zeros(8, PAGE, 656, dtype=torch.uint8, device=dev),
                   torch.zeros(8, PAGE, 128, dtype=torch.float16, device=dev))
    q = (torch.randn(T, H, P + 64, generator=g, device=dev) / 4).to(torch.float16)
    kv_c = torch.randn(T, 512, generator=g, device=dev).to(torch.float16)
    k_pe = torch.randn(T, 64, generator=g, device=dev).to(torch.float16)
    idx_k = torch.randn(T, 128, generator=g, device=dev).to(torch.float16)
    slot = torch.arange(T, device=dev, dtype=torch.int32) * 3
    want = m.q_latent(q, w)
    out = {}
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        L._prologue(q, kv_c, k_pe, idx_k, slot)  # warm-up outside the capture
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            out["ql"], out["hist"] = L._prologue(q, kv_c, k_pe, idx_k, slot)
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(3):
        out["hist"].fill_(7)
        out["ql"].fill_(0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert not out["hist"].any()
        assert torch.equal(out["ql"].view(torch.int16), want.view(torch.int16))
