"""Per-tile fp8_ds_mla scales through every fp8 attention kernel.

Production caches carry four different NoPE tile scales per row (the
reference reads one per 128-dim tile, sm70_mla_decode.cu:74-100, :970-998).
These cases feed rows whose tile scales are 2^-6, 2^-3, 1 and 8 in a random
order per row, with O(1) values and O(1) scores, through each kernel the
decode plan can pick for an fp8 cache:

  c3       B=4, 64 heads, top-2048 at 180k context: the LDS-DMA split decode
           and the split merge (the headline configuration)
  dma_h16  B=3, 16 heads, top-512: the LDS-DMA split decode, one head group
  pipe     B=16, 64 heads: the 64-head pipelined kernel with 16 key splits
  regst    B=2, 16 heads, top-17408: the register-staged split decode
  prefill  B=256, 64 heads: the pipelined prefill kernel, one split
  c4       the last 4096-token launch of the 64k causal prefill

The CPU tests show, on the same inputs, that reading a tile with the next
tile's scale on the QK side alone, or on the PV side alone, falls outside
the tolerance (2e-3 relative / 1e-3 absolute on o, 1e-4 on lse); the GPU
tests hold the kernels to that tolerance against the oracle."""
import pytest
import torch

from oracle import dsa_oracle as O
import tile_scales as TS

SCALE = 576 ** -0.5
PAGE = 64

PRIVATE = {
    # name: seed, B, H, topk, ctx
    "c3": (1, 4, 64, 2048, 184320),
    "dma_h16": (2, 3, 16, 512, 5000),
    "pipe": (3, 16, 64, 2048, 8192),
    "regst": (5, 2, 16, 17408, 20000),
}
SHARED = {
    # name: seed, B, H, topk, n_rows, seqs, causal spread, sampled tokens
    "prefill": (4, 256, 64, 2048, 4096, [2048 + 7 * i for i in range(256)], False,
                [0, 1, 77, 128, 200, 255]),
    "c4": (6, 4096, 64, 2048, 65536, list(range(65536 - 4095, 65537)), True,
           [0, 1, 2047, 4095]),
}


def oracle(q, sel):
    """The oracle on compact caches: token b's selected rows laid out
    contiguously, every entry valid."""
    B, n = sel.shape[:2]
    kv_c = sel.reshape(-1, PAGE, 656)
    idx_c = torch.arange(B * n, dtype=torch.int32).view(B, n)
    bt_c = torch.arange(kv_c.shape[0], dtype=torch.int32)[None].repeat(B, 1)
    seq_c = torch.full((B,), B * n, dtype=torch.int32)
    return O.sparse_mla(q, kv_c, idx_c, bt_c, seq_c, SCALE)


def build(name):
    """(q, idx, bt, seq, cache maker, sampled tokens, selected rows of those
    tokens), all on the CPU."""
    if name in PRIVATE:
        seed, B, H, topk, ctx = PRIVATE[name]
        q, idx, bt, seq, sel, phys, pool = TS.paged_case(seed, B, H, topk, ctx)
        toks = list(range(B))
        return q, idx, bt, seq, (lambda dev: TS.paged_cache(sel, phys, pool, PAGE, dev)), toks, sel
    seed, B, H, topk, n_rows, seqs, spread, toks = SHARED[name]
    q, idx, bt, seq, flat = TS.shared_case(seed, B, H, topk, n_rows, seqs, causal_spread=spread)
    sel = TS.selected(flat, idx[toks], bt[toks])
    return (q, idx, bt, seq, (lambda dev: flat.view(-1, PAGE, 656).to(dev)), toks, sel)


CASES = list(PRIVATE) + list(SHARED)


@pytest.mark.parametrize("name", CASES)
def test_tile_scale_mutants_fail(name):
    """CPU: the unmutated separable attention equals the oracle; a rotated
    tile-scale index on either side alone breaks the tolerance."""
    q, idx, bt, seq, _, toks, sel = build(name)
    ro, rl = oracle(q[toks], sel)
    ao, al = TS.attention(q[toks], sel, sel, SCALE)
    assert TS.within(ao, al, ro, rl)
    assert float(ro.abs().mean()) > 50 * TS.ATOL
    assert TS.mutants_fail(q[toks], sel, SCALE, ro, rl)


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_tile_scales_gpu(ops, dev, name):
    q, idx, bt, seq, cache, toks, sel = build(name)
    B, H = q.shape[:2]
    print(f"tile scales {name}: B={B} H={H} topk={idx.shape[1]}", flush=True)
    kv = cache(dev)
    o = torch.full((B, H, 512), float("nan"), dtype=torch.float16, device=dev)
    lse = torch.full((B, H), float("nan"), device=dev)
    ops.sm70_sparse_mla_decode(o, lse, q.to(dev), kv, idx.to(dev), bt.to(dev), seq.to(dev),
                               SCALE)
    ro, rl = oracle(q[toks], sel)
    TS.check(o[toks].float().cpu(), lse[toks].cpu(), ro, rl)


def _layer_mutants_fail(c, q_lat):
    """Per token (valid entries differ in number), the layer's attention on
    its own selected rows with a rotated tile-scale index on one side."""
    page = c["lat2"].shape[1]
    flat = c["lat2"].reshape(-1, 656)
    qk_bad = pv_bad = False
    for b in range(q_lat.shape[0]):
        sel = c["ridx"][b][c["ridx"][b] >= 0].long()
        phys = c["bt_tok"][b].long()[sel // page] * page + sel % page
        rows_b = flat[phys][None]
        ro, rl = c["ro"][b:b + 1], c["rl"][b:b + 1]
        assert TS.within(*TS.attention(q_lat[b:b + 1], rows_b, rows_b, c["scale"]), ro, rl)
        bad = TS.rotate_scales(rows_b)
        qk_bad |= not TS.within(*TS.attention(q_lat[b:b + 1], bad, rows_b, c["scale"]), ro, rl)
        pv_bad |= not TS.within(*TS.attention(q_lat[b:b + 1], rows_b, bad, c["scale"]), ro, rl)
    return qk_bad and pv_bad


@pytest.mark.parametrize("step", ["decode", "spec2", "prefill"])
def test_layer_tile_mutants_fail(step):
    """CPU, on the layer-step tests' tile-scale inputs: the oracle chain's
    attention is O(1), and a rotated tile-scale index on the QK or the PV
    side breaks the tolerance."""
    import test_gpu_dsa_layer as L
    c = L.prefill_case(True) if step == "prefill" else L.decode_case(
        1 if step == "decode" else 2, True)
    assert float(c["ro"].abs().mean()) > 50 * TS.ATOL
    q_lat = O.q_latent(c["q"], c["W_UK_T"])
    if step == "prefill":
        q_lat, keep = q_lat[::20], slice(None, None, 20)
        c = dict(c, ridx=c["ridx"][keep], bt_tok=c["bt_tok"][keep], ro=c["ro"][keep],
                 rl=c["rl"][keep])
    assert _layer_mutants_fail(c, q_lat)
