"""GPU parity of one DSA layer step (glm5-on-v100_amd/dsa_layer.py) against
the oracle's restatement of the reference's callers (oracle/dsa_oracle.py
dsa_layer_decode / dsa_layer_prefill): cache writes bit-exact, top-k
indices bit-exact (dyadic indexer inputs make every score exact), q_latent
exact (dyadic q_nope and W_UK_T), attention within the op tolerances
(2e-3 relative / 1e-3 absolute, lse 1e-4), and the W_UV projection of the
kernel's own output within fp16 rounding."""
import pytest
import torch

from oracle import dsa_oracle as O
import tile_scales as TS

pytestmark = pytest.mark.gpu

PAGE = 64


def dyadic(g, shape, num, den):
    return (torch.randint(-num, num + 1, shape, generator=g) / den).to(torch.float16)


def make_layer(seed, H, P, V, nblk, tile=False):
    """tile=False: latents N(0,1)/24 with amax/448 tile scales.  tile=True:
    O(1) latents whose four tile scales are 2^-6, 2^-3, 1 and 8 in a random
    order per row, and W_UK_T large enough for O(1) scores."""
    g = torch.Generator().manual_seed(seed)
    if tile:
        latent = TS.rows(torch.randn(nblk * PAGE, 576, generator=g), g).view(nblk, PAGE, 656)
    else:
        lat = torch.randn(nblk * PAGE, 576, generator=g) / 24.0
        latent = O.dsmla_rows(lat, per_tile=True).view(nblk, PAGE, 656)
    idxk = dyadic(g, (nblk, PAGE, 128), 8, 8)
    W_UK_T = dyadic(g, (H, P, 512), 1, 2) if tile else dyadic(g, (H, P, 512), 2, 16)
    W_UV = (torch.randn(H, 512, V, generator=g) / 24.0).to(torch.float16)
    return g, latent, idxk, W_UK_T, W_UV


def step_tokens(g, T, H, P, tile=False):
    q = torch.cat([dyadic(g, (T, H, P), 2, 4),
                   (torch.randn(T, H, 64, generator=g) / 4).to(torch.float16)], dim=-1)
    idx_q = dyadic(g, (T, 32, 128), 8, 8)
    idx_w = dyadic(g, (T, 32), 4, 4)
    if tile:
        # O(1) new rows whose tile amax is pinned to 7, so that the writer's
        # amax/448 scale is 2^-6 and fp16(e4m3 * scale) is exact
        kv_c = torch.randn(T, 512, generator=g).clamp(-6.9, 6.9)
        kv_c[:, ::128] = 7.0
        kv_c = kv_c.to(torch.float16)
        k_pe = torch.randn(T, 64, generator=g).to(torch.float16)
    else:
        kv_c = (torch.randn(T, 512, generator=g) / 24.0).to(torch.float16)
        k_pe = (torch.randn(T, 64, generator=g) / 24.0).to(torch.float16)
    idx_k = dyadic(g, (T, 128), 8, 8)
    return q, idx_q, idx_w, kv_c, k_pe, idx_k


def slots_of(bt_rows, pos):
    return torch.tensor([int(bt_rows[i][p // PAGE]) * PAGE + p % PAGE for i, p in enumerate(pos)])


def build(pkg, dev, latent, idxk, W_UK_T, W_UV, scale):
    m = pkg.dsa_layer
    w = m.DsaLayerWeights(W_UK_T.to(dev), W_UV.to(dev), scale)
    return m.DsaLayer(w, latent.clone().to(dev), idxk.clone().to(dev))


def check_out(got, want, o_gpu, ro, lse, rl, W_UV):
    torch.testing.assert_close(o_gpu.float().cpu(), ro, rtol=2e-3, atol=1e-3)
    fin = torch.isfinite(rl)
    assert torch.equal(fin, torch.isfinite(lse.cpu()))
    assert (lse.cpu()[fin] - rl[fin]).abs().max().item() <= 1e-4
    # v_up of the kernel's own output: fp16 bmm vs fp64
    own = O.v_up(o_gpu.cpu(), W_UV)
    tol = 2e-3 * own.abs().max().item() + 1e-4
    assert (got.float().cpu().double() - own).abs().max().item() <= tol
    # and end to end against the oracle's chain
    tol2 = 2e-2 * want.abs().max().item() + 1e-3
    assert (got.float().cpu().double() - want).abs().max().item() <= tol2


def decode_case(next_n, tile):
    """CPU inputs of one decode step (4 tokens: 4 requests, or 2 requests x 2
    speculative tokens) and the oracle chain's results on them."""
    H, P, V, nblk = 64, 32, 64, 160
    g, latent, idxk, W_UK_T, W_UV = make_layer(40 + next_n, H, P, V, nblk, tile)
    R = 4 // next_n
    B = R * next_n
    lens = [3000, 2600, 900, 2049][:R]
    mb = 50
    bt = torch.stack([torch.randperm(nblk, generator=g)[:mb] for _ in range(R)]).to(torch.int32)
    seq = torch.tensor(lens, dtype=torch.int32)
    q, idx_q, idx_w, kv_c, k_pe, idx_k = step_tokens(g, B, H, P, tile)
    # the step's tokens sit at the last next_n positions of each request
    pos = [lens[r] - next_n + j for r in range(R) for j in range(next_n)]
    bt_tok = bt.repeat_interleave(next_n, dim=0)
    slot = slots_of(bt_tok, pos)
    scale = (P + 64) ** -0.5
    lat2 = O.concat_and_cache_mla(latent, kv_c, k_pe, slot, "fp8_ds_mla")
    idxk2 = O.indexer_k_store(idxk, idx_k, slot.to(torch.int32))
    sl_tok = torch.tensor(pos, dtype=torch.int32) + 1
    want, ridx, ro, rl = O.dsa_layer_decode(q, idx_q, idx_w, bt_tok, sl_tok, lat2, idxk2,
                                            W_UK_T, W_UV, scale)
    return dict(latent=latent, idxk=idxk, W_UK_T=W_UK_T, W_UV=W_UV, scale=scale, q=q,
                idx_q=idx_q, idx_w=idx_w, bt=bt, seq=seq, kv_c=kv_c, k_pe=k_pe, idx_k=idx_k,
                slot=slot, lat2=lat2, idxk2=idxk2, bt_tok=bt_tok, want=want, ridx=ridx, ro=ro,
                rl=rl)


@pytest.mark.parametrize("next_n,tile", [(1, False), (2, False), (1, True), (2, True)],
                         ids=["decode", "spec2", "decode_tiles", "spec2_tiles"])
def test_decode_step(pkg, dev, next_n, tile):
    """tile=True: the O(1) rows with very different per-tile scales, through
    the fused split merge + W_UV epilogue."""
    c = decode_case(next_n, tile)
    layer = build(pkg, dev, c["latent"], c["idxk"], c["W_UK_T"], c["W_UV"], c["scale"])
    got = layer.decode(*(c[k].to(dev) for k in ("q", "idx_q", "idx_w", "bt", "seq", "kv_c",
                                                 "k_pe", "idx_k", "slot")))
    assert torch.equal(layer.latent_cache.cpu(), c["lat2"])
    assert torch.equal(layer.idx_k_cache.cpu(), c["idxk2"])
    assert torch.equal(layer.last_idx.cpu(), c["ridx"])
    check_out(got, c["want"], layer.last_o, c["ro"], layer.last_lse, c["rl"], c["W_UV"])


def prefill_case(tile):
    """CPU inputs of one prefill step (two requests, 100 and 60 new tokens
    after 2200 and 500 cached ones, 16 heads) and the oracle chain's
    results."""
    H, P, V, nblk = 16, 32, 32, 120
    g, latent, idxk, W_UK_T, W_UV = make_layer(50, H, P, V, nblk, tile)
    prior, new = [2200, 500], [100, 60]
    bounds = [0, new[0], new[0] + new[1]]
    mb = 40
    bt = torch.stack([torch.randperm(nblk, generator=g)[:mb] for _ in range(2)]).to(torch.int32)
    T = sum(new)
    q, idx_q, idx_w, kv_c, k_pe, idx_k = step_tokens(g, T, H, P, tile)
    pos = [prior[r] + j for r in range(2) for j in range(new[r])]
    req = [r for r in range(2) for _ in range(new[r])]
    slot = slots_of(bt[req], pos)
    causal = torch.tensor(pos, dtype=torch.int32) + 1
    scale = (P + 64) ** -0.5
    lat2 = O.concat_and_cache_mla(latent, kv_c, k_pe, slot, "fp8_ds_mla")
    idxk2 = O.indexer_k_store(idxk, idx_k, slot.to(torch.int32))
    want, ridx, ro, rl = O.dsa_layer_prefill(q, idx_q, idx_w, bounds, bt, causal, lat2, idxk2,
                                             W_UK_T, W_UV, scale)
    return dict(latent=latent, idxk=idxk, W_UK_T=W_UK_T, W_UV=W_UV, scale=scale, q=q,
                idx_q=idx_q, idx_w=idx_w, bounds=bounds, bt=bt, causal=causal, kv_c=kv_c,
                k_pe=k_pe, idx_k=idx_k, slot=slot, lat2=lat2, bt_tok=bt[req], want=want,
                ridx=ridx, ro=ro, rl=rl)


@pytest.mark.parametrize("tile", [False, True], ids=["prefill", "prefill_tiles"])
def test_prefill_step(pkg, dev, tile):
    c = prefill_case(tile)
    layer = build(pkg, dev, c["latent"], c["idxk"], c["W_UK_T"], c["W_UV"], c["scale"])
    got = layer.prefill(c["q"].to(dev), c["idx_q"].to(dev), c["idx_w"].to(dev), c["bounds"],
                        c["bt"].to(dev), c["causal"].to(dev), c["kv_c"].to(dev),
                        c["k_pe"].to(dev), c["idx_k"].to(dev), c["slot"].to(dev), sub_rows=64)
    assert torch.equal(layer.latent_cache.cpu(), c["lat2"])
    assert torch.equal(layer.last_idx.cpu(), c["ridx"])
    check_out(got, c["want"], layer.last_o, c["ro"], layer.last_lse, c["rl"], c["W_UV"])
