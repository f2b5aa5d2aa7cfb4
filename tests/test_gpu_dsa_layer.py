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

pytestmark = pytest.mark.gpu

PAGE = 64


def dyadic(g, shape, num, den):
    return (torch.randint(-num, num + 1, shape, generator=g) / den).to(torch.float16)


def make_layer(seed, H, P, V, nblk):
    g = torch.Generator().manual_seed(seed)
    lat = torch.randn(nblk * PAGE, 576, generator=g) / 24.0
    latent = O.dsmla_rows(lat, per_tile=True).view(nblk, PAGE, 656)
    idxk = dyadic(g, (nblk, PAGE, 128), 8, 8)
    W_UK_T = dyadic(g, (H, P, 512), 2, 16)
    W_UV = (torch.randn(H, 512, V, generator=g) / 24.0).to(torch.float16)
    return g, latent, idxk, W_UK_T, W_UV


def step_tokens(g, T, H, P):
    q = torch.cat([dyadic(g, (T, H, P), 2, 4),
                   (torch.randn(T, H, 64, generator=g) / 4).to(torch.float16)], dim=-1)
    idx_q = dyadic(g, (T, 32, 128), 8, 8)
    idx_w = dyadic(g, (T, 32), 4, 4)
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


@pytest.mark.parametrize("next_n", [1, 2], ids=["decode", "spec2"])
def test_decode_step(pkg, dev, next_n):
    H, P, V, nblk = 64, 32, 64, 160
    g, latent, idxk, W_UK_T, W_UV = make_layer(40 + next_n, H, P, V, nblk)
    R = 4 // next_n
    B = R * next_n
    lens = [3000, 2600, 900, 2049][:R]
    mb = 50
    bt = torch.stack([torch.randperm(nblk, generator=g)[:mb] for _ in range(R)]).to(torch.int32)
    seq = torch.tensor(lens, dtype=torch.int32)
    q, idx_q, idx_w, kv_c, k_pe, idx_k = step_tokens(g, B, H, P)
    # the step's tokens sit at the last next_n positions of each request
    pos = [lens[r] - next_n + j for r in range(R) for j in range(next_n)]
    bt_tok = bt.repeat_interleave(next_n, dim=0)
    slot = slots_of(bt_tok, pos)
    scale = (P + 64) ** -0.5
    layer = build(pkg, dev, latent, idxk, W_UK_T, W_UV, scale)
    got = layer.decode(q.to(dev), idx_q.to(dev), idx_w.to(dev), bt.to(dev), seq.to(dev),
                       kv_c.to(dev), k_pe.to(dev), idx_k.to(dev), slot.to(dev))
    lat2 = O.concat_and_cache_mla(latent, kv_c, k_pe, slot, "fp8_ds_mla")
    idxk2 = O.indexer_k_store(idxk, idx_k, slot.to(torch.int32))
    assert torch.equal(layer.latent_cache.cpu(), lat2)
    assert torch.equal(layer.idx_k_cache.cpu(), idxk2)
    sl_tok = torch.tensor(pos, dtype=torch.int32) + 1
    want, ridx, ro, rl = O.dsa_layer_decode(q, idx_q, idx_w, bt_tok, sl_tok, lat2, idxk2,
                                            W_UK_T, W_UV, scale)
    assert torch.equal(layer.last_idx.cpu(), ridx)
    check_out(got, want, layer.last_o, ro, layer.last_lse, rl, W_UV)


def test_prefill_step(pkg, dev):
    H, P, V, nblk = 16, 32, 32, 120
    g, latent, idxk, W_UK_T, W_UV = make_layer(50, H, P, V, nblk)
    prior, new = [2200, 500], [100, 60]
    bounds = [0, new[0], new[0] + new[1]]
    mb = 40
    bt = torch.stack([torch.randperm(nblk, generator=g)[:mb] for _ in range(2)]).to(torch.int32)
    T = sum(new)
    q, idx_q, idx_w, kv_c, k_pe, idx_k = step_tokens(g, T, H, P)
    pos = [prior[r] + j for r in range(2) for j in range(new[r])]
    req = [r for r in range(2) for _ in range(new[r])]
    slot = slots_of(bt[req], pos)
    causal = torch.tensor(pos, dtype=torch.int32) + 1
    scale = (P + 64) ** -0.5
    layer = build(pkg, dev, latent, idxk, W_UK_T, W_UV, scale)
    got = layer.prefill(q.to(dev), idx_q.to(dev), idx_w.to(dev), bounds, bt.to(dev),
                        causal.to(dev), kv_c.to(dev), k_pe.to(dev), idx_k.to(dev),
                        slot.to(dev), sub_rows=64)
    lat2 = O.concat_and_cache_mla(latent, kv_c, k_pe, slot, "fp8_ds_mla")
    idxk2 = O.indexer_k_store(idxk, idx_k, slot.to(torch.int32))
    assert torch.equal(layer.latent_cache.cpu(), lat2)
    want, ridx, ro, rl = O.dsa_layer_prefill(q, idx_q, idx_w, bounds, bt, causal, lat2, idxk2,
                                             W_UK_T, W_UV, scale)
    assert torch.equal(layer.last_idx.cpu(), ridx)
    check_out(got, want, layer.last_o, ro, layer.last_lse, rl, W_UV)
