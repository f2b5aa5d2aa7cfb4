"""GPU parity: dense MLA decode (sm70_mla_decode), fp16 latent cache.

Against the oracle's restatement of the reference kernel
(oracle/dsa_oracle.py mla_decode): o within 2e-3 relative / 1e-3 absolute
and lse within 1e-4 of the exact (fp64) result, and within the same bounds
of the reference's own fp16 running-O arithmetic (fp16_acc=True)."""
import math

import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu

SCALE = 576 ** -0.5
RTOL, ATOL, LSE_ATOL = 2e-3, 1e-3, 1e-4


def make(seed, B, H, nblk, page, seqs, mb=None):
    g = torch.Generator().manual_seed(seed)
    kv = (torch.randn(nblk * page, 576, generator=g) / 24.0).to(torch.float16).view(nblk, page, 576)
    mb = mb or max((max(seqs) + page - 1) // page, 1)
    bt = torch.stack([torch.randperm(nblk, generator=g)[:mb] for _ in range(B)]).to(torch.int32)
    q = (torch.randn(B, H, 576, generator=g) / 24.0 * 6).to(torch.float16)
    return q, kv, bt, torch.tensor(seqs, dtype=torch.int32)


def run(ops, dev, q, kv, bt, seq):
    B, H = q.shape[:2]
    o = torch.full((B, H, 512), float("nan"), dtype=torch.float16, device=dev)
    lse = torch.full((B, H), float("nan"), device=dev)
    ops.sm70_mla_decode(o, lse, q.to(dev), kv.to(dev), bt.to(dev), seq.to(dev), SCALE)
    return o.float().cpu(), lse.cpu()


def check(o, lse, ro, rl):
    assert torch.equal(torch.isinf(lse), torch.isinf(rl))
    fin = torch.isfinite(rl)
    if fin.any():
        assert (lse[fin] - rl[fin]).abs().max().item() <= LSE_ATOL
    torch.testing.assert_close(o, ro, rtol=RTOL, atol=ATOL)


CASES = [
    # seed, B, H, nblk, page, seqs
    (0, 1, 32, 10, 16, [100]),
    (1, 4, 64, 60, 64, [3000, 2048, 700, 1]),
    (2, 2, 128, 90, 64, [5000, 33]),
    (3, 3, 32, 40, 48, [1400, 0, 500]),          # page not a power of two, empty token
    (4, 1, 64, 700, 64, [40000]),                # long context: many splits
    (5, 256, 64, 40, 16, [90 + (i % 200) for i in range(256)]),  # 64-head prefill configuration
]


@pytest.mark.parametrize("case", CASES, ids=[f"c{c[0]}" for c in CASES])
def test_dense_decode(ops, dev, case):
    seed, B, H, nblk, page, seqs = case
    q, kv, bt, seq = make(seed, B, H, nblk, page, seqs)
    o, lse = run(ops, dev, q, kv, bt, seq)
    assert not torch.isnan(o).any() and not torch.isnan(lse).any()
    ro, rl = O.mla_decode(q, kv, bt, seq, SCALE)
    check(o, lse, ro, rl)
    if B * max(seqs) <= 20000:
        r16, l16 = O.mla_decode(q, kv, bt, seq, SCALE, fp16_acc=True)
        check(o, lse, r16, l16)


def test_unresolvable_rows_are_zero_keys(ops, dev):
    """Positions below seq_len on a -1 block are zero keys with score 0, as
    in the reference (sm70_mla_decode.cu:762-771)."""
    q, kv, bt, seq = make(7, 3, 32, 40, 64, [900, 300, 200])
    bt[0, 3] = -1
    bt[1, :] = -1            # every position unresolvable: o = 0, lse = ln 300
    bt[2, 1] = 10 ** 6       # block past the cache
    o, lse = run(ops, dev, q, kv, bt, seq)
    ro, rl = O.mla_decode(q, kv, bt, seq, SCALE)
    check(o, lse, ro, rl)
    assert torch.all(o[1] == 0)
    assert (lse[1] - math.log(300)).abs().max() <= LSE_ATOL


def test_dense_equals_sparse_with_all_positions(ops, dev):
    """On-GPU second oracle: dense decode == sparse decode with idx = 0..L-1
    (seq_len <= topk, every row resolvable), two different kernels."""
    q, kv, bt, seq = make(8, 4, 64, 40, 64, [2048, 1500, 64, 999])
    o, lse = run(ops, dev, q, kv, bt, seq)
    idx = torch.arange(2048, dtype=torch.int32).expand(4, 2048).contiguous()
    os_ = torch.empty(4, 64, 512, dtype=torch.float16, device=dev)
    ls = torch.empty(4, 64, device=dev)
    ops.sm70_sparse_mla_decode(os_, ls, q.to(dev), kv.to(dev), idx.to(dev), bt.to(dev),
                               seq.to(dev), SCALE)
    torch.testing.assert_close(o, os_.float().cpu(), rtol=RTOL, atol=ATOL)
    assert (lse - ls.cpu()).abs().max() <= LSE_ATOL


def test_rejects_like_reference(ops, dev):
    q, kv, bt, seq = make(9, 1, 16, 4, 16, [10])
    o = torch.empty(1, 16, 512, dtype=torch.float16, device=dev)
    lse = torch.empty(1, 16, device=dev)
    with pytest.raises(RuntimeError, match="multiple of 32"):
        ops.sm70_mla_decode(o, lse, q.to(dev), kv.to(dev), bt.to(dev), seq.to(dev), SCALE)
    q, kv, bt, seq = make(9, 1, 32, 4, 16, [10])
    o = torch.empty(1, 32, 512, dtype=torch.float16, device=dev)
    lse = torch.empty(1, 32, device=dev)
    kv8 = torch.zeros(4, 16, 656, dtype=torch.uint8, device=dev)
    with pytest.raises(RuntimeError, match="fp16"):
        ops.sm70_mla_decode(o, lse, q.to(dev), kv8, bt.to(dev), seq.to(dev), SCALE)
