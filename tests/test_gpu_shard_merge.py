"""GPU parity, bit-exact: key-shard indexer merge (sm70_indexer_shard_merge)
against the oracle's restatement of sm70_mla_decode.cu:2055-2182."""
import math

import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def make(seed, tp, R, K, tie_levels=None, short_rows=(), stride=100000, span=50000):
    """Each shard scores its own range of positions (key sharding: shard s
    owns [s stride, s stride + span)) and keeps its top K; short rows have
    fewer than K valid keys per shard (-inf, -1).  A row's positions span
    less than 131072 values (the kernel's bitmap ordering) when
    (tp - 1) stride + span does."""
    g = torch.Generator().manual_seed(seed)
    if tie_levels:
        vals = torch.randint(-tie_levels, tie_levels + 1, (tp, R, K), generator=g).float() / 4
    else:
        vals = torch.randn(tp, R, K, generator=g)
    pos = torch.empty(tp, R, K, dtype=torch.int32)
    for s in range(tp):
        base = s * stride
        for r in range(R):
            pos[s, r] = (base + torch.randperm(span, generator=g)[:K]).to(torch.int32)
    for r, n in short_rows:
        vals[:, r, n:] = -math.inf
        pos[:, r, n:] = -1
    return torch.cat([vals, pos.view(torch.float32)], dim=2).contiguous()


@pytest.mark.parametrize("tp", [2, 3, 4])
@pytest.mark.parametrize("ties", [None, 6], ids=["distinct", "ties"])
@pytest.mark.parametrize("spread", ["bitmap", "sort"])
def test_merge_dst_base(ops, dev, tp, ties, spread):
    K, R = 2048, 37
    geo = dict(stride=16384, span=16384) if spread == "bitmap" else {}
    allf = make(tp * 10 + (ties or 0), tp, R, K, ties, short_rows=[(3, 100), (4, 0), (5, 2047)],
                **geo)
    out = torch.full((R + 9, K), 7, dtype=torch.int32, device=dev)
    ops.sm70_indexer_shard_merge(out, allf.to(dev), torch.empty(0, dtype=torch.int32, device=dev),
                                 5, K)
    want = O.shard_merge_rows(allf, K)
    got = out.cpu()
    assert torch.equal(got[5:5 + R], want)
    assert torch.all(got[:5] == 7) and torch.all(got[5 + R:] == 7)  # other rows untouched
    assert torch.all(got[5 + 4] == -1)


def test_merge_dst_rows(ops, dev):
    K, R, tp = 2048, 20, 4
    allf = make(3, tp, R, K, 3)
    perm = torch.randperm(R, generator=torch.Generator().manual_seed(1)).to(torch.int32)
    out = torch.zeros(R, K, dtype=torch.int32, device=dev)
    ops.sm70_indexer_shard_merge(out, allf.to(dev), perm.to(dev), -1, K)
    want = O.shard_merge_rows(allf, K)
    assert torch.equal(out.cpu()[perm.long()], want)


def test_general_k_through_the_c_abi(pkg, dev):
    """The C ABI takes any power-of-two K <= 2048 with tp*K a multiple of 512."""
    for tp, K in ((2, 256), (1, 512), (8, 1024), (16, 512)):
        R = 9
        allf = make(tp + K, tp, R, K, 5, short_rows=[(2, 10)])
        out = torch.zeros(R, K, dtype=torch.int32, device=dev)
        a = allf.to(dev)
        pkg._lib.call("mi355_dsa_indexer_shard_merge", out.data_ptr(), K, R, a.data_ptr(), tp, R,
                      K, None, 0, torch.cuda.current_stream().cuda_stream)
        assert torch.equal(out.cpu(), O.shard_merge_rows(allf, K)), (tp, K)


def test_rejects_like_reference(ops, dev):
    allf = torch.zeros(5, 2, 4096, device=dev)
    out = torch.zeros(2, 2048, dtype=torch.int32, device=dev)
    e = torch.empty(0, dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError, match="tp in"):
        ops.sm70_indexer_shard_merge(out, allf, e, 0, 2048)
    with pytest.raises(RuntimeError, match="K=2048"):
        ops.sm70_indexer_shard_merge(out, torch.zeros(2, 2, 2048, device=dev), e, 0, 1024)
    with pytest.raises(RuntimeError, match="dst_rows"):
        ops.sm70_indexer_shard_merge(out, torch.zeros(2, 2, 4096, device=dev), e, -1, 2048)


def test_duplicate_positions_fall_back_to_the_sort(ops, dev):
    """Shards that (against key sharding) report the same positions: the
    output keeps the duplicates, in ascending order, as the sort gives."""
    K, R, tp = 2048, 6, 2
    allf = make(21, tp, R, K, 4, stride=0, span=3000)  # both shards draw from [0, 3000)
    out = torch.zeros(R, K, dtype=torch.int32, device=dev)
    ops.sm70_indexer_shard_merge(out, allf.to(dev), torch.empty(0, dtype=torch.int32, device=dev),
                                 0, K)
    want = O.shard_merge_rows(allf, K)
    assert torch.equal(out.cpu(), want)
    assert any(len(set(row.tolist())) < K for row in want)  # the case really has duplicates
