"""Pins the oracle's key-shard merge (sm70_mla_decode.cu:2055-2182) against
a brute-force sort on (score, -column) tuples, the reference's own torch.topk
path (sparse_attn_indexer.py:1008-1031) on distinct scores, and KATs for
ties, -inf and NaN."""
import math

import pytest
import torch

from oracle import dsa_oracle as O


def payload(vals, pos):
    """vals, pos: [tp, R, K] -> allf [tp, R, 2K] fp32."""
    return torch.cat([vals.float(), pos.to(torch.int32).view(torch.float32)], dim=2)


def brute(vals, pos, K):
    tp, R, _ = vals.shape
    out = []
    for r in range(R):
        cands = []
        for s in range(tp):
            for c in range(K):
                v = float(vals[s, r, c])
                cands.append((v, -(s * K + c), int(pos[s, r, c])))
        cands.sort(reverse=True)
        sel = [p if v != -math.inf else -1 for v, _, p in cands[:K]]
        out.append(sorted(sel))
    return torch.tensor(out, dtype=torch.int32)


@pytest.mark.parametrize("tp,K", [(2, 8), (4, 16), (3, 32)])
def test_brute_force_with_ties_and_inf(tp, K):
    g = torch.Generator().manual_seed(tp * K)
    R = 5
    vals = torch.randint(-3, 4, (tp, R, K), generator=g).float()   # many ties
    vals[0, 1, : K // 2] = -math.inf
    vals[:, 2, :] = -math.inf                                       # whole row -inf
    pos = torch.stack([torch.randperm(10 * K, generator=g)[: tp * K].view(tp, K)
                       for _ in range(R)], dim=1)
    got = O.shard_merge_rows(payload(vals, pos), K)
    assert torch.equal(got, brute(vals, pos, K))
    assert torch.all(got[2] == -1)


def test_matches_reference_topk_path_on_distinct_scores():
    g = torch.Generator().manual_seed(7)
    tp, R, K = 4, 6, 64
    vals = torch.randn(tp, R, K, generator=g)
    vals[1, 3, 10:] = -math.inf
    pos = torch.stack([torch.randperm(1000, generator=g)[: tp * K].view(tp, K)
                       for _ in range(R)], dim=1).to(torch.int32)
    allf = payload(vals, pos)
    av = allf[:, :, :K].permute(1, 0, 2).reshape(R, tp * K)
    ai = allf[:, :, K:].permute(1, 0, 2).reshape(R, tp * K).contiguous().view(torch.int32)
    mv, mp = torch.topk(av, K, dim=1)
    mi = torch.where(torch.isinf(mv), torch.full_like(ai.gather(1, mp), -1), ai.gather(1, mp))
    assert torch.equal(O.shard_merge_rows(allf, K), mi.sort(dim=1).values.to(torch.int32))


def test_nan_keys_follow_the_monotone_map():
    """+NaN maps above +inf (selected, position kept); -NaN maps below -inf
    (selected only to fill the row, as -1)."""
    K = 4
    vals = torch.tensor([[[float("nan"), 1.0, 2.0, 3.0]], [[-1.0, -2.0, -3.0, -4.0]]])
    neg_nan = torch.tensor([0xFFC00000], dtype=torch.int64).to(torch.int32).view(torch.float32)
    vals[1, 0, 3] = neg_nan
    pos = torch.tensor([[[100, 101, 102, 103]], [[200, 201, 202, 203]]])
    got = O.shard_merge_rows(payload(vals, pos), K)
    assert got.tolist() == [[100, 101, 102, 103]]
    vals2 = torch.full((2, 1, 4), -math.inf)
    vals2[0, 0, 0] = 5.0
    vals2[1, 0, 1] = neg_nan
    got2 = O.shard_merge_rows(payload(vals2, pos), K)
    assert got2.tolist() == [[-1, -1, -1, 100]]
