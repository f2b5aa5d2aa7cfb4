"""Writes the golden fixtures of the DSA hot path (tests/golden/*.npz).

Each fixture holds seeded inputs and the outputs of the CPU oracle
(oracle/dsa_oracle.py), whose functions are pinned independently by the
tests/test_oracle_*.py checks (known answers, closed forms, brute force).
The reference itself cannot run here (CUDA sources, vLLM imports), so the
fixtures freeze the pinned oracle: tests/test_golden.py checks that the
oracle still reproduces them and tests/test_gpu_golden.py runs the HIP
kernels on the same inputs.

Usage: python tests/golden/make_golden.py   (rewrites the .npz files)
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import dsa_oracle as O  # noqa: E402

SCALE = 576 ** -0.5


def _np(t):
    return t.contiguous().numpy()


def k_store():
    g = torch.Generator().manual_seed(101)
    n_tok, nblk, page = 48, 8, 16
    k = (torch.randn(n_tok, 128, generator=g) * 3).to(torch.float16)
    k[5] = 0  # amax 0 -> scale FLT_MIN
    k[6, :4] = torch.tensor([448.0 * 7, -448.0 * 7, 448.0 * 7 / 448 * 0.5, 1.0])  # saturating row
    slot = torch.randperm(nblk * page, generator=g)[:n_tok].to(torch.int32)
    slot[3] = -1
    slot[9] = nblk * page + 5  # out of range: skipped
    c16 = torch.zeros(nblk, page, 128, dtype=torch.float16)
    c8 = torch.zeros(nblk, page, 132, dtype=torch.uint8)
    return dict(k=_np(k), slot=_np(slot), cache16=_np(c16), cache8=_np(c8),
                out16=_np(O.indexer_k_store(c16, k, slot)),
                out8=_np(O.indexer_k_store(c8, k, slot)))


def indexer():
    g = torch.Generator().manual_seed(202)
    B, nblk, page, max_kv = 3, 12, 16, 176
    q = torch.randn(B, 32, 128, generator=g).to(torch.float16)
    w = (torch.randn(B, 32, generator=g) / 32 ** 0.5).to(torch.float16)
    lat = torch.randn(nblk * page, 128, generator=g).to(torch.float16)
    c16 = lat.view(nblk, page, 128)
    c8 = O.indexer_k_store(torch.zeros(nblk, page, 132, dtype=torch.uint8), lat,
                           torch.arange(nblk * page, dtype=torch.int32))
    bt = torch.stack([torch.randperm(nblk, generator=g)[:11] for _ in range(B)]).to(torch.int32)
    seq = torch.tensor([170, 64, 0], dtype=torch.int32)
    s16, h16 = O.indexer_logits(q, c16, w, bt, seq, max_kv, with_hist=True)
    s8, h8 = O.indexer_logits(q, c8, w, bt, seq, max_kv, with_hist=True)
    return dict(q=_np(q), w=_np(w), cache16=_np(c16), cache8=_np(c8), bt=_np(bt), seq=_np(seq),
                score16=_np(s16), hist16=_np(h16), score8=_np(s8), hist8=_np(h8))


def topk():
    g = torch.Generator().manual_seed(303)
    R, W, K = 4, 5000, 2048
    s = torch.randn(R, W, generator=g)
    s[1] = torch.round(s[1] * 4) / 4           # heavy ties
    s[2, :] = 0.5                              # all equal
    s[2, 100] = -0.0
    seq = torch.tensor([5000, 4999, 3000, 1500], dtype=torch.int32)
    return dict(score=_np(s), seq=_np(seq), k=np.int32(K), idx=_np(O.topk_rows(s, seq, K)))


def sparse_mla():
    g = torch.Generator().manual_seed(404)
    B, H, nblk, page, topk = 3, 8, 6, 16, 64
    lat = torch.randn(nblk * page, 576, generator=g) / 24.0
    kv16 = lat.to(torch.float16).view(nblk, page, 576)
    kv8 = O.dsmla_rows(lat).view(nblk, page, 656)
    bt = torch.stack([torch.randperm(nblk, generator=g)[:5] for _ in range(B)]).to(torch.int32)
    seq = torch.tensor([75, 50, 60], dtype=torch.int32)
    q = (torch.randn(B, H, 576, generator=g) / 4).to(torch.float16)
    idx = torch.full((B, topk), -1, dtype=torch.int32)
    for b in range(B):
        n = min(int(seq[b]), topk)
        idx[b, :n] = torch.randperm(int(seq[b]), generator=g)[:n].sort().values.to(torch.int32)
    idx[2] = -1  # no valid key
    idx[1, 5] = 10 ** 6  # >= seq_len: masked
    o16, l16 = O.sparse_mla(q, kv16, idx, bt, seq, SCALE)
    o8, l8 = O.sparse_mla(q, kv8, idx, bt, seq, SCALE)
    return dict(q=_np(q), kv16=_np(kv16), kv8=_np(kv8), bt=_np(bt), seq=_np(seq), idx=_np(idx),
                scale=np.float32(SCALE), o16=_np(o16), lse16=_np(l16), o8=_np(o8), lse8=_np(l8))


def fp8_linear():
    g = torch.Generator().manual_seed(505)
    N, K, M = 72, 272, 3
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.float16)
    w8, s = O.attn_fp8_quantize(w)
    x = torch.randn(M, K, generator=g).to(torch.float16)
    return dict(w8=_np(w8), s=_np(s), x=_np(x),
                deq=_np(O.attn_fp8_dequant(w8, s)), y=_np(O.attn_fp8_gemv(x, w8, s)))


FIXTURES = {"k_store": k_store, "indexer": indexer, "topk": topk, "sparse_mla": sparse_mla,
            "fp8_linear": fp8_linear}


def generate(name):
    return FIXTURES[name]()


if __name__ == "__main__":
    for name, fn in FIXTURES.items():
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **fn())
        print(path, os.path.getsize(path))
