"""Seeded synthetic inputs of the benchmark configurations, built on the GPU.

There is no model checkpoint or dataset on the path, so the benchmark and
the full-size tests feed the kernels synthetic tensors with the shapes and
distributions of the reference's serving configuration: paged caches with
a random block permutation, fp16 activations ~ N(0,1) (scaled as stated per
config) and fp8 caches quantised before storage.
"""
from __future__ import annotations

import torch

DSMLA_ROW_BYTES = 656


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def quantize_dsmla_rows(lat: torch.Tensor) -> torch.Tensor:
    """[n,576] float -> [n,656] uint8 fp8_ds_mla rows on lat's device: one
    NoPE scale amax/448 per row written into all 4 tile slots, e4m3 RNE
    with saturation, RoPE copied as fp16 (row layout of the reference's
    fp8_ds_mla cache: 512 e4m3 | 4 fp32 scales | 64 fp16)."""
    n = lat.shape[0]
    x = lat.to(torch.float32)
    nope = x[:, :512]
    amax = nope.abs().amax(dim=1, keepdim=True)
    scale = torch.clamp(amax / 448.0, min=torch.finfo(torch.float32).tiny)
    q = (nope / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8)
    sb = scale.expand(n, 4).contiguous().view(torch.uint8).reshape(n, 16)
    rb = x[:, 512:].to(torch.float16).contiguous().view(torch.uint8).reshape(n, 128)
    return torch.cat([q, sb, rb], dim=1).contiguous()


def paged_block_table(B: int, blocks_per_seq: int, pool_blocks: int, g, device) -> torch.Tensor:
    """Each sequence gets a distinct random subset of the physical pool."""
    perm = torch.randperm(pool_blocks, generator=g, device=device)
    need = B * blocks_per_seq
    assert need <= pool_blocks
    return perm[:need].view(B, blocks_per_seq).to(torch.int32).contiguous()


def latent_cache(n_rows: int, fp8: bool, g, device, page: int = 64, chunk: int = 1 << 18):
    """Latent cache [n_rows/page, page, 576 | 656], values N(0,1)/sqrt(576)."""
    assert n_rows % page == 0
    width = DSMLA_ROW_BYTES if fp8 else 576
    out = torch.empty(n_rows, width, dtype=torch.uint8 if fp8 else torch.float16, device=device)
    for lo in range(0, n_rows, chunk):
        hi = min(lo + chunk, n_rows)
        lat = torch.randn(hi - lo, 576, generator=g, device=device) / 24.0
        out[lo:hi] = quantize_dsmla_rows(lat) if fp8 else lat.to(torch.float16)
    return out.view(n_rows // page, page, width)


def sorted_unique_positions(B: int, topk: int, ctx: int, g, device) -> torch.Tensor:
    """idx [B, topk]: distinct positions in [0, ctx), ascending (the order the
    top-k kernels emit)."""
    rows = []
    for _ in range(B):
        if ctx <= topk:
            r = torch.full((topk,), -1, dtype=torch.int64, device=device)
            r[:ctx] = torch.arange(ctx, device=device)
        else:
            r = torch.randperm(ctx, generator=g, device=device)[:topk].sort().values
        rows.append(r)
    return torch.stack(rows).to(torch.int32).contiguous()


def decode_inputs(B=4, H=64, ctx=184320, topk=2048, fp8=True, page=64, pool_factor=1,
                  seed=3, device="cuda"):
    """Config C3: sparse MLA decode over a paged fp8_ds_mla (or fp16) cache."""
    g = _gen(seed, device)
    bps = (ctx + page - 1) // page
    pool = B * bps * pool_factor
    kv = latent_cache(pool * page, fp8, g, device, page)
    bt = paged_block_table(B, bps, pool, g, device)
    seq = torch.full((B,), ctx, dtype=torch.int32, device=device)
    q = (torch.randn(B, H, 576, generator=g, device=device) / 24.0).to(torch.float16)
    idx = sorted_unique_positions(B, topk, ctx, g, device)
    return dict(q=q, kv=kv, idx=idx, bt=bt, seq=seq, scale=576 ** -0.5)


def indexer_decode_inputs(B=4, ctx=65536, page=64, dup_frac=0.01, seed=2, device="cuda",
                          fp8=False):
    """Config C2: indexer logits + top-k at decode, with ~1% duplicated keys.
    fp8=True also returns the keys quantised into 132-byte fp8 rows
    (`kc8`, written by the indexer-K store op) in the same paged layout."""
    g = _gen(seed, device)
    bps = (ctx + page - 1) // page
    pool = B * bps
    k = torch.randn(pool * page, 128, generator=g, device=device).to(torch.float16)
    ndup = int(dup_frac * pool * page)
    if ndup:
        perm = torch.randperm(pool * page, generator=g, device=device)
        k[perm[ndup:2 * ndup]] = k[perm[:ndup]]  # disjoint source / target rows
    bt = paged_block_table(B, bps, pool, g, device)
    q = torch.randn(B, 32, 128, generator=g, device=device).to(torch.float16)
    w = (torch.randn(B, 32, generator=g, device=device) / 32 ** 0.5).to(torch.float16)
    seq = torch.full((B,), ctx, dtype=torch.int32, device=device)
    kc = k.view(pool, page, 128)
    out = dict(q=q, k=k, kc=kc, w=w, bt=bt, seq=seq, max_kv=bps * page)
    if fp8:
        from . import _sm70_ops
        kc8 = torch.empty(pool, page, 132, dtype=torch.uint8, device=device)
        slots = torch.arange(pool * page, dtype=torch.int32, device=device)
        _sm70_ops.sm70_indexer_k_store(kc8, k, slots)
        out["kc8"] = kc8
    return out
