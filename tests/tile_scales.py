"""fp8_ds_mla inputs whose four NoPE tile scales differ by large factors.

Each row's 512 NoPE values are O(1) (N(0,1) before quantisation), but the
four 128-dim tiles are encoded with the scales 2^-6, 2^-3, 2^0 and 2^3 in a
random order per row.  A kernel that reads a tile with another tile's scale
(or another row's) is therefore off by a factor of at least 8 on that
tile's share of the score or of the output.  Powers of two also make
fp16(e4m3 * scale) exact, so the kernels' exact products and the
reference's fp16-rounded dequantisation (sm70_mla_decode.cu:81-100) agree
on these rows, and the outputs stay O(1), far above the 1e-3 absolute
tolerance.

Test infrastructure only: the mutant attention below plants one mistake
(a rotated tile-scale index, on the QK or the PV side) on the CPU, so that
a test can show its tolerance would catch that mistake.
"""
from __future__ import annotations

import torch

from oracle import dsa_oracle as O

EXPS = (-6.0, -3.0, 0.0, 3.0)
RTOL, ATOL, LSE_ATOL = 2e-3, 1e-3, 1e-4


def rows(x: torch.Tensor, g: torch.Generator) -> torch.Tensor:
    """x [n, 576] float -> [n, 656] uint8 fp8_ds_mla rows (512 e4m3 | 4 fp32
    tile scales | 64 fp16 RoPE), tile scales a per-row permutation of
    2^EXPS."""
    n = x.shape[0]
    x = x.to(torch.float32)
    perm = torch.argsort(torch.rand(n, 4, generator=g), dim=1)
    scale = torch.exp2(torch.tensor(EXPS)[perm]).contiguous()
    codes = O.e4m3_encode(x[:, :512].reshape(n, 4, 128) / scale[:, :, None]).reshape(n, 512)
    sb = scale.view(torch.uint8).reshape(n, 16)
    rb = x[:, 512:].to(torch.float16).contiguous().view(torch.uint8).reshape(n, 128)
    return torch.cat([codes, sb, rb], dim=1).contiguous()


def rotate_scales(r: torch.Tensor) -> torch.Tensor:
    """The same rows with tile t reading tile (t + 1) % 4's scale."""
    out = r.clone()
    sc = r[..., 512:528].reshape(*r.shape[:-1], 4, 4)
    out[..., 512:528] = sc.roll(-1, dims=-2).reshape(*r.shape[:-1], 16)
    return out


def attention(q: torch.Tensor, k_rows: torch.Tensor, v_rows: torch.Tensor, scale: float):
    """Sparse attention of q [B, H, 576] over per-token compact row lists
    (k_rows / v_rows [B, n, 656]: every row valid), keys read from k_rows
    and values from v_rows, fp64; the oracle's arithmetic
    (dsa_oracle.sparse_mla) with the two sides separable."""
    B, n = k_rows.shape[:2]
    qs = O.scaled_q(q, scale).double()
    o = torch.empty(B, q.shape[1], 512, dtype=torch.float64)
    lse = torch.empty(B, q.shape[1], dtype=torch.float64)
    ok = torch.arange(n, dtype=torch.int64)
    for b in range(B):
        kv = O.latent_rows_fp16(k_rows[b].reshape(n, 1, 656), ok).double()
        vv = O.latent_rows_fp16(v_rows[b].reshape(n, 1, 656), ok).double()
        s = qs[b] @ kv.T
        m = s.max(dim=1, keepdim=True).values
        p = torch.exp(s - m)
        l = p.sum(dim=1, keepdim=True)
        o[b] = (p @ vv[:, :512]) / l
        lse[b] = (m + torch.log(l)).squeeze(1)
    return o.float(), lse.float()


def within(o, lse, ro, rl) -> bool:
    """The GPU tests' acceptance rule: o within 2e-3 relative / 1e-3
    absolute, lse within 1e-4."""
    ok_o = bool(((o - ro).abs() <= ATOL + RTOL * ro.abs()).all())
    return ok_o and float((lse - rl).abs().max()) <= LSE_ATOL


def check(o, lse, ro, rl):
    torch.testing.assert_close(o, ro, rtol=RTOL, atol=ATOL)
    assert float((lse - rl).abs().max()) <= LSE_ATOL
    # the outputs are O(1): a uniform error of a few tenths of a percent shows
    assert float(ro.abs().mean()) > 50 * ATOL


def mutants_fail(q, sel_rows, scale, ro, rl):
    """A rotated tile-scale index on the QK side alone and on the PV side
    alone must each fall outside the tolerance against the oracle."""
    bad = rotate_scales(sel_rows)
    mq = attention(q, bad, sel_rows, scale)
    mv = attention(q, sel_rows, bad, scale)
    return (not within(*mq, ro, rl)) and (not within(*mv, ro, rl))


def paged_case(seed: int, B: int, H: int, topk: int, ctx: int, page: int = 64,
               qmag: float = 2.0):
    """One decode batch over a paged cache: every token at context ctx
    selects topk distinct sorted positions; only the selected rows carry
    data.  Returns CPU tensors (q, idx, bt, seq, sel_rows [B, topk, 656],
    phys_rows [B, topk]) and the pool size in pages."""
    g = torch.Generator().manual_seed(seed)
    bps = (ctx + page - 1) // page
    pool = B * bps
    bt = torch.randperm(pool, generator=g)[:B * bps].view(B, bps).to(torch.int32)
    idx = torch.stack([torch.randperm(ctx, generator=g)[:topk].sort().values
                       for _ in range(B)]).to(torch.int32)
    phys = bt.long().gather(1, idx.long() // page) * page + idx.long() % page
    sel = rows(torch.randn(B * topk, 576, generator=g), g).view(B, topk, 656)
    q = (torch.randn(B, H, 576, generator=g) * qmag).to(torch.float16)
    seq = torch.full((B,), ctx, dtype=torch.int32)
    return q, idx, bt, seq, sel, phys, pool


def paged_cache(sel: torch.Tensor, phys: torch.Tensor, pool: int, page: int, dev):
    """The paged cache on dev: zeros except the selected rows."""
    kv = torch.zeros(pool * page, 656, dtype=torch.uint8, device=dev)
    kv[phys.reshape(-1).to(dev)] = sel.reshape(-1, 656).to(dev)
    return kv.view(pool, page, 656)


def shared_case(seed: int, B: int, H: int, topk: int, n_rows: int, seqs, page: int = 64,
                qmag: float = 2.0, causal_spread: bool = False):
    """A prefill-shaped batch: B tokens of one sequence share a block-table
    row over a cache of n_rows rows (all carrying data); token b selects
    min(topk, seqs[b]) distinct sorted positions below seqs[b] (random, or
    spread evenly over the causal range), -1 padded.  Returns CPU tensors
    (q, idx, bt, seq, flat_rows [n_rows, 656])."""
    g = torch.Generator().manual_seed(seed)
    nblk = n_rows // page
    flat = rows(torch.randn(n_rows, 576, generator=g), g)
    bt = torch.randperm(nblk, generator=g).to(torch.int32)[None].expand(B, nblk).contiguous()
    seq = torch.tensor(seqs, dtype=torch.int32)
    idx = torch.full((B, topk), -1, dtype=torch.int32)
    u = torch.rand(B, generator=g, dtype=torch.float64)
    for b in range(B):
        L = int(seq[b])
        n = min(L, topk)
        if causal_spread:
            j = torch.arange(n, dtype=torch.float64)
            idx[b, :n] = torch.floor((j + u[b]) * L / n).to(torch.int32)
        else:
            idx[b, :n] = torch.randperm(L, generator=g)[:n].sort().values.to(torch.int32)
    q = (torch.randn(B, H, 576, generator=g) * qmag).to(torch.float16)
    return q, idx, bt, seq, flat


def selected(flat: torch.Tensor, idx: torch.Tensor, bt: torch.Tensor, page: int = 64):
    """Rows selected by the valid entries of every token, [B, n, 656]; all
    tokens must select the same number of positions."""
    ok = idx >= 0
    n = int(ok[0].sum())
    assert bool((ok.sum(1) == n).all())
    pos = idx[:, :n].long()
    phys = bt.long().gather(1, pos // page) * page + pos % page
    return flat[phys.reshape(-1)].view(idx.shape[0], n, 656)
