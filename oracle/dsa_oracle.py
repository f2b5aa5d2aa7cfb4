"""CPU restatement of the DSA hot-path ops -- TEST INFRASTRUCTURE ONLY.

Every function cites the reference file:line it restates (paths relative to
the bayley/glm5-on-v100 tree).  Inputs/outputs are CPU torch tensors with the
same layouts as the GPU ops.  Float math runs in fp32 or fp64 as noted;
integer/byte work is exact.
"""
from __future__ import annotations

import math

import numpy as np
import torch

FLT_MIN = float(np.finfo(np.float32).tiny)
DSMLA_ROW_BYTES = 656
IDXK_FP8_ROW_BYTES = 132
TOPK_NBIN = 4096


# ---------------------------------------------------------------------------
# e4m3 codec and monotone key
# ---------------------------------------------------------------------------
def e4m3_encode(x: torch.Tensor) -> torch.Tensor:
    """fp32 -> OCP e4m3 bytes with round-to-nearest-even and SATFINITE.

    Restates __nv_cvt_float_to_fp8(v, __NV_SATFINITE, __NV_E4M3)
    (sm70_mla_decode.cu:704) and the weight quantizer's clamp-then-cast
    (glue.patch:1529-1530).  torch's own cast is not saturating (it maps
    values above 464 to NaN), so the value is clamped to +-448 first; NaN
    stays NaN (0x7f with its sign).
    """
    xf = x.to(torch.float32)
    c = torch.where(torch.isnan(xf), xf, xf.clamp(-448.0, 448.0))
    return c.to(torch.float8_e4m3fn).view(torch.uint8)


def e4m3_decode(b: torch.Tensor) -> torch.Tensor:
    """e4m3 bytes -> exact fp32 values (sm70_attn_fp8.cu:16-20)."""
    return b.contiguous().view(torch.float8_e4m3fn).to(torch.float32)


def mono_key(x: torch.Tensor) -> torch.Tensor:
    """Monotone uint32 key of fp32 values as int64 (sm70_mla_decode.cu:43-46)."""
    u = x.contiguous().to(torch.float32).view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    neg = (u & 0x80000000) != 0
    return torch.where(neg, (~u) & 0xFFFFFFFF, u | 0x80000000)


# ---------------------------------------------------------------------------
# paged cache helpers
# ---------------------------------------------------------------------------
def resolve_rows(pos: torch.Tensor, bt_row: torch.Tensor, page: int,
                 n_rows: int) -> torch.Tensor:
    """Logical positions -> physical cache rows, -1 where the page index is
    beyond the table or the row is outside the cache
    (sm70_mla_decode.cu:186-193, :227-233, :983-989)."""
    pos = pos.to(torch.int64)
    pg = torch.div(pos, page, rounding_mode="floor")
    ok = (pos >= 0) & (pg < bt_row.numel())
    blk = torch.where(ok, bt_row.to(torch.int64)[pg.clamp(0, max(bt_row.numel() - 1, 0))],
                      torch.full_like(pos, -1))
    row = blk * page + (pos - pg * page)
    ok = ok & (row >= 0) & (row < n_rows)
    return torch.where(ok, row, torch.full_like(row, -1))


def idxk_rows_fp32(k_cache: torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
    """Gather indexer-K rows as fp32 (rows == -1 -> zeros).  fp16 cache:
    exact; fp8 132-B cache: e4m3 * per-row scale in fp32
    (idxk_fp8_load4, sm70_mla_decode.cu:106-115)."""
    ok = rows >= 0
    out = torch.zeros(rows.numel(), 128, dtype=torch.float32)
    if not bool(ok.any()):
        return out
    if k_cache.dtype == torch.float16:
        out[ok] = k_cache.reshape(-1, k_cache.shape[-1])[rows[ok]].to(torch.float32)
    else:
        fb = k_cache.reshape(-1, IDXK_FP8_ROW_BYTES)[rows[ok]]
        out[ok] = e4m3_decode(fb[:, :128].contiguous()) * fb[:, 128:132].contiguous().view(torch.float32)
    return out


def latent_rows_fp16(kv_cache: torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
    """Gather latent rows as the fp16 values the attention consumes
    (rows == -1 -> zeros).  fp8_ds_mla rows are dequantized as
    fp16_rn(e4m3 * tile_scale) for the 512 NoPE dims and copied for the 64
    fp16 RoPE dims (dsmla_load4, sm70_mla_decode.cu:81-100, then the fp16
    store into the key tile at :1006-1012).  Only the gathered rows are
    decoded."""
    ok = rows >= 0
    width = 576
    out = torch.zeros(rows.numel(), width, dtype=torch.float16)
    if not bool(ok.any()):
        return out
    if kv_cache.dtype == torch.float16:
        out[ok] = kv_cache.reshape(-1, kv_cache.shape[-1])[rows[ok]]
        return out
    fb = kv_cache.reshape(-1, DSMLA_ROW_BYTES)[rows[ok]]
    vals = e4m3_decode(fb[:, :512].contiguous()).view(-1, 4, 128)
    sc = fb[:, 512:528].contiguous().view(torch.float32).view(-1, 4, 1)
    nope = (vals * sc).reshape(-1, 512).to(torch.float16)
    rope = fb[:, 528:656].contiguous().view(torch.float16)
    out[ok] = torch.cat([nope, rope], dim=1)
    return out


# ---------------------------------------------------------------------------
# indexer-K store (sm70_mla_decode.cu:654-706, host :2910-2939)
# ---------------------------------------------------------------------------
def idxk_fp8_row(k_row: torch.Tensor) -> torch.Tensor:
    """One 128-dim fp16 key -> 132 bytes [128 e4m3 | fp32 scale] with
    scale = max(amax/448, FLT_MIN) (sm70_mla_decode.cu:690-705)."""
    v = k_row.to(torch.float32).reshape(-1, 128)
    amax = v.abs().amax(dim=1, keepdim=True)
    scale = torch.clamp(amax / 448.0, min=FLT_MIN)
    q = e4m3_encode(v / scale)
    sb = scale.to(torch.float32).contiguous().view(torch.uint8).reshape(-1, 4)
    return torch.cat([q, sb], dim=1)


def indexer_k_store(kv_cache: torch.Tensor, k: torch.Tensor,
                    slot: torch.Tensor) -> torch.Tensor:
    """Returns a copy of kv_cache with k[t] scattered into row slot[t];
    slots < 0 or >= n_rows are skipped.  Later tokens win on duplicate
    slots only in the sense that the reference is race-free per token; tests
    use unique slots."""
    out = kv_cache.clone()
    if out.dtype == torch.float16:
        flat = out.view(-1, k.shape[1])
        n_rows = flat.shape[0]
        for t in range(k.shape[0]):
            r = int(slot[t])
            if 0 <= r < n_rows:
                flat[r] = k[t]
        return out
    flat = out.view(-1, IDXK_FP8_ROW_BYTES)
    n_rows = flat.shape[0]
    rows = idxk_fp8_row(k)
    s = slot.to(torch.int64)
    ok = (s >= 0) & (s < n_rows)
    flat[s[ok]] = rows[ok]
    return out


# ---------------------------------------------------------------------------
# indexer logits (sm70_mla_decode.cu:150-329 decode, :542-653 packed)
# ---------------------------------------------------------------------------
def indexer_logits(q: torch.Tensor, k_cache: torch.Tensor, w: torch.Tensor,
                   bt: torch.Tensor, seq_lens: torch.Tensor, max_kv: int,
                   dtype=torch.float64, with_hist: bool = False):
    """score[b,p] = sum_h relu(q[b,h].K[row(b,p)]) * w[b,h] for p < seq_len,
    -inf for seq_len <= p < max_kv; K of an unresolvable row is 0.
    Returns (score fp32 [B,max_kv], hist int32 [B,4096] or None).  The dot
    and head sum run in `dtype` (fp64 default) and are rounded to fp32 once;
    for the fp8 cache the per-row scale multiplies the dot before the relu
    (sm70_mla_decode.cu:309-313)."""
    B = q.shape[0]
    page = k_cache.shape[-2]
    n_rows = k_cache.numel() // (k_cache.shape[-1])
    score = torch.full((B, max_kv), float("-inf"), dtype=torch.float32)
    hist = torch.zeros(B, TOPK_NBIN, dtype=torch.int32) if with_hist else None
    fp8 = k_cache.dtype == torch.uint8
    for b in range(B):
        L = min(int(seq_lens[b]), max_kv)
        if L <= 0:
            continue
        pos = torch.arange(L)
        rows = resolve_rows(pos, bt[b], page, n_rows)
        if fp8:
            flat_b = k_cache.reshape(-1, IDXK_FP8_ROW_BYTES)
            kv = torch.zeros(L, 128, dtype=dtype)
            sc = torch.zeros(L, dtype=dtype)
            ok = rows >= 0
            kv[ok] = e4m3_decode(flat_b[rows[ok], :128].contiguous()).to(dtype)
            sc[ok] = flat_b[rows[ok], 128:132].contiguous().view(torch.float32).reshape(-1).to(dtype)
            dots = (q[b].to(dtype) @ kv.T) * sc  # [32, L]
        else:
            kv = idxk_rows_fp32(k_cache, rows).to(dtype)
            dots = q[b].to(dtype) @ kv.T
        s = (torch.relu(dots) * w[b].to(dtype)[:, None]).sum(dim=0)
        score[b, :L] = s.to(torch.float32)
        if with_hist:
            bins = (mono_key(score[b, :L]) >> 20).to(torch.int64)
            hist[b] = torch.bincount(bins, minlength=TOPK_NBIN).to(torch.int32)
    return score, hist


def pack_indexer_q(q: torch.Tensor) -> torch.Tensor:
    """[n,32,128] -> [32, ceil(n/16), 8, 16, 16] (zero-padded rows), the
    packing of reference/sparse_attn_indexer.py:136-145."""
    n = q.shape[0]
    n16 = (n + 15) // 16 * 16
    if n16 != n:
        q = torch.nn.functional.pad(q, (0, 0, 0, 0, 0, n16 - n))
    return (q.reshape(n16 // 16, 16, 32, 8, 16).permute(2, 0, 3, 1, 4).contiguous())


def unpack_indexer_q(qp: torch.Tensor, n: int) -> torch.Tensor:
    """Inverse of pack_indexer_q."""
    nqt = qp.shape[1]
    return qp.permute(1, 3, 0, 2, 4).reshape(nqt * 16, 32, 128)[:n]


def indexer_logits_packed(qp: torch.Tensor, k_cache, w, bt, seq_lens, max_kv,
                          dtype=torch.float64, qt: int = 32):
    """Prefill logits from packed Q (sm70_mla_decode.cu:542-653).  Two
    things differ from the decode kernel's contract:
      * every 32-query tile gathers its keys with the block-table row of the
        tile's first query, qbase = tile * 32 (:556, :566; QT = 32, :548);
        rows of the tile below it are not consulted (callers pass one row,
        expanded, sparse_attn_indexer.py:764-781);
      * an fp8 key is dequantised to fp16 before the dot:
        fp16_rn(fp32(e4m3 * scale)) (idxk_fp8_load4 :106-115, then
        __float2half into the key tile, :561-580); fp16 keys are used as
        stored."""
    B = w.shape[0]
    q = unpack_indexer_q(qp, B)
    first = (torch.arange(B) // qt) * qt
    bt_tile = bt.index_select(0, first)
    if k_cache.dtype == torch.uint8:
        flat = k_cache.reshape(-1, IDXK_FP8_ROW_BYTES)
        k16 = (e4m3_decode(flat[:, :128].contiguous()) *
               flat[:, 128:132].contiguous().view(torch.float32)).to(torch.float16)
        k_cache = k16.view(*k_cache.shape[:-1], 128)
    return indexer_logits(q, k_cache, w, bt_tile, seq_lens, max_kv, dtype)[0]


# ---------------------------------------------------------------------------
# top-k selection (contract of sm70_mla_decode.cu:1187-1212 made exact)
# ---------------------------------------------------------------------------
def topk_rows(score: torch.Tensor, seq_lens: torch.Tensor, k: int) -> torch.Tensor:
    """idx[r,:] = positions p < min(seq_len[r], width) of the k largest
    scores (32-bit monotone-key order, equal keys -> lower position first),
    emitted in ascending position order, -1 padded.  numpy lexsort brute
    force."""
    score = score.contiguous()
    R, W = score.shape
    out = np.full((R, k), -1, dtype=np.int32)
    keys = mono_key(score).numpy()
    for r in range(R):
        L = max(0, min(int(seq_lens[r]), W))
        if L == 0:
            continue
        kr = keys[r, :L]
        pos = np.arange(L)
        order = np.lexsort((pos, -kr))  # primary: key desc, secondary: pos asc
        sel = np.sort(order[:k])
        out[r, :sel.size] = sel
    return torch.from_numpy(out)


# ---------------------------------------------------------------------------
# sparse MLA attention (sm70_mla_decode.cu:918-1184; triton_mla.py:494-554)
# ---------------------------------------------------------------------------
def scaled_q(q: torch.Tensor, scale: float) -> torch.Tensor:
    """q * scale rounded to fp16 with the scale itself rounded to fp16
    (__hmul(q, __float2half(scale)), sm70_mla_decode.cu:1016-1018)."""
    s16 = float(torch.tensor(scale, dtype=torch.float16))
    return (q.to(torch.float32) * s16).to(torch.float16)


def sparse_mla(q: torch.Tensor, kv_cache: torch.Tensor, idx: torch.Tensor,
               bt: torch.Tensor, seq_lens: torch.Tensor, scale: float,
               dtype=torch.float64, empty_lse: float | None = None,
               zero_unresolved: bool | None = None):
    """Reference sparse attention for every token/head.  A selected entry j
    takes part iff 0 <= idx < seq_len (sm70_mla_decode.cu:1047-1053).  Its
    row is bt[b, idx / page] * page + idx % page; when that row does not
    resolve (negative block, or row outside the cache) the reference's two
    kernels differ, and the op follows the reference's dispatch
    (sm70_mla_decode.cu:2511):
      * B >= 32 and H <= 16 (its prefill kernel): the key is masked
        (row -1 -> invalid, :1617-1628, :1705);
      * otherwise (its split-decode kernel): the key reads as a zero row and
        stays in the softmax with score 0 (:970-992 zero-fills the tile,
        :1047-1053 tests only the position range).
    zero_unresolved=None picks that rule; True/False forces one.  An entry
    whose page index is past the block table's width is masked either way
    (the reference reads its table out of bounds there, which defines
    nothing).  Returns (o fp32 [B,H,512], lse fp32 [B,H]); tokens with no
    key get o = 0 and lse = empty_lse, by default the op's: -1e30 on the
    prefill-kernel shapes (lse = m_init + ln 1, :1789-1793), else -inf
    (merge convention, :1175-1183)."""
    B, H, D = q.shape
    page = kv_cache.shape[-2]
    row_w = kv_cache.shape[-1]
    n_rows = kv_cache.numel() // row_w
    o = torch.zeros(B, H, 512, dtype=torch.float32)
    prefill_shape = B >= 32 and H <= 16
    if empty_lse is None:
        empty_lse = -1e30 if prefill_shape else float("-inf")
    if zero_unresolved is None:
        zero_unresolved = not prefill_shape
    lse = torch.full((B, H), empty_lse, dtype=torch.float32)
    qs = scaled_q(q, scale).to(dtype)
    for b in range(B):
        sel = idx[b].to(torch.int64)
        L = int(seq_lens[b])
        valid = (sel >= 0) & (sel < L)
        in_table = valid & (torch.div(sel, page, rounding_mode="floor") < bt.shape[1])
        rows = resolve_rows(torch.where(valid, sel, torch.zeros_like(sel)),
                            bt[b], page, n_rows)
        rows = torch.where(valid, rows, torch.full_like(rows, -1))
        use = rows >= 0
        if zero_unresolved:
            use = use | in_table  # unresolved rows stay as zero keys
        if not bool(use.any()):
            continue
        kv = latent_rows_fp16(kv_cache, rows[use]).to(dtype)  # [n, 576]
        s = qs[b] @ kv.T  # [H, n]
        m = s.max(dim=1, keepdim=True).values
        p = torch.exp(s - m)
        l = p.sum(dim=1, keepdim=True)
        o[b] = ((p @ kv[:, :512]) / l).to(torch.float32)
        lse[b] = (m + torch.log(l)).squeeze(1).to(torch.float32)
    return o, lse


def dense_mla(q: torch.Tensor, kv_cache: torch.Tensor, bt: torch.Tensor,
              seq_lens: torch.Tensor, scale: float, dtype=torch.float64):
    """Dense causal MLA decode over positions [0, seq_len): the plain-torch
    path of reference/triton_mla.py:494-554 (gather -> bmm -> mask ->
    softmax -> bmm), with q scaled as the sparse kernel does."""
    B = q.shape[0]
    max_kv = bt.shape[1] * kv_cache.shape[-2]
    idx = torch.arange(max_kv, dtype=torch.int32).expand(B, max_kv).contiguous()
    return sparse_mla(q, kv_cache, idx, bt, seq_lens, scale, dtype)


def mla_decode(q: torch.Tensor, kv_cache: torch.Tensor, bt: torch.Tensor,
               seq_lens: torch.Tensor, scale: float, fp16_acc: bool = False, tile: int = 32):
    """Dense MLA decode, the reference's sm70_mla_decode
    (sm70_mla_decode.cu:717-898, host :1474-1534): positions [0, seq_len) of
    an fp16 latent cache, q * fp16(scale) rounded to fp16 (:793-794), V = the
    first 512 dims, lse = m + ln l, and o = 0 / lse = -inf for a token with no
    valid position (:887-895).

    A position below seq_len whose row does not resolve (page index past the
    table, negative block, row outside the cache) reads a zero row and stays
    in the softmax with score 0 (:762-771, :826-832).  Positions at or past
    the table's width (max_blocks * page) are not attended: the reference
    reads its block table out of bounds there (:766), which defines nothing.

    fp16_acc=False: exact (fp64) attention.
    fp16_acc=True: the kernel's own arithmetic tile by tile (`tile` keys,
    :759): running max from -1e30 (:746), p = exp(s - m) rounded to fp16 for
    PV while l sums the unrounded p (:839-841), and the running O kept in
    fp16 -- rescaled by alpha and rounded (:850-851), then the tile's P V
    (fp32 sum) added and rounded again (:873-875); o = fp16(O / l)."""
    B, H, _ = q.shape
    page = kv_cache.shape[-2]
    n_rows = kv_cache.numel() // 576
    flat = kv_cache.reshape(n_rows, 576)
    o = torch.zeros(B, H, 512, dtype=torch.float32)
    lse = torch.full((B, H), float("-inf"), dtype=torch.float32)
    qs = scaled_q(q, scale).to(torch.float64)
    for b in range(B):
        L = min(int(seq_lens[b]), bt.shape[1] * page)
        if not fp16_acc:
            if L <= 0:
                continue
            rows = resolve_rows(torch.arange(L), bt[b], page, n_rows)
            kv = torch.zeros(L, 576, dtype=torch.float64)
            ok = rows >= 0
            kv[ok] = flat[rows[ok]].to(torch.float64)
            sc = qs[b] @ kv.T                                  # [H, L]
            mx = sc.max(dim=1, keepdim=True).values
            p = torch.exp(sc - mx)
            l = p.sum(dim=1, keepdim=True)
            o[b] = ((p @ kv[:, :512]) / l).to(torch.float32)
            lse[b] = (mx + torch.log(l)).squeeze(1).to(torch.float32)
            continue
        m = torch.full((H,), -1e30, dtype=torch.float64)
        l = torch.zeros(H, dtype=torch.float64)
        acc = torch.zeros(H, 512, dtype=torch.float16)
        for base in range(0, L, tile):
            pos = torch.arange(base, min(base + tile, L))
            rows = resolve_rows(pos, bt[b], page, n_rows)
            kv = torch.zeros(tile, 576, dtype=torch.float64)
            ok = rows >= 0
            kv[:len(pos)][ok] = flat[rows[ok]].to(torch.float64)
            s = qs[b] @ kv.T                                  # [H, tile]
            s[:, len(pos):] = float("-inf")
            m_cur = torch.maximum(m, s.max(dim=1).values)
            alpha = torch.exp(m - m_cur)
            p = torch.where(torch.isinf(s), torch.zeros_like(s), torch.exp(s - m_cur[:, None]))
            l = l * alpha + p.sum(dim=1)
            m = m_cur
            acc = (acc.to(torch.float64) * alpha[:, None]).to(torch.float16)
            pv = p.to(torch.float16).to(torch.float64) @ kv[:, :512]
            acc = (acc.to(torch.float64) + pv).to(torch.float16)
        pos_l = l > 0
        inv = torch.where(pos_l, 1.0 / torch.where(pos_l, l, torch.ones_like(l)), torch.zeros_like(l))
        o[b] = (acc.to(torch.float64) * inv[:, None]).to(torch.float16).to(torch.float32)
        lse[b] = torch.where(pos_l, m + torch.log(torch.where(pos_l, l, torch.ones_like(l))),
                             torch.full_like(m, float("-inf"))).to(torch.float32)
    return o, lse


def varlen_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     cu_q, cu_k, scale: float, causal: bool):
    """Dense varlen attention as the reference's MLA prefill backend computes
    it (vllm/v1/attention/backends/mla/prefill/sm70_triton.py:54-187), here
    in fp64 without tiling: per sequence, s = scale * q k^T; with `causal`,
    key j is masked for query i when j > i + (k_len - q_len) (:117-123,
    :145-152); softmax over the unmasked keys.  A query with no key (k_len 0,
    or every key masked) gets out = 0 and lse = -inf (:106-112, :175-185).
    Returns out fp64 [total_q, H, Dv] and lse fp64 [H, total_q]."""
    cu_q = [int(x) for x in cu_q]
    cu_k = [int(x) for x in cu_k]
    total_q, H, _ = q.shape
    out = torch.zeros(total_q, H, v.shape[2], dtype=torch.float64)
    lse = torch.full((H, total_q), float("-inf"), dtype=torch.float64)
    for i in range(len(cu_q) - 1):
        qs, qe, ks, ke = cu_q[i], cu_q[i + 1], cu_k[i], cu_k[i + 1]
        q_len, k_len = qe - qs, ke - ks
        if q_len == 0 or k_len == 0:
            continue
        qi = q[qs:qe].double().transpose(0, 1)           # [H, q_len, D]
        ki = k[ks:ke].double().transpose(0, 1)
        vi = v[ks:ke].double().transpose(0, 1)
        sc = torch.matmul(qi, ki.transpose(1, 2)) * scale  # [H, q_len, k_len]
        if causal:
            qpos = torch.arange(q_len)[:, None] + (k_len - q_len)
            sc = sc.masked_fill(torch.arange(k_len)[None, :] > qpos, float("-inf"))
        m = sc.max(dim=2, keepdim=True).values
        has = torch.isfinite(m)
        msafe = torch.where(has, m, torch.zeros_like(m))
        p = torch.exp(sc - msafe)
        l = p.sum(dim=2, keepdim=True)
        o = torch.matmul(p, vi) / torch.where(l > 0, l, torch.ones_like(l))
        out[qs:qe] = o.transpose(0, 1)
        lse[:, qs:qe] = torch.where(l > 0, msafe + torch.log(l),
                                    torch.full_like(l, float("-inf"))).squeeze(2)
    return out, lse


def shard_merge_rows(allf: torch.Tensor, K: int) -> torch.Tensor:
    """Exact top-K merge of key-shard candidates, the reference's fused merge
    (sm70_mla_decode.cu:2055-2182): allf fp32 [tp, R, 2K] (K scores, then K
    positions as int32 bits, per shard and row).  Per row, the K largest
    64-bit keys (mono(score) << 32) | (tp*K - 1 - col), col = s*K + c
    (:2090-2100); a selection with mono <= mono(-inf) = 0x007FFFFF gives -1
    (:2145-2152); positions sorted ascending (:2156-2173).  Returns int32
    [R, K]."""
    tp, R, _ = allf.shape
    ncand = tp * K
    vals = allf[:, :, :K].permute(1, 0, 2).reshape(R, ncand).contiguous()
    pos = allf[:, :, K:].permute(1, 0, 2).reshape(R, ncand).contiguous().view(torch.int32)
    u = vals.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    mono = torch.where(u >= 0x80000000, (~u) & 0xFFFFFFFF, u | 0x80000000)
    col = torch.arange(ncand, dtype=torch.int64)
    key = (mono << 32) | (ncand - 1 - col)
    # keys are below 2^64; compare as int64 after flipping the sign bit
    skey = key ^ (-(2 ** 63))
    top = torch.argsort(skey, dim=1, descending=True)[:, :K]
    sel_mono = mono.gather(1, top)
    sel_pos = pos.to(torch.int64).gather(1, top)
    sel = torch.where(sel_mono > 0x007FFFFF, sel_pos, torch.full_like(sel_pos, -1))
    return sel.sort(dim=1).values.to(torch.int32)


# ---------------------------------------------------------------------------
# fp8_ds_mla latent-cache writer (generator side; the reference's writer
# concat_and_cache_ds_mla is not vendored, only its 656-B layout is:
# sm70_mla_decode.cu:74-100, triton_mla.py:92-95)
# ---------------------------------------------------------------------------
def dsmla_rows(latent: torch.Tensor, per_tile: bool = False) -> torch.Tensor:
    """[n,576] fp16/fp32 -> [n,656] uint8 rows.  NoPE scale = amax/448 over
    the 512 NoPE dims written into all 4 tile slots (per_tile=False), or
    one amax/448 per 128-dim tile (per_tile=True); RoPE copied as fp16."""
    x = latent.to(torch.float32)
    n = x.shape[0]
    nope = x[:, :512].reshape(n, 4, 128)
    if per_tile:
        amax = nope.abs().amax(dim=2, keepdim=True)
    else:
        amax = nope.abs().amax(dim=(1, 2), keepdim=True).expand(n, 4, 1)
    scale = torch.clamp(amax / 448.0, min=FLT_MIN).contiguous()
    qb = e4m3_encode(nope / scale).reshape(n, 512)
    sb = scale.reshape(n, 4).contiguous().view(torch.uint8).reshape(n, 16)
    rb = x[:, 512:576].to(torch.float16).contiguous().view(torch.uint8).reshape(n, 128)
    return torch.cat([qb, sb, rb], dim=1).contiguous()


def concat_and_cache_mla(kv_cache: torch.Tensor, kv_c: torch.Tensor, k_pe: torch.Tensor,
                         slot: torch.Tensor, kv_cache_dtype: str) -> torch.Tensor:
    """Returns a copy of the latent cache with token t written to row
    slot[t] (slots < 0 or >= n_rows skipped), following vLLM's
    concat_and_cache_mla:
      * "auto": row = [kv_c | k_pe] in fp16 (576 halves);
      * "fp8_ds_mla": row = 512 e4m3 bytes with one scale per 128-dim tile,
        scale = max(amax/448, FLT_MIN) (amax of |kv_c| over the tile as the
        reference's fixed hunk computes it, patches/glm5-v100-sm70-glue.patch:
        517-531), e4m3 = RNE-satfinite(v/scale); then the 4 fp32 scales; then
        k_pe's 16-bit values unchanged (fp16 or bf16 bits)."""
    out = kv_cache.clone()
    T = slot.shape[0]
    s = slot.to(torch.int64)
    if kv_cache_dtype == "auto":
        flat = out.view(-1, 576)
        rows = torch.cat([kv_c[:T].to(torch.float16), k_pe[:T].to(torch.float16)], dim=1)
    else:
        flat = out.view(-1, DSMLA_ROW_BYTES)
        x = kv_c[:T].to(torch.float32).reshape(T, 4, 128)
        amax = torch.nan_to_num(x.abs(), nan=0.0).amax(dim=2, keepdim=True)
        scale = torch.clamp(amax / 448.0, min=FLT_MIN)
        qb = e4m3_encode(x / scale).reshape(T, 512)
        sb = scale.reshape(T, 4).contiguous().view(torch.uint8).reshape(T, 16)
        rb = k_pe[:T].contiguous().view(torch.uint8).reshape(T, 128)
        rows = torch.cat([qb, sb, rb], dim=1)
    n_rows = flat.shape[0]
    ok = (s >= 0) & (s < n_rows)
    flat[s[ok]] = rows[ok]
    return out


# ---------------------------------------------------------------------------
# fp8 weight-only projections (glue.patch:1515-1532; sm70_attn_fp8.cu)
# ---------------------------------------------------------------------------
def attn_fp8_quantize(weight: torch.Tensor):
    """[128,128]-block e4m3 quantization of an [N,K] weight: pad to 128
    multiples, scale = clamp(amax/448, 1e-12), q = clamp(w/scale, +-448) ->
    e4m3, crop (restates _sm70_attn_fp8_quantize, glue.patch:1515-1532)."""
    n, k = weight.shape
    nb, kb = (n + 127) // 128, (k + 127) // 128
    padded = torch.zeros(nb * 128, kb * 128, dtype=torch.float32)
    padded[:n, :k] = weight.float()
    blocks = padded.view(nb, 128, kb, 128)
    scale = (blocks.abs().amax(dim=(1, 3)) / 448.0).clamp(min=1e-12)
    qv = (blocks / scale[:, None, :, None]).clamp(-448.0, 448.0)
    q8 = qv.to(torch.float8_e4m3fn).view(torch.uint8)
    q8 = q8.view(nb * 128, kb * 128)[:n, :k].contiguous()
    return q8, scale.contiguous()


def expand_block_scale(s: torch.Tensor, n: int, k: int) -> torch.Tensor:
    return s.repeat_interleave(128, 0).repeat_interleave(128, 1)[:n, :k]


def attn_fp8_dequant(w: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """fp16_rn(fp32(e4m3(w) * s)) (sm70_attn_fp8.cu:122-144)."""
    n, k = w.shape
    return (e4m3_decode(w) * expand_block_scale(s, n, k)).to(torch.float16)


def attn_fp8_gemv(x: torch.Tensor, w: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """y = x @ deq(W)^T in fp64 (sm70_attn_fp8.cu:51-116 computes the same
    sum with fp16/fp32 partial sums)."""
    n, k = w.shape
    deq = e4m3_decode(w).double() * expand_block_scale(s, n, k).double()
    return x.double() @ deq.T


# ---------------------------------------------------------------------------
# one DSA layer step: the reference's callers of the ops
# (sparse_attn_indexer.py:528-881, triton_mla.py:212-301 and :365-492)
# ---------------------------------------------------------------------------
def q_latent(q: torch.Tensor, W_UK_T: torch.Tensor) -> torch.Tensor:
    """[T, H, P + 64] -> [T, H, 576] fp16: q_nope @ W_UK_T per head in fp64,
    rounded to fp16, then q_pe (triton_mla.py:413-418)."""
    P = W_UK_T.shape[1]
    ql = torch.einsum("thp,hpl->thl", q[..., :P].double(), W_UK_T.double())
    return torch.cat([ql, q[..., P:].double()], dim=-1).to(torch.float16)


def v_up(o: torch.Tensor, W_UV: torch.Tensor) -> torch.Tensor:
    """o [T, H, 512] (the kernel's fp16 output) @ W_UV per head, fp64
    (triton_mla.py:486-492): [T, H * V]."""
    T, H, _ = o.shape
    return torch.einsum("thl,hlv->thv", o.to(torch.float16).double(),
                        W_UV.double()).reshape(T, -1)


def dsa_layer_decode(q, idx_q, idx_w, block_table, seq_lens, latent_cache, idx_k_cache,
                     W_UK_T, W_UV, scale, topk=2048):
    """Decode step with per-token rows already expanded (block_table and
    seq_lens [B]): indexer logits -> top-k -> sparse attention -> v_up.
    Returns (out, idx, o, lse)."""
    page = idx_k_cache.shape[1]
    max_kv = block_table.shape[1] * page
    score, _ = indexer_logits(idx_q, idx_k_cache, idx_w, block_table, seq_lens, max_kv)
    idx = topk_rows(score, seq_lens, topk)
    o, lse = sparse_mla(q_latent(q, W_UK_T), latent_cache, idx, block_table, seq_lens, scale)
    return v_up(o, W_UV), idx, o, lse


def dsa_layer_prefill_topk(idx_q, idx_w, bounds, block_table, causal_len, idx_k_cache,
                           topk=2048, kt=64):
    """Prefill top-k rows: per request r (token rows [bounds[r], bounds[r+1])),
    scores over the request's block-table row up to each token's causal
    length; the reference's sub-chunking and the 64-key launch rounding do
    not change the selected sets (sparse_attn_indexer.py:760-881)."""
    T = idx_q.shape[0]
    page = idx_k_cache.shape[1]
    out = torch.full((T, topk), -1, dtype=torch.int32)
    for r in range(len(bounds) - 1):
        lo, hi = bounds[r], bounds[r + 1]
        if hi <= lo:
            continue
        cl = causal_len[lo:hi].to(torch.int32)
        max_kv = max(min(block_table.shape[1] * page,
                         (int(cl.max()) + kt - 1) // kt * kt), page)
        bt = block_table[r:r + 1].expand(hi - lo, -1)
        score, _ = indexer_logits(idx_q[lo:hi], idx_k_cache, idx_w[lo:hi], bt, cl, max_kv)
        out[lo:hi] = topk_rows(score, cl, topk)
    return out


def dsa_layer_prefill(q, idx_q, idx_w, bounds, block_table, causal_len, latent_cache,
                      idx_k_cache, W_UK_T, W_UV, scale, topk=2048):
    """Prefill step: top-k per token, attention with per-token causal lengths
    and per-token block-table rows, v_up.  Returns (out, idx, o, lse)."""
    idx = dsa_layer_prefill_topk(idx_q, idx_w, bounds, block_table, causal_len, idx_k_cache,
                                 topk)
    req = torch.repeat_interleave(torch.arange(len(bounds) - 1),
                                  torch.tensor([bounds[r + 1] - bounds[r]
                                                for r in range(len(bounds) - 1)]))
    bt = block_table.index_select(0, req)
    o, lse = sparse_mla(q_latent(q, W_UK_T), latent_cache, idx, bt,
                        causal_len.to(torch.int32), scale)
    return v_up(o, W_UV), idx, o, lse
