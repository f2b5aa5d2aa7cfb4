"""One DSA attention layer step on top of the hot-path ops: the caller side
of the kernels, as the reference's model runner drives them.

Decode (reference/sparse_attn_indexer.py:528-639 with the fused decode top-k,
then reference/triton_mla.py:212-301 _forward_mqa_sparse and the layer's
v_up projection):
  1. write the step's tokens into the latent cache (concat_and_cache_mla)
     and the indexer-K cache (sm70_indexer_k_store);
  2. indexer logits with the level-1 histogram, then sm70_decode_topk;
  3. q_nope -> latent through W_UK_T (bmm over heads), concatenated with q_pe;
  4. sparse MLA attention over the top-k rows;
  5. o -> values through W_UV (bmm over heads).
Steps 3 and 5 run the per-head projection kernel (mi355_dsa_head_proj)
instead of the reference's transposes, bmm and concatenation.  With the
step's tokens given (the usual decode shapes) the step is five launches:
the cache writes fused into the indexer logits launch
(mi355_dsa_decode_layer_indexer), the top-k scan and select with step 3 run
in the select launch (mi355_dsa_decode_layer_topk, which also leaves the
layer's histogram zero for the next step), the attention, and the split merge
fused with step 5 (mi355_dsa_decode_layer_attention).  All are bit-identical
to the separate ops.  Everything runs in order on the caller's stream: a
second stream for the latent write and step 3 (which do not feed the
indexer) made a captured decode layer slower (106.7 vs 96.0 us at 180k
context), the cross-stream join costing more than the overlap hides.
Speculative decode rows (B tokens over B / next_n requests) are expanded per
token as the reference does (triton_mla.py:267-279).

Prefill (sparse_attn_indexer.py:641-881 without tensor-parallel key
sharding, then triton_mla.py:380-492 _forward_mha_sparse): per request and
per `sub_rows`-row sub-chunk, the packed indexer logits over the causal reach
of the sub-chunk (rounded up to the 64-key tile) and persistent_topk with the
per-token causal lengths; then the attention with per-token causal lengths and
per-token block-table rows, and the W_UV projection.  The reference splits a
request into 128-row sub-chunks to bound the fp32 score buffer (sub_rows x
reach) on a 32 GB card; here `sub_rows` defaults to 1024 (256 MB at 64k
reach), which on a 64k causal prefill takes the logits from 36 % to 45 % of
the fp16 MFMA peak (fewer, fuller launches; 2048 is level, larger is slower
once the buffer leaves the 256 MB MALL).

All buffers come from torch's caching allocator; nothing here synchronises
the host except the per-sub-chunk causal reach, which the reference also reads
on the host (memoized per chunk, :774-789) and which callers can pass in.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _cache_ops, _lib, _sm70_ops
from .ops import _check, _stream

KT = 64  # key tile the prefill logits launch is rounded to (sparse_attn_indexer.py:753)


@dataclass
class DsaLayerWeights:
    """W_UK_T [H, P, 512] and W_UV [H, 512, V] fp16 (built from kv_b_proj as
    triton_mla.py:388-412 does), softmax scale of the 576-dim latent q.
    The projection kernel reads each head's weight transposed (k
    contiguous); those copies are made once here, as the reference makes
    W_UK_T once after loading."""
    W_UK_T: torch.Tensor
    W_UV: torch.Tensor
    scale: float

    def __post_init__(self):
        _check(self.W_UK_T.dtype == torch.float16 and self.W_UV.dtype == torch.float16,
               "W_UK_T and W_UV must be fp16")
        _check(self.W_UK_T.dim() == 3 and self.W_UK_T.shape[2] == 512
               and self.W_UV.dim() == 3 and self.W_UV.shape[1] == 512
               and self.W_UV.shape[0] == self.W_UK_T.shape[0],
               "W_UK_T must be [H, P, 512] and W_UV [H, 512, V]")
        self.uk_t = self.W_UK_T.transpose(1, 2).contiguous()   # [H, 512, P]
        self.uv_t = self.W_UV.transpose(1, 2).contiguous()     # [H, V, 512]

    @property
    def n_heads(self) -> int:
        return self.W_UK_T.shape[0]

    @property
    def nope_dim(self) -> int:
        return self.W_UK_T.shape[1]

    @property
    def v_dim(self) -> int:
        return self.W_UV.shape[2]


def _rows8(x: torch.Tensor) -> torch.Tensor:
    """x with unit last stride, 16-byte aligned, token / head strides that
    are multiples of 8 elements (what the kernel loads 16 B at a time)."""
    ok = (x.stride(2) == 1 and x.stride(1) % 8 == 0 and x.stride(0) % 8 == 0
          and x.data_ptr() % 16 == 0)
    return x if ok else x.contiguous()


def head_proj(out: torch.Tensor, x: torch.Tensor, wt: torch.Tensor, tail: int) -> None:
    """out[t, h, :N] = x[t, h, :K] @ wt[h].T, out[t, h, N:N+tail] = x[t, h, K:K+tail];
    x [T, H, >= K + tail], wt [H, N, K], out [T, H, >= N + tail] (fp16)."""
    _check(x.is_cuda and wt.is_cuda and out.is_cuda, "all tensors must be on the GPU")
    _check(x.dtype == torch.float16 and wt.dtype == torch.float16 and out.dtype == torch.float16,
           "head_proj: fp16 tensors expected")
    _check(wt.is_contiguous() and out.stride(2) == 1, "head_proj: wt contiguous, out rows dense")
    H, N, K = wt.shape
    T = x.shape[0]
    _check(x.shape[1] == H and out.shape[:2] == (T, H), "head_proj: token / head shapes differ")
    with torch.cuda.device(x.device):
        _lib.call("mi355_dsa_head_proj", out.data_ptr(), out.stride(0), out.stride(1),
                  x.data_ptr(), x.stride(0), x.stride(1), wt.data_ptr(), T, H, N, K, tail,
                  _stream(x))


def q_latent(q: torch.Tensor, w: DsaLayerWeights) -> torch.Tensor:
    """q [T, H, P + 64] -> [T, H, 576] fp16: bmm(q_nope, W_UK_T) | q_pe
    (triton_mla.py:413-418), one launch."""
    _check(q.dim() == 3 and q.shape[2] == w.nope_dim + 64, "q must be [T, H, P + 64]")
    q = _rows8(q)
    out = torch.empty(q.shape[0], q.shape[1], 576, dtype=torch.float16, device=q.device)
    head_proj(out, q, w.uk_t, 64)
    return out


def v_up(o: torch.Tensor, w: DsaLayerWeights) -> torch.Tensor:
    """o [T, H, 512] -> [T, H * V]: bmm over heads with W_UV
    (triton_mla.py:486-492), one launch."""
    T, H, _ = o.shape
    out = torch.empty(T, H * w.v_dim, dtype=torch.float16, device=o.device)
    head_proj(out.view(T, H, w.v_dim), _rows8(o), w.uv_t, 0)
    return out


class DsaLayer:
    """One layer's caches and weights; decode() / prefill() run a step."""

    _HIST_ROWS = 64  # tokens the fused indexer launch takes per step

    def __init__(self, weights: DsaLayerWeights, latent_cache: torch.Tensor,
                 idx_k_cache: torch.Tensor, topk: int = 2048):
        self.w = weights
        self.latent_cache = latent_cache   # [n_blocks, page, 656] u8 or [.., 576] fp16
        self.idx_k_cache = idx_k_cache     # [n_blocks, page, 128] fp16 or [.., 132] u8
        self.topk = topk
        self.kv_dtype = "fp8_ds_mla" if latent_cache.dtype == torch.uint8 else "auto"
        # the writer's (unused) scale argument, made once: a fill per step costs a launch
        self._one = torch.ones((), device=latent_cache.device)
        self._hists: dict = {}

    # -- cache writes -------------------------------------------------------
    def store(self, kv_c: torch.Tensor, k_pe: torch.Tensor, idx_k: torch.Tensor,
              slot_mapping: torch.Tensor) -> None:
        """Writes the step's tokens into both paged caches (slot < 0 skipped)."""
        self.store_latent(kv_c, k_pe, slot_mapping)
        self.store_index_key(idx_k, slot_mapping)

    def store_latent(self, kv_c: torch.Tensor, k_pe: torch.Tensor,
                     slot_mapping: torch.Tensor) -> None:
        _cache_ops.concat_and_cache_mla(kv_c, k_pe, self.latent_cache, slot_mapping,
                                        self.kv_dtype, self._one)

    def store_index_key(self, idx_k: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        _sm70_ops.sm70_indexer_k_store(self.idx_k_cache, idx_k.to(torch.float16).contiguous(),
                                       slot_mapping.to(torch.int32))

    # -- decode -------------------------------------------------------------
    def decode_topk(self, idx_q: torch.Tensor, idx_w: torch.Tensor,
                    block_table: torch.Tensor, seq_lens: torch.Tensor,
                    hist: torch.Tensor | None = None) -> torch.Tensor:
        """Indexer logits + fused histogram + decode top-k: idx [B, topk].
        hist, if given, is an already cleared int32 [B, 4096]."""
        B = idx_q.shape[0]
        page = self.idx_k_cache.shape[1]
        max_kv = block_table.shape[1] * page
        score = torch.empty(B, max_kv, dtype=torch.float32, device=idx_q.device)
        if hist is None:
            hist = torch.zeros(B, 4096, dtype=torch.int32, device=idx_q.device)
        idx = torch.empty(B, self.topk, dtype=torch.int32, device=idx_q.device)
        _sm70_ops.sm70_indexer_logits(score, idx_q.contiguous(), self.idx_k_cache,
                                      idx_w.contiguous(), block_table, seq_lens, hist)
        _sm70_ops.sm70_decode_topk(idx, score, seq_lens, hist, self.topk)
        return idx

    def decode(self, q: torch.Tensor, idx_q: torch.Tensor, idx_w: torch.Tensor,
               block_table: torch.Tensor, seq_lens: torch.Tensor,
               kv_c: torch.Tensor | None = None, k_pe: torch.Tensor | None = None,
               idx_k: torch.Tensor | None = None,
               slot_mapping: torch.Tensor | None = None) -> torch.Tensor:
        """q [B, H, P + 64], idx_q [B, 32, 128], idx_w [B, 32]; block_table
        [R, max_blocks] and seq_lens [R] per request (R = B / next_n, seq_lens
        counting the step's tokens).  With kv_c / k_pe / idx_k / slot_mapping
        the step's tokens are first written to the caches.  Returns
        out [B, H * V]."""
        B, R = q.shape[0], seq_lens.shape[0]
        bt = block_table.to(torch.int32)
        sl = seq_lens.to(torch.int32)
        if B != R:  # spec-as-decode: per-token rows (triton_mla.py:267-279)
            assert B % R == 0, f"non-uniform decode batch: {B} tokens, {R} requests"
            n = B // R
            offs = torch.arange(n, device=q.device, dtype=torch.int32)
            sl = (sl.unsqueeze(1) - (n - 1) + offs).reshape(-1).contiguous()
            bt = bt.repeat_interleave(n, dim=0).contiguous()
        hist = None
        fusable = kv_c is not None and self._fusable(q, kv_c, k_pe, idx_k, slot_mapping)
        if fusable and self._indexer_fusable(q, idx_q, idx_w):
            # one launch: both cache writes and the indexer logits; then the
            # top-k (leaving the layer's histogram zero) with q_latent beside it
            ql, idx = self._indexer_step(q, idx_q, idx_w, bt, sl, kv_c, k_pe, idx_k,
                                         slot_mapping)
        else:
            if fusable:
                # one launch: q_latent, both cache writes and the histogram clear
                ql, hist = self._prologue(q, kv_c, k_pe, idx_k, slot_mapping)
            else:
                if kv_c is not None:
                    self.store(kv_c, k_pe, idx_k, slot_mapping)
                ql = q_latent(q, self.w)
            idx = self.decode_topk(idx_q, idx_w, bt, sl, hist)
        o, lse, out = self._attention(ql, idx, bt, sl)
        self.last_idx, self.last_o, self.last_lse = idx, o, lse
        return out

    def _attention(self, ql, idx, bt, sl):
        """Sparse MLA decode over the top-k rows and the W_UV projection
        (mi355_dsa_decode_layer_attention: the split merge and the projection
        in one launch where the decode splits the keys).  Returns o [B, H,
        512], lse [B, H] and out [B, H * V]."""
        B, H = ql.shape[0], ql.shape[1]
        lat = self.latent_cache
        kv_fp8 = lat.dtype == torch.uint8
        o = torch.empty(B, H, 512, dtype=torch.float16, device=ql.device)
        lse = torch.empty(B, H, dtype=torch.float32, device=ql.device)
        out = torch.empty(B, H * self.w.v_dim, dtype=torch.float16, device=ql.device)
        _check(lat.is_contiguous(), "latent cache must be contiguous")
        idx, bt, sl = idx.contiguous(), bt.contiguous(), sl.contiguous()
        topk = idx.shape[1]
        L = _lib.lib()
        ws_bytes = L.mi355_dsa_sparse_mla_workspace_size(B, H, topk)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=ql.device)
        uv = self.w.uv_t
        with torch.cuda.device(ql.device):
            _lib.call("mi355_dsa_decode_layer_attention", out.data_ptr(), out.stride(0),
                      o.data_ptr(), lse.data_ptr(), ql.data_ptr(), B, H, lat.data_ptr(),
                      int(kv_fp8), lat.numel() // lat.shape[-1], lat.shape[-2], idx.data_ptr(),
                      topk, bt.data_ptr(), bt.shape[1], sl.data_ptr(), float(self.w.scale),
                      uv.data_ptr(), uv.shape[1], ws.data_ptr(), ws_bytes, _stream(ql))
        return o, lse, out

    def _fusable(self, q, kv_c, k_pe, idx_k, slot_mapping) -> bool:
        """The fused decode prologue covers the layer's usual shapes: one
        slot per token, 16-bit latent inputs of one dtype (fp16 for an fp16
        cache), fp16-castable indexer keys of 128 dims."""
        B = q.shape[0]
        fp8 = self.kv_dtype == "fp8_ds_mla"
        return (slot_mapping.numel() == B and slot_mapping.dtype in (torch.int32, torch.int64)
                and kv_c.dim() == 2 and k_pe.dim() == 2 and kv_c.shape[0] >= B
                and k_pe.shape[0] >= B and kv_c.shape[1] == 512 and k_pe.shape[1] == 64
                and kv_c.dtype == k_pe.dtype
                and (kv_c.dtype == torch.float16 or (fp8 and kv_c.dtype == torch.bfloat16))
                and idx_k.dim() == 2 and idx_k.shape[0] >= B and idx_k.shape[1] == 128
                and q.dim() == 3 and q.shape[2] == self.w.nope_dim + 64)

    def _indexer_fusable(self, q, idx_q, idx_w) -> bool:
        """The fused prologue + logits launch takes at most 64 new tokens and
        the logits op's own operand forms."""
        B = q.shape[0]
        return (B <= self._HIST_ROWS and idx_q.dtype == torch.float16 and idx_q.dim() == 3
                and tuple(idx_q.shape) == (B, 32, 128) and idx_w.dtype == torch.float16
                and idx_w.numel() == B * 32)

    def _zero_hist(self, B: int, device) -> torch.Tensor:
        """Rows [0, B) of the layer's top-k histogram on `device`, zero
        between steps: the fused logits launch adds into them and the
        consuming top-k clears exactly the rows it used, so one [64, 4096]
        buffer per device (the fused path takes at most 64 tokens) serves
        every batch size.  The buffer is state shared by the layer's steps:
        one DsaLayer must not be stepped on two streams at once."""
        assert B <= self._HIST_ROWS
        key = str(device)
        h = self._hists.get(key)
        if h is None:
            h = torch.zeros(self._HIST_ROWS, 4096, dtype=torch.int32, device=device)
            self._hists[key] = h
        return h[:B]

    def _indexer_step(self, q, idx_q, idx_w, bt, sl, kv_c, k_pe, idx_k, slot_mapping):
        """mi355_dsa_decode_layer_indexer (the latent and indexer-K writes and
        the indexer logits with the histogram, one launch), then
        mi355_dsa_decode_layer_topk (the top-k, which leaves the histogram
        zero, with q_latent run beside its select).  Returns (q_latent, idx)."""
        B, H = q.shape[0], q.shape[1]
        q = _rows8(q)
        ql = torch.empty(B, H, 576, dtype=torch.float16, device=q.device)

        def rows16(x):
            ok = x.stride(1) == 1 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0
            return x if ok else x.contiguous()

        kv_c, k_pe = rows16(kv_c[:B]), rows16(k_pe[:B])
        ik = idx_k[:B].to(torch.float16).contiguous()
        slot = slot_mapping.contiguous()
        islot = slot.to(torch.int32)
        lat, ikc = self.latent_cache, self.idx_k_cache
        fp8 = self.kv_dtype == "fp8_ds_mla"
        ik_fp8 = ikc.dtype == torch.uint8
        kv_rows = lat.numel() // (656 if fp8 else 576)
        ik_rows = ikc.numel() // (132 if ik_fp8 else 128)
        page = ikc.shape[1]
        max_kv = bt.shape[1] * page
        score = torch.empty(B, max_kv, dtype=torch.float32, device=q.device)
        hist = self._zero_hist(B, q.device)
        iq, iw = idx_q.contiguous(), idx_w.contiguous()
        bt, sl = bt.contiguous(), sl.contiguous()
        idx = torch.empty(B, self.topk, dtype=torch.int32, device=q.device)
        L = _lib.lib()
        ws_bytes = L.mi355_dsa_decode_topk_workspace_size(B, max_kv, self.topk)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
        uk = self.w.uk_t
        st = _stream(q)
        with torch.cuda.device(q.device):
            _lib.call("mi355_dsa_decode_layer_indexer", B, lat.data_ptr(), int(fp8), kv_rows,
                      kv_c.data_ptr(), kv_c.stride(0), k_pe.data_ptr(), k_pe.stride(0),
                      int(kv_c.dtype == torch.bfloat16), slot.data_ptr(),
                      int(slot.dtype == torch.int64), ikc.data_ptr(), int(ik_fp8), ik_rows,
                      ik.data_ptr(), islot.data_ptr(), score.data_ptr(), B, max_kv,
                      iq.data_ptr(), iw.data_ptr(), page, bt.data_ptr(), bt.shape[1],
                      sl.data_ptr(), hist.data_ptr(), st)
            self.last_score = score
            _lib.call("mi355_dsa_decode_layer_topk", idx.data_ptr(), score.data_ptr(),
                      sl.data_ptr(), hist.data_ptr(), B, max_kv, self.topk, ws.data_ptr(),
                      ws_bytes, ql.data_ptr(), ql.stride(0), ql.stride(1), q.data_ptr(),
                      q.stride(0), q.stride(1), uk.data_ptr(), B, H, uk.shape[1], uk.shape[2],
                      64, st)
        return ql, idx

    def _prologue(self, q, kv_c, k_pe, idx_k, slot_mapping):
        """mi355_dsa_decode_layer_prologue: q_latent (returned), the latent
        and indexer-K cache writes, and a cleared histogram (returned)."""
        B, H = q.shape[0], q.shape[1]
        q = _rows8(q)
        ql = torch.empty(B, H, 576, dtype=torch.float16, device=q.device)
        hist = torch.empty(B, 4096, dtype=torch.int32, device=q.device)

        def rows16(x):
            ok = x.stride(1) == 1 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0
            return x if ok else x.contiguous()

        kv_c, k_pe = rows16(kv_c[:B]), rows16(k_pe[:B])
        ik = idx_k[:B].to(torch.float16).contiguous()
        slot = slot_mapping.contiguous()
        islot = slot.to(torch.int32)
        lat, ikc = self.latent_cache, self.idx_k_cache
        fp8 = self.kv_dtype == "fp8_ds_mla"
        ik_fp8 = ikc.dtype == torch.uint8
        kv_rows = lat.numel() // (656 if fp8 else 576)
        ik_rows = ikc.numel() // (132 if ik_fp8 else 128)
        uk = self.w.uk_t
        with torch.cuda.device(q.device):
            _lib.call("mi355_dsa_decode_layer_prologue", ql.data_ptr(), ql.stride(0), ql.stride(1),
                      q.data_ptr(), q.stride(0), q.stride(1), uk.data_ptr(), B, H, uk.shape[1],
                      uk.shape[2], 64, lat.data_ptr(), int(fp8), kv_rows, kv_c.data_ptr(),
                      kv_c.stride(0), k_pe.data_ptr(), k_pe.stride(0),
                      int(kv_c.dtype == torch.bfloat16), slot.data_ptr(),
                      int(slot.dtype == torch.int64), ikc.data_ptr(), int(ik_fp8), ik_rows,
                      ik.data_ptr(), islot.data_ptr(), hist.data_ptr(), hist.numel(), _stream(q))
        return ql, hist

    # -- prefill ------------------------------------------------------------
    def prefill_topk(self, idx_q: torch.Tensor, idx_w: torch.Tensor, bounds: list[int],
                     block_table: torch.Tensor, causal_len: torch.Tensor,
                     sub_rows: int = 1024, reach: list[int] | None = None) -> torch.Tensor:
        """Top-k rows of the prefill tokens: request r owns token rows
        [bounds[r], bounds[r+1]) and block-table row r; causal_len[t] is
        token t's context length (its position + 1).  `reach` optionally gives
        each sub-chunk's max causal length (else read from causal_len)."""
        T = idx_q.shape[0]
        page = self.idx_k_cache.shape[1]
        full_kv = block_table.shape[1] * page
        out = torch.full((T, self.topk), -1, dtype=torch.int32, device=idx_q.device)
        ws = torch.empty(1 << 20, dtype=torch.uint8, device=idx_q.device)
        max_len = int(causal_len.max()) if reach is None else max(reach)
        k = 0
        for r in range(len(bounds) - 1):
            lo, hi = bounds[r], bounds[r + 1]
            for lo2 in range(lo, hi, sub_rows):
                hi2 = min(lo2 + sub_rows, hi)
                n = hi2 - lo2
                cl = causal_len[lo2:hi2].to(torch.int32).contiguous()
                cmax = int(cl.max()) if reach is None else reach[k]
                k += 1
                max_kv = max(min(full_kv, (cmax + KT - 1) // KT * KT), page)
                cols = min(block_table.shape[1], (max_kv + page - 1) // page)
                seg_bt = block_table[r:r + 1, :cols].to(torch.int32).expand(n, cols).contiguous()
                score = torch.empty(n, max_kv, dtype=torch.float32, device=idx_q.device)
                qs = idx_q[lo2:hi2]
                n16 = (n + 15) // 16 * 16
                if n16 != n:
                    qs = torch.nn.functional.pad(qs, (0, 0, 0, 0, 0, n16 - n))
                qp = qs.reshape(n16 // 16, 16, 32, 8, 16).permute(2, 0, 3, 1, 4).contiguous()
                _sm70_ops.sm70_indexer_logits_packed(score, qp, self.idx_k_cache,
                                                     idx_w[lo2:hi2].contiguous(), seg_bt, cl)
                _sm70_ops.persistent_topk(score, cl.view(n, 1), out[lo2:hi2], ws, self.topk,
                                          max_len)
        return out

    def prefill(self, q: torch.Tensor, idx_q: torch.Tensor, idx_w: torch.Tensor,
                bounds: list[int], block_table: torch.Tensor, causal_len: torch.Tensor,
                kv_c: torch.Tensor | None = None, k_pe: torch.Tensor | None = None,
                idx_k: torch.Tensor | None = None, slot_mapping: torch.Tensor | None = None,
                sub_rows: int = 1024, reach: list[int] | None = None) -> torch.Tensor:
        """Prefill tokens q [T, H, P + 64] (see prefill_topk for the
        metadata).  Returns out [T, H * V]."""
        if kv_c is not None:
            self.store(kv_c, k_pe, idx_k, slot_mapping)
        T = q.shape[0]
        idx = self.prefill_topk(idx_q, idx_w, bounds, block_table, causal_len, sub_rows, reach)
        req = torch.repeat_interleave(
            torch.arange(len(bounds) - 1, device=q.device),
            torch.tensor([bounds[r + 1] - bounds[r] for r in range(len(bounds) - 1)],
                         device=q.device))
        per_tok_bt = block_table.to(torch.int32).index_select(0, req).contiguous()
        ql = q_latent(q, self.w)
        o = torch.empty(T, self.w.n_heads, 512, dtype=torch.float16, device=q.device)
        lse = torch.empty(T, self.w.n_heads, dtype=torch.float32, device=q.device)
        _sm70_ops.sm70_sparse_mla_decode(o, lse, ql, self.latent_cache, idx, per_tok_bt,
                                         causal_len.to(torch.int32).contiguous(), self.w.scale)
        self.last_idx, self.last_o, self.last_lse = idx, o, lse
        return v_up(o, self.w)
