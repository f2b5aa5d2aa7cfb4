"""torch custom-op registration of the DSA hot-path ops.

Schemas are the reference's, verbatim (patches/glm5-v100-sm70-glue.patch:
494-565; persistent_topk from its call sites, reference/
sparse_attn_indexer.py:632-639 and :873-880).  Each op validates its tensors
the way the reference's TORCH_CHECKs do (same conditions, RuntimeError),
then calls the C ABI on the current stream.  Only the CUDA (= HIP on ROCm)
dispatch key has a kernel: CPU tensors raise, there is no silent fallback.
Outputs are mutated in place and the ops return nothing, so they are
capture-safe (no host sync, workspace from torch's caching allocator).

Ops are registered in the namespace named by MI355_DSA_NAMESPACE (default
"mi355_dsa"); "_C" registers them as torch.ops._C.<name>, the names the
reference's callers resolve (reference/_sm70_ops.py:23-29).
"""
from __future__ import annotations

import os

import torch

from . import _lib

NAMESPACE = os.environ.get("MI355_DSA_NAMESPACE", "mi355_dsa")

SCHEMAS = {
    "sm70_mla_decode": (
        "sm70_mla_decode(Tensor! o, Tensor! lse, Tensor q, Tensor kv_cache, "
        "Tensor block_table, Tensor seq_lens, float scale) -> ()"),
    "sm70_indexer_shard_merge": (
        "sm70_indexer_shard_merge(Tensor! out, Tensor allf, Tensor dst_rows, "
        "int dst_base, int topk) -> ()"),
    "sm70_sparse_mla_decode": (
        "sm70_sparse_mla_decode(Tensor! o, Tensor! lse, Tensor q, "
        "Tensor kv_cache, Tensor idx, Tensor block_table, Tensor seq_lens, "
        "float scale) -> ()"),
    "sm70_indexer_logits": (
        "sm70_indexer_logits(Tensor! score, Tensor q, Tensor k_cache, "
        "Tensor weights, Tensor block_table, Tensor seq_lens, "
        "Tensor!? hist) -> ()"),
    "sm70_indexer_logits_packed": (
        "sm70_indexer_logits_packed(Tensor! score, Tensor q_packed, "
        "Tensor k_cache, Tensor weights, Tensor block_table, Tensor seq_lens) "
        "-> ()"),
    "sm70_decode_topk": (
        "sm70_decode_topk(Tensor! idx, Tensor score, Tensor seq_lens, "
        "Tensor hist, int k) -> ()"),
    "sm70_indexer_k_store": (
        "sm70_indexer_k_store(Tensor! kv_cache, Tensor k, Tensor slot_mapping) "
        "-> ()"),
    "sm70_attn_fp8_gemv": "sm70_attn_fp8_gemv(Tensor! y, Tensor x, Tensor w, Tensor s) -> ()",
    "sm70_attn_fp8_dequant": "sm70_attn_fp8_dequant(Tensor! out, Tensor w, Tensor s) -> ()",
    "persistent_topk": (
        "persistent_topk(Tensor logits, Tensor lengths, Tensor! output, "
        "Tensor workspace, int k, int max_seq_len) -> ()"),
    # vLLM cache op (vllm/_custom_ops.py concat_and_cache_mla), the writer of
    # the latent cache the sparse MLA kernels read
    "concat_and_cache_mla": (
        "concat_and_cache_mla(Tensor kv_c, Tensor k_pe, Tensor! kv_cache, "
        "Tensor slot_mapping, str kv_cache_dtype, Tensor scale) -> ()"),
}

DSMLA_ROW_BYTES = 656
IDXK_FP8_ROW_BYTES = 132


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _contig(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


def _out_ok(t: torch.Tensor, name: str) -> None:
    _check(t.is_contiguous(), f"{name} must be contiguous")


# ---------------------------------------------------------------------------
# implementations (CUDA dispatch key)
# ---------------------------------------------------------------------------
def mla_decode_impl(o, lse, q, kv_cache, block_table, seq_lens, scale):
    """Dense decode, sm70_mla_decode.cu:1474-1501 checks (fp16 cache only,
    n_head a multiple of 32)."""
    _check(q.is_cuda and kv_cache.is_cuda, "q and kv_cache must be on the GPU")
    _check(q.dtype == torch.float16, "q must be fp16")
    _check(kv_cache.dtype == torch.float16, "kv_cache must be fp16")
    _check(o.dtype == torch.float16, "o must be fp16")
    _check(lse.dtype == torch.float32, "lse must be fp32")
    _check(block_table.dtype == torch.int32, "block_table must be int32")
    _check(seq_lens.dtype == torch.int32, "seq_lens must be int32")
    _check(q.dim() == 3 and q.size(2) == 576, "q last dim must be 576")
    B, H = q.size(0), q.size(1)
    _check(H % 32 == 0 and H > 0, "n_head must be a multiple of 32")
    _check(o.dim() == 3 and o.size(0) == B and o.size(1) == H and o.size(2) == 512,
           "o last dim must be 512")
    _check(lse.dim() == 2 and lse.size(0) == B and lse.size(1) == H, "lse must be [B, H]")
    _check(block_table.dim() == 2 and block_table.size(0) == B, "block_table must be [B, max_blocks]")
    _check(seq_lens.numel() == B, "seq_lens must be [B]")
    _check(kv_cache.size(-1) == 576, "kv_cache last dim must be 576")
    _check(kv_cache.is_contiguous(), "kv_cache must be contiguous")
    _out_ok(o, "o")
    _out_ok(lse, "lse")
    if B == 0:
        return
    q, block_table, seq_lens = _contig(q), _contig(block_table), _contig(seq_lens)
    page = kv_cache.size(-2)
    n_rows = kv_cache.numel() // 576
    max_blocks = block_table.size(1)
    L = _lib.lib()
    ws_bytes = L.mi355_dsa_mla_decode_workspace_size(B, H, max_blocks * page)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        _lib.call("mi355_dsa_mla_decode", o.data_ptr(), lse.data_ptr(), q.data_ptr(), B, H,
                  kv_cache.data_ptr(), n_rows, page, block_table.data_ptr(), max_blocks,
                  seq_lens.data_ptr(), float(scale), ws.data_ptr(), ws_bytes, _stream(q))


def indexer_shard_merge_impl(out, allf, dst_rows, dst_base, topk):
    """sm70_mla_decode.cu:2411-2436 checks (K = 2048, tp in [2, 4])."""
    _check(allf.is_cuda and allf.is_contiguous() and allf.dim() == 3,
           "allf must be contiguous [tp, R, 2K] cuda")
    _check(allf.dtype == torch.float32, "allf must be fp32")
    _check(out.dtype == torch.int32 and out.dim() == 2, "out must be int32 [rows, >= K]")
    tp, R = allf.size(0), allf.size(1)
    _check(topk == 2048 and allf.size(2) == 2 * topk, "shard merge kernel supports K=2048 only")
    _check(2 <= tp <= 4, "shard merge kernel supports tp in [2,4]")
    _check(dst_base >= 0 or dst_rows.numel() == R, "need dst_rows when dst_base < 0")
    _check((tp * topk) % 512 == 0, "ncand must be a multiple of 512")
    _check(out.is_cuda and out.stride(1) == 1, "out must be a row-major cuda tensor")
    if R == 0:
        return
    dr = None
    if dst_base < 0:
        dr = dst_rows.to(torch.int32).contiguous()
    with torch.cuda.device(allf.device):
        _lib.call("mi355_dsa_indexer_shard_merge", out.data_ptr(), out.stride(0), out.size(0),
                  allf.data_ptr(), tp, R, topk, dr.data_ptr() if dr is not None else None,
                  int(dst_base), _stream(allf))


def sparse_mla_decode_impl(o, lse, q, kv_cache, idx, block_table, seq_lens, scale):
    """sm70_mla_decode.cu:2457-2616 checks."""
    _check(q.is_cuda and kv_cache.is_cuda, "q and kv_cache must be on the GPU")
    _check(q.dtype == torch.float16, "q must be fp16")
    kv_fp8 = kv_cache.dtype == torch.uint8
    _check(kv_fp8 or kv_cache.dtype == torch.float16,
           "kv_cache must be fp16 or uint8 (fp8_ds_mla)")
    _check(o.dtype == torch.float16, "o must be fp16")
    _check(lse.dtype == torch.float32, "lse must be fp32")
    _check(idx.dtype == torch.int32, "idx must be int32")
    _check(block_table.dtype == torch.int32, "block_table must be int32")
    _check(seq_lens.dtype == torch.int32, "seq_lens must be int32")
    _check(q.dim() == 3 and q.size(2) == 576, "q last dim must be 576")
    B, H = q.size(0), q.size(1)
    _check(H > 0, "n_head must be > 0")
    _check(o.dim() == 3 and o.size(0) == B and o.size(1) == H and o.size(2) == 512,
           "o last dim must be 512")
    _check(lse.dim() == 2 and lse.size(0) == B and lse.size(1) == H, "lse must be [B, H]")
    _check(idx.dim() == 2 and idx.size(0) == B, "idx must be [B, topk]")
    _check(block_table.dim() == 2 and block_table.size(0) == B, "block_table must be [B, max_blocks]")
    _check(seq_lens.numel() == B, "seq_lens must be [B]")
    if kv_fp8:
        _check(kv_cache.size(-1) == DSMLA_ROW_BYTES,
               "fp8 kv_cache last dim must be 656 (fp8_ds_mla layout)")
    else:
        _check(kv_cache.size(-1) == 576, "fp16 kv_cache last dim must be 576")
    _check(kv_cache.is_contiguous(), "kv_cache must be contiguous")
    _out_ok(o, "o")
    _out_ok(lse, "lse")
    if B == 0:
        return
    q, idx, block_table, seq_lens = (_contig(q), _contig(idx), _contig(block_table),
                                     _contig(seq_lens))
    topk = idx.size(1)
    page = kv_cache.size(-2)
    n_rows = kv_cache.numel() // (DSMLA_ROW_BYTES if kv_fp8 else 576)
    L = _lib.lib()
    ws_bytes = L.mi355_dsa_sparse_mla_workspace_size(B, H, topk)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        _lib.call("mi355_dsa_sparse_mla_decode", o.data_ptr(), lse.data_ptr(), q.data_ptr(),
                  B, H, kv_cache.data_ptr(), int(kv_fp8), n_rows, page, idx.data_ptr(), topk,
                  block_table.data_ptr(), block_table.size(1), seq_lens.data_ptr(),
                  float(scale), ws.data_ptr(), ws_bytes, _stream(q))


def _indexer_common_checks(score, k_cache, weights, block_table, seq_lens):
    k_fp8 = k_cache.dtype == torch.uint8
    _check(k_fp8 or k_cache.dtype == torch.float16, "k_cache must be fp16 or uint8 (fp8)")
    _check(weights.dtype == torch.float16, "weights must be fp16")
    _check(score.dtype == torch.float32, "score must be fp32")
    _check(block_table.dtype == torch.int32, "block_table must be int32")
    _check(seq_lens.dtype == torch.int32, "seq_lens must be int32")
    if k_fp8:
        _check(k_cache.size(-1) == IDXK_FP8_ROW_BYTES,
               "fp8 indexer k_cache last dim must be 132")
    else:
        _check(k_cache.size(-1) == 128, "fp16 indexer k_cache last dim must be 128")
    page = k_cache.size(-2)
    _check(page > 0 and (page & (page - 1)) == 0,
           "indexer cache page size must be a power of two")
    _check(k_cache.is_contiguous(), "k_cache must be contiguous")
    _out_ok(score, "score")
    n_rows = k_cache.numel() // (IDXK_FP8_ROW_BYTES if k_fp8 else 128)
    return k_fp8, page, n_rows


def indexer_logits_impl(score, q, k_cache, weights, block_table, seq_lens, hist=None):
    """sm70_mla_decode.cu:2626-2764 checks (hist is accepted for any B: the
    kernel builds the histogram on every path)."""
    _check(q.dtype == torch.float16, "q must be fp16")
    k_fp8, page, n_rows = _indexer_common_checks(score, k_cache, weights, block_table, seq_lens)
    _check(q.dim() == 3 and q.size(2) == 128, "indexer head_dim must be 128")
    _check(q.size(1) == 32, "kernel specialized for 32 indexer heads")
    B = q.size(0)
    _check(score.dim() == 2 and score.size(0) == B, "score must be [B, max_kv]")
    _check(weights.numel() == B * 32, "weights must be [B, 32]")
    _check(block_table.dim() == 2 and block_table.size(0) == B, "block_table must be [B, max_blocks]")
    _check(seq_lens.numel() == B, "seq_lens must be [B]")
    if hist is not None:
        _check(hist.dtype == torch.int32 and hist.is_contiguous() and hist.dim() == 2
               and hist.size(0) == B and hist.size(1) == 4096,
               "hist must be contiguous int32 [B, 4096]")
    if B == 0 or score.size(1) == 0:
        return
    q, weights, block_table, seq_lens = (_contig(q), _contig(weights), _contig(block_table),
                                         _contig(seq_lens))
    with torch.cuda.device(q.device):
        _lib.call("mi355_dsa_indexer_logits", score.data_ptr(), B, score.size(1), q.data_ptr(),
                  32, 128, k_cache.data_ptr(), int(k_fp8), n_rows, page, weights.data_ptr(),
                  block_table.data_ptr(), block_table.size(1), seq_lens.data_ptr(),
                  _ptr(hist), _stream(q))


def indexer_logits_packed_impl(score, q_packed, k_cache, weights, block_table, seq_lens):
    """sm70_mla_decode.cu:2771-2836 checks."""
    _check(q_packed.dtype == torch.float16 and q_packed.is_contiguous(),
           "q_packed must be contiguous fp16")
    k_fp8, page, n_rows = _indexer_common_checks(score, k_cache, weights, block_table, seq_lens)
    B = score.size(0)
    n_qt = (B + 15) // 16
    _check(q_packed.dim() == 5 and q_packed.size(0) == 32 and q_packed.size(1) == n_qt
           and q_packed.size(2) == 8 and q_packed.size(3) == 16 and q_packed.size(4) == 16,
           "q_packed must be [32, ceil(B/16), 8, 16, 16]")
    _check(weights.numel() == B * 32, "weights must be [B, 32]")
    _check(block_table.dim() == 2 and block_table.size(0) == B,
           "block_table must be [B, max_blocks]")
    _check(seq_lens.numel() == B, "seq_lens must be [B]")
    if B == 0 or score.size(1) == 0:
        return
    weights, block_table, seq_lens = _contig(weights), _contig(block_table), _contig(seq_lens)
    with torch.cuda.device(score.device):
        _lib.call("mi355_dsa_indexer_logits_packed", score.data_ptr(), B, score.size(1),
                  q_packed.data_ptr(), k_cache.data_ptr(), int(k_fp8), n_rows, page,
                  weights.data_ptr(), block_table.data_ptr(), block_table.size(1),
                  seq_lens.data_ptr(), _stream(score))


def decode_topk_impl(idx, score, seq_lens, hist, k):
    """sm70_mla_decode.cu:2844-2905 checks."""
    _check(score.is_cuda and idx.is_cuda, "score and idx must be on the GPU")
    _check(score.dtype == torch.float32, "score must be fp32")
    _check(idx.dtype == torch.int32, "idx must be int32")
    _check(seq_lens.dtype == torch.int32, "seq_lens must be int32")
    _check(score.is_contiguous() and idx.is_contiguous(), "score and idx must be contiguous")
    B, max_kv, K = score.size(0), score.size(1), int(k)
    _check(idx.dim() == 2 and idx.size(0) == B and idx.size(1) == K, "idx must be [B, K]")
    _check(K >= 1, "k must be >= 1")
    _check(hist.dtype == torch.int32 and hist.is_contiguous() and hist.dim() == 2
           and hist.size(0) == B and hist.size(1) == 4096,
           "hist must be contiguous int32 [B, 4096]")
    _check(seq_lens.numel() == B, "seq_lens must be [B]")
    if B == 0:
        return
    seq_lens = _contig(seq_lens)
    L = _lib.lib()
    ws_bytes = L.mi355_dsa_decode_topk_workspace_size(B, max_kv, K)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=score.device)
    with torch.cuda.device(score.device):
        _lib.call("mi355_dsa_decode_topk", idx.data_ptr(), score.data_ptr(), seq_lens.data_ptr(),
                  hist.data_ptr(), B, max_kv, K, ws.data_ptr(), ws_bytes, _stream(score))


def persistent_topk_impl(logits, lengths, output, workspace, k, max_seq_len):
    """Row top-k with per-row lengths (vLLM persistent_topk as called at
    reference/sparse_attn_indexer.py:873-880)."""
    _check(logits.dtype == torch.float32 and logits.dim() == 2, "logits must be fp32 [n, max_kv]")
    _check(output.dtype == torch.int32 and output.dim() == 2, "output must be int32 [n, k]")
    _check(lengths.dtype == torch.int32, "lengths must be int32")
    n, W, K = logits.size(0), logits.size(1), int(k)
    _check(output.size(0) == n and output.size(1) == K, "output must be [n, k]")
    _check(lengths.numel() == n, "lengths must have one entry per row")
    _check(K >= 1, "k must be >= 1")
    if n == 0:
        return
    logits, lengths = _contig(logits), _contig(lengths)
    tmp = output if output.is_contiguous() else torch.empty_like(output, memory_format=torch.contiguous_format)
    L = _lib.lib()
    ws_bytes = L.mi355_dsa_persistent_topk_workspace_size(n, W, K)
    if ws_bytes and workspace.numel() * workspace.element_size() >= ws_bytes and workspace.is_contiguous():
        ws = workspace
    else:
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=logits.device)
    with torch.cuda.device(logits.device):
        _lib.call("mi355_dsa_persistent_topk", logits.data_ptr(), n, W, lengths.data_ptr(),
                  tmp.data_ptr(), K, int(max_seq_len), ws.data_ptr(), ws_bytes, _stream(logits))
    if tmp is not output:
        output.copy_(tmp)


def indexer_k_store_impl(kv_cache, k, slot_mapping):
    """sm70_mla_decode.cu:2910-2939 checks."""
    _check(kv_cache.is_cuda and k.is_cuda, "kv_cache and k must be on the GPU")
    k_fp8 = kv_cache.dtype == torch.uint8
    _check(k_fp8 or kv_cache.dtype == torch.float16, "kv_cache must be fp16 or uint8 (fp8)")
    _check(k.dtype == torch.float16, "k must be fp16")
    _check(slot_mapping.dtype == torch.int32, "slot_mapping must be int32")
    head_dim, n_tok = k.size(-1), k.size(0)
    if n_tok == 0:
        return
    _check(slot_mapping.numel() >= n_tok, "slot_mapping shorter than k")
    _check(kv_cache.is_contiguous(), "kv_cache must be contiguous")
    if k_fp8:
        _check(head_dim == 128, "fp8 indexer store requires head_dim == 128")
        _check(kv_cache.size(-1) == IDXK_FP8_ROW_BYTES, "fp8 indexer kv_cache last dim must be 132")
        n_rows = kv_cache.numel() // IDXK_FP8_ROW_BYTES
    else:
        n_rows = kv_cache.numel() // head_dim
    k, slot_mapping = _contig(k), _contig(slot_mapping)
    with torch.cuda.device(k.device):
        _lib.call("mi355_dsa_indexer_k_store", kv_cache.data_ptr(), int(k_fp8), n_rows,
                  k.data_ptr(), n_tok, head_dim, slot_mapping.data_ptr(), _stream(k))


def concat_and_cache_mla_impl(kv_c, k_pe, kv_cache, slot_mapping, kv_cache_dtype, scale):
    """vLLM concat_and_cache_mla for kv_cache_dtype "auto" (fp16 rows of
    kv_lora_rank + pe_dim) and "fp8_ds_mla" (656-byte rows); the token count
    is slot_mapping's length (kv_c / k_pe may carry padding rows)."""
    _check(kv_cache_dtype in ("auto", "fp8_ds_mla"),
           f"concat_and_cache_mla: unsupported kv_cache_dtype {kv_cache_dtype!r}")
    _check(kv_c.is_cuda and k_pe.is_cuda and kv_cache.is_cuda and slot_mapping.is_cuda,
           "all tensors must be on the GPU")
    _check(kv_c.dim() == 2 and k_pe.dim() == 2, "kv_c and k_pe must be 2-D")
    _check(kv_c.size(1) == 512 and k_pe.size(1) == 64,
           "kv_lora_rank must be 512 and the rope dim 64")
    _check(slot_mapping.dtype in (torch.int64, torch.int32), "slot_mapping must be int64 or int32")
    n_tok = slot_mapping.size(0)
    _check(kv_c.size(0) >= n_tok and k_pe.size(0) >= n_tok, "fewer kv_c / k_pe rows than slots")
    _check(kv_cache.is_contiguous(), "kv_cache must be contiguous")
    fp8 = kv_cache_dtype == "fp8_ds_mla"
    if fp8:
        _check(kv_cache.dtype == torch.uint8 and kv_cache.size(-1) == DSMLA_ROW_BYTES,
               "fp8_ds_mla kv_cache must be uint8 with last dim 656")
        _check(kv_c.dtype in (torch.float16, torch.bfloat16) and k_pe.dtype == kv_c.dtype,
               "kv_c and k_pe must be fp16 or bf16 of one dtype")
        n_rows = kv_cache.numel() // DSMLA_ROW_BYTES
    else:
        _check(kv_cache.dtype == torch.float16 and kv_cache.size(-1) == 576,
               "auto kv_cache must be fp16 with last dim 576")
        _check(kv_c.dtype == torch.float16 and k_pe.dtype == torch.float16,
               "kv_c and k_pe must be fp16")
        n_rows = kv_cache.numel() // 576
    if n_tok == 0:
        return

    def rows16(x):
        ok = (x.stride(1) == 1 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0)
        return x if ok else x.contiguous()

    kv_c, k_pe, slot_mapping = rows16(kv_c), rows16(k_pe), _contig(slot_mapping)
    with torch.cuda.device(kv_c.device):
        _lib.call("mi355_dsa_concat_and_cache_mla", kv_cache.data_ptr(), int(fp8), n_rows,
                  kv_c.data_ptr(), kv_c.stride(0), k_pe.data_ptr(), k_pe.stride(0),
                  int(kv_c.dtype == torch.bfloat16), n_tok, slot_mapping.data_ptr(),
                  int(slot_mapping.dtype == torch.int64), _stream(kv_c))


def attn_fp8_gemv_impl(y, x, w, s):
    """sm70_attn_fp8.cu:148-191 checks."""
    _check(x.is_cuda and w.is_cuda and s.is_cuda and y.is_cuda, "all tensors must be on the GPU")
    _check(x.dtype == torch.float16, "x must be fp16")
    _check(y.dtype == torch.float16, "y must be fp16")
    _check(w.dtype == torch.uint8, "w must be uint8 (e4m3 bits)")
    _check(s.dtype == torch.float32, "s must be fp32")
    _check(x.dim() == 2 and w.dim() == 2 and y.dim() == 2 and s.dim() == 2, "all tensors must be 2-D")
    M, K, N = x.size(0), x.size(1), w.size(0)
    _check(1 <= M <= 8, f"sm70_attn_fp8_gemv: M must be 1..8, got {M}")
    _check(K % 16 == 0 and N % 8 == 0, "bad N/K alignment")
    _check(w.size(1) == K and y.size(0) == M and y.size(1) == N, "shape mismatch")
    _check(s.size(0) == (N + 127) // 128 and s.size(1) == (K + 127) // 128, "scale shape mismatch")
    _check(x.is_contiguous() and w.is_contiguous() and y.is_contiguous() and s.is_contiguous(),
           "all tensors must be contiguous")
    with torch.cuda.device(x.device):
        _lib.call("mi355_dsa_attn_fp8_gemv", y.data_ptr(), x.data_ptr(), w.data_ptr(),
                  s.data_ptr(), M, N, K, _stream(x))


def attn_fp8_dequant_impl(out, w, s):
    """sm70_attn_fp8.cu:193-215 checks."""
    _check(out.is_cuda and w.is_cuda and s.is_cuda, "all tensors must be on the GPU")
    _check(out.dtype == torch.float16, "out must be fp16")
    _check(w.dtype == torch.uint8, "w must be uint8 (e4m3 bits)")
    _check(s.dtype == torch.float32, "s must be fp32")
    _check(out.dim() == 2 and w.dim() == 2 and s.dim() == 2, "all tensors must be 2-D")
    N, K = w.size(0), w.size(1)
    _check(K % 16 == 0, "K must be a multiple of 16")
    _check(out.size(0) == N and out.size(1) == K, "out must be [N, K]")
    _check(s.size(0) == (N + 127) // 128 and s.size(1) == (K + 127) // 128, "scale shape mismatch")
    _check(out.is_contiguous() and w.is_contiguous() and s.is_contiguous(),
           "all tensors must be contiguous")
    with torch.cuda.device(w.device):
        _lib.call("mi355_dsa_attn_fp8_dequant", out.data_ptr(), w.data_ptr(), s.data_ptr(),
                  N, K, _stream(w))


def attn_fp8_quantize(weight):
    """Load-time [128,128]-block e4m3 quantization of an fp16 [N,K] weight on
    the GPU: returns (uint8 e4m3 bits [N,K], fp32 scale [ceil(N/128),
    ceil(K/128)]), the same values as _sm70_attn_fp8_quantize
    (patches/glm5-v100-sm70-glue.patch:1515-1532)."""
    _check(weight.is_cuda, "weight must be on the GPU")
    _check(weight.dim() == 2, "weight must be 2-D [N, K]")
    w = _contig(weight.to(torch.float16))
    N, K = w.size(0), w.size(1)
    q = torch.empty(N, K, dtype=torch.uint8, device=w.device)
    s = torch.empty((N + 127) // 128, (K + 127) // 128, dtype=torch.float32, device=w.device)
    if N and K:
        with torch.cuda.device(w.device):
            _lib.call("mi355_dsa_attn_fp8_quantize", q.data_ptr(), s.data_ptr(), w.data_ptr(),
                      N, K, _stream(w))
    return q, s


IMPLS = {
    "sm70_indexer_shard_merge": indexer_shard_merge_impl,
    "sm70_mla_decode": mla_decode_impl,
    "sm70_sparse_mla_decode": sparse_mla_decode_impl,
    "sm70_indexer_logits": indexer_logits_impl,
    "sm70_indexer_logits_packed": indexer_logits_packed_impl,
    "sm70_decode_topk": decode_topk_impl,
    "sm70_indexer_k_store": indexer_k_store_impl,
    "sm70_attn_fp8_gemv": attn_fp8_gemv_impl,
    "sm70_attn_fp8_dequant": attn_fp8_dequant_impl,
    "persistent_topk": persistent_topk_impl,
    "concat_and_cache_mla": concat_and_cache_mla_impl,
}

_registered = {}


CACHE_OPS = ("concat_and_cache_mla",)


def register(namespace: str | None = None, names=None) -> str:
    """Registers the ops `names` (default: every op) in `namespace`
    (idempotent per namespace); returns the namespace."""
    ns = namespace or NAMESPACE
    if ns in _registered:
        return ns
    lib = torch.library.Library(ns, "FRAGMENT")
    for name, schema in SCHEMAS.items():
        if names is not None and name not in names:
            continue
        if hasattr(getattr(torch.ops, ns), name):
            continue  # defined elsewhere (e.g. a real vLLM _C build)
        lib.define(schema)
        lib.impl(name, IMPLS[name], "CUDA")

        def _fake(*args, **kwargs):
            return None

        torch.library.register_fake(f"{ns}::{name}", _fake, lib=lib)
    _registered[ns] = lib
    return ns


def register_cache_ops(namespace: str = "_C_cache_ops") -> str:
    """Registers the latent-cache writer alone in the namespace vLLM's
    _custom_ops.concat_and_cache_mla resolves (torch.ops._C_cache_ops)."""
    return register(namespace, CACHE_OPS)


def op(name: str):
    """The registered torch op `name` (registering on first use)."""
    ns = register()
    return getattr(getattr(torch.ops, ns), name)
