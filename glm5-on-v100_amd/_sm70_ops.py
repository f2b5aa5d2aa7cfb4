"""Drop-in replacement for the DSA part of vllm/_sm70_ops.py.

Same function names, argument order and semantics as the reference's
wrappers (reference/_sm70_ops.py:1802-1961); they dispatch to the torch ops
registered by ops.py, which run the gfx950 HIP kernels.  `_op` raises
RuntimeError for a missing op exactly like the reference (:23-29).
"""
from __future__ import annotations

import torch

from . import ops as _ops


def _op(name: str):
    ns = _ops.register()
    space = getattr(torch.ops, ns)
    if not hasattr(space, name):
        raise RuntimeError(
            f"MI355X DSA op {ns}::{name} is not available. "
            "Build libmi355_dsa.so (gfx950) to enable it.")
    return getattr(space, name)


def sm70_attn_fp8_gemv(y: torch.Tensor, x: torch.Tensor, w: torch.Tensor,
                       s: torch.Tensor) -> None:
    """Matrix-vector product with an fp8 weight: y (fp16 [M, N]) receives
    x (fp16 [M, K], 1 <= M <= 8) times the transpose of the dequantized
    weight, where w holds one e4m3 byte per weight element [N, K] and s
    (fp32) one multiplier per 128 x 128 block of w."""
    _op("sm70_attn_fp8_gemv")(y, x, w, s)


def _sm70_attn_fp8_quantize(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """[128,128]-block e4m3 quantization of an fp16 [N,K] weight, on the GPU.

    Returns (uint8 e4m3 bits [N,K], fp32 scale_inv [ceil(N/128), ceil(K/128)]),
    like the model loader's function of the same name."""
    from . import ops as _ops
    return _ops.attn_fp8_quantize(weight)


def sm70_attn_fp8_dequant(out: torch.Tensor, w: torch.Tensor, s: torch.Tensor) -> None:
    """Expands the e4m3 weight w [N, K] with its 128 x 128 block multipliers s
    into fp16 values written to out [N, K] (used for batches too large for
    the GEMV)."""
    _op("sm70_attn_fp8_dequant")(out, w, s)


def sm70_mla_decode(o: torch.Tensor, lse: torch.Tensor, q: torch.Tensor,
                    kv_cache: torch.Tensor, block_table: torch.Tensor,
                    seq_lens: torch.Tensor, scale: float) -> None:
    """Dense MLA decode over positions [0, seq_len): writes o [B,H,512] fp16,
    lse [B,H] fp32 (reference/_sm70_ops.py:1774-1784)."""
    _op("sm70_mla_decode")(o, lse, q, kv_cache, block_table, seq_lens, scale)


def sm70_indexer_shard_merge(out: torch.Tensor, allf: torch.Tensor, dst_rows: torch.Tensor,
                             dst_base: int, topk: int) -> None:
    """Exact top-K merge of the all-gathered key-shard candidates allf
    [tp, R, 2K] into out rows dst_base + r (or dst_rows[r] when dst_base < 0),
    positions ascending, -1 for -inf selections (the TP prefill indexer's
    fused merge, reference/sparse_attn_indexer.py:985-1006)."""
    _op("sm70_indexer_shard_merge")(out, allf, dst_rows, dst_base, topk)


def sm70_sparse_mla_decode(o: torch.Tensor, lse: torch.Tensor, q: torch.Tensor,
                           kv_cache: torch.Tensor, idx: torch.Tensor,
                           block_table: torch.Tensor, seq_lens: torch.Tensor,
                           scale: float) -> None:
    """Sparse (top-k) MLA attention: writes o [B,H,512] fp16, lse [B,H] fp32."""
    _op("sm70_sparse_mla_decode")(o, lse, q, kv_cache, idx, block_table, seq_lens, scale)


def sm70_indexer_logits(score: torch.Tensor, q: torch.Tensor, k_cache: torch.Tensor,
                        weights: torch.Tensor, block_table: torch.Tensor,
                        seq_lens: torch.Tensor, hist: torch.Tensor | None = None) -> None:
    """Fills score [B, max_kv] (fp32) with each position's indexer logit:
    the weighted sum over the 32 indexer heads of relu(q . k); positions at
    or past seq_len get -inf.  When hist (int32 [B, 4096], zeroed by the
    caller) is given, the same launch counts every valid score into its
    12-bit monotone-key bin, the first level that sm70_decode_topk uses."""
    _op("sm70_indexer_logits")(score, q, k_cache, weights, block_table, seq_lens, hist)


def sm70_indexer_logits_packed(score: torch.Tensor, q_packed: torch.Tensor,
                               k_cache: torch.Tensor, weights: torch.Tensor,
                               block_table: torch.Tensor, seq_lens: torch.Tensor) -> None:
    """Packed-Q indexer logits (prefill path); q_packed is
    [32, ceil(B/16), 8, 16, 16] fp16 contiguous."""
    _op("sm70_indexer_logits_packed")(score, q_packed, k_cache, weights, block_table, seq_lens)


def sm70_decode_topk(idx: torch.Tensor, score: torch.Tensor, seq_lens: torch.Tensor,
                     hist: torch.Tensor, k: int) -> None:
    """Decode top-k select: idx [B, k] <- top-k positions of score
    (p < seq_lens), ascending, -1 padded.  Graph-capture safe."""
    _op("sm70_decode_topk")(idx, score, seq_lens, hist, k)


def sm70_indexer_k_store(kv_cache: torch.Tensor, k: torch.Tensor,
                         slot_mapping: torch.Tensor) -> None:
    """Graph-safe indexer-K scatter into the paged cache (skips slot < 0)."""
    _op("sm70_indexer_k_store")(kv_cache, k, slot_mapping)


def persistent_topk(logits: torch.Tensor, lengths: torch.Tensor, output: torch.Tensor,
                    workspace: torch.Tensor, k: int, max_seq_len: int) -> None:
    """Row-wise top-k used by the prefill indexer (vLLM persistent_topk)."""
    _op("persistent_topk")(logits, lengths, output, workspace, k, max_seq_len)
