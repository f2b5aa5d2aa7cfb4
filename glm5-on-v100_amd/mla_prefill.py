"""Dense varlen MLA prefill attention on the gfx950 kernel
(csrc/varlen_attn.hip, C ABI mi355_dsa_varlen_attention).

Drop-in for the reference's SM70 MLA prefill backend
(reference/vllm/v1/attention/backends/mla/prefill/sm70_triton.py):
`varlen_attention` has the signature and results of its `_varlen_attention`
(:54-187) -- ragged batches by cu_seqlens, causal with the diagonal aligned to
the end of the key sequence, LSE [H, total_q] in fp32, -inf (and a zero
output) for a query with no key -- and `SM70MLAPrefill` has the backend's two
entry points, `run_prefill_new_tokens` (:229-244) and
`run_prefill_context_chunk` (:246-266), with the metadata passed in.

The reference computes in fp32 from fp16/bf16 inputs; the kernel multiplies
fp16 (bf16) inputs exactly into fp32 accumulators and rounds P to fp16 (bf16
P is kept as a hi + lo pair) for the PV product.  The reference backend also
lists fp32 (sm70_triton.py:193), where it computes in fp32 throughout; fp32
inputs here run a kernel of their own on the fp32 MFMA, in fp32 arithmetic
end to end (P included) over the whole fp32 range, with an fp32 output.
"""
from __future__ import annotations

import torch

from . import _lib
from .ops import _check, _stream


# the C ABI's dtype argument
_DTYPE_CODE = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def _cu(t: torch.Tensor, dev) -> torch.Tensor:
    return t.to(device=dev, dtype=torch.int32).contiguous()


def varlen_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor,
                     softmax_scale: float, causal: bool, return_softmax_lse: bool,
                     max_seqlen_q: int | None = None):
    """q [total_q, H, Dq], k [total_k, H, Dq], v [total_k, H, Dv] (fp16, bf16
    or fp32, last dim contiguous); cu_seqlens_* int [num_seqs + 1].  Returns
    out [total_q, H, Dv] (q.dtype) and, if asked, lse [H, total_q] fp32.
    max_seqlen_q saves the host read of the longest query run."""
    _check(q.is_cuda and k.is_cuda and v.is_cuda, "q, k and v must be on the GPU")
    _check(q.dtype in _DTYPE_CODE, "varlen_attention: fp16, bf16 or fp32 inputs")
    _check(k.dtype == q.dtype and v.dtype == q.dtype, "q, k and v must share one dtype")
    _check(q.dim() == 3 and k.dim() == 3 and v.dim() == 3, "q, k, v must be [tokens, heads, dim]")
    total_q, H, d_qk = q.shape
    total_k = k.shape[0]
    _check(k.shape[1] == H and v.shape[1] == H, "q, k and v must have the same head count")
    _check(k.shape[2] == d_qk, "k head dim must equal q's")
    _check(v.shape[0] == total_k, "k and v must have the same token count")
    d_v = v.shape[2]
    num_seqs = cu_seqlens_q.numel() - 1
    _check(num_seqs >= 0 and cu_seqlens_k.numel() == num_seqs + 1,
           "cu_seqlens_q and cu_seqlens_k must have num_seqs + 1 entries")
    out = torch.empty(total_q, H, d_v, dtype=q.dtype, device=q.device)
    lse = (torch.empty(H, total_q, dtype=torch.float32, device=q.device)
           if return_softmax_lse else None)
    if num_seqs > 0 and total_q > 0:
        per16 = 16 // q.element_size()  # elements per 16-byte piece

        def rows(x):
            ok = x.stride(2) == 1 and x.stride(0) % per16 == 0 and x.stride(1) % per16 == 0 \
                and x.data_ptr() % 16 == 0
            return x if ok else x.contiguous()
        q, k, v = rows(q), rows(k), rows(v)
        cq, ck = _cu(cu_seqlens_q, q.device), _cu(cu_seqlens_k, q.device)
        if max_seqlen_q is None:
            max_seqlen_q = int((cq[1:] - cq[:-1]).max()) if num_seqs else 0
        with torch.cuda.device(q.device):
            _lib.call("mi355_dsa_varlen_attention", out.data_ptr(),
                      lse.data_ptr() if lse is not None else None,
                      q.data_ptr(), k.data_ptr(), v.data_ptr(), _DTYPE_CODE[q.dtype],
                      num_seqs, H, d_qk, d_v, q.stride(0), q.stride(1), k.stride(0), k.stride(1),
                      v.stride(0), v.stride(1), out.stride(0), out.stride(1), cq.data_ptr(),
                      ck.data_ptr(), max_seqlen_q, total_q, float(softmax_scale), int(causal),
                      _stream(q))
    if return_softmax_lse:
        return out, lse
    return out


class SM70MLAPrefill:
    """The two attention entry points of the reference's SM70 MLA prefill
    backend, with the prefill metadata passed explicitly."""

    def __init__(self, scale: float):
        self.scale = scale

    def run_prefill_new_tokens(self, q, k, v, query_start_loc, return_softmax_lse: bool):
        """Causal self-attention of each request's new tokens (sm70_triton.py:229-244)."""
        return varlen_attention(q, k, v, query_start_loc, query_start_loc, self.scale,
                                causal=True, return_softmax_lse=return_softmax_lse)

    def run_prefill_context_chunk(self, q, k, v, query_start_loc, chunk_cu_seq_lens):
        """Non-causal attention of the new tokens to one gathered context chunk,
        with LSE for the chunk merge (sm70_triton.py:246-266)."""
        return varlen_attention(q, k, v, query_start_loc, chunk_cu_seq_lens, self.scale,
                                causal=False, return_softmax_lse=True)
