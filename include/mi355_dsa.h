/*
 * mi355_dsa.h -- C ABI of the MI355X (gfx950) DSA sparse-attention kernels.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream
 * (passed as void*; NULL selects the null stream), launches asynchronously on
 * that stream and returns MI355_DSA_OK or an error code.  On error nothing is
 * launched and mi355_dsa_last_error() returns the message of the calling
 * thread's last failure.  No entry point allocates device memory: scratch
 * comes from a caller-provided workspace whose size the matching
 * *_workspace_size() function reports.  No entry point synchronises the
 * stream except mi355_dsa_selfcheck().
 *
 * Each function replaces one host launcher of the reference (file:line
 * citations are relative to the bayley/glm5-on-v100 tree); the argument
 * meaning, tensor layouts and masking conventions follow it.  The torch op
 * schemas that wrap these functions are the reference's
 * (patches/glm5-v100-sm70-glue.patch:494-565).
 *
 * Dtype codes: fp16 tensors are IEEE binary16; "fp8" caches are uint8 rows
 * in the layouts described per function; all index tensors are int32.
 */
#ifndef MI355_DSA_H_
#define MI355_DSA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI355_DSA_OK 0
#define MI355_DSA_EINVAL 1 /* bad argument (shape / size / alignment) */
#define MI355_DSA_EHIP 2   /* HIP runtime error at launch */
#define MI355_DSA_ECHECK 3 /* device self-check mismatch */

/* Message of the calling thread's last error ("" if none). */
const char* mi355_dsa_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int mi355_dsa_abi_version(void);

/*
 * Device self-check, synchronous on `stream`: verifies the MFMA accumulator
 * placement the kernels assume, the ds_read_b64_tr_b16 lane mapping of the
 * attention PV step, and both e4m3 decodes used in the gathers.  Unlike the
 * other entry points it allocates (and frees) a few KB of device memory and
 * synchronises the stream; call it once at start-up, outside graph capture.
 * Replaces the reference's first-launch WMMA layout probe
 * (csrc/attention/sm70_mla_decode.cu:511-540, :2807-2818).
 * Returns MI355_DSA_ECHECK on a mismatch.
 */
int mi355_dsa_selfcheck(void* stream);

/*
 * Indexer-K cache scatter: kv_cache row slot_mapping[t] <- k[t] for every
 * token t with 0 <= slot < n_rows (other slots are skipped on device).
 *   kv_fp8 == 0: kv_cache fp16 rows of head_dim halves (plain copy).
 *   kv_fp8 == 1: kv_cache rows of 132 bytes = 128 e4m3 + fp32 scale, with
 *                scale = max(amax/448, FLT_MIN), e4m3 = RNE-satfinite(k/scale);
 *                head_dim must be 128.
 *   k: fp16 [n_tok, head_dim] contiguous; n_rows = rows in kv_cache.
 * Replaces sm70_indexer_k_store (csrc/attention/sm70_mla_decode.cu:2910-2939).
 */
int mi355_dsa_indexer_k_store(void* kv_cache, int kv_fp8, int64_t n_rows,
                              const void* k, int64_t n_tok, int head_dim,
                              const int32_t* slot_mapping, void* stream);

/*
 * MLA latent cache writer: kv_cache row slot_mapping[t] <- token t for every
 * t < n_tok with 0 <= slot < n_rows (other slots are skipped on device).
 *   kv_c: [n_tok, >= 512] 16-bit rows (row stride kv_c_stride elements),
 *   k_pe: [n_tok, >= 64] 16-bit rows (row stride k_pe_stride elements),
 *         in_bf16 = 1: bf16 inputs, else fp16; rows 16-byte aligned.
 *   kv_fp8 == 0 ("auto"): kv_cache rows of 576 fp16 = [kv_c | k_pe]
 *                (fp16 inputs only).
 *   kv_fp8 == 1 ("fp8_ds_mla"): kv_cache rows of 656 bytes = 512 e4m3 with
 *                one scale per 128-dim tile, scale = max(amax/448, FLT_MIN),
 *                e4m3 = RNE-satfinite(kv_c/scale); then the 4 fp32 scales;
 *                then k_pe's 64 16-bit values unchanged.
 *   slot_mapping: int64 (slot_i64 = 1) or int32 [n_tok].
 * Replaces vLLM's concat_and_cache_mla for kv_cache_dtype "auto" and
 * "fp8_ds_mla" (concat_and_cache_ds_mla_kernel; the reference carries only
 * its amax fix, patches/glm5-v100-sm70-glue.patch:517-531).
 */
int mi355_dsa_concat_and_cache_mla(void* kv_cache, int kv_fp8, int64_t n_rows,
                                   const void* kv_c, int64_t kv_c_stride,
                                   const void* k_pe, int64_t k_pe_stride,
                                   int in_bf16, int64_t n_tok,
                                   const void* slot_mapping, int slot_i64,
                                   void* stream);

/*
 * Dense MLA decode over a paged fp16 latent cache: for each token b and head
 * h, attention of q[b,h,:576] * scale over the cache rows of positions
 * [0, seq_lens[b]) (row(p) = bt[b, p/page]*page + p%page; a position whose
 * page index is >= max_blocks or whose row is outside [0, n_kv_rows) is
 * skipped).  V = the first 512 dims of a row.  q * scale is rounded to fp16
 * (scale itself rounded to fp16 first) and P to fp16 before PV; O is
 * accumulated in fp32.  o fp16 [B,H,512], lse fp32 [B,H] (natural log; a
 * token with no valid position gets o = 0, lse = -inf).  kv_cache rows are
 * 576 fp16; n_kv_rows counts them.  Needs workspace of
 * mi355_dsa_mla_decode_workspace_size(B, n_head, max_blocks * page_size)
 * bytes (16-byte aligned; 0 means none).
 * Replaces sm70_mla_decode (csrc/attention/sm70_mla_decode.cu:717-898, host
 * :1474-1534), whose kernel keeps the running O in fp16 between 32-key tiles.
 */
size_t mi355_dsa_mla_decode_workspace_size(int B, int n_head, int max_kv);
int mi355_dsa_mla_decode(void* o, float* lse, const void* q, int B, int n_head,
                         const void* kv_cache, int64_t n_kv_rows, int page_size,
                         const int32_t* block_table, int max_blocks,
                         const int32_t* seq_lens, float scale, void* workspace,
                         size_t workspace_bytes, void* stream);

/*
 * Exact top-K merge of key-sharded indexer candidates.  allf fp32
 * [tp, R, 2K]: per shard s and row r, K scores then K positions (int32
 * bits).  Row r's output is the K candidates of largest
 * (mono(score) << 32) | (tp*K - 1 - (s*K + c)) -- by score, ties to the lower
 * column -- as positions (-1 for a selection at or below mono(-inf)), sorted
 * ascending, written to out row dst_base + r (dst_base >= 0) or dst_rows[r]
 * (int32 device array; rows outside [0, out_rows) are skipped).  out is int32
 * with row stride out_stride >= K.  K a power of two <= 2048; tp*K a multiple
 * of 512, at most 8192.
 * Replaces sm70_indexer_shard_merge (csrc/attention/sm70_mla_decode.cu:
 * 2055-2182, host :2411-2436); the all-gather that produces allf is the
 * caller's.
 */
int mi355_dsa_indexer_shard_merge(int32_t* out, int64_t out_stride, int64_t out_rows,
                                  const float* allf, int tp, int R, int K,
                                  const int32_t* dst_rows, int dst_base, void* stream);

/*
 * Dense varlen attention (MLA prefill, multi-head form):
 *   out[t,h,:] = softmax(scale * q[t,h,:] . k[j,h,:]) v[j,h,:]
 * over the keys j of token t's sequence s: queries cu_seqlens_q[s] ..
 * cu_seqlens_q[s+1]-1, keys cu_seqlens_k[s] .. cu_seqlens_k[s+1]-1 (int32
 * device arrays of num_seqs + 1).  causal != 0: query i (0-based in its
 * sequence of q_len) sees keys j <= i + k_len - q_len.  lse (nullable) is
 * fp32 [n_head, total_q], natural log; a query with no key gets out = 0 and
 * lse = -inf.  q/k/v/out are fp16 (dtype = 0), bf16 (dtype = 1) or fp32
 * (dtype = 2, computed in fp32 arithmetic on the fp32 MFMA) with unit
 * last-dim stride and the given element strides (multiples of one 16-byte
 * piece: 8 elements, 4 for fp32; out: 4), q/k/v 16-byte aligned, out 8-byte
 * (fp32: 16-byte) aligned.  (d_qk, d_v) in {(192,128), (128,128), (64,64),
 * (256,256)}.  max_q_len = the longest query run.
 * Replaces the reference's dense MLA prefill attention, _varlen_attention
 * (vllm/v1/attention/backends/mla/prefill/sm70_triton.py:54-187).
 */
int mi355_dsa_varlen_attention(void* out, float* lse, const void* q, const void* k,
                               const void* v, int dtype, int num_seqs, int n_head, int d_qk,
                               int d_v, int64_t q_tok_stride, int64_t q_head_stride,
                               int64_t k_tok_stride, int64_t k_head_stride,
                               int64_t v_tok_stride, int64_t v_head_stride,
                               int64_t o_tok_stride, int64_t o_head_stride,
                               const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                               int max_q_len, int total_q, float softmax_scale, int causal,
                               void* stream);

/*
 * Per-head projection of an MLA layer (fp16 in and out, fp32 accumulation):
 *   out[t,h,n]   = sum_k x[t,h,k] * wt[h,n,k]    (t < T, h < H, n < N, k < K)
 *   out[t,h,N+i] = x[t,h,K+i]                    (i < tail)
 * x and out are addressed with element strides (token, head); wt is the
 * per-head weight transposed, [H, N, K] contiguous.  K must be a multiple of
 * 32 (of 64 when 256 <= K < 512, of 128 when K >= 512) and at most 1024; N a
 * multiple of 64 (K < 256), 32 (256 <= K < 512) or 16 (K >= 512); tail a
 * multiple of 8.  x and wt 16-byte aligned with strides that are multiples of
 * 8 elements (out too when tail > 0).
 * Replaces the torch.bmm calls around the attention op with their transposes
 * and concatenation: q_nope @ W_UK_T concatenated with q_pe
 * (reference/triton_mla.py:388-418: x = q, K = qk_nope_head_dim, N = 512,
 * tail = 64, wt = W_UK_T transposed) and o @ W_UV (:486-492: x = o, K = 512,
 * N = v_head_dim, tail = 0, wt = W_UV transposed).
 */
int mi355_dsa_head_proj(void* out, int64_t out_tok_stride, int64_t out_head_stride,
                        const void* x, int64_t x_tok_stride, int64_t x_head_stride,
                        const void* wt, int T, int H, int N, int K, int tail,
                        void* stream);

/*
 * Attention of one DSA decode layer step with its W_UV projection: o and lse
 * as mi355_dsa_sparse_mla_decode (same arguments, same workspace size), then
 * out[b, h*V + n] = sum_k o[b,h,k] * uv_t[h,n,k] as mi355_dsa_head_proj
 * (x = o, K = 512, N = V, tail 0; out rows out_tok_stride apart).  When the
 * decode splits the keys, B <= 16 and V is a multiple of 32, the split
 * merge and the projection run as one launch; o, lse and out are
 * bit-identical either way.  Replaces, for the layer harness, the caller's
 * sparse attention plus W_UV bmm (reference/triton_mla.py:292-301, :486-492);
 * it has no single counterpart in the reference.
 */
int mi355_dsa_decode_layer_attention(
    void* out, int64_t out_tok_stride, void* o, float* lse, const void* q, int B, int n_head,
    const void* kv_cache, int kv_fp8, int64_t n_kv_rows, int page_size, const int32_t* idx,
    int topk, const int32_t* block_table, int max_blocks, const int32_t* seq_lens, float scale,
    const void* uv_t, int V, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Fused prologue of one DSA decode layer step: the work before the indexer
 * that depends only on the step's inputs, as one launch.  Equal, bit for
 * bit, to the four calls
 *   mi355_dsa_head_proj(q_lat, ..., q, ..., wt_uk, T, H, N, K, tail)
 *   mi355_dsa_concat_and_cache_mla(kv_cache, kv_fp8, kv_rows, kv_c, kv_c_stride,
 *                                  k_pe, k_pe_stride, in_bf16, T, slot_mapping, slot_i64)
 *   mi355_dsa_indexer_k_store(idx_cache, idx_fp8, idx_rows, idx_k, T, 128, idx_slot)
 *   a clear of hist (hist_words int32, a multiple of 4, 16-byte aligned)
 * with the argument rules of each (the projection always takes the
 * decode-shaped kernel; idx_k is fp16 [T, 128], 16-byte aligned).  T is the
 * step's token count for all four.  It has no single counterpart in the
 * reference: it replaces, for the layer harness, the indexer-K store and
 * zeroed histogram of reference/sparse_attn_indexer.py:553-555 and :601 and
 * the latent write and q_nope @ W_UK_T of vLLM's MLA layer (the projection
 * restated at reference/triton_mla.py:406-418).
 */
int mi355_dsa_decode_layer_prologue(
    void* q_lat, int64_t ql_tok_stride, int64_t ql_head_stride, const void* q,
    int64_t q_tok_stride, int64_t q_head_stride, const void* wt_uk, int T, int H, int N, int K,
    int tail, void* kv_cache, int kv_fp8, int64_t kv_rows, const void* kv_c,
    int64_t kv_c_stride, const void* k_pe, int64_t k_pe_stride, int in_bf16,
    const void* slot_mapping, int slot_i64, void* idx_cache, int idx_fp8, int64_t idx_rows,
    const void* idx_k, const int32_t* idx_slot, int32_t* hist, int64_t hist_words,
    void* stream);

/*
 * The cache writes and the indexer logits of one DSA decode layer step as one
 * launch: the latent-cache and indexer-K writes of the step's T tokens (the
 * arguments of mi355_dsa_decode_layer_prologue from kv_cache to idx_slot)
 * and the logits with the level-1 histogram as mi355_dsa_indexer_logits
 * over idx_cache (32 heads x 128 dims; score [B, max_kv], idx_q [B, 32, 128],
 * idx_w [B, 32], the cache's page size, block_table [B, max_blocks],
 * seq_lens [B]).  hist [B, 4096] must be zero on entry
 * (mi355_dsa_decode_layer_topk leaves it so); T <= 64.  Results equal, bit
 * for bit, the separate calls (the reference's indexer-K store,
 * sparse_attn_indexer.py:553-555, then its logits, :586-590).
 */
int mi355_dsa_decode_layer_indexer(
    int T, void* kv_cache, int kv_fp8, int64_t kv_rows, const void* kv_c, int64_t kv_c_stride,
    const void* k_pe, int64_t k_pe_stride, int in_bf16, const void* slot_mapping, int slot_i64,
    void* idx_cache, int idx_fp8, int64_t idx_rows, const void* idx_k, const int32_t* idx_slot,
    float* score, int B, int max_kv, const void* idx_q, const void* idx_w, int idx_page_size,
    const int32_t* block_table, int max_blocks, const int32_t* seq_lens, int32_t* hist,
    void* stream);

/*
 * Indexer logits (decode and generic path):
 *   score[b,p] = sum_h relu(q[b,h,:] . K[row(b,p),:]) * w[b,h]   (p < seq_len[b])
 *   score[b,p] = -inf                                          (seq_len[b] <= p < max_kv)
 * with row(b,p) = bt[b, p/page]*page + p%page; a row outside [0,n_kv_rows)
 * or a page index >= max_blocks reads K = 0.  q fp16 [B,32,128], w fp16
 * [B,32], bt int32 [B,max_blocks], seq_lens int32 [B], score fp32
 * [B,max_kv].  k_fp8 selects the 132-byte fp8 rows (see k_store), else fp16
 * rows of 128 halves.  page_size must be a power of two.  hist (nullable)
 * is a caller-zeroed int32 [B,4096]; when given, hist[b, mono(score)>>20]
 * is incremented for every p < seq_len[b] (mono = monotone fp32 key).
 * Replaces sm70_indexer_logits (csrc/attention/sm70_mla_decode.cu:2626-2764).
 */
int mi355_dsa_indexer_logits(float* score, int B, int max_kv, const void* q,
                             int n_ihead, int head_dim, const void* k_cache,
                             int k_fp8, int64_t n_kv_rows, int page_size,
                             const void* weights, const int32_t* block_table,
                             int max_blocks, const int32_t* seq_lens,
                             int32_t* hist, void* stream);

/*
 * Prefill indexer logits from pre-packed Q.  Same math as
 * mi355_dsa_indexer_logits without hist; q_packed is fp16
 * [32, ceil(B/16), 8, 16, 16] with q_packed[h][t][kt][r][c] = q[16t+r, h,
 * 16kt+c] (rows >= B zero).  As in the reference, the key tile of a query
 * tile is gathered with the block-table row of the tile's first query: all
 * rows of a call are expected to share one table (the per-segment caller
 * expands a single request row).
 * Replaces sm70_indexer_logits_packed (csrc/attention/sm70_mla_decode.cu:2771-2836).
 */
int mi355_dsa_indexer_logits_packed(float* score, int B, int max_kv,
                                    const void* q_packed, const void* k_cache,
                                    int k_fp8, int64_t n_kv_rows, int page_size,
                                    const void* weights,
                                    const int32_t* block_table, int max_blocks,
                                    const int32_t* seq_lens, void* stream);

/*
 * Decode top-k: idx[b,:] = the positions p < seq_len[b] of the k largest
 * score[b,p] (exact 32-bit order; equal scores prefer the lower position),
 * written in ascending position order and padded with -1.  hist is the
 * [B,4096] level-1 histogram built by mi355_dsa_indexer_logits.  The
 * workspace holds candidate lists only (no state between calls); per-row
 * arrival counters of the one-launch path live in a library-owned device
 * array, one slot per stream and per captured call.
 * Replaces sm70_decode_topk (csrc/attention/sm70_mla_decode.cu:2844-2905).
 */
size_t mi355_dsa_decode_topk_workspace_size(int B, int max_kv, int k);
int mi355_dsa_decode_topk(int32_t* idx, const float* score,
                          const int32_t* seq_lens, const int32_t* hist, int B,
                          int max_kv, int k, void* workspace,
                          size_t workspace_bytes, void* stream);

/*
 * The top-k phase of one DSA decode layer step (the layer harness): the
 * decode top-k as mi355_dsa_decode_topk (same first nine arguments), which
 * also leaves hist zero (16-byte aligned) for the next step's
 * mi355_dsa_decode_layer_indexer, and the q_nope -> latent projection as
 * mi355_dsa_head_proj (x = q, wt = W_UK_T^T [H, N, K], carried tail
 * columns).  On the one-launch and two-kernel top-k paths with K < 256 the
 * projection runs in the launch that selects, on CUs the select leaves
 * idle.  Results are
 * bit-identical to the two calls.  The reference zeroes a fresh histogram
 * each step (reference/sparse_attn_indexer.py:601) and projects q in the MLA
 * layer (triton_mla.py:413-418).
 */
int mi355_dsa_decode_layer_topk(
    int32_t* idx, const float* score, const int32_t* seq_lens, int32_t* hist, int B, int max_kv,
    int k, void* workspace, size_t workspace_bytes, void* q_lat, int64_t ql_tok_stride,
    int64_t ql_head_stride, const void* q, int64_t q_tok_stride, int64_t q_head_stride,
    const void* wt_uk, int T, int H, int N, int K, int tail, void* stream);

/*
 * Row-wise top-k for prefill: same selection contract as decode_topk, per
 * row r of score [n_rows, row_stride] with valid length seq_lens[r]
 * (clamped to row_stride); idx [n_rows, k].  Builds its own histograms.
 * Replaces vLLM's persistent_topk as called at
 * reference/sparse_attn_indexer.py:873-880 (max_seq_len is accepted for
 * signature parity and only bounds-checked).
 */
size_t mi355_dsa_persistent_topk_workspace_size(int n_rows, int row_stride,
                                                int k);
int mi355_dsa_persistent_topk(const float* score, int n_rows, int row_stride,
                              const int32_t* seq_lens, int32_t* idx, int k,
                              int max_seq_len, void* workspace,
                              size_t workspace_bytes, void* stream);

/*
 * Sparse (top-k) MLA attention over the paged latent cache, decode and
 * prefill.  For each token b and head h:
 *   s_j  = fp16(q[b,h,:] * fp16(scale)) . K_j      (576 dims)
 *   o    = sum_j softmax(s)_j V_j                   (V_j = K_j[0:512])
 *   lse  = max_j s_j + ln sum_j exp(s_j - max)      (-inf when no key valid)
 * over the selected keys j = idx[b,i] with 0 <= j < seq_len[b].  A selected
 * key whose row does not resolve inside the cache (negative block, row past
 * the cache) follows the reference's dispatch (:2511): for B >= 32 and
 * H <= 16 it is masked and an empty token's lse is -1e30 (its prefill
 * kernel, :1617-1628, :1789-1793); otherwise it is a zero key with score 0
 * (its split-decode kernel, :970-992).  q fp16 [B,H,576], o fp16 [B,H,512],
 * lse fp32 [B,H], idx int32 [B,topk] (logical positions, -1 unused),
 * bt int32 [B,max_blocks], seq_lens int32 [B].  kv_fp8 == 0: fp16 rows of
 * 576 halves; kv_fp8 == 1: 656-byte fp8_ds_mla rows.
 * Replaces sm70_sparse_mla_decode (csrc/attention/sm70_mla_decode.cu:2457-2616).
 */
size_t mi355_dsa_sparse_mla_workspace_size(int B, int n_head, int topk);
int mi355_dsa_sparse_mla_decode(void* o, float* lse, const void* q, int B,
                                int n_head, const void* kv_cache, int kv_fp8,
                                int64_t n_kv_rows, int page_size,
                                const int32_t* idx, int topk,
                                const int32_t* block_table, int max_blocks,
                                const int32_t* seq_lens, float scale,
                                void* workspace, size_t workspace_bytes,
                                void* stream);

/*
 * mi355_dsa_sparse_mla_decode without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * that forbid allocation).  It has no counterpart in the reference.  The
 * split partials go to a library-owned device array of
 * mi355_dsa_sparse_mla_noalloc_max_bytes() bytes (32 MiB) per device, held
 * from the library's load until the process ends; a call needing more
 * (mi355_dsa_sparse_mla_workspace_size(B, n_head, topk) larger than that,
 * e.g. B >= 128 at 16 heads and topk 2048; no 64-head shape at topk 2048)
 * returns MI355_DSA_EINVAL and
 * launches nothing.  Every call on one device shares that device's array:
 * calls that overlap on one device (different streams) race and must be
 * serialised by the caller.  Results equal mi355_dsa_sparse_mla_decode's bit
 * for bit.  Neither entry point calls hipMalloc or hipFree.
 */
size_t mi355_dsa_sparse_mla_noalloc_max_bytes(void);
int mi355_dsa_sparse_mla_decode_noalloc(void* o, float* lse, const void* q,
                                        int B, int n_head,
                                        const void* kv_cache, int kv_fp8,
                                        int64_t n_kv_rows, int page_size,
                                        const int32_t* idx, int topk,
                                        const int32_t* block_table,
                                        int max_blocks,
                                        const int32_t* seq_lens, float scale,
                                        void* stream);

/*
 * fp8-e4m3 weight-only GEMV: y[m,n] = sum_k x[m,k] * e4m3(w[n,k]) * s[n/128,k/128]
 * x fp16 [M,K], w uint8 [N,K], s fp32 [ceil(N/128), ceil(K/128)], y fp16
 * [M,N]; 1 <= M <= 8, K % 16 == 0, N % 8 == 0, all contiguous.
 * Replaces sm70_attn_fp8_gemv (csrc/attention/sm70_attn_fp8.cu:148-191).
 */
int mi355_dsa_attn_fp8_gemv(void* y, const void* x, const uint8_t* w,
                            const float* s, int M, int N, int K, void* stream);

/*
 * fp8-e4m3 block dequant: out[n,k] = fp16_rn(e4m3(w[n,k]) * s[n/128,k/128]).
 * Replaces sm70_attn_fp8_dequant (csrc/attention/sm70_attn_fp8.cu:193-215).
 */
int mi355_dsa_attn_fp8_dequant(void* out, const uint8_t* w, const float* s,
                               int N, int K, void* stream);

/*
 * Load-time weight quantizer: w fp16 [N,K] (row-major, contiguous) ->
 * q e4m3 bytes [N,K] and s fp32 [ceil(N/128), ceil(K/128)] with, per
 * 128x128 block, s = max(amax/448, 1e-12) and q = e4m3_rne(clamp(w/s,
 * +-448)).  Produces the inputs of mi355_dsa_attn_fp8_gemv / _dequant.
 * Replaces _sm70_attn_fp8_quantize (patches/glm5-v100-sm70-glue.patch:
 * 1515-1532), which the reference runs in PyTorch at model load.
 */
int mi355_dsa_attn_fp8_quantize(uint8_t* q, float* s, const void* w, int N, int K, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MI355_DSA_H_ */
