// Fused prologue of one DSA decode layer step (the layer harness,
// glm5-on-v100_amd/dsa_layer.py): the four pieces of work that precede the
// indexer and do not depend on each other run as one launch instead of four.
//
//   * q_latent: q_nope [T, H, K] through W_UK_T (head_proj_block, with q's
//     RoPE columns carried), as mi355_dsa_head_proj;
//   * the latent-cache write of the step's tokens (concat_cache_mla_block),
//     as mi355_dsa_concat_and_cache_mla;
//   * the indexer-K cache write (k_store_*_block), as
//     mi355_dsa_indexer_k_store;
//   * clearing the [B, 4096] top-k histogram that the indexer logits fill.
//
// In the reference's model runner these are separate launches
// (reference/sparse_attn_indexer.py:553-555 for the indexer-K store and :601
// for the zeroed histogram; the latent write and q_nope @ W_UK_T run in
// vLLM's MLA layer, a projection the reference's prefill path restates at
// triton_mla.py:406-418).  At decode sizes
// each is one small round of loads and stores (~1.6 us of launch in a HIP
// graph, plus a memory round trip); one launch overlaps them.  Every
// workgroup runs exactly one piece, chosen by its index range, with the same
// code as the standalone kernel, so the results are bit-identical to the
// four separate calls.
#include <algorithm>

#include "cache_write.h"
#include "capi_internal.h"
#include "dsa_common.h"
#include "head_proj.h"
#include "indexer_decode.h"

namespace mi355dsa {
namespace {

struct PrologueArgs {
  // q_latent (decode-shaped head projection)
  HpArgs hp;
  int hp_kw;      // 1, 2 or 4: k split of the projection's waves
  int hp_gx;      // workgroups per token chunk
  int hp_wgs;     // hp_gx * token chunks
  // latent-cache write
  const uint8_t* kv_c;
  int64_t kv_c_stride;  // bytes
  const uint8_t* k_pe;
  int64_t k_pe_stride;  // bytes
  const void* slot;
  uint8_t* kv;
  int64_t kv_rows;
  int lat_kind;  // 0: fp16 rows, 1: fp8_ds_mla from fp16, 2: fp8_ds_mla from bf16
  int slot_i64;
  int lat_wgs;
  // indexer-K write (head_dim 128)
  const u32x4* ik;
  const int32_t* ik_slot;
  void* ik_cache;
  int64_t ik_rows;
  int ik_fp8;
  int ik_wgs;
  // histogram to clear
  u32x4* hist;
  int64_t hist_vec;  // 16-byte units
  int hz_wgs;
  int64_t n_tok;
};

constexpr int kHzPerWg = 4096;  // 16-byte units cleared per workgroup

template <bool FP8, bool BF16>
__device__ __forceinline__ void latent_block(const PrologueArgs& a, int bx) {
  if (a.slot_i64)
    concat_cache_mla_block<FP8, BF16, int64_t>(a.kv_c, a.kv_c_stride, a.k_pe, a.k_pe_stride,
                                               reinterpret_cast<const int64_t*>(a.slot), a.kv,
                                               a.n_tok, a.kv_rows, bx);
  else
    concat_cache_mla_block<FP8, BF16, int32_t>(a.kv_c, a.kv_c_stride, a.k_pe, a.k_pe_stride,
                                               reinterpret_cast<const int32_t*>(a.slot), a.kv,
                                               a.n_tok, a.kv_rows, bx);
}

// Workgroup id of the prologue's grid: one piece, chosen by index range.
__device__ __forceinline__ void prologue_piece(const PrologueArgs& a, int id) {
  if (id < a.lat_wgs) {
    if (a.lat_kind == 0) latent_block<false, false>(a, id);
    else if (a.lat_kind == 1) latent_block<true, false>(a, id);
    else latent_block<true, true>(a, id);
    return;
  }
  id -= a.lat_wgs;
  if (id < a.ik_wgs) {
    if (a.ik_fp8)
      k_store_fp8_block(a.ik, a.ik_slot, reinterpret_cast<uint8_t*>(a.ik_cache), a.n_tok,
                        a.ik_rows, id);
    else
      k_store_f16_vec_block(a.ik, a.ik_slot, reinterpret_cast<u32x4*>(a.ik_cache), a.n_tok,
                            kIdxHeadDim / 8, a.ik_rows, id, threadIdx.x, kIdxHeadDim / 8,
                            256 / (kIdxHeadDim / 8));
    return;
  }
  id -= a.ik_wgs;
  if (id < a.hz_wgs) {
    const u32x4 z = {0u, 0u, 0u, 0u};
    const int64_t hi = min((int64_t)(id + 1) * kHzPerWg, a.hist_vec);
    for (int64_t i = (int64_t)id * kHzPerWg + threadIdx.x; i < hi; i += 256) a.hist[i] = z;
    return;
  }
  id -= a.hz_wgs;
  const int bx = id % a.hp_gx, by = id / a.hp_gx;
  if (a.hp_kw == 1) head_proj_block<4, 1>(a.hp, bx, by);
  else if (a.hp_kw == 2) head_proj_block<2, 2>(a.hp, bx, by);
  else head_proj_block<1, 4>(a.hp, bx, by);
}

__global__ void __launch_bounds__(256) decode_prologue_kernel(PrologueArgs a) {
  prologue_piece(a, blockIdx.x);
}

// The step's two cache writes, then its indexer logits: n_pro cache-write
// workgroups at the front of the grid, then n_tiles logits workgroups per
// token row.  The logits workgroups that read
// a row the step's indexer-K write targets write that row themselves first
// (indexer_logits_block with NEWK), so no workgroup waits on another; the
// histogram must already be zero (the consuming top-k leaves it so).
struct LayerIdxArgs {
  PrologueArgs pro;
  int n_pro;
  IdxDecArgs idx;
  IdxNewKeys nk;
  int n_tiles;
};

template <bool KFP8>
__global__ void __launch_bounds__(256) decode_layer_indexer_kernel(LayerIdxArgs a) {
  int id = blockIdx.x;
  if (id < a.pro.lat_wgs) {  // the latent-cache write
    if (a.pro.lat_kind == 0) latent_block<false, false>(a.pro, id);
    else if (a.pro.lat_kind == 1) latent_block<true, false>(a.pro, id);
    else latent_block<true, true>(a.pro, id);
    return;
  }
  id -= a.pro.lat_wgs;
  if (id < a.pro.ik_wgs) {  // the indexer-K write
    if (KFP8)
      k_store_fp8_block(a.pro.ik, a.pro.ik_slot, reinterpret_cast<uint8_t*>(a.pro.ik_cache),
                        a.pro.n_tok, a.pro.ik_rows, id);
    else
      k_store_f16_vec_block(a.pro.ik, a.pro.ik_slot, reinterpret_cast<u32x4*>(a.pro.ik_cache),
                            a.pro.n_tok, kIdxHeadDim / 8, a.pro.ik_rows, id, threadIdx.x,
                            kIdxHeadDim / 8, 256 / (kIdxHeadDim / 8));
    return;
  }
  id = blockIdx.x;
  if (id < a.n_pro) return;
  const int i = id - a.n_pro;
  indexer_logits_block<KFP8, true>(a.idx, i % a.n_tiles, i / a.n_tiles, a.nk);
}

}  // namespace
}  // namespace mi355dsa

using namespace mi355dsa;

// Arguments and grid of the prologue's pieces, with the checks of the
// standalone calls.  q_lat null: no projection; hist null (hist_words 0): no
// clear.
static int make_prologue(
    PrologueArgs& a, int64_t& total, void* q_lat, int64_t ql_tok_stride,
    int64_t ql_head_stride, const void* q, int64_t q_tok_stride, int64_t q_head_stride,
    const void* wt_uk, int T, int H, int N, int K, int tail, void* kv_cache, int kv_fp8,
    int64_t kv_rows, const void* kv_c, int64_t kv_c_stride, const void* k_pe,
    int64_t k_pe_stride, int in_bf16, const void* slot_mapping, int slot_i64, void* idx_cache,
    int idx_fp8, int64_t idx_rows, const void* idx_k, const int32_t* idx_slot, int32_t* hist,
    int64_t hist_words) {
  DSA_CHECK(T >= 1, "decode_layer: bad sizes");
  DSA_CHECK(kv_cache && kv_c && k_pe && slot_mapping && idx_cache && idx_k && idx_slot &&
                (hist || hist_words == 0),
            "decode_layer: null pointer argument");
  a = PrologueArgs{};
  int64_t hp_wgs = 0;
  if (q_lat != nullptr) {
    // q_latent: the checks of mi355_dsa_head_proj (decode-shaped kernel)
    const int rc = hp_decode_setup(a.hp, a.hp_kw, a.hp_gx, hp_wgs, "decode_layer", q_lat,
                                   ql_tok_stride, ql_head_stride, q, q_tok_stride,
                                   q_head_stride, wt_uk, T, H, N, K, tail);
    if (rc) return rc;
  }
  // latent write: the checks of mi355_dsa_concat_and_cache_mla
  DSA_CHECK(kv_rows >= 0, "decode_layer: kv_rows must be >= 0");
  DSA_CHECK(aligned_to(kv_cache, 16) && aligned_to(kv_c, 16) && aligned_to(k_pe, 16),
            "decode_layer: kv_cache, kv_c and k_pe must be 16-byte aligned");
  DSA_CHECK(kv_c_stride >= kValueDim && k_pe_stride >= kLatentDim - kValueDim &&
                kv_c_stride % 8 == 0 && k_pe_stride % 8 == 0,
            "decode_layer: kv_c / k_pe row strides must be >= their widths and "
            "multiples of 8 elements");
  DSA_CHECK(!in_bf16 || kv_fp8, "decode_layer: the fp16 latent cache takes fp16 inputs");
  // indexer-K write (head_dim 128): the checks of mi355_dsa_indexer_k_store
  DSA_CHECK(idx_rows >= 0, "decode_layer: idx_rows must be >= 0");
  DSA_CHECK(aligned_to(idx_k, 16), "decode_layer: idx_k must be 16-byte aligned");
  DSA_CHECK(idx_fp8 ? aligned_to(idx_cache, 4) : aligned_to(idx_cache, 16),
            "decode_layer: idx_cache is misaligned");
  // histogram
  DSA_CHECK(hist_words >= 0 && hist_words % 4 == 0 && (hist_words == 0 || aligned_to(hist, 16)),
            "decode_layer: hist must be 16-byte aligned, a multiple of 4 words");

  a.kv_c = reinterpret_cast<const uint8_t*>(kv_c);
  a.kv_c_stride = kv_c_stride * 2;
  a.k_pe = reinterpret_cast<const uint8_t*>(k_pe);
  a.k_pe_stride = k_pe_stride * 2;
  a.slot = slot_mapping;
  a.kv = reinterpret_cast<uint8_t*>(kv_cache);
  a.kv_rows = kv_rows;
  a.lat_kind = !kv_fp8 ? 0 : (in_bf16 ? 2 : 1);
  a.slot_i64 = slot_i64 ? 1 : 0;
  a.lat_wgs = (T + 3) / 4;
  a.ik = reinterpret_cast<const u32x4*>(idx_k);
  a.ik_slot = idx_slot;
  a.ik_cache = idx_cache;
  a.ik_rows = idx_rows;
  a.ik_fp8 = idx_fp8 ? 1 : 0;
  a.ik_wgs = (T + 15) / 16;  // fp8: 16 tokens per workgroup; fp16: 16 lanes x 16 tokens
  a.hist = reinterpret_cast<u32x4*>(hist);
  a.hist_vec = hist_words / 4;
  a.hz_wgs = (int)((a.hist_vec + kHzPerWg - 1) / kHzPerWg);
  a.n_tok = T;
  a.hp_wgs = (int)hp_wgs;
  total = (int64_t)a.lat_wgs + a.ik_wgs + a.hz_wgs + hp_wgs;
  DSA_CHECK(total < ((int64_t)1 << 31), "decode_layer: grid too large");
  return MI355_DSA_OK;
}

extern "C" int mi355_dsa_decode_layer_prologue(
    void* q_lat, int64_t ql_tok_stride, int64_t ql_head_stride, const void* q,
    int64_t q_tok_stride, int64_t q_head_stride, const void* wt_uk, int T, int H, int N, int K,
    int tail, void* kv_cache, int kv_fp8, int64_t kv_rows, const void* kv_c,
    int64_t kv_c_stride, const void* k_pe, int64_t k_pe_stride, int in_bf16,
    const void* slot_mapping, int slot_i64, void* idx_cache, int idx_fp8, int64_t idx_rows,
    const void* idx_k, const int32_t* idx_slot, int32_t* hist, int64_t hist_words,
    void* stream) {
  clear_error();
  PrologueArgs a;
  int64_t total = 0;
  const int rc = make_prologue(a, total, q_lat, ql_tok_stride,
                               ql_head_stride, q, q_tok_stride, q_head_stride, wt_uk, T, H, N, K,
                               tail, kv_cache, kv_fp8, kv_rows, kv_c, kv_c_stride, k_pe,
                               k_pe_stride, in_bf16, slot_mapping, slot_i64, idx_cache, idx_fp8,
                               idx_rows, idx_k, idx_slot, hist, hist_words);
  if (rc) return rc;
  DSA_CHECK(q_lat != nullptr && hist != nullptr, "decode_layer_prologue: null pointer argument");
  decode_prologue_kernel<<<dim3((unsigned)total), 256, 0, as_stream(stream)>>>(a);
  DSA_LAUNCH_CHECK("decode_layer_prologue");
  return MI355_DSA_OK;
}

// The step's two cache writes and its indexer logits as one launch.  Results
// equal, bit for bit, mi355_dsa_concat_and_cache_mla and
// mi355_dsa_indexer_k_store followed by mi355_dsa_indexer_logits over
// idx_cache: the logits workgroups that read a row the step writes write
// that row first, with the store's own code.  The histogram must be zero on
// entry (mi355_dsa_decode_layer_topk leaves it so); the step's tokens are at
// most kIdxMaxNew.
extern "C" int mi355_dsa_decode_layer_indexer(
    int T, void* kv_cache, int kv_fp8, int64_t kv_rows, const void* kv_c, int64_t kv_c_stride,
    const void* k_pe, int64_t k_pe_stride, int in_bf16, const void* slot_mapping, int slot_i64,
    void* idx_cache, int idx_fp8, int64_t idx_rows, const void* idx_k, const int32_t* idx_slot,
    float* score, int B, int max_kv, const void* idx_q, const void* idx_w, int idx_page_size,
    const int32_t* block_table, int max_blocks, const int32_t* seq_lens, int32_t* hist,
    void* stream) {
  clear_error();
  LayerIdxArgs a{};
  int64_t n_pro = 0;
  int rc = make_prologue(a.pro, n_pro, nullptr, 0, 0, nullptr, 0, 0, nullptr, T, 0, 0, 0, 0,
                         kv_cache, kv_fp8, kv_rows, kv_c, kv_c_stride, k_pe, k_pe_stride,
                         in_bf16, slot_mapping, slot_i64, idx_cache, idx_fp8, idx_rows, idx_k,
                         idx_slot, nullptr, 0);
  if (rc) return rc;
  DSA_CHECK(T <= kIdxMaxNew, "decode_layer_indexer: at most %d new tokens, got %d", kIdxMaxNew, T);
  // the checks of mi355_dsa_indexer_logits (32 heads x 128 dims)
  DSA_CHECK(B >= 1 && B <= 65535 && max_kv >= 0 && max_blocks >= 0,
            "decode_layer_indexer: bad sizes");
  DSA_CHECK(score && idx_q && idx_w && block_table && seq_lens && hist,
            "decode_layer_indexer: null pointer argument");
  DSA_CHECK(idx_page_size > 0 && (idx_page_size & (idx_page_size - 1)) == 0,
            "decode_layer_indexer: indexer cache page size must be a power of two");
  DSA_CHECK(aligned_to(idx_q, 16), "decode_layer_indexer: idx_q must be 16-byte aligned");
  DSA_CHECK(aligned_to(hist, 4), "decode_layer_indexer: hist must be 4-byte aligned");
  IdxDecArgs& d = a.idx;
  d.Q = reinterpret_cast<const f16*>(idx_q);
  d.Kv = idx_cache;
  d.W = reinterpret_cast<const f16*>(idx_w);
  d.block_table = block_table;
  d.seq_lens = seq_lens;
  d.score = score;
  d.hist = reinterpret_cast<uint32_t*>(hist);
  d.n_kv_rows = idx_rows;
  d.max_blocks = max_blocks;
  d.page_shift = ilog2_pow2(idx_page_size);
  d.max_kv = max_kv;
  d.hist8 = aligned_to(hist, 8) ? 1 : 0;
  d.span = idx_span_launch(idx_fp8, B, max_kv);
  a.nk.ik = reinterpret_cast<const u32x4*>(idx_k);
  a.nk.slot = idx_slot;
  a.nk.T = T;
  a.nk.dst = idx_cache;
  a.n_pro = (int)n_pro;
  a.n_tiles = (max_kv + kIdxPPB - 1) / kIdxPPB;
  const int64_t total = n_pro + (int64_t)a.n_tiles * B;
  DSA_CHECK(total < ((int64_t)1 << 31), "decode_layer_indexer: grid too large");
  hipStream_t st = as_stream(stream);
  if (idx_fp8)
    decode_layer_indexer_kernel<true><<<dim3((unsigned)total), 256, 0, st>>>(a);
  else
    decode_layer_indexer_kernel<false><<<dim3((unsigned)total), 256, 0, st>>>(a);
  DSA_LAUNCH_CHECK("decode_layer_indexer");
  return MI355_DSA_OK;
}
