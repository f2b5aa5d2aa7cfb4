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

__global__ void __launch_bounds__(256) decode_prologue_kernel(PrologueArgs a) {
  int id = blockIdx.x;
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

}  // namespace
}  // namespace mi355dsa

using namespace mi355dsa;

extern "C" int mi355_dsa_decode_layer_prologue(
    void* q_lat, int64_t ql_tok_stride, int64_t ql_head_stride, const void* q,
    int64_t q_tok_stride, int64_t q_head_stride, const void* wt_uk, int T, int H, int N, int K,
    int tail, void* kv_cache, int kv_fp8, int64_t kv_rows, const void* kv_c,
    int64_t kv_c_stride, const void* k_pe, int64_t k_pe_stride, int in_bf16,
    const void* slot_mapping, int slot_i64, void* idx_cache, int idx_fp8, int64_t idx_rows,
    const void* idx_k, const int32_t* idx_slot, int32_t* hist, int64_t hist_words,
    void* stream) {
  clear_error();
  DSA_CHECK(T >= 1 && H > 0 && N > 0 && K > 0 && tail >= 0, "decode_layer_prologue: bad sizes");
  DSA_CHECK(q_lat && q && wt_uk && kv_cache && kv_c && k_pe && slot_mapping && idx_cache &&
                idx_k && idx_slot && hist,
            "decode_layer_prologue: null pointer argument");
  // q_latent: the checks of mi355_dsa_head_proj (decode-shaped kernel)
  const int KW = K >= 512 ? 4 : (K >= 256 ? 2 : 1);
  const int NW = 4 / KW;
  DSA_CHECK(K % (32 * KW) == 0 && K / KW <= 32 * kHpMaxKb,
            "decode_layer_prologue: K = %d must be a multiple of %d and at most %d", K, 32 * KW,
            32 * kHpMaxKb * 4);
  DSA_CHECK(N % (16 * NW) == 0, "decode_layer_prologue: N = %d must be a multiple of %d", N,
            16 * NW);
  DSA_CHECK(tail % 8 == 0, "decode_layer_prologue: tail must be a multiple of 8");
  DSA_CHECK(aligned_to(q, 16) && aligned_to(wt_uk, 16) && q_tok_stride % 8 == 0 &&
                q_head_stride % 8 == 0,
            "decode_layer_prologue: q and wt must be 16-byte aligned with strides multiple of 8");
  DSA_CHECK(q_head_stride >= K + tail && q_tok_stride >= (int64_t)H * q_head_stride,
            "decode_layer_prologue: q strides too small for K + tail per head");
  DSA_CHECK(ql_head_stride >= N + tail && ql_tok_stride >= (int64_t)H * ql_head_stride,
            "decode_layer_prologue: q_lat strides too small for N + tail per head");
  DSA_CHECK(tail == 0 || (aligned_to(q_lat, 16) && ql_tok_stride % 8 == 0 &&
                          ql_head_stride % 8 == 0 && N % 8 == 0),
            "decode_layer_prologue: q_lat must be 16-byte aligned with strides multiple of 8");
  // latent write: the checks of mi355_dsa_concat_and_cache_mla
  DSA_CHECK(kv_rows >= 0, "decode_layer_prologue: kv_rows must be >= 0");
  DSA_CHECK(aligned_to(kv_cache, 16) && aligned_to(kv_c, 16) && aligned_to(k_pe, 16),
            "decode_layer_prologue: kv_cache, kv_c and k_pe must be 16-byte aligned");
  DSA_CHECK(kv_c_stride >= kValueDim && k_pe_stride >= kLatentDim - kValueDim &&
                kv_c_stride % 8 == 0 && k_pe_stride % 8 == 0,
            "decode_layer_prologue: kv_c / k_pe row strides must be >= their widths and "
            "multiples of 8 elements");
  DSA_CHECK(!in_bf16 || kv_fp8, "decode_layer_prologue: the fp16 latent cache takes fp16 inputs");
  // indexer-K write (head_dim 128): the checks of mi355_dsa_indexer_k_store
  DSA_CHECK(idx_rows >= 0, "decode_layer_prologue: idx_rows must be >= 0");
  DSA_CHECK(aligned_to(idx_k, 16), "decode_layer_prologue: idx_k must be 16-byte aligned");
  DSA_CHECK(idx_fp8 ? aligned_to(idx_cache, 4) : aligned_to(idx_cache, 16),
            "decode_layer_prologue: idx_cache is misaligned");
  // histogram
  DSA_CHECK(hist_words >= 0 && hist_words % 4 == 0 && aligned_to(hist, 16),
            "decode_layer_prologue: hist must be 16-byte aligned, a multiple of 4 words");

  PrologueArgs a{};
  HpArgs& hp = a.hp;
  hp.x = reinterpret_cast<const f16*>(q);
  hp.x_st = q_tok_stride;
  hp.x_sh = q_head_stride;
  hp.wt = reinterpret_cast<const f16*>(wt_uk);
  hp.out = reinterpret_cast<f16*>(q_lat);
  hp.o_st = ql_tok_stride;
  hp.o_sh = ql_head_stride;
  hp.T = T;
  hp.H = H;
  hp.N = N;
  hp.K = K;
  hp.tail = tail;
  hp.out8 = aligned_to(q_lat, 8) && ql_tok_stride % 4 == 0 && ql_head_stride % 4 == 0;
  hp.n_blocks = N / (16 * NW);
  a.hp_kw = KW;
  a.hp_gx = H * hp.n_blocks;
  const int tiles = (T + 15) / 16;
  const int n_chunks = std::max(1, std::min(tiles, 2048 / std::max(a.hp_gx, 1)));
  hp.t_chunk = (tiles + n_chunks - 1) / n_chunks * 16;
  const int64_t hp_wgs = (int64_t)a.hp_gx * ((T + hp.t_chunk - 1) / hp.t_chunk);

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
  const int64_t total = (int64_t)a.lat_wgs + a.ik_wgs + a.hz_wgs + hp_wgs;
  DSA_CHECK(total < ((int64_t)1 << 31), "decode_layer_prologue: grid too large");
  decode_prologue_kernel<<<dim3((unsigned)total), 256, 0, as_stream(stream)>>>(a);
  DSA_LAUNCH_CHECK("decode_layer_prologue");
  return MI355_DSA_OK;
}
