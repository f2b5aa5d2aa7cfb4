// Cache scatters: the indexer-K cache (fp16 copy and 132-byte fp8 rows) and
// the MLA latent cache (576 fp16 or 656-byte fp8_ds_mla rows).
// Indexer K follows sm70_indexer_k_store (reference
// csrc/attention/sm70_mla_decode.cu:654-706, host :2910-2939); the latent
// writer follows vLLM's concat_and_cache_mla with kv_cache_dtype
// "fp8_ds_mla" (concat_and_cache_ds_mla_kernel; only the amax hunk is in the
// reference, patches/glm5-v100-sm70-glue.patch:30-62): per 128-dim tile
// scale = max(amax/448, FLT_MIN), e4m3 = RNE-satfinite(v/scale), RoPE copied
// as 16-bit values.  Tokens whose slot is negative or beyond the cache are
// skipped on the device, so the ops are safe under graph capture with
// padded slot mappings.
//
// Layout on gfx950: 16 lanes own one 128-dim group (16 B each, one
// coalesced 256-B read per group); the fp8 paths reduce |v| over those 16
// lanes with DPP and write 8 e4m3 bytes per lane.
#include <float.h>

#include "cache_write.h"
#include "capi_internal.h"
#include "dsa_common.h"

namespace mi355dsa {

// fp16 copy, element-wise fallback for unaligned buffers / odd head_dim.
__global__ void __launch_bounds__(256) k_store_f16_scalar_kernel(
    const uint16_t* __restrict__ k, const int32_t* __restrict__ slot,
    uint16_t* __restrict__ kv, int64_t n_tok, int head_dim, int64_t n_rows) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.y + threadIdx.y;
  if (t >= n_tok) return;
  const int64_t row = slot[t];
  if (row < 0 || row >= n_rows) return;
  for (int d = threadIdx.x; d < head_dim; d += blockDim.x)
    kv[row * head_dim + d] = k[t * head_dim + d];
}

__global__ void __launch_bounds__(256) k_store_f16_vec_kernel(
    const u32x4* __restrict__ k, const int32_t* __restrict__ slot,
    u32x4* __restrict__ kv, int64_t n_tok, int chunks, int64_t n_rows) {
  k_store_f16_vec_block(k, slot, kv, n_tok, chunks, n_rows, blockIdx.x,
                        threadIdx.y * blockDim.x + threadIdx.x, blockDim.x, blockDim.y);
}

__global__ void __launch_bounds__(256) k_store_fp8_kernel(
    const u32x4* __restrict__ k, const int32_t* __restrict__ slot,
    uint8_t* __restrict__ kv, int64_t n_tok, int64_t n_rows) {
  k_store_fp8_block(k, slot, kv, n_tok, n_rows, blockIdx.x);
}

template <bool FP8, bool BF16, typename SlotT>
__global__ void __launch_bounds__(256) concat_cache_mla_kernel(
    const uint8_t* __restrict__ kv_c, int64_t kv_c_stride, const uint8_t* __restrict__ k_pe,
    int64_t k_pe_stride, const SlotT* __restrict__ slot, uint8_t* __restrict__ kv,
    int64_t n_tok, int64_t n_rows) {
  concat_cache_mla_block<FP8, BF16, SlotT>(kv_c, kv_c_stride, k_pe, k_pe_stride, slot, kv,
                                           n_tok, n_rows, blockIdx.x);
}

}  // namespace mi355dsa

using namespace mi355dsa;

extern "C" int mi355_dsa_indexer_k_store(void* kv_cache, int kv_fp8,
                                         int64_t n_rows, const void* k,
                                         int64_t n_tok, int head_dim,
                                         const int32_t* slot_mapping,
                                         void* stream) {
  clear_error();
  DSA_CHECK(n_tok >= 0, "n_tok must be >= 0");
  if (n_tok == 0) return MI355_DSA_OK;
  DSA_CHECK(kv_cache && k && slot_mapping, "null pointer argument");
  DSA_CHECK(head_dim > 0, "head_dim must be > 0");
  DSA_CHECK(n_rows >= 0, "n_rows must be >= 0");
  hipStream_t st = as_stream(stream);
  if (kv_fp8) {
    DSA_CHECK(head_dim == 128, "fp8 indexer store requires head_dim == 128");
    DSA_CHECK(aligned_to(k, 16), "k must be 16-byte aligned");
    DSA_CHECK(aligned_to(kv_cache, 4), "kv_cache must be 4-byte aligned");
    const int64_t blocks = (n_tok + 15) / 16;
    k_store_fp8_kernel<<<dim3((unsigned)blocks), 256, 0, st>>>(
        reinterpret_cast<const u32x4*>(k), slot_mapping,
        reinterpret_cast<uint8_t*>(kv_cache), n_tok, n_rows);
    DSA_LAUNCH_CHECK("indexer_k_store(fp8)");
    return MI355_DSA_OK;
  }
  if (head_dim % 8 == 0 && aligned_to(k, 16) && aligned_to(kv_cache, 16)) {
    const int chunks = head_dim / 8;
    const int cx = chunks < 256 ? chunks : 256;
    const int ty = 256 / cx;
    const int64_t blocks = (n_tok + ty - 1) / ty;
    k_store_f16_vec_kernel<<<dim3((unsigned)blocks), dim3(cx, ty), 0, st>>>(
        reinterpret_cast<const u32x4*>(k), slot_mapping,
        reinterpret_cast<u32x4*>(kv_cache), n_tok, chunks, n_rows);
  } else {
    const int cx = head_dim < 256 ? head_dim : 256;
    const int ty = 256 / cx;
    const int64_t blocks = (n_tok + ty - 1) / ty;
    k_store_f16_scalar_kernel<<<dim3((unsigned)blocks), dim3(cx, ty), 0, st>>>(
        reinterpret_cast<const uint16_t*>(k), slot_mapping,
        reinterpret_cast<uint16_t*>(kv_cache), n_tok, head_dim, n_rows);
  }
  DSA_LAUNCH_CHECK("indexer_k_store(fp16)");
  return MI355_DSA_OK;
}

extern "C" int mi355_dsa_concat_and_cache_mla(void* kv_cache, int kv_fp8, int64_t n_rows,
                                              const void* kv_c, int64_t kv_c_stride,
                                              const void* k_pe, int64_t k_pe_stride,
                                              int in_bf16, int64_t n_tok,
                                              const void* slot_mapping, int slot_i64,
                                              void* stream) {
  clear_error();
  DSA_CHECK(n_tok >= 0 && n_rows >= 0, "n_tok and n_rows must be >= 0");
  if (n_tok == 0) return MI355_DSA_OK;
  DSA_CHECK(kv_cache && kv_c && k_pe && slot_mapping, "null pointer argument");
  DSA_CHECK(aligned_to(kv_cache, 16) && aligned_to(kv_c, 16) && aligned_to(k_pe, 16),
            "kv_cache, kv_c and k_pe must be 16-byte aligned");
  DSA_CHECK(kv_c_stride >= kValueDim && k_pe_stride >= kLatentDim - kValueDim &&
                kv_c_stride % 8 == 0 && k_pe_stride % 8 == 0,
            "kv_c / k_pe row strides must be >= their widths and multiples of 8 elements");
  DSA_CHECK(!in_bf16 || kv_fp8, "the fp16 latent cache takes fp16 inputs");
  const int64_t blocks = (n_tok + 3) / 4;
  DSA_CHECK(blocks <= INT32_MAX, "too many tokens");
  hipStream_t st = as_stream(stream);
  const uint8_t* a = reinterpret_cast<const uint8_t*>(kv_c);
  const uint8_t* r = reinterpret_cast<const uint8_t*>(k_pe);
  uint8_t* kv = reinterpret_cast<uint8_t*>(kv_cache);
  const int64_t sa = kv_c_stride * 2, sr = k_pe_stride * 2;
#define CCM_LAUNCH(FP8, BF16)                                                               \
  do {                                                                                      \
    if (slot_i64)                                                                           \
      concat_cache_mla_kernel<FP8, BF16, int64_t><<<dim3((unsigned)blocks), 256, 0, st>>>(  \
          a, sa, r, sr, reinterpret_cast<const int64_t*>(slot_mapping), kv, n_tok, n_rows); \
    else                                                                                    \
      concat_cache_mla_kernel<FP8, BF16, int32_t><<<dim3((unsigned)blocks), 256, 0, st>>>(  \
          a, sa, r, sr, reinterpret_cast<const int32_t*>(slot_mapping), kv, n_tok, n_rows); \
  } while (0)
  if (!kv_fp8)
    CCM_LAUNCH(false, false);
  else if (in_bf16)
    CCM_LAUNCH(true, true);
  else
    CCM_LAUNCH(true, false);
#undef CCM_LAUNCH
  DSA_LAUNCH_CHECK("concat_and_cache_mla");
  return MI355_DSA_OK;
}
