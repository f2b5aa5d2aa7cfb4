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

#include "capi_internal.h"
#include "dsa_common.h"

namespace mi355dsa {

// fp16 copy, 16-byte chunks.  blockDim = (cx, ty): cx lanes stride over the
// row's chunks, ty tokens per block.
__global__ void __launch_bounds__(256) k_store_f16_vec_kernel(
    const u32x4* __restrict__ k, const int32_t* __restrict__ slot,
    u32x4* __restrict__ kv, int64_t n_tok, int chunks, int64_t n_rows) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.y + threadIdx.y;
  if (t >= n_tok) return;
  // the lane's first chunk is loaded with the slot, before the slot is
  // checked: one memory round trip instead of two
  const int64_t row = slot[t];
  const u32x4* src = k + t * chunks;
  const int c0 = threadIdx.x;
  const u32x4 v0 = src[c0 < chunks ? c0 : 0];
  asm volatile("" ::"v"(v0));  // keeps the load ahead of the check (not sunk past it)
  if (row < 0 || row >= n_rows) return;
  u32x4* dst = kv + row * chunks;
  if (c0 < chunks) dst[c0] = v0;
  for (int c = c0 + blockDim.x; c < chunks; c += blockDim.x) dst[c] = src[c];
}

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

// fp8 132-byte rows: scale = max(amax/448, FLT_MIN); byte = e4m3(v/scale).
// 16 tokens per 256-thread block; lanes (16j .. 16j+15) own token j.
__global__ void __launch_bounds__(256) k_store_fp8_kernel(
    const u32x4* __restrict__ k, const int32_t* __restrict__ slot,
    uint8_t* __restrict__ kv, int64_t n_tok, int64_t n_rows) {
  const int sub = threadIdx.x & 15;
  const int64_t t = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  int64_t row = -1;
  u32x4 raw = {0u, 0u, 0u, 0u};
  if (t < n_tok) {
    row = slot[t];
    raw = k[t * 16 + sub];
  }
  // Whole-vector bit_cast: hipcc (ROCm 7.2) lowers a bit_cast of a single
  // vector element inside an unrolled loop to a load of element 0 only.
  const f16x8 h8 = __builtin_bit_cast(f16x8, raw);
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; i++) v[i] = (float)h8[i];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[i]));
  amax = max16(amax);  // the 16 lanes of this token
  if (t >= n_tok || row < 0 || row >= n_rows) return;
  const float scale = fmaxf(amax / 448.0f, FLT_MIN);
  const u32x2 q = e4m3_quant8(v, amax, scale);
  uint8_t* rp = kv + row * (int64_t)kIdxkFp8RowBytes;
  uint32_t* dw = reinterpret_cast<uint32_t*>(rp + 8 * sub);  // 4-B aligned
  dw[0] = q[0];
  dw[1] = q[1];
  if (sub == 0) *reinterpret_cast<float*>(rp + 128) = scale;
}

// MLA latent rows.  One wave per token: lane l holds latent dims 8l .. 8l+7
// (16-lane group = one 128-dim fp8 tile), lanes 0..7 also carry RoPE dims
// 8l .. 8l+7.  T16: uint16_t bit pattern of fp16 (BF16 = false) or bf16.
// fp8_ds_mla row (656 B): [0,512) e4m3, [512,528) 4 fp32 tile scales,
// [528,656) RoPE as the input's 16-bit values.  fp16 ("auto") row: 576 halves.
template <bool FP8, bool BF16, typename SlotT>
__global__ void __launch_bounds__(256) concat_cache_mla_kernel(
    const uint8_t* __restrict__ kv_c, int64_t kv_c_stride, const uint8_t* __restrict__ k_pe,
    int64_t k_pe_stride, const SlotT* __restrict__ slot, uint8_t* __restrict__ kv,
    int64_t n_tok, int64_t n_rows) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= n_tok) return;  // wave-uniform
  // the token's data is loaded with its slot, before the slot is checked:
  // one memory round trip instead of two (lanes 8.. re-read a RoPE piece
  // they do not store)
  const int64_t row = (int64_t)slot[t];
  const u32x4 raw = *reinterpret_cast<const u32x4*>(kv_c + t * kv_c_stride + 16 * lane);
  const u32x4 rope = *reinterpret_cast<const u32x4*>(k_pe + t * k_pe_stride + 16 * (lane & 7));
  asm volatile("" ::"v"(raw), "v"(rope));  // keeps the loads ahead of the check
  if (row < 0 || row >= n_rows) return;  // wave-uniform
  if constexpr (!FP8) {
    uint8_t* rp = kv + row * (int64_t)(kLatentDim * 2);
    *reinterpret_cast<u32x4*>(rp + 16 * lane) = raw;
    if (lane < 8) *reinterpret_cast<u32x4*>(rp + 2 * kValueDim + 16 * lane) = rope;
    return;
  } else {
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t w = raw[i];
      if constexpr (BF16) {
        v[2 * i] = __uint_as_float(w << 16);
        v[2 * i + 1] = __uint_as_float(w & 0xffff0000u);
      } else {
        const f16x2 h = __builtin_bit_cast(f16x2, w);
        v[2 * i] = (float)h[0];
        v[2 * i + 1] = (float)h[1];
      }
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[i]));
    amax = max16(amax);  // the 16 lanes of this 128-dim tile
    const float scale = fmaxf(amax / 448.0f, FLT_MIN);
    const u32x2 q = e4m3_quant8(v, amax, scale);
    uint8_t* rp = kv + row * (int64_t)kDsmlaRowBytes;
    *reinterpret_cast<u32x2*>(rp + 8 * lane) = q;
    if ((lane & 15) == 0) *reinterpret_cast<float*>(rp + kValueDim + 4 * (lane >> 4)) = scale;
    if (lane < 8) *reinterpret_cast<u32x4*>(rp + kValueDim + 16 + 16 * lane) = rope;
  }
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
