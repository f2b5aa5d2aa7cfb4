// Indexer-K cache scatter (fp16 copy and 132-byte fp8 rows).
// Behaviour follows sm70_indexer_k_store (reference
// csrc/attention/sm70_mla_decode.cu:654-706, host :2910-2939): tokens whose
// slot is negative or beyond the cache are skipped on the device, so the op
// is safe under graph capture with padded slot mappings.
//
// Layout on gfx950: 16 lanes own one 128-dim token row (16 B each, one
// coalesced 256-B read per row); the fp8 path reduces |k| over those 16
// lanes with cross-lane shuffles and writes 8 e4m3 bytes per lane.
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
  const int64_t row = slot[t];
  if (row < 0 || row >= n_rows) return;
  const u32x4* src = k + t * chunks;
  u32x4* dst = kv + row * chunks;
  for (int c = threadIdx.x; c < chunks; c += blockDim.x) dst[c] = src[c];
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
  // reduce over the 16 lanes of this token (xor masks stay inside the group)
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) amax = fmaxf(amax, shfl_xor_f(amax, m));
  if (t >= n_tok || row < 0 || row >= n_rows) return;
  const float scale = fmaxf(amax / 448.0f, FLT_MIN);
  uint32_t q0 = 0, q1 = 0;
  if (amax <= 65504.0f) {
    // Finite row.  v / scale via the reciprocal with one Markstein
    // correction (r = RN(1/scale), y = RN(v r), rho = v - y scale exactly,
    // q = RN(y + rho r), the sign of v restored for v = -0), then the
    // hardware RNE fp32 -> e4m3 conversion.  Both were checked exhaustively
    // on gfx950 against IEEE division and the integer SATFINITE encoder:
    // identical codes for every fp16 amax and every fp16 v with |v| <= amax,
    // both signs (all such quotients lie within +-448).
    const float r = 1.0f / scale;
    float q[8];
    bool nan = false;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float y = v[i] * r;
      q[i] = __builtin_copysignf(__builtin_fmaf(__builtin_fmaf(-y, scale, v[i]), r, y), v[i]);
      nan |= v[i] != v[i];
    }
    q0 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
    q0 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], (int)q0, true);
    q1 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[4], q[5], 0, false);
    q1 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[6], q[7], (int)q1, true);
    if (nan) {  // NaN inputs keep the encoder's code (sign | 0x7f)
#pragma unroll
      for (int i = 0; i < 8; i++) {
        if (v[i] != v[i]) {
          const uint32_t code = f32_to_e4m3_satfinite(v[i] / scale);
          const int sh = 8 * (i & 3);
          if (i < 4) q0 = (q0 & ~(0xffu << sh)) | (code << sh);
          else q1 = (q1 & ~(0xffu << sh)) | (code << sh);
        }
      }
    }
  } else {  // an infinite input: IEEE division and the integer encoder
#pragma unroll
    for (int i = 0; i < 4; i++) {
      q0 |= f32_to_e4m3_satfinite(v[i] / scale) << (8 * i);
      q1 |= f32_to_e4m3_satfinite(v[4 + i] / scale) << (8 * i);
    }
  }
  uint8_t* rp = kv + row * (int64_t)kIdxkFp8RowBytes;
  uint32_t* dw = reinterpret_cast<uint32_t*>(rp + 8 * sub);  // 4-B aligned
  dw[0] = q0;
  dw[1] = q1;
  if (sub == 0) *reinterpret_cast<float*>(rp + 128) = scale;
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
