// Cache-scatter workgroup bodies (see k_store.hip for the formats and the
// design): shared by the standalone kernels of k_store.hip and the fused
// decode-layer prologue (dsa_layer.hip).  Every body is one 256-thread
// workgroup whose index is passed in.
#pragma once

#include <float.h>

#include "dsa_common.h"

namespace mi355dsa {

// fp16 copy, 16-byte chunks: workgroup bx of cx x ty threads (thread tid
// = lane tid % cx of token tid / cx); cx lanes stride over the row's chunks,
// ty tokens per workgroup.
__device__ __forceinline__ void k_store_f16_vec_block(
    const u32x4* __restrict__ k, const int32_t* __restrict__ slot,
    u32x4* __restrict__ kv, int64_t n_tok, int chunks, int64_t n_rows, int bx, int tid, int cx,
    int ty) {
  const int64_t t = (int64_t)bx * ty + tid / cx;
  if (t >= n_tok) return;
  // the lane's first chunk is loaded with the slot, before the slot is
  // checked: one memory round trip instead of two
  const int64_t row = slot[t];
  const u32x4* src = k + t * chunks;
  const int c0 = tid % cx;
  const u32x4 v0 = src[c0 < chunks ? c0 : 0];
  asm volatile("" ::"v"(v0));  // keeps the load ahead of the check (not sunk past it)
  if (row < 0 || row >= n_rows) return;
  u32x4* dst = kv + row * chunks;
  if (c0 < chunks) dst[c0] = v0;
  for (int c = c0 + cx; c < chunks; c += cx) dst[c] = src[c];
}

// One fp8 132-byte row: scale = max(amax/448, FLT_MIN); byte = e4m3(v/scale).
// The 16 lanes of one DPP row (sub = 0..15, all active) hold the fp16 key,
// lane sub dims 8 sub .. +8 in raw.  rp null: the lanes take part in the
// row maximum and store nothing.
__device__ __forceinline__ void k_fp8_row_store(const u32x4 raw, uint8_t* rp, int sub) {
  // Whole-vector bit_cast: hipcc (ROCm 7.2) lowers a bit_cast of a single
  // vector element inside an unrolled loop to a load of element 0 only.
  const f16x8 h8 = __builtin_bit_cast(f16x8, raw);
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; i++) v[i] = (float)h8[i];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[i]));
  amax = max16(amax);  // the 16 lanes of this row
  if (rp == nullptr) return;
  const float scale = fmaxf(amax / 448.0f, FLT_MIN);
  const u32x2 q = e4m3_quant8(v, amax, scale);
  uint32_t* dw = reinterpret_cast<uint32_t*>(rp + 8 * sub);  // 4-B aligned
  dw[0] = q[0];
  dw[1] = q[1];
  if (sub == 0) *reinterpret_cast<float*>(rp + 128) = scale;
}

// fp8 132-byte rows, 16 tokens per 256-thread block; lanes (16j .. 16j+15)
// own token j.
__device__ __forceinline__ void k_store_fp8_block(
    const u32x4* __restrict__ k, const int32_t* __restrict__ slot,
    uint8_t* __restrict__ kv, int64_t n_tok, int64_t n_rows, int bx) {
  const int sub = threadIdx.x & 15;
  const int64_t t = (int64_t)bx * 16 + (threadIdx.x >> 4);
  int64_t row = -1;
  u32x4 raw = {0u, 0u, 0u, 0u};
  if (t < n_tok) {
    row = slot[t];
    raw = k[t * 16 + sub];
  }
  const bool store = t < n_tok && row >= 0 && row < n_rows;
  k_fp8_row_store(raw, store ? kv + row * (int64_t)kIdxkFp8RowBytes : nullptr, sub);
}

// MLA latent rows.  One wave per token: lane l holds latent dims 8l .. 8l+7
// (16-lane group = one 128-dim fp8 tile), lanes 0..7 also carry RoPE dims
// 8l .. 8l+7.  T16: uint16_t bit pattern of fp16 (BF16 = false) or bf16.
// fp8_ds_mla row (656 B): [0,512) e4m3, [512,528) 4 fp32 tile scales,
// [528,656) RoPE as the input's 16-bit values.  fp16 ("auto") row: 576 halves.
template <bool FP8, bool BF16, typename SlotT>
__device__ __forceinline__ void concat_cache_mla_block(
    const uint8_t* __restrict__ kv_c, int64_t kv_c_stride, const uint8_t* __restrict__ k_pe,
    int64_t k_pe_stride, const SlotT* __restrict__ slot, uint8_t* __restrict__ kv,
    int64_t n_tok, int64_t n_rows, int bx) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)bx * 4 + (threadIdx.x >> 6);
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
