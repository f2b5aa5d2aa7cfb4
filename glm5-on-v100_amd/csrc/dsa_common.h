// Device-side building blocks shared by the DSA sparse-attention kernels
// (gfx950 / CDNA4, wave64).
//
// Storage formats (byte layouts fixed by the op contract):
//   * fp8_ds_mla latent row, 656 B: [0,512) e4m3 NoPE latents (4 tiles of
//     128), [512,528) 4 fp32 tile scales, [528,656) 64 fp16 RoPE values.
//     Dequant of dim d < 512 is e4m3(byte[d]) * scale[d / 128].
//     (reference: csrc/attention/sm70_mla_decode.cu:74-100)
//   * fp8 indexer-K row, 132 B: [0,128) e4m3, [128,132) fp32 per-row scale.
//     (reference: csrc/attention/sm70_mla_decode.cu:102-115)
//   * fp16 latent row: 576 halves; fp16 indexer-K row: 128 halves.
//
// MFMA operand layouts used throughout (v_mfma_f32_16x16x32_f16 and
// v_mfma_f32_16x16x16_f16, one 64-lane wave, g = lane / 16, c = lane % 16):
//   A (16 x K): lane holds row c, k-slots g*KPL .. g*KPL+KPL-1
//   B (K x 16): lane holds column c, the same k-slots
//   D (16 x 16, fp32): lane holds column c, rows 4g .. 4g+3
// (KPL = 8 for the x32 form, 4 for the x16 form.)  Only D's placement is
// observable: any permutation of the contraction index that A and B share
// gives the same product, which the kernels use to pick load-friendly
// k-slot -> dimension mappings.  mi355_dsa_selfcheck() verifies D's placement
// on the device.
#pragma once

#include <float.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mi355dsa {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// 16-byte vector that only promises 4-byte alignment (132-B indexer rows).
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

constexpr int kDsmlaRowBytes = 656;  // fp8_ds_mla latent row
constexpr int kIdxkFp8RowBytes = 132;  // fp8 indexer-K row
constexpr int kLatentDim = 576;        // qk dim (512 NoPE + 64 RoPE)
constexpr int kValueDim = 512;         // v dim
constexpr int kIdxHeadDim = 128;       // indexer head dim
constexpr int kIdxHeads = 32;          // indexer heads
constexpr int kTopkBins = 4096;        // 12-bit level histogram

__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x16(f16x4 a, f16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// Monotone unsigned key of an fp32 value: larger float -> larger key, with
// -0 < +0 and -inf the smallest non-NaN key (0x007FFFFF).
// (reference: sm70_mla_decode.cu:43-46)
__device__ __forceinline__ uint32_t mono_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// ---------------------------------------------------------------------------
// OCP e4m3 (e4m3fn: bias 7, no inf, max 448) codec, exact, integer based.
// ---------------------------------------------------------------------------

// 4 e4m3 bytes -> 4 exact fp16 values (every e4m3 value, denormals included,
// is an fp16 value), with the gfx950 conversion at scale 1: two values per
// instruction
__device__ __forceinline__ f16x4 e4m3x4_to_f16x4(uint32_t w) {
  const f16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w, 1.0f, false);
  const f16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w, 1.0f, true);
  const u32x2 pk = {__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
  return __builtin_bit_cast(f16x4, pk);
}

// e4m3 byte -> fp16 bit pattern of value/256.  Exact for every finite byte,
// including denormals (they land on fp16 denormals): the 4-bit exponent
// field moves into the low bits of fp16's 5-bit field, i.e. the bias grows
// by 8.  Two bytes at a time: x01 holds byte0 in bits [0,8) and byte1 in
// bits [16,24).
__device__ __forceinline__ uint32_t e4m3x2_to_f16x2_div256(uint32_t x01) {
  return ((x01 & 0x00800080u) << 8) | ((x01 & 0x007f007fu) << 7);
}

// Spread bytes (b0,b1) / (b2,b3) of a dword into the two 16-bit lanes.
__device__ __forceinline__ uint32_t spread_lo(uint32_t w) {
  return (w & 0xffu) | ((w << 8) & 0xff0000u);
}
__device__ __forceinline__ uint32_t spread_hi(uint32_t w) {
  return ((w >> 16) & 0xffu) | ((w >> 8) & 0xff0000u);
}

// 4 e4m3 bytes (one dword) -> 4 exact fp32 values divided by 256.
__device__ __forceinline__ void e4m3x4_to_f32_div256(uint32_t w, float out[4]) {
  const uint32_t lo = e4m3x2_to_f16x2_div256(spread_lo(w));
  const uint32_t hi = e4m3x2_to_f16x2_div256(spread_hi(w));
  const f16x2 a = __builtin_bit_cast(f16x2, lo);
  const f16x2 b = __builtin_bit_cast(f16x2, hi);
  out[0] = (float)a[0];
  out[1] = (float)a[1];
  out[2] = (float)b[0];
  out[3] = (float)b[1];
}

// fp32 -> e4m3 byte, round-to-nearest-even with saturation to +-448
// (SATFINITE).  NaN maps to 0x7F (sign kept).
__device__ __forceinline__ uint32_t f32_to_e4m3_satfinite(float x) {
  const uint32_t bits = __float_as_uint(x);
  const uint32_t sign = (bits >> 24) & 0x80u;
  const uint32_t mag = bits & 0x7fffffffu;
  if (mag > 0x7f800000u) return sign | 0x7fu;  // NaN
  const float a = __uint_as_float(mag);
  uint32_t code;
  if (a >= 448.0f) {
    code = 0x7eu;
  } else if (a < 0.015625f) {  // below the smallest normal 2^-6
    // denormal grid step is 2^-9; a*512 is exact; rintf rounds half-even.
    code = (uint32_t)__builtin_rintf(a * 512.0f);  // 0..8 (8 == 2^-6 normal)
  } else {
    // keep 3 mantissa bits with RNE; a carry walks into the exponent.
    const uint32_t r = mag + 0x7ffffu + ((mag >> 20) & 1u);
    code = (r >> 20) - (120u << 3);
    if (code > 0x7eu) code = 0x7eu;
  }
  return sign | code;
}

// 8 values -> 8 e4m3 bytes of v / scale, RNE with SATFINITE, given
// scale = max(amax / 448, FLT_MIN) of a group whose |values| <= amax.
// For 2^-80 <= amax <= FLT_MAX (every finite fp16 amax but 0; bf16 amax
// away from the bottom of the fp32 range, where the reciprocal and the
// correction would leave normal numbers): v / scale via the reciprocal with
// one Markstein correction
// (r = RN(1/scale), y = RN(v r), rho = v - y scale exactly, q = RN(y + rho r),
// the sign of v restored for v = -0), then the hardware RNE conversion
// v_cvt_pk_fp8_f32.  Both steps were checked exhaustively on gfx950 against
// IEEE division and f32_to_e4m3_satfinite: identical codes for every fp16
// and every bf16 amax and every v of the same type with |v| <= amax, both
// signs (all such quotients lie within +-448).  NaN inputs keep the
// encoder's code (sign | 0x7f); any other amax (0, tiny, infinite) takes
// IEEE division and the integer encoder.
__device__ __forceinline__ u32x2 e4m3_quant8(const float v[8], float amax, float scale) {
  uint32_t q0 = 0, q1 = 0;
  if (amax <= FLT_MAX && amax >= 0x1p-80f) {
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
    if (nan) {
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
  } else {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      q0 |= f32_to_e4m3_satfinite(v[i] / scale) << (8 * i);
      q1 |= f32_to_e4m3_satfinite(v[4 + i] / scale) << (8 * i);
    }
  }
  return (u32x2){q0, q1};
}

// DPP lane exchange inside rows of 16 lanes (CTRL: a quad_perm, row_mirror
// or row_half_mirror code); the result depends only on the row's values.
template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
// max over aligned groups of 16 lanes, bitwise equal in all 16
__device__ __forceinline__ float max16(float v) {
  v = fmaxf(v, dppf<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dppf<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dppf<0x141>(v));  // row_half_mirror: quad 0 <-> quad 1
  return fmaxf(v, dppf<0x140>(v));  // row_mirror: half-row 0 <-> half-row 1
}

// ---------------------------------------------------------------------------
// Wave-level helpers.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float shfl_xor_f(float v, int m) {
  return __shfl_xor(v, m, 64);
}
// v + v of lane ^ 16, and v + v of lane ^ 32, as VALU lane swaps (gfx950
// v_permlane16/32_swap) instead of LDS permutes.  Each swap hands lane l the
// partner value in one of its two results and keeps its own in the other, so
// the sum of the two results is the pair sum (bitwise: addition commutes).
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// max(d, 0) of an MFMA result in one instruction: such a value is never a
// signalling NaN, so the quieting max the compiler puts before fmaxf is not
// needed (a NaN gives 0, as d > 0 ? d : 0 does).
__device__ __forceinline__ float relu_mfma(float d) {
  float r;
  asm("v_max_f32 %0, 0, %1" : "=v"(r) : "v"(d));
  return r;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor_f(v, m));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += shfl_xor_f(v, m);
  return v;
}

__host__ __device__ __forceinline__ int ilog2_pow2(int v) {
  int s = 0;
  while ((1 << s) < v) s++;
  return s;
}

// Inclusive prefix sum over the 64 lanes of a wave (all lanes active):
// row_shr DPP steps within each 16-lane row, then the row totals read with
// v_readlane.  No LDS traffic.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, true);  // row_shr:1
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, true);  // row_shr:2
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, true);  // row_shr:4
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, true);  // row_shr:8
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)x, 15);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)x, 31);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)x, 47);
  const int row = (int)(threadIdx.x & 63) >> 4;
  return x + (row >= 1 ? r0 : 0u) + (row >= 2 ? r1 : 0u) + (row >= 3 ? r2 : 0u);
}

// Block-wide exclusive prefix sum over NT threads; *total gets the full sum.
// wsum needs NT/64 + 1 words.
template <int NT>
__device__ uint32_t block_excl_scan_n(uint32_t v, uint32_t* wsum, uint32_t* total) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t x = wave_incl_scan(v);
  if (lane == 63) wsum[wave] = x;
  __syncthreads();
  if (wave == 0) {  // exclusive scan of the NW wave sums, in wave 0's lanes
    const uint32_t t = lane < NW ? wsum[lane] : 0u;
    const uint32_t y = wave_incl_scan(t);
    if (lane < NW) wsum[lane] = y - t;
    if (lane == NW - 1) wsum[NW] = y;
  }
  __syncthreads();
  const uint32_t res = wsum[wave] + x - v;
  *total = wsum[NW];
  __syncthreads();
  return res;
}

// Block-wide exclusive prefix sum with one barrier: every wave reads all the
// wave totals and scans them itself.  wsum holds 2 * NT/64 words, one half
// per parity; consecutive calls must alternate the parity, so that a call's
// writes never meet the previous call's reads (two calls of one parity are
// separated by the barrier of the call between them).  *total gets the sum.
template <int NT>
__device__ uint32_t block_excl_scan1(uint32_t v, uint32_t* wsum, int parity, uint32_t* total) {
  constexpr int NW = NT / 64;
  static_assert(NW >= 1 && NW <= 64, "one wave scans the wave totals");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t* ws = wsum + parity * NW;
  const uint32_t x = wave_incl_scan(v);
  if (lane == 63) ws[wave] = x;
  __syncthreads();
  const uint32_t t = lane < NW ? ws[lane] : 0u;
  const uint32_t y = wave_incl_scan(t);  // inclusive over the wave totals
  const uint32_t before =
      wave == 0 ? 0u : (uint32_t)__builtin_amdgcn_readlane((int)y, wave - 1);
  *total = (uint32_t)__builtin_amdgcn_readlane((int)y, NW - 1);
  return before + x - v;
}

// Reductions over the 64 lanes of a wave (all lanes active), the same value
// in every lane: DPP steps within each 16-lane row, then the four row results
// read with v_readlane (no LDS traffic, unlike a shuffle).
template <typename Op>
__device__ __forceinline__ int wave_reduce_i32(int x, Op op) {
  x = op(x, __builtin_amdgcn_mov_dpp(x, 0xB1, 0xf, 0xf, false));   // quad_perm [1,0,3,2]
  x = op(x, __builtin_amdgcn_mov_dpp(x, 0x4E, 0xf, 0xf, false));   // quad_perm [2,3,0,1]
  x = op(x, __builtin_amdgcn_mov_dpp(x, 0x141, 0xf, 0xf, false));  // row_half_mirror
  x = op(x, __builtin_amdgcn_mov_dpp(x, 0x140, 0xf, 0xf, false));  // row_mirror
  return op(op(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16)),
            op(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48)));
}
__device__ __forceinline__ int wave_min_i32(int x) {
  return wave_reduce_i32(x, [](int a, int b) { return a < b ? a : b; });
}
__device__ __forceinline__ int wave_max_i32(int x) {
  return wave_reduce_i32(x, [](int a, int b) { return a > b ? a : b; });
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
  return (uint32_t)wave_reduce_i32((int)x, [](int a, int b) {
    return (uint32_t)a < (uint32_t)b ? a : b;
  });
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  return (uint32_t)wave_reduce_i32((int)x, [](int a, int b) {
    return (uint32_t)a > (uint32_t)b ? a : b;
  });
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t x) {
  return (uint32_t)wave_reduce_i32((int)x, [](int a, int b) {
    return (int)((uint32_t)a + (uint32_t)b);
  });
}

// Workgroup barrier that waits only for this wave's LDS operations (not for
// vector-memory loads in flight, which __syncthreads would drain).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// global_load_lds_dwordx4: lane l's 16 bytes at gptr land at lds + 16 l (the
// LDS base goes through M0, so it must be wave-uniform).  Issued as inline
// asm so the compiler does not treat every later LDS read as depending on
// the gathers in flight (it would otherwise wait for all of them): callers
// wait for completion themselves with s_waitcnt vmcnt before a barrier.
__device__ __forceinline__ void dma16(const void* gptr, const void* lds) {
  const uint32_t off = (uint32_t)(uintptr_t)lds;
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(gptr), "{m0}"(off) : "memory");
}
// global_load_lds_dword: lane l's 4 bytes at gptr land at lds + 4 l.
__device__ __forceinline__ void dma4(const void* gptr, const void* lds) {
  const uint32_t off = (uint32_t)(uintptr_t)lds;
  asm volatile("global_load_lds_dword %0, off" ::"v"(gptr), "{m0}"(off) : "memory");
}
// dma16 of the 16 bytes at gptr + IMM (IMM in the instruction's offset
// field, so that several loads share one address register).  The offset
// field applies to the LDS address too, so M0 carries lds - IMM (the caller
// passes lds >= IMM).
template <int IMM>
__device__ __forceinline__ void dma16_at(const void* gptr, const void* lds) {
  static_assert(IMM >= 0 && IMM < 4096, "offset field");
  const uint32_t off = (uint32_t)(uintptr_t)lds - (uint32_t)IMM;
  asm volatile("global_load_lds_dwordx4 %0, off offset:%2" ::"v"(gptr), "{m0}"(off), "n"(IMM)
               : "memory");
}
// dma4 of the 4 bytes at gptr + IMM, landing at lds + 4 l (M0 = lds - IMM).
template <int IMM>
__device__ __forceinline__ void dma4_at(const void* gptr, const void* lds) {
  static_assert(IMM >= 0 && IMM < 4096, "offset field");
  const uint32_t off = (uint32_t)(uintptr_t)lds - (uint32_t)IMM;
  asm volatile("global_load_lds_dword %0, off offset:%2" ::"v"(gptr), "{m0}"(off), "n"(IMM)
               : "memory");
}

}  // namespace mi355dsa
