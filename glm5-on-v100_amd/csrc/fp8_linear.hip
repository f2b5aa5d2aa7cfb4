// fp8-e4m3 weight-only projections: block dequant and the small-M GEMV.
// Semantics follow sm70_attn_fp8_dequant / sm70_attn_fp8_gemv (reference
// csrc/attention/sm70_attn_fp8.cu:51-215): w is row-major e4m3 [N,K] with
// fp32 block scales s[ceil(N/128), ceil(K/128)], dequant = e4m3(w) * s.
//
// GEMV design for gfx950: the HBM-bound stream of W is fed straight into
// v_mfma_f32_16x16x32_f16.  Each wave owns NB column blocks of 16 weight
// rows; x (M <= 8 rows, zero padded to 16) is the A operand, the dequantised
// weights the B operand.  e4m3 bytes become exact fp16 with the hardware
// conversion (v_cvt_scalef32_pk_f16_fp8 at scale 1, two per instruction), so
// the fp16 products are exact and accumulate in fp32; the block scale is
// applied once per 128-wide k block.  Waves of a workgroup split K and are
// reduced through LDS.  Long-K shapes stream the weights through a per-wave
// LDS ring filled by LDS-DMA (fp8_gemv_dma_kernel), several k blocks in
// flight per wave without holding them in registers.
#include "capi_internal.h"
#include "dsa_common.h"

namespace mi355dsa {

// ---------------------------------------------------------------------------
// dequant: one thread per 16 weights; grid = (N, ceil(K/16/256))
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) fp8_dequant_kernel(
    const uint8_t* __restrict__ w, const float* __restrict__ s,
    f16* __restrict__ out, int K, int KB) {
  const int n = blockIdx.x;
  const int chunk = blockIdx.y * 256 + threadIdx.x;
  const int k0 = chunk * 16;
  if (k0 >= K) return;
  const int64_t off = (int64_t)n * K + k0;
  const float sc = s[(int64_t)(n >> 7) * KB + (k0 >> 7)];
  const u32x4 raw = *reinterpret_cast<const u32x4*>(w + off);
  f16x8 o0, o1;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const f16x4 v = e4m3x4_to_f16x4(raw[i]);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const f16 h = (f16)((float)v[j] * sc);
      if (i < 2)
        o0[4 * i + j] = h;
      else
        o1[4 * (i - 2) + j] = h;
    }
  }
  *reinterpret_cast<f16x8*>(out + off) = o0;
  *reinterpret_cast<f16x8*>(out + off + 8) = o1;
}

// ---------------------------------------------------------------------------
// GEMV.  k-slot mapping inside a 128-wide k block: step s (0..3), lane group
// g, slot e  ->  k = 32g + 8s + e.  A lane therefore reads 32 contiguous
// weight bytes and 64 contiguous x bytes per k block; the 4 lanes of a row
// cover its 128-byte line.
//
// Wave w of a workgroup takes k blocks w, w + WAVES, ... of the workgroup's
// 16 NB weight rows, one block at a time (load, then MFMAs).  Latency is
// hidden by occupancy rather than by a register ring: at ~56-74 VGPRs a SIMD
// holds 6-8 waves, and on this part that streams faster than deeper
// per-wave prefetch at lower occupancy (measured).  Loads of k blocks past
// the end are clamped to the last block (in bounds, scale 0).
// ---------------------------------------------------------------------------
template <int NB>
struct GemvFrag {
  f16x8 a[4];  // x, A operand
  u32x4 b0[NB], b1[NB];
  float sc[NB];  // block scale (0 past the end)
};

template <int NB, int WAVES>
__global__ void __launch_bounds__(WAVES * 64) fp8_gemv_kernel(
    const f16* __restrict__ x, const uint8_t* __restrict__ w,
    const float* __restrict__ s, f16* __restrict__ y, int M, int N, int K,
    int KB) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int n_base = blockIdx.x * (16 * NB);

  f32x4 acc[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) acc[j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  const bool xrow = c < M;
  const f16* xr = x + (int64_t)(xrow ? c : 0) * K;
  // weight rows of this lane (clamped into the matrix; rows >= N get scale 0)
  const uint8_t* wr[NB];
  const float* sr[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) {
    wr[j] = w + (int64_t)min(n_base + 16 * j + c, N - 1) * K + 32 * g;
    sr[j] = s + (int64_t)(min(n_base + 16 * j, N - 1) >> 7) * KB;
  }

  auto load = [&](int kb, GemvFrag<NB>& f) {
    const bool ok = kb < KB;
    kb = min(kb, KB - 1);
    const int kvalid = K - kb * 128;  // multiple of 16
    const int kofs = kb * 128 + 32 * g;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      f.a[q] = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
      if (xrow && (32 * g + 8 * q) < kvalid)
        f.a[q] = *reinterpret_cast<const f16x8*>(xr + kofs + 8 * q);
    }
#pragma unroll
    for (int j = 0; j < NB; j++) {
      f.b0[j] = (u32x4){0u, 0u, 0u, 0u};
      f.b1[j] = (u32x4){0u, 0u, 0u, 0u};
      const uint8_t* p = wr[j] + kb * 128;
      if (32 * g < kvalid) f.b0[j] = *reinterpret_cast<const u32x4*>(p);
      if (32 * g + 16 < kvalid) f.b1[j] = *reinterpret_cast<const u32x4*>(p + 16);
      // every row of a 16-row column block shares one 128x128 scale block
      f.sc[j] = (ok && n_base + 16 * j < N) ? sr[j][kb] : 0.f;
    }
  };

  const int nk = (KB + WAVES - 1) / WAVES;  // uniform trip count
  for (int i = 0; i < nk; i++) {
    GemvFrag<NB> f;
    load(wave + WAVES * i, f);
#pragma unroll
    for (int j = 0; j < NB; j++) {
      f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint32_t d0 = (q < 2) ? f.b0[j][2 * q] : f.b1[j][2 * (q - 2)];
        const uint32_t d1 = (q < 2) ? f.b0[j][2 * q + 1] : f.b1[j][2 * (q - 2) + 1];
        const f16x4 h0 = e4m3x4_to_f16x4(d0), h1 = e4m3x4_to_f16x4(d1);
        const f16x8 h = {h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
        t = mfma16x16x32(f.a[q], h, t);
      }
#pragma unroll
      for (int r = 0; r < 4; r++) acc[j][r] += f.sc[j] * t[r];
    }
  }

  // reduce the WAVES partial sums through LDS
  __shared__ float red[WAVES][NB][4][64];
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int r = 0; r < 4; r++) red[wave][j][r][lane] = acc[j][r];
  __syncthreads();
  // D layout: lane (col c, group g), reg r -> x row m = 4g + r, weight row c.
  for (int e = threadIdx.x; e < NB * 4 * 64; e += WAVES * 64) {
    const int j = e / 256, r = (e / 64) & 3, l = e & 63;
    const int m = 4 * (l >> 4) + r;
    const int n = n_base + 16 * j + (l & 15);
    if (m >= M || n >= N) continue;
    float v = 0.f;
#pragma unroll
    for (int wv = 0; wv < WAVES; wv++) v += red[wv][j][r][l];
    y[(int64_t)m * N + n] = (f16)v;
  }
}

// ---------------------------------------------------------------------------
// GEMV with the weights streamed through a per-wave LDS ring by LDS-DMA
// (K a multiple of 128, M <= 4).  The register kernel above keeps one k block
// per wave in flight, so a wave's k blocks form a chain of dependent memory
// round trips; deeper prefetch in registers cost more occupancy than it hid
// (measured).  Here each wave keeps D k blocks in flight in LDS without
// holding them in VGPRs.  A workgroup owns R (16 or 8) weight rows; per slot
// the R rows x 128 B are stored as [16-byte piece hq][row], so that lane
// (c, g) reads pieces 2g and 2g + 1 of row c with conflict-free 16-byte
// reads (lanes c >= R, and x rows >= M, read a zero line), and the 4 x rows
// of the block take 256 B each, chunk k of row r at chunk k ^ 4r (the rows'
// reads then fall in different banks).  A wave waits with an explicit vmcnt for its
// oldest slot only, reads it, then reuses the slot for the block D steps
// ahead (past its last block it reloads the block it just read, so the count
// in flight stays uniform).  The MFMA arithmetic per k block is the register
// kernel's.
// ---------------------------------------------------------------------------
constexpr int kGdSlotX = 4 * 256;  // 4 x rows x 128 halves

template <int R>
struct GdShape {
  static constexpr int kSlotW = R * 128;          // weight rows x 128 B
  static constexpr int kSlot = kSlotW + kGdSlotX;
  static constexpr int kPer = R / 8 + 1;          // DMA instructions per slot
};

template <int R, int WAVES, int D>
__global__ void __launch_bounds__(WAVES * 64) fp8_gemv_dma_kernel(
    const f16* __restrict__ x, const uint8_t* __restrict__ w, const float* __restrict__ s,
    f16* __restrict__ y, int M, int N, int K, int KB) {
  using G = GdShape<R>;
  extern __shared__ __align__(16) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int n_base = blockIdx.x * R;
  uint8_t* ring = smem + wave * D * G::kSlot;
  uint8_t* zero = smem + WAVES * D * G::kSlot;                       // 64 B of zeros
  float* s_sc = reinterpret_cast<float*>(zero + 64);                 // this row block's KB scales

  // the R rows share one 128-row scale block
  const float* srow = s + (int64_t)(n_base >> 7) * KB;
  for (int i = threadIdx.x; i < KB; i += WAVES * 64) s_sc[i] = srow[i];
  if (threadIdx.x < 16) reinterpret_cast<uint32_t*>(zero)[threadIdx.x] = 0u;
  __syncthreads();

  // DMA sources of this lane.  Weights, instruction j: slot position
  // 64 j + lane = hq R + r, i.e. row r = lane % R (clamped into the matrix),
  // piece hq = (64 j + lane) / R.  x: row min(g, M - 1), 16-byte chunk
  // c ^ 4g of the block's 256 bytes, landing at chunk c of LDS row g.
  const uint8_t* wsrc = w + (int64_t)min(n_base + lane % R, N - 1) * K;
  const uint8_t* xsrc = reinterpret_cast<const uint8_t*>(x) +
                        (int64_t)min(g, M - 1) * K * 2 + 16 * (c ^ (4 * g));
  auto issue = [&](int kb, int slot) {
    uint8_t* sl = ring + slot * G::kSlot;
#pragma unroll
    for (int j = 0; j < R / 8; j++)
      dma16(wsrc + (int64_t)kb * 128 + 16 * ((64 * j + lane) / R), sl + 1024 * j);
    dma16(xsrc + (int64_t)kb * 256, sl + G::kSlotW);
  };

  const int nk = (KB + WAVES - 1) / WAVES;  // uniform trip count
#pragma unroll
  for (int d = 0; d < D; d++) issue(min(wave + WAVES * d, KB - 1), d);

  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const bool wrow = c < R, xrow = c < M;
  for (int i = 0; i < nk; i++) {
    const int slot = i % D;
    const int kb = wave + WAVES * i;
    // the oldest slot's DMAs are done once at most (D - 1) * kPer newer ones
    // remain in flight
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((D - 1) * G::kPer) : "memory");
    const uint8_t* sl = ring + slot * G::kSlot;
    const uint8_t* w0 = wrow ? sl + ((2 * g) * R + c) * 16 : zero;
    const uint8_t* w1 = wrow ? sl + ((2 * g + 1) * R + c) * 16 : zero;
    const u32x4 b0 = *reinterpret_cast<const u32x4*>(w0);
    const u32x4 b1 = *reinterpret_cast<const u32x4*>(w1);
    const uint8_t* xa = xrow ? sl + G::kSlotW + c * 256 + 64 * (g ^ c) : zero;
    const int xs = xrow ? 16 : 0;
    f16x8 a[4];
#pragma unroll
    for (int q = 0; q < 4; q++) a[q] = *reinterpret_cast<const f16x8*>(xa + xs * q);
    const float sc = kb < KB ? s_sc[kb] : 0.f;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slot is read: reuse it
    const int nxt = kb + WAVES * D;
    issue(nxt < KB ? nxt : min(kb, KB - 1), slot);
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint32_t d0 = (q < 2) ? b0[2 * q] : b1[2 * (q - 2)];
      const uint32_t d1 = (q < 2) ? b0[2 * q + 1] : b1[2 * (q - 2) + 1];
      const f16x4 h0 = e4m3x4_to_f16x4(d0), h1 = e4m3x4_to_f16x4(d1);
      const f16x8 h = {h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
      t = mfma16x16x32(a[q], h, t);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) acc[r] += sc * t[r];
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the ring's last reloads
  __syncthreads();

  // reduce the WAVES partial sums through LDS (the ring is free now)
  float* red = reinterpret_cast<float*>(smem);  // [WAVES][4][64]
#pragma unroll
  for (int r = 0; r < 4; r++) red[(wave * 4 + r) * 64 + lane] = acc[r];
  __syncthreads();
  for (int e = threadIdx.x; e < 4 * 64; e += WAVES * 64) {
    const int r = e >> 6, l = e & 63;
    const int m = 4 * (l >> 4) + r;
    const int n = n_base + (l & 15);
    if (m >= M || (l & 15) >= R || n >= N) continue;
    float v = 0.f;
#pragma unroll
    for (int wv = 0; wv < WAVES; wv++) v += red[(wv * 4 + r) * 64 + l];
    y[(int64_t)m * N + n] = (f16)v;
  }
}

// ---------------------------------------------------------------------------
// Load-time quantizer (reference _sm70_attn_fp8_quantize, glue.patch:
// 1515-1532): per 128x128 block scale = max(amax / 448, 1e-12) and
// q = e4m3_rne(clamp(w / scale, +-448)); partial edge blocks take the amax
// of their valid elements (the reference pads with zeros).  One workgroup per
// block, thread t covers 64 columns of row t / 2.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) fp8_quantize_kernel(const f16* __restrict__ w,
                                                           uint8_t* __restrict__ q,
                                                           float* __restrict__ s, int N, int K) {
  const int nb = blockIdx.y, kb = blockIdx.x, KB = gridDim.x;
  const int r = nb * 128 + (threadIdx.x >> 1);
  const int k0 = kb * 128 + 64 * (threadIdx.x & 1);
  const bool vec = (K % 8) == 0 && k0 + 64 <= K;
  float v[64];
  if (r < N && vec) {
    const f16x8* src = reinterpret_cast<const f16x8*>(w + (int64_t)r * K + k0);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const f16x8 h = src[i];
#pragma unroll
      for (int e = 0; e < 8; e++) v[8 * i + e] = (float)h[e];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 64; i++)
      v[i] = (r < N && k0 + i < K) ? (float)w[(int64_t)r * K + k0 + i] : 0.f;
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 64; i++) amax = fmaxf(amax, fabsf(v[i]));
  amax = wave_max(amax);
  __shared__ float wmax[4];
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const float scale = fmaxf(amax / 448.0f, 1e-12f);  // IEEE division, as the reference
  if (threadIdx.x == 0) s[(int64_t)nb * KB + kb] = scale;
  if (r >= N) return;
  uint32_t word[16];
#pragma unroll
  for (int i = 0; i < 16; i++) {
    uint32_t x = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float t = fminf(fmaxf(v[4 * i + e] / scale, -448.0f), 448.0f);
      x |= f32_to_e4m3_satfinite(t) << (8 * e);
    }
    word[i] = x;
  }
  uint8_t* dst = q + (int64_t)r * K + k0;
  if (vec && ((uintptr_t)dst & 15) == 0) {
#pragma unroll
    for (int i = 0; i < 4; i++)
      reinterpret_cast<u32x4*>(dst)[i] = (u32x4){word[4 * i], word[4 * i + 1], word[4 * i + 2], word[4 * i + 3]};
  } else {
    for (int i = 0; i < 64; i++)
      if (k0 + i < K) dst[i] = (uint8_t)(word[i >> 2] >> (8 * (i & 3)));
  }
}

template <int NB, int WAVES>
static void launch_gemv(const f16* x, const uint8_t* w, const float* s, f16* y,
                        int M, int N, int K, int KB, hipStream_t st) {
  const int blocks = (N + 16 * NB - 1) / (16 * NB);
  fp8_gemv_kernel<NB, WAVES><<<blocks, WAVES * 64, 0, st>>>(x, w, s, y, M, N, K, KB);
}

template <int R, int WAVES, int D>
static int launch_gemv_dma(const f16* x, const uint8_t* w, const float* s, f16* y, int M,
                           int N, int K, int KB, hipStream_t st) {
  const size_t lds = (size_t)WAVES * D * GdShape<R>::kSlot + 64 + 4 * (size_t)KB;
  const int rc = reserve_lds(reinterpret_cast<const void*>(fp8_gemv_dma_kernel<R, WAVES, D>), lds,
                             "attn_fp8_gemv");
  if (rc) return rc;
  fp8_gemv_dma_kernel<R, WAVES, D><<<(N + R - 1) / R, WAVES * 64, lds, st>>>(x, w, s, y, M, N,
                                                                              K, KB);
  return MI355_DSA_OK;
}

}  // namespace mi355dsa

using namespace mi355dsa;

extern "C" int mi355_dsa_attn_fp8_gemv(void* y, const void* x, const uint8_t* w,
                                       const float* s, int M, int N, int K,
                                       void* stream) {
  clear_error();
  DSA_CHECK(M >= 1 && M <= 8, "sm70_attn_fp8_gemv: M must be 1..8, got %d", M);
  DSA_CHECK(K > 0 && N > 0 && K % 16 == 0 && N % 8 == 0, "bad N/K alignment");
  DSA_CHECK(y && x && w && s, "null pointer argument");
  DSA_CHECK(aligned_to(x, 16) && aligned_to(w, 16),
            "x and w must be 16-byte aligned");
  const int KB = (K + 127) / 128;
  hipStream_t st = as_stream(stream);
  const f16* xp = reinterpret_cast<const f16*>(x);
  f16* yp = reinterpret_cast<f16*>(y);
  // Large N: 32 rows x 8 waves per workgroup (768 workgroups at N = 24576,
  // three resident per CU).  Smaller N with a long K (at least 64 k blocks,
  // M <= 4): the LDS-ring kernel, 8 rows x 4 waves x 4 blocks in flight per
  // wave (768 workgroups at N = 6144: 44.4 -> 30.7 us at M = 1).  Otherwise
  // 16 rows x 16 waves, so that K is spread over enough waves to keep the
  // matrix streaming (at K = 6144 a wave has only 3 k blocks, and the ring
  // gains nothing).
  if (N >= 16384) {
    launch_gemv<2, 8>(xp, w, s, yp, M, N, K, KB, st);
  } else if (K % 128 == 0 && K >= 8192 && M <= 4) {
    const int rc = launch_gemv_dma<8, 4, 4>(xp, w, s, yp, M, N, K, KB, st);
    if (rc) return rc;
  } else {
    launch_gemv<1, 16>(xp, w, s, yp, M, N, K, KB, st);
  }
  DSA_LAUNCH_CHECK("attn_fp8_gemv");
  return MI355_DSA_OK;
}

extern "C" int mi355_dsa_attn_fp8_dequant(void* out, const uint8_t* w,
                                          const float* s, int N, int K,
                                          void* stream) {
  clear_error();
  DSA_CHECK(K > 0 && N >= 0 && K % 16 == 0, "K must be a multiple of 16");
  if (N == 0) return MI355_DSA_OK;
  DSA_CHECK(out && w && s, "null pointer argument");
  DSA_CHECK(aligned_to(out, 16) && aligned_to(w, 16),
            "out and w must be 16-byte aligned");
  const int KB = (K + 127) / 128;
  const int chunks = K / 16;
  dim3 grid(N, (chunks + 255) / 256);
  fp8_dequant_kernel<<<grid, 256, 0, as_stream(stream)>>>(
      w, s, reinterpret_cast<f16*>(out), K, KB);
  DSA_LAUNCH_CHECK("attn_fp8_dequant");
  return MI355_DSA_OK;
}

extern "C" int mi355_dsa_attn_fp8_quantize(uint8_t* q, float* s, const void* w, int N, int K,
                                           void* stream) {
  clear_error();
  DSA_CHECK(N >= 0 && K >= 0, "N and K must be >= 0");
  if (N == 0 || K == 0) return MI355_DSA_OK;
  DSA_CHECK(q && s && w, "null pointer argument");
  DSA_CHECK(aligned_to(w, 2), "w must be 2-byte aligned");
  const int NB = (N + 127) / 128, KB = (K + 127) / 128;
  DSA_CHECK(NB <= 65535, "N too large");
  const bool vec_ok = aligned_to(w, 16) && K % 8 == 0;
  (void)vec_ok;
  fp8_quantize_kernel<<<dim3(KB, NB), 256, 0, as_stream(stream)>>>(
      reinterpret_cast<const f16*>(w), q, s, N, K);
  DSA_LAUNCH_CHECK("attn_fp8_quantize");
  return MI355_DSA_OK;
}
