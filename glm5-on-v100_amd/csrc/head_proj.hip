// Per-head projections of an MLA attention layer (gfx950, wave64 MFMA):
//
//   out[t, h, n] = sum_k x[t, h, k] * W[h, k, n]      (n < N, k < K)
//   out[t, h, N + i] = x[t, h, K + i]                  (i < tail)
//
// The layer uses it twice per step (reference/triton_mla.py:388-418 and
// :486-492): q_nope [T, H, P] through W_UK_T [H, P, 512], with the 64 RoPE
// values of q carried into columns 512..575 (tail = 64); and the attention
// output o [T, H, 512] through W_UV [H, 512, V].  The reference runs both as
// torch.bmm over heads plus transposes and a concatenation.
//
// The weight arrives transposed per head, wt[h, n, k] (k contiguous), which
// the layer materialises once when its weights are prepared: an MFMA B
// fragment (column n, eight consecutive k) is then one 16-byte load.  At
// decode sizes (T of a few tokens) the call is weight-bound, so every weight
// byte is read exactly once: each workgroup owns one head and a block of
// columns, holds its weight slice in registers, and streams its tokens past
// it in 16-row MFMA tiles.  Four waves split the block along n (NW) and/or
// k (KW, partial sums reduced through LDS), so both shapes of the layer give
// 512 workgroups per call: W_UK_T (K = 128, N = 512) as NW = 4, and W_UV
// (K = 512, N = 128) as KW = 4.  Large T is split over a second grid axis.
// Prefill calls (T >= 512) take a wide variant that covers a head's whole N
// per workgroup, so each token fragment is loaded once per wave and feeds
// eight MFMAs.  Both compute D^T = W^T X^T, so a lane stores four
// consecutive output columns of one token.  Accumulation is fp32; out is
// rounded to fp16 once (RNE).
#include <algorithm>

#include "capi_internal.h"
#include "dsa_common.h"
#include "head_proj.h"

namespace mi355dsa {
namespace {

template <int NW, int KW>
__global__ __launch_bounds__(256) void head_proj_kernel(HpArgs a) {
  head_proj_block<NW, KW>(a, blockIdx.x, blockIdx.y);
}

// Prefill shapes (many tokens): a workgroup covers all N columns of a head
// for a run of tokens.  Wave (wn, wk) of NW x KW holds NTW column tiles of
// 16 x its K / KW slice of the weight in registers, so every token fragment
// it loads feeds NTW MFMAs (the decode-shaped kernel above feeds one); the
// next 16-token tile is prefetched; with KW > 1 the partial sums meet in
// LDS, each wave reducing and storing NTW / KW of the tiles; the carried
// columns are copied inside the token loop.
constexpr int kHpWideKb = 4;     // 32-wide k blocks per wave (K = 128 KW)
constexpr int kHpWideNt = 8;     // column tiles per wave
constexpr int kHpWideMinT = 512; // tokens from which a call takes the wide kernel
constexpr int kHpWideWgs = 512;  // workgroups per call (two per CU)

template <int NW, int KW, bool TAIL>
__global__ __launch_bounds__(256) void head_proj_wide_kernel(HpArgs a) {
  constexpr int NTW = kHpWideNt, KB = kHpWideKb;
  constexpr int NSH = NTW / KW;  // tiles each wave reduces and stores
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 4, c = lane & 15;
  const int h = blockIdx.x / a.n_blocks, nb = blockIdx.x % a.n_blocks;
  const int wn = wave % NW, wk = wave / NW;
  const int nw0 = (nb * NW + wn) * NTW * 16;  // first column of the wave
  const int k0 = wk * 32 * KB + 8 * g;

  f16x8 b[NTW][KB];
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    const f16* wrow = a.wt + ((int64_t)h * a.N + nw0 + 16 * j + c) * a.K + k0;
#pragma unroll
    for (int i = 0; i < KB; ++i) b[j][i] = *reinterpret_cast<const f16x8*>(wrow + 32 * i);
  }
  // The weight loads complete here, once: vmcnt also counts stores, so a
  // wait for them inside the token loop would drain the output stores.
#pragma unroll
  for (int j = 0; j < NTW; ++j)
#pragma unroll
    for (int i = 0; i < KB; ++i) asm volatile("" ::"v"(b[j][i]));
  __shared__ f32x4 red[KW > 1 ? KW * NW * NTW * 64 : 1];

  // Every load and store of the token loop is unconditional, so the
  // compiler's wait before a tile's MFMAs covers that tile's loads only.
  // Token indices are clamped to the chunk's last token: a lane past the
  // end loads, computes and stores that token's row again (the same bits).
  const int t_begin = blockIdx.y * a.t_chunk;
  const int t_last = min(a.T, t_begin + a.t_chunk) - 1;
  auto load_x = [&](int t0, f16x8 (&xv)[KB]) {
    const int ta = min(t0 + c, t_last);
    const f16* xrow = a.x + (int64_t)ta * a.x_st + (int64_t)h * a.x_sh + k0;
#pragma unroll
    for (int i = 0; i < KB; ++i) xv[i] = *reinterpret_cast<const f16x8*>(xrow + 32 * i);
  };
  // carried columns: 8 of them for one token of the tile per thread (the
  // 16 * tail / 8 pieces of a tile, repeated over the 256 threads).  The
  // repeats are deliberate: the store stays unconditional, so the loop's
  // waits keep counting it.  At the layer's shapes (q_latent: K 128, N 512;
  // v_up: K 512, N 128) n_blocks is 1, the repeated stores of a piece come
  // from one workgroup and meet in one L2 line, and HBM sees each carried
  // byte once; with n_blocks > 1 every column block stores them again.
  const int per_tok = TAIL ? a.tail / 8 : 1;
  const int item = TAIL ? (int)threadIdx.x % (16 * per_tok) : 0;
  const int tail_dt = item / per_tok, tail_v = (item % per_tok) * 8;

  f16x8 cur[KB], nxt[KB];
  load_x(t_begin, cur);
  // the first tile completes before the loop too, so that the loop head
  // needs no wait for it
#pragma unroll
  for (int i = 0; i < KB; ++i) asm volatile("" ::"v"(cur[i]));
  for (int t0 = t_begin; t0 <= t_last; t0 += 16) {
    f16x8 tailv;
    int tt = 0;
    if constexpr (TAIL) {
      tt = min(t0 + tail_dt, t_last);
      tailv = *reinterpret_cast<const f16x8*>(a.x + (int64_t)tt * a.x_st +
                                              (int64_t)h * a.x_sh + a.K + tail_v);
    }
    load_x(t0 + 16, nxt);  // the last step re-reads the chunk's last token
    f32x4 acc[NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      acc[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < KB; ++i) acc[j] = mfma16x16x32(b[j][i], cur[i], acc[j]);
    }
    // D column of this lane: token ta, rows (output columns) 4g .. 4g+3
    const int ta = min(t0 + c, t_last);
    f16* orow = a.out + (int64_t)ta * a.o_st + (int64_t)h * a.o_sh + nw0 + 4 * g;
    if constexpr (KW > 1) {
#pragma unroll
      for (int j = 0; j < NTW; ++j) red[((wk * NW + wn) * NTW + j) * 64 + lane] = acc[j];
      __syncthreads();
#pragma unroll
      for (int jj = 0; jj < NSH; ++jj) {
        const int j = wk * NSH + jj;
        f32x4 v = red[((0 * NW + wn) * NTW + j) * 64 + lane];
#pragma unroll
        for (int q = 1; q < KW; ++q) v += red[((q * NW + wn) * NTW + j) * 64 + lane];
        const f16x4 o = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
        *reinterpret_cast<f16x4*>(orow + 16 * j) = o;
      }
      __syncthreads();
    } else {
#pragma unroll
      for (int j = 0; j < NTW; ++j) {
        const f16x4 o = {(f16)acc[j][0], (f16)acc[j][1], (f16)acc[j][2], (f16)acc[j][3]};
        *reinterpret_cast<f16x4*>(orow + 16 * j) = o;
      }
    }
    if constexpr (TAIL)
      *reinterpret_cast<f16x8*>(a.out + (int64_t)tt * a.o_st + (int64_t)h * a.o_sh + a.N +
                                tail_v) = tailv;
#pragma unroll
    for (int i = 0; i < KB; ++i) cur[i] = nxt[i];
  }
}

template <int NW, int KW>
void launch_hp(const HpArgs& a0, int n_chunks, hipStream_t st) {
  HpArgs a = a0;
  a.n_blocks = a.N / (16 * NW);
  dim3 grid(a.H * a.n_blocks, n_chunks);
  head_proj_kernel<NW, KW><<<grid, 256, 0, st>>>(a);
}

}  // namespace
}  // namespace mi355dsa

using namespace mi355dsa;

extern "C" int mi355_dsa_head_proj(void* out, int64_t out_tok_stride, int64_t out_head_stride,
                                   const void* x, int64_t x_tok_stride, int64_t x_head_stride,
                                   const void* wt, int T, int H, int N, int K, int tail,
                                   void* stream) {
  clear_error();
  DSA_CHECK(T >= 0 && H > 0 && N > 0 && K > 0 && tail >= 0, "head_proj: bad sizes");
  if (T == 0) return MI355_DSA_OK;
  DSA_CHECK(out && x && wt, "head_proj: null pointer argument");
  const int KW = K >= 512 ? 4 : (K >= 256 ? 2 : 1);
  const int NW = 4 / KW;
  DSA_CHECK(K % (32 * KW) == 0 && K / KW <= 32 * kHpMaxKb,
            "head_proj: K = %d must be a multiple of %d and at most %d", K, 32 * KW,
            32 * kHpMaxKb * 4);
  DSA_CHECK(N % (16 * NW) == 0, "head_proj: N = %d must be a multiple of %d", N, 16 * NW);
  DSA_CHECK(tail % 8 == 0, "head_proj: tail must be a multiple of 8");
  DSA_CHECK(aligned_to(x, 16) && aligned_to(wt, 16) && x_tok_stride % 8 == 0 &&
                x_head_stride % 8 == 0,
            "head_proj: x and wt must be 16-byte aligned with strides multiple of 8");
  DSA_CHECK(x_head_stride >= K + tail && x_tok_stride >= (int64_t)H * x_head_stride,
            "head_proj: x strides too small for K + tail per head");
  DSA_CHECK(out_head_stride >= N + tail && out_tok_stride >= (int64_t)H * out_head_stride,
            "head_proj: out strides too small for N + tail per head");
  DSA_CHECK(tail == 0 || (aligned_to(out, 16) && out_tok_stride % 8 == 0 &&
                          out_head_stride % 8 == 0 && N % 8 == 0),
            "head_proj: out must be 16-byte aligned with strides multiple of 8 when tail > 0");
  HpArgs a{};
  a.x = reinterpret_cast<const f16*>(x);
  a.x_st = x_tok_stride;
  a.x_sh = x_head_stride;
  a.wt = reinterpret_cast<const f16*>(wt);
  a.out = reinterpret_cast<f16*>(out);
  a.o_st = out_tok_stride;
  a.o_sh = out_head_stride;
  a.T = T;
  a.H = H;
  a.N = N;
  a.K = K;
  a.tail = tail;
  a.out8 = aligned_to(out, 8) && out_tok_stride % 4 == 0 && out_head_stride % 4 == 0;
  hipStream_t st = as_stream(stream);
  // many tokens: the wide kernel (whole head per workgroup) when the shape
  // fits it; K = 128 KW and N a multiple of its column span
  const int wide_cols = (4 / KW) * kHpWideNt * 16;
  if (T >= kHpWideMinT && K == 32 * kHpWideKb * KW && N % wide_cols == 0 && a.out8 &&
      2 * tail <= 256) {
    a.n_blocks = N / wide_cols;
    const int gxw = H * a.n_blocks;
    const int tiles = (T + 15) / 16;
    const int n_chunks = std::max(1, std::min(tiles, kHpWideWgs / std::max(gxw, 1)));
    a.t_chunk = (tiles + n_chunks - 1) / n_chunks * 16;
    const dim3 grid(gxw, (T + a.t_chunk - 1) / a.t_chunk);
    if (tail > 0) {
      if (KW == 4)
        head_proj_wide_kernel<1, 4, true><<<grid, 256, 0, st>>>(a);
      else if (KW == 2)
        head_proj_wide_kernel<2, 2, true><<<grid, 256, 0, st>>>(a);
      else
        head_proj_wide_kernel<4, 1, true><<<grid, 256, 0, st>>>(a);
    } else {
      if (KW == 4)
        head_proj_wide_kernel<1, 4, false><<<grid, 256, 0, st>>>(a);
      else if (KW == 2)
        head_proj_wide_kernel<2, 2, false><<<grid, 256, 0, st>>>(a);
      else
        head_proj_wide_kernel<4, 1, false><<<grid, 256, 0, st>>>(a);
    }
    DSA_LAUNCH_CHECK("head_proj");
    return MI355_DSA_OK;
  }
  // weight-sized grid along x; split tokens along y until ~2048 workgroups
  const int gx = H * (N / (16 * NW));
  const int tiles = (T + 15) / 16;
  const int n_chunks = std::max(1, std::min(tiles, 2048 / std::max(gx, 1)));
  a.t_chunk = (tiles + n_chunks - 1) / n_chunks * 16;
  const int chunks = (T + a.t_chunk - 1) / a.t_chunk;
  if (KW == 4)
    launch_hp<1, 4>(a, chunks, st);
  else if (KW == 2)
    launch_hp<2, 2>(a, chunks, st);
  else
    launch_hp<4, 1>(a, chunks, st);
  DSA_LAUNCH_CHECK("head_proj");
  return MI355_DSA_OK;
}
