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
// Accumulation is fp32; out is rounded to fp16 once (RNE).
#include <algorithm>

#include "capi_internal.h"
#include "dsa_common.h"

namespace mi355dsa {
namespace {

constexpr int kHpMaxKb = 8;  // 32-wide k blocks per wave (K / KW <= 256)

struct HpArgs {
  const f16* x;
  int64_t x_st, x_sh;  // element strides of a token and of a head
  const f16* wt;       // [H, N, K]
  f16* out;
  int64_t o_st, o_sh;
  int T, H, N, K, tail;
  int n_blocks;  // workgroups per head along n
  int t_chunk;   // tokens per workgroup along grid y (multiple of 16)
};

template <int NW, int KW>
__global__ __launch_bounds__(256) void head_proj_kernel(HpArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 4, c = lane & 15;
  const int h = blockIdx.x / a.n_blocks, nb = blockIdx.x % a.n_blocks;
  const int wn = wave % NW, wk = wave / NW;
  const int n = (nb * NW + wn) * 16 + c;
  const int kp = a.K / KW;
  const int nkb = kp / 32;
  const int k0 = wk * kp + 8 * g;

  f16x8 b[kHpMaxKb];
  const f16* wrow = a.wt + ((int64_t)h * a.N + n) * a.K + k0;
#pragma unroll
  for (int i = 0; i < kHpMaxKb; ++i)
    if (i < nkb) b[i] = *reinterpret_cast<const f16x8*>(wrow + 32 * i);

  __shared__ f32x4 red[KW > 1 ? (KW - 1) * NW * 64 : 1];
  const int t_begin = blockIdx.y * a.t_chunk;
  const int t_end = min(a.T, t_begin + a.t_chunk);
  const f16x8 zero = {};
  for (int t0 = t_begin; t0 < t_end; t0 += 16) {
    const int ta = t0 + c;  // A row of this lane
    const bool live = ta < t_end;
    const f16* xrow = a.x + (int64_t)(live ? ta : t_begin) * a.x_st + (int64_t)h * a.x_sh + k0;
    f16x8 av[kHpMaxKb];
#pragma unroll
    for (int i = 0; i < kHpMaxKb; ++i)
      if (i < nkb) av[i] = live ? *reinterpret_cast<const f16x8*>(xrow + 32 * i) : zero;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kHpMaxKb; ++i)
      if (i < nkb) acc = mfma16x16x32(av[i], b[i], acc);
    if constexpr (KW > 1) {
      if (wk > 0) red[((wk - 1) * NW + wn) * 64 + lane] = acc;
      __syncthreads();
      if (wk == 0) {
#pragma unroll
        for (int j = 0; j < KW - 1; ++j) acc += red[(j * NW + wn) * 64 + lane];
      }
      __syncthreads();
    }
    if (wk == 0) {
      // D: lane holds column n, rows 4g .. 4g+3 of the tile
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = t0 + 4 * g + j;
        if (t < t_end) a.out[(int64_t)t * a.o_st + (int64_t)h * a.o_sh + n] = (f16)acc[j];
      }
    }
  }

  // carried columns (q's RoPE part): the n-block-0 workgroup of each head
  if (a.tail > 0 && nb == 0) {
    const int per_tok = a.tail / 8;
    const int n_items = (t_end - t_begin) * per_tok;
    for (int it = threadIdx.x; it < n_items; it += 256) {
      const int t = t_begin + it / per_tok, v = (it % per_tok) * 8;
      const f16x8 val = *reinterpret_cast<const f16x8*>(
          a.x + (int64_t)t * a.x_st + (int64_t)h * a.x_sh + a.K + v);
      *reinterpret_cast<f16x8*>(a.out + (int64_t)t * a.o_st + (int64_t)h * a.o_sh + a.N + v) = val;
    }
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
  // weight-sized grid along x; split tokens along y until ~2048 workgroups
  const int gx = H * (N / (16 * NW));
  const int tiles = (T + 15) / 16;
  const int n_chunks = std::max(1, std::min(tiles, 2048 / std::max(gx, 1)));
  a.t_chunk = (tiles + n_chunks - 1) / n_chunks * 16;
  const int chunks = (T + a.t_chunk - 1) / a.t_chunk;
  hipStream_t st = as_stream(stream);
  if (KW == 4)
    launch_hp<1, 4>(a, chunks, st);
  else if (KW == 2)
    launch_hp<2, 2>(a, chunks, st);
  else
    launch_hp<4, 1>(a, chunks, st);
  DSA_LAUNCH_CHECK("head_proj");
  return MI355_DSA_OK;
}
