// Decode-shaped per-head projection workgroup (see head_proj.hip for the
// design): shared by mi355_dsa_head_proj's kernel and the fused decode-layer
// prologue (dsa_layer.hip).
#pragma once

#include <algorithm>

#include "capi_internal.h"
#include "dsa_common.h"

namespace mi355dsa {

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
  int out8;      // out rows take 8-byte stores (aligned base and strides)
};

// Body of one 256-thread workgroup (bx, by) of the decode-shaped grid; also
// run by the fused decode-layer prologue (dsa_layer.hip).
// tid: the thread's index among the workgroup's 256 (a 1024-thread launch
// runs four of these blocks side by side when KW == 1, which has no barrier).
template <int NW, int KW>
__device__ __forceinline__ void head_proj_block(const HpArgs& a, int bx, int by,
                                                int tid = threadIdx.x) {
  const int wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c = lane & 15;
  const int h = bx / a.n_blocks, nb = bx % a.n_blocks;
  const int wn = wave % NW, wk = wave / NW;
  const int n0 = (nb * NW + wn) * 16;  // the wave's 16 output columns
  const int n = n0 + c;                 // weight row this lane loads
  const int kp = a.K / KW;
  const int nkb = kp / 32;
  const int k0 = wk * kp + 8 * g;

  f16x8 b[kHpMaxKb];
  const f16* wrow = a.wt + ((int64_t)h * a.N + n) * a.K + k0;
#pragma unroll
  for (int i = 0; i < kHpMaxKb; ++i)
    if (i < nkb) b[i] = *reinterpret_cast<const f16x8*>(wrow + 32 * i);

  __shared__ f32x4 red[KW > 1 ? (KW - 1) * NW * 64 : 1];
  const int t_begin = by * a.t_chunk;
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
    // D^T = W^T X^T: the weight fragment is the A operand, the tokens' the
    // B operand, so a lane's D column is one token and its four rows are
    // consecutive output columns (one 8-byte store)
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kHpMaxKb; ++i)
      if (i < nkb) acc = mfma16x16x32(b[i], av[i], acc);
    if constexpr (KW > 1) {
      if (wk > 0) red[((wk - 1) * NW + wn) * 64 + lane] = acc;
      __syncthreads();
      if (wk == 0) {
#pragma unroll
        for (int j = 0; j < KW - 1; ++j) acc += red[(j * NW + wn) * 64 + lane];
      }
      __syncthreads();
    }
    if (wk == 0 && live) {
      // lane: token ta, columns n0 + 4g .. +3
      f16* op = a.out + (int64_t)ta * a.o_st + (int64_t)h * a.o_sh + n0 + 4 * g;
      if (a.out8) {
        const f16x4 o = {(f16)acc[0], (f16)acc[1], (f16)acc[2], (f16)acc[3]};
        *reinterpret_cast<f16x4*>(op) = o;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) op[j] = (f16)acc[j];
      }
    }
  }

  // carried columns (q's RoPE part): the n-block-0 workgroup of each head
  if (a.tail > 0 && nb == 0) {
    const int per_tok = a.tail / 8;
    const int n_items = (t_end - t_begin) * per_tok;
    for (int it = tid; it < n_items; it += 256) {
      const int t = t_begin + it / per_tok, v = (it % per_tok) * 8;
      const f16x8 val = *reinterpret_cast<const f16x8*>(
          a.x + (int64_t)t * a.x_st + (int64_t)h * a.x_sh + a.K + v);
      *reinterpret_cast<f16x8*>(a.out + (int64_t)t * a.o_st + (int64_t)h * a.o_sh + a.N + v) = val;
    }
  }
}

// Host side: arguments and grid of the decode-shaped projection, with the
// checks mi355_dsa_head_proj makes for it.  kw: the k split of the waves;
// gx: workgroups per token chunk; wgs: all workgroups.
inline int hp_decode_setup(HpArgs& a, int& kw, int& gx, int64_t& wgs, const char* who,
                           void* out, int64_t o_st, int64_t o_sh, const void* x, int64_t x_st,
                           int64_t x_sh, const void* wt, int T, int H, int N, int K, int tail) {
  DSA_CHECK(T >= 1 && H > 0 && N > 0 && K > 0 && tail >= 0, "%s: bad projection sizes", who);
  DSA_CHECK(out && x && wt, "%s: null pointer argument", who);
  const int KW = K >= 512 ? 4 : (K >= 256 ? 2 : 1);
  const int NW = 4 / KW;
  DSA_CHECK(K % (32 * KW) == 0 && K / KW <= 32 * kHpMaxKb,
            "%s: K = %d must be a multiple of %d and at most %d", who, K, 32 * KW,
            32 * kHpMaxKb * 4);
  DSA_CHECK(N % (16 * NW) == 0, "%s: N = %d must be a multiple of %d", who, N, 16 * NW);
  DSA_CHECK(tail % 8 == 0, "%s: tail must be a multiple of 8", who);
  DSA_CHECK(aligned_to(x, 16) && aligned_to(wt, 16) && x_st % 8 == 0 && x_sh % 8 == 0,
            "%s: q and wt must be 16-byte aligned with strides multiple of 8", who);
  DSA_CHECK(x_sh >= K + tail && x_st >= (int64_t)H * x_sh,
            "%s: q strides too small for K + tail per head", who);
  DSA_CHECK(o_sh >= N + tail && o_st >= (int64_t)H * o_sh,
            "%s: q_lat strides too small for N + tail per head", who);
  DSA_CHECK(tail == 0 || (aligned_to(out, 16) && o_st % 8 == 0 && o_sh % 8 == 0 && N % 8 == 0),
            "%s: q_lat must be 16-byte aligned with strides multiple of 8", who);
  a = HpArgs{};
  a.x = reinterpret_cast<const f16*>(x);
  a.x_st = x_st;
  a.x_sh = x_sh;
  a.wt = reinterpret_cast<const f16*>(wt);
  a.out = reinterpret_cast<f16*>(out);
  a.o_st = o_st;
  a.o_sh = o_sh;
  a.T = T;
  a.H = H;
  a.N = N;
  a.K = K;
  a.tail = tail;
  a.out8 = aligned_to(out, 8) && o_st % 4 == 0 && o_sh % 4 == 0;
  a.n_blocks = N / (16 * NW);
  kw = KW;
  gx = H * a.n_blocks;
  const int tiles = (T + 15) / 16;
  const int n_chunks = std::max(1, std::min(tiles, 2048 / std::max(gx, 1)));
  a.t_chunk = (tiles + n_chunks - 1) / n_chunks * 16;
  wgs = (int64_t)gx * ((T + a.t_chunk - 1) / a.t_chunk);
  return MI355_DSA_OK;
}

}  // namespace mi355dsa
