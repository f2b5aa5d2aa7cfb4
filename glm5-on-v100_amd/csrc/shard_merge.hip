// Exact top-K merge of key-sharded indexer candidates (gfx950).
//
// Input allf [tp, R, 2K] fp32: for shard s and row r, K candidate scores
// then K candidate positions (int32 bits; -1 with score -inf when the shard
// had fewer than K).  Row r of the output gets the K candidates of largest
//   key(s, c) = (mono(score) << 32) | (tp*K - 1 - (s*K + c)),
// i.e. by score with ties to the lower column (s*K + c) -- the column order
// in which torch.topk over the [R, tp*K] layout breaks ties -- with a
// selection whose score maps to mono <= mono(-inf) written as -1, and the K
// positions sorted ascending.  Destination row: dst_base + r, or dst_rows[r]
// when dst_base < 0 (a destination outside [0, out_rows) is skipped).
// (Reference: sm70_indexer_shard_merge, csrc/attention/sm70_mla_decode.cu:
// 2055-2182, host :2411-2436.)
//
// One 512-thread workgroup per row.  Each thread holds tp*K/512 (<= 16)
// candidates' monotone keys in registers (column tid + 512 i for its i-th).  A 12+12+8
// bit radix select on LDS histograms finds the K-th largest score key T and
// how many candidates equal to T are taken; those are the lowest columns
// among the equal ones, ranked by block scans in column order (only when
// that choice can change the output).  The selected positions are collected
// in LDS and put in ascending order by a bitmap over their span (distinct
// positions spanning fewer than 131072 values: one block scan) or, failing
// that, a bitonic sort.
#include "capi_internal.h"
#include "dsa_common.h"

namespace mi355dsa {
namespace {

constexpr int kSmThreads = 512;
constexpr int kSmWaves = kSmThreads / 64;
constexpr int kSmMaxK = 2048;

struct SmShared {
  uint32_t hist[kTopkBins];  // radix histograms, then the position bitmap
  int32_t sel[kSmMaxK];
  uint32_t wsum[kSmWaves + 1];
  int T;
  uint32_t above;
  uint32_t cnt, eq_cnt, n_neg;
  int pmin, pmax;
};
constexpr int kSmBitmapBits = kTopkBins * 32;  // 131072 positions

// exclusive prefix sum over the block; *total gets the sum
__device__ uint32_t sm_scan(uint32_t v, SmShared& sh, uint32_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) sh.wsum[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t run = 0;
    for (int w = 0; w < kSmWaves; w++) {
      const uint32_t t = sh.wsum[w];
      sh.wsum[w] = run;
      run += t;
    }
    sh.wsum[kSmWaves] = run;
  }
  __syncthreads();
  const uint32_t res = sh.wsum[wave] + x - v;
  *total = sh.wsum[kSmWaves];
  __syncthreads();
  return res;
}

// bin T of an nbins histogram with above(T) < need <= above(T) + hist[T]
// (above = keys in higher bins); need <= total.
__device__ void sm_threshold(SmShared& sh, int nbins, uint32_t need, int* T, uint32_t* above) {
  const int per = nbins / kSmThreads > 0 ? nbins / kSmThreads : 1;
  const int lo = threadIdx.x * per;
  uint32_t cs = 0;
  if (lo < nbins)
    for (int i = 0; i < per; i++) cs += sh.hist[lo + i];
  uint32_t total;
  const uint32_t excl = sm_scan(cs, sh, &total);
  if (threadIdx.x == 0) sh.T = -1;
  __syncthreads();
  if (lo < nbins) {
    uint32_t a = total - excl - cs;
    for (int bin = lo + per - 1; bin >= lo; bin--) {
      const uint32_t h = sh.hist[bin];
      if (a < need && a + h >= need) {
        sh.T = bin;
        sh.above = a;
      }
      a += h;
    }
  }
  __syncthreads();
  *T = sh.T;
  *above = sh.above;
  __syncthreads();
}

__device__ __forceinline__ uint32_t mono_of(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

constexpr int kSmMaxPer = 16;  // candidates per thread (tp*K <= 8192)

__global__ void __launch_bounds__(kSmThreads) shard_merge_kernel(
    const float* __restrict__ allf, const int32_t* __restrict__ dst_rows,
    int32_t* __restrict__ out, int64_t out_stride, int64_t out_rows, int R, int K,
    int nper, int dst_base) {
  __shared__ SmShared sh;
  const int r = blockIdx.x;
  const int tid = threadIdx.x;

  // ---- candidates: column col = tid + 512 i = s K + c ----
  // The loops over i skip (continue) rather than stop at nper, so they
  // unroll with fixed registers; the loads are unconditional (steps past
  // nper re-read column tid, whose value is never used), so all of a
  // thread's loads are in flight together.  A break made a runtime loop:
  // one load, then one wait, per step.
  uint32_t key[kSmMaxPer];
#pragma unroll
  for (int i = 0; i < kSmMaxPer; i++) {
    const int col = tid + (i < nper ? i : 0) * kSmThreads;
    const int s = col / K, c = col - s * K;
    key[i] = mono_of(allf[((int64_t)s * R + r) * (2 * K) + c]);
  }

  // ---- radix select of the K-th largest score key ----
  for (int i = tid; i < kTopkBins; i += kSmThreads) sh.hist[i] = 0u;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kSmMaxPer; i++) {
    if (i >= nper) continue;
    atomicAdd(&sh.hist[key[i] >> 20], 1u);
  }
  __syncthreads();
  int T;
  uint32_t above;
  sm_threshold(sh, kTopkBins, (uint32_t)K, &T, &above);
  uint32_t need = (uint32_t)K - above;
  uint32_t prefix = (uint32_t)T;
  int shift = 20;
  if (sh.hist[T] > need) {
    __syncthreads();
    for (int i = tid; i < kTopkBins; i += kSmThreads) sh.hist[i] = 0u;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kSmMaxPer; i++) {
      if (i >= nper) continue;
      if ((key[i] >> 20) == prefix) atomicAdd(&sh.hist[(key[i] >> 8) & 0xFFFu], 1u);
    }
    __syncthreads();
    sm_threshold(sh, kTopkBins, need, &T, &above);
    need -= above;
    prefix = (prefix << 12) | (uint32_t)T;
    shift = 8;
    if (sh.hist[T] > need) {
      __syncthreads();
      for (int i = tid; i < 256; i += kSmThreads) sh.hist[i] = 0u;
      __syncthreads();
#pragma unroll
      for (int i = 0; i < kSmMaxPer; i++) {
        if (i >= nper) continue;
        if ((key[i] >> 8) == prefix) atomicAdd(&sh.hist[key[i] & 0xFFu], 1u);
      }
      __syncthreads();
      sm_threshold(sh, 256, need, &T, &above);
      need -= above;
      prefix = (prefix << 8) | (uint32_t)T;
      shift = 0;
    }
  }
  // selected: (key >> shift) > prefix, plus the `need` lowest columns with
  // (key >> shift) == prefix (all of whose keys equal the K-th key when
  // shift == 0; when the select stopped early, that bin is taken whole).
  // The column order among equal keys only matters when fewer than all of
  // them are taken and they are above mono(-inf) (else every one is -1).
  const bool rank_eq = shift == 0 && sh.hist[T] > need && prefix > 0x007FFFFFu;

  // ---- collect the selected positions ----
  if (tid == 0) {
    sh.cnt = 0;
    sh.eq_cnt = 0;
    sh.n_neg = 0;
    sh.pmin = 0x7FFFFFFF;
    sh.pmax = -1;
  }
  __syncthreads();
  int lmin = 0x7FFFFFFF, lmax = -1;  // this thread's selected positions
  uint32_t lneg = 0;
  auto emit = [&](int i) {
    const int col = tid + i * kSmThreads;
    const int s = col / K, c = col - s * K;
    int32_t idx = -1;
    if (key[i] > 0x007FFFFFu)  // above mono(-inf)
      idx = __float_as_int(allf[((int64_t)s * R + r) * (2 * K) + K + c]);
    const uint32_t slot = atomicAdd(&sh.cnt, 1u);
    if (slot < (uint32_t)K) sh.sel[slot] = idx;
    if (idx < 0) {
      lneg++;
    } else {
      lmin = min(lmin, idx);
      lmax = max(lmax, idx);
    }
  };
  if (rank_eq) {
    uint32_t eq_base = 0;
#pragma unroll
    for (int i = 0; i < kSmMaxPer; i++) {
      if (i >= nper) continue;  // uniform: every thread runs the same scans
      const uint32_t kk = key[i] >> shift;
      if (kk > prefix) emit(i);
      const uint32_t eq = kk == prefix ? 1u : 0u;
      uint32_t tot;
      const uint32_t rank = eq_base + sm_scan(eq, sh, &tot);  // column order
      if (eq && rank < need) emit(i);
      eq_base += tot;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kSmMaxPer; i++) {
      if (i >= nper) continue;
      const uint32_t kk = key[i] >> shift;
      if (kk > prefix || (kk == prefix && atomicAdd(&sh.eq_cnt, 1u) < need)) emit(i);
    }
  }
  // one LDS atomic per wave for the span and the -1 count
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    lmin = min(lmin, __shfl_xor(lmin, o, 64));
    lmax = max(lmax, __shfl_xor(lmax, o, 64));
    lneg += __shfl_xor(lneg, o, 64);
  }
  if ((tid & 63) == 0) {
    atomicMin(&sh.pmin, lmin);
    atomicMax(&sh.pmax, lmax);
    atomicAdd(&sh.n_neg, lneg);
  }
  __syncthreads();

  const int dst = dst_base >= 0 ? dst_base + r : dst_rows[r];
  if (dst < 0 || dst >= out_rows) return;  // a destination outside out is skipped (uniform)
  int32_t* orow = out + (int64_t)dst * out_stride;

  // ---- ascending order: bitmap compaction when the positions span fewer
  // than 131072 values and are distinct (key-sharded candidates are) ----
  const uint32_t n_neg = sh.n_neg;
  const int pmin = sh.pmin, pmax = sh.pmax;
  if (n_neg == (uint32_t)K || (int64_t)pmax - pmin < kSmBitmapBits) {
    for (int i = tid; i < kTopkBins; i += kSmThreads) sh.hist[i] = 0u;
    __syncthreads();
    for (int i = tid; i < K; i += kSmThreads) {
      const int32_t v = sh.sel[i];
      if (v >= 0) atomicOr(&sh.hist[(v - pmin) >> 5], 1u << ((v - pmin) & 31));
    }
    __syncthreads();
    constexpr int WPT = kTopkBins / kSmThreads;  // 8 bitmap words per thread
    uint32_t words[WPT], cnt = 0;
#pragma unroll
    for (int u = 0; u < WPT; u++) {
      words[u] = sh.hist[tid * WPT + u];
      cnt += __popc(words[u]);
    }
    uint32_t total;
    uint32_t o = n_neg + sm_scan(cnt, sh, &total);
    if (total + n_neg == (uint32_t)K) {  // uniform: all distinct
      for (int i = tid; i < (int)n_neg; i += kSmThreads) orow[i] = -1;
#pragma unroll
      for (int u = 0; u < WPT; u++) {
        uint32_t wv = words[u];
        while (wv) {
          const int b = __ffs(wv) - 1;
          wv &= wv - 1;
          orow[o++] = pmin + 32 * (tid * WPT + u) + b;
        }
      }
      return;
    }
    // duplicated positions: fall through to the sort
  }

  // ---- bitonic sort ascending (K a power of two) ----
  for (int k2 = 2; k2 <= K; k2 <<= 1) {
    for (int j = k2 >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < K; i += kSmThreads) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const int32_t a = sh.sel[i], b = sh.sel[ixj];
          const bool up = (i & k2) == 0;
          if ((a > b) == up) {
            sh.sel[i] = b;
            sh.sel[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int i = tid; i < K; i += kSmThreads) orow[i] = sh.sel[i];
}

}  // namespace
}  // namespace mi355dsa

using namespace mi355dsa;

extern "C" int mi355_dsa_indexer_shard_merge(int32_t* out, int64_t out_stride, int64_t out_rows,
                                             const float* allf, int tp, int R, int K,
                                             const int32_t* dst_rows, int dst_base,
                                             void* stream) {
  clear_error();
  DSA_CHECK(tp >= 1 && R >= 0 && K >= 1, "shard_merge: bad sizes");
  DSA_CHECK(K <= kSmMaxK && (K & (K - 1)) == 0, "shard_merge: K must be a power of two <= %d",
            kSmMaxK);
  const int64_t ncand = (int64_t)tp * K;
  DSA_CHECK(ncand % kSmThreads == 0 && ncand / kSmThreads <= 16 && ncand >= K,
            "shard_merge: tp * K must be a multiple of 512 and at most 8192");
  if (R == 0) return MI355_DSA_OK;
  DSA_CHECK(out && allf, "shard_merge: null pointer argument");
  DSA_CHECK(dst_base >= 0 || dst_rows, "shard_merge: need dst_rows when dst_base < 0");
  DSA_CHECK(dst_base < 0 || (int64_t)dst_base + R <= out_rows,
            "shard_merge: rows dst_base .. dst_base + R exceed out");
  DSA_CHECK(out_stride >= K, "shard_merge: out rows shorter than K");
  hipStream_t st = as_stream(stream);
  shard_merge_kernel<<<R, kSmThreads, 0, st>>>(allf, dst_rows, out, out_stride, out_rows, R, K,
                                                (int)(ncand / kSmThreads), dst_base);
  return check_launch("indexer_shard_merge");
}
