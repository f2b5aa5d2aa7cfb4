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
// candidates' monotone keys and positions in registers (column tid + 512 i
// for its i-th).  A radix select on LDS histograms (a first digit of at most
// 12 bits starting below the bits that all of the row's keys share, then
// digits of 8) finds the K-th largest score key T and how many candidates
// equal to T are taken; those are the lowest columns among the equal ones,
// ranked by block scans in column order (only when that choice can change
// the output).  The selected positions are collected
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
  uint32_t cnt, n_neg;
  int pmin, pmax;
  uint32_t kmin, kmax;
};
constexpr int kSmBitmapBits = kTopkBins * 32;  // 131072 positions

// exclusive prefix sum over the block (DPP wave scans); *total gets the sum
__device__ __forceinline__ uint32_t sm_scan(uint32_t v, SmShared& sh, uint32_t* total) {
  return block_excl_scan_n<kSmThreads>(v, sh.wsum, total);
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

// VEC: tp*K a multiple of 2048 and a 16-byte aligned payload; a thread's
// i-th candidate is column 2048 (i / 4) + 4 tid + i % 4, four of them per
// 16-byte load.  Otherwise column tid + 512 i, one per load.
template <bool VEC>
__global__ void __launch_bounds__(kSmThreads, 8) shard_merge_kernel(
    const float* __restrict__ allf, const int32_t* __restrict__ dst_rows,
    int32_t* __restrict__ out, int64_t out_stride, int64_t out_rows, int R, int K,
    int nper, int dst_base) {
  __shared__ SmShared sh;
  const int r = blockIdx.x;
  const int tid = threadIdx.x;

  // ---- candidates (column col = s K + c) ----
  // The loops over i skip (continue) rather than stop at nper, so they
  // unroll with fixed registers; the loads are unconditional (steps past
  // nper re-read the first ones, whose values are never used), so all of a
  // thread's loads are in flight together.  A break made a runtime loop:
  // one load, then one wait, per step.  Positions are loaded with the
  // scores: about a quarter of the candidates are selected, spread over the
  // row, so reading only theirs later would touch the same cache lines
  // after a second round trip.
  uint32_t key[kSmMaxPer];
  int32_t pos[kSmMaxPer];
  if constexpr (VEC) {
#pragma unroll
    for (int j = 0; j < kSmMaxPer / 4; j++) {
      const int col = 2048 * (4 * j < nper ? j : 0) + 4 * tid;
      const int s = col / K, c = col - s * K;  // c % 4 == 0: a group stays in one shard
      const float* rowp = allf + ((int64_t)s * R + r) * (2 * K);
      const u32x4 sv = *reinterpret_cast<const u32x4*>(rowp + c);
      const u32x4 pv = *reinterpret_cast<const u32x4*>(rowp + K + c);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        key[4 * j + e] = mono_of(__uint_as_float(sv[e]));
        pos[4 * j + e] = (int32_t)pv[e];
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < kSmMaxPer; i++) {
      const int col = tid + (i < nper ? i : 0) * kSmThreads;
      const int s = col / K, c = col - s * K;
      const float* rowp = allf + ((int64_t)s * R + r) * (2 * K);
      key[i] = mono_of(rowp[c]);
      pos[i] = __float_as_int(rowp[K + c]);
    }
  }

  // ---- the bits the row's keys share: the first digit starts below them ----
  // (normally distributed scores share their sign and most exponent bits; a
  // digit over those bits would put every key in a few bins, whose LDS
  // atomics then serialise)
  uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
#pragma unroll
  for (int i = 0; i < kSmMaxPer; i++) {
    if (i >= nper) continue;
    kmin = min(kmin, key[i]);
    kmax = max(kmax, key[i]);
  }
  kmin = wave_min_u32(kmin);
  kmax = wave_max_u32(kmax);
  if (tid == 0) {
    sh.kmin = 0xFFFFFFFFu;
    sh.kmax = 0u;
  }
  for (int i = tid; i < kTopkBins; i += kSmThreads) sh.hist[i] = 0u;
  __syncthreads();
  if ((tid & 63) == 0) {
    atomicMin(&sh.kmin, kmin);
    atomicMax(&sh.kmax, kmax);
  }
  __syncthreads();
  const uint32_t diff = sh.kmin ^ sh.kmax;
  // highest differing bit hb; the keys agree on every bit above it
  const int hb = diff ? 31 - __clz(diff) : 0;

  // ---- radix select of the K-th largest key: a digit of at most 12 bits
  // from bit hb down, then digits of 8; prefix = key >> shift of the K-th key ----
  int lo = hb >= 11 ? hb - 11 : 0;
  int nb = hb - lo + 1;
#pragma unroll
  for (int i = 0; i < kSmMaxPer; i++) {
    if (i >= nper) continue;
    atomicAdd(&sh.hist[(key[i] >> lo) & ((1u << nb) - 1u)], 1u);
  }
  __syncthreads();
  int T;
  uint32_t above;
  sm_threshold(sh, kTopkBins, (uint32_t)K, &T, &above);
  uint32_t need = (uint32_t)K - above;
  int shift = lo;
  // every key agrees with kmin above bit hb: the K-th key's prefix
  uint32_t prefix = ((hb == 31 ? 0u : (sh.kmin >> (hb + 1)) << nb)) | (uint32_t)T;
  const int lane = tid & 63;
  uint32_t n_at = sh.hist[T];  // candidates with (key >> shift) == prefix
  // further digits of 8 bits: a threshold bin holds a few hundred keys, and
  // a 256-bin histogram is cleared and scanned in one step per thread
  while (n_at > need && shift > 0) {  // uniform
    const int lo2 = shift >= 8 ? shift - 8 : 0;
    const int nb2 = shift - lo2;
    __syncthreads();
    for (int i = tid; i < (1 << nb2); i += kSmThreads) sh.hist[i] = 0u;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kSmMaxPer; i++) {
      if (i >= nper) continue;
      if ((key[i] >> shift) == prefix) atomicAdd(&sh.hist[(key[i] >> lo2) & ((1u << nb2) - 1u)], 1u);
    }
    __syncthreads();
    sm_threshold(sh, 1 << nb2, need, &T, &above);
    need -= above;
    prefix = (prefix << nb2) | (uint32_t)T;
    shift = lo2;
    n_at = sh.hist[T];
  }
  // selected: (key >> shift) > prefix, plus the `need` lowest columns with
  // (key >> shift) == prefix (all of whose keys equal the K-th key when
  // shift == 0; when the select stopped early, that bin is taken whole).
  // The column order among equal keys only matters when fewer than all of
  // them are taken and they are above mono(-inf) (else every one is -1).
  const bool rank_eq = shift == 0 && n_at > need && prefix > 0x007FFFFFu;

  // ---- collect the selected positions ----
  if (tid == 0) {
    sh.cnt = 0;
    sh.n_neg = 0;
    sh.pmin = 0x7FFFFFFF;
    sh.pmax = -1;
  }
  __syncthreads();
  int lmin = 0x7FFFFFFF, lmax = -1;  // this thread's selected positions
  uint32_t lneg = 0;
  auto put = [&](int i, uint32_t slot) {
    const int32_t idx = key[i] > 0x007FFFFFu ? pos[i] : -1;  // above mono(-inf)
    if (slot < (uint32_t)K) sh.sel[slot] = idx;
    if (idx < 0) {
      lneg++;
    } else {
      lmin = min(lmin, idx);
      lmax = max(lmax, idx);
    }
  };
  // the wave's selected candidates of step i take consecutive slots: one LDS
  // atomic per wave and step
  auto emit = [&](int i, bool take) {
    const uint64_t m = __ballot(take);
    uint32_t base = 0;
    if (lane == 0 && m) base = atomicAdd(&sh.cnt, (uint32_t)__popcll(m));
    base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
    if (!take) return;
    put(i, base + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                            __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u)));
  };
  if (rank_eq && !VEC) {
    uint32_t eq_base = 0;
#pragma unroll
    for (int i = 0; i < kSmMaxPer; i++) {
      if (i >= nper) continue;  // uniform: every thread runs the same scans
      const uint32_t kk = key[i] >> shift;
      const uint32_t eq = kk == prefix ? 1u : 0u;
      uint32_t tot;
      const uint32_t rank = eq_base + sm_scan(eq, sh, &tot);  // column order
      emit(i, kk > prefix || (eq && rank < need));
      eq_base += tot;
    }
  } else if (rank_eq) {
    // column order with four consecutive columns per thread and step j:
    // one scan of the thread's count per step, then its own order
    uint32_t eq_base = 0;
#pragma unroll
    for (int j = 0; j < kSmMaxPer / 4; j++) {
      if (4 * j >= nper) continue;  // uniform
      uint32_t eqm = 0;
#pragma unroll
      for (int e = 0; e < 4; e++) eqm |= ((key[4 * j + e] >> shift) == prefix ? 1u : 0u) << e;
      uint32_t tot;
      uint32_t rank = eq_base + sm_scan(__popc(eqm), sh, &tot);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t kk = key[4 * j + e] >> shift;
        const bool eq = (eqm >> e) & 1u;
        emit(4 * j + e, kk > prefix || (eq && rank < need));
        rank += eq ? 1u : 0u;
      }
      eq_base += tot;
    }
  } else {
    // Any `need` of the equal ones will do: the bin is taken whole, or all
    // of them are at or below mono(-inf).  One block scan of the packed
    // (greater | equal << 16) counts numbers the slots: greater keys first,
    // then the equal ones (per-step LDS atomics made a chain of dependent
    // LDS round trips, ~5 us per row).
    uint32_t gt_mask = 0, eq_mask = 0;
#pragma unroll
    for (int i = 0; i < kSmMaxPer; i++) {
      if (i >= nper) continue;
      const uint32_t kk = key[i] >> shift;
      gt_mask |= (kk > prefix ? 1u : 0u) << i;
      eq_mask |= (kk == prefix ? 1u : 0u) << i;
    }
    uint32_t tot;
    const uint32_t ex = sm_scan(__popc(gt_mask) | (__popc(eq_mask) << 16), sh, &tot);
    uint32_t gslot = ex & 0xFFFFu, erank = ex >> 16;
    const uint32_t n_gt = tot & 0xFFFFu;
#pragma unroll
    for (int i = 0; i < kSmMaxPer; i++) {
      if (i >= nper) continue;
      if ((gt_mask >> i) & 1u) {
        put(i, gslot++);
      } else if ((eq_mask >> i) & 1u) {
        if (erank < need) put(i, n_gt + erank);
        erank++;
      }
    }
  }
  // one LDS atomic per wave for the span and the -1 count
  lmin = wave_min_i32(lmin);
  lmax = wave_max_i32(lmax);
  lneg = wave_sum_u32(lneg);
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
  const int nper = (int)(ncand / kSmThreads);
  if (ncand % 2048 == 0 && aligned_to(allf, 16))
    shard_merge_kernel<true><<<R, kSmThreads, 0, st>>>(allf, dst_rows, out, out_stride, out_rows,
                                                        R, K, nper, dst_base);
  else
    shard_merge_kernel<false><<<R, kSmThreads, 0, st>>>(allf, dst_rows, out, out_stride,
                                                         out_rows, R, K, nper, dst_base);
  return check_launch("indexer_shard_merge");
}
