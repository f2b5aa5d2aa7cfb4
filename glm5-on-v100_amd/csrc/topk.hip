// Exact per-row top-k selection for the DSA indexer (decode and prefill).
//
// Contract (reference sm70_decode_topk, csrc/attention/sm70_mla_decode.cu:
// 1187-1212, host :2844-2905, made exact): idx[r,:] holds the positions
// p < min(seq_len[r], width) of the k largest scores under the 32-bit
// monotone key order; among equal keys the lower position wins; positions
// are written in ascending order and the tail is padded with -1.  When
// seq_len <= k every valid position is selected.
//
// Design for gfx950: no inter-workgroup synchronisation (the reference's
// co-resident spin grid needs a forward-progress guarantee that a plain
// launch does not give).  Three kernels share the exact radix select on LDS
// histograms (a 12-bit level-1 digit, then 10- or 12-bit digits):
//  * topk_row2_kernel, one 1024-thread workgroup per row, two per CU: the
//    row is read once or twice (a candidate list in LDS, position bitmaps
//    and one block scan give the ordered output); persistent_topk and decode
//    calls with many rows.
//  * topk_row_kernel / topk_row_select: the same contract in up to four
//    reads with an ordered compaction pass; rows too wide for the bitmaps
//    and the decode select kernel's fallback.
//  * topk_scan_kernel + topk_select_kernel: decode calls with few rows,
//    spread over the row's 1024-key tiles.
// The decode paths start from the level-1 histogram the indexer kernel
// already built.  Every path is deterministic.
#include "capi_internal.h"
#include "dsa_common.h"
#include "head_proj.h"

namespace mi355dsa {

constexpr int kTkThreads = 1024;
constexpr int kTkWaves = kTkThreads / 64;
constexpr int kTkV = 16;                         // positions per thread, final pass
constexpr int kTkChunk = kTkThreads * kTkV;      // 16384 positions per chunk
constexpr int kTkChunkPad = kTkChunk + kTkChunk / kTkV;

struct TopkShared {
  uint32_t hist[kTopkBins];
  float chunk[kTkChunkPad];
  uint32_t wsum[kTkWaves + 1];
  int T;
  uint32_t above;
};

__device__ uint32_t block_excl_scan(uint32_t v, uint32_t* wsum, uint32_t* total) {
  return block_excl_scan_n<kTkThreads>(v, wsum, total);
}

// Bin T of an nbins histogram with above(T) < need <= above(T) + hist[T],
// where above(T) counts keys in bins > T.  Requires need <= total.  SH has
// hist, wsum (kTkWaves + 1 words), T and above.
template <class SH>
__device__ void find_threshold(SH& sh, int nbins, uint32_t need, int* T, uint32_t* above) {
  const int per = nbins >= kTkThreads ? nbins / kTkThreads : 1;
  const int lo = threadIdx.x * per;
  uint32_t cs = 0;
  if (lo < nbins)
    for (int i = 0; i < per; i++) cs += sh.hist[lo + i];
  uint32_t total;
  const uint32_t excl = block_excl_scan(cs, sh.wsum, &total);
  if (threadIdx.x == 0) sh.T = -1;
  __syncthreads();
  if (lo < nbins) {
    uint32_t a = total - excl - cs;  // keys in bins above this thread's chunk
    for (int bin = lo + per - 1; bin >= lo; bin--) {
      const uint32_t h = sh.hist[bin];
      if (a < need && a + h >= need) {
        sh.T = bin;
        sh.above = a;
        break;
      }
      a += h;
    }
  }
  __syncthreads();
  *T = sh.T;
  *above = sh.above;
  __syncthreads();
}


// Applies f(p, key) to every position p < L of the row; each thread keeps
// kTkU independent loads in flight per step (a plain strided loop would
// wait for one load per iteration).
constexpr int kTkU = 16;
template <int U = kTkU, typename F>
__device__ __forceinline__ void row_pass(const float* __restrict__ row, int L, F f) {
  for (int base = 0; base < L; base += kTkThreads * U) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int p = base + u * kTkThreads + (int)threadIdx.x;
      v[u] = (p < L) ? row[p] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int p = base + u * kTkThreads + (int)threadIdx.x;
      if (p < L) f(p, mono_key(v[u]));
    }
  }
}

// Whole-row selection by one 1024-thread workgroup (L > K): 3-level radix
// select on LDS histograms, then an ordered compaction pass.  hist_row (may
// be null) is the row's level-1 histogram; one that does not count exactly
// L keys is rebuilt from the row.
__device__ void topk_row_select(TopkShared& sh, const float* __restrict__ row, int L, int K,
                                int32_t* __restrict__ out, const uint32_t* __restrict__ hist_row) {
  // ---- level 1: bits [20,32) ----
  bool rebuild = hist_row == nullptr;
  if (hist_row != nullptr) {
    const uint32_t* h = hist_row;
    uint32_t part = 0;
    for (int i = threadIdx.x; i < kTopkBins; i += kTkThreads) {
      sh.hist[i] = h[i];
      part += h[i];
    }
    uint32_t total;
    block_excl_scan(part, sh.wsum, &total);
    // a histogram that does not describe this row exactly is rebuilt
    rebuild = (total != (uint32_t)L);
  }
  if (rebuild) {
    for (int i = threadIdx.x; i < kTopkBins; i += kTkThreads) sh.hist[i] = 0u;
    __syncthreads();
    row_pass(row, L, [&](int, uint32_t key) { atomicAdd(&sh.hist[key >> 20], 1u); });
    __syncthreads();
  }
  int T;
  uint32_t above;
  find_threshold(sh, kTopkBins, (uint32_t)K, &T, &above);
  uint32_t need = (uint32_t)K - above;
  uint32_t prefix = (uint32_t)T;
  int shift = 20;
  uint32_t bin_count = (T >= 0) ? sh.hist[T] : 0u;

  // ---- level 2: bits [8,20) of keys in bin T ----
  if (bin_count > need) {
    __syncthreads();
    for (int i = threadIdx.x; i < kTopkBins; i += kTkThreads) sh.hist[i] = 0u;
    __syncthreads();
    row_pass(row, L, [&](int, uint32_t key) {
      if ((key >> 20) == prefix) atomicAdd(&sh.hist[(key >> 8) & 0xfffu], 1u);
    });
    __syncthreads();
    find_threshold(sh, kTopkBins, need, &T, &above);
    need -= above;
    prefix = (prefix << 12) | (uint32_t)T;
    shift = 8;
    bin_count = (T >= 0) ? sh.hist[T] : 0u;
    // ---- level 3: bits [0,8) ----
    if (bin_count > need) {
      __syncthreads();
      for (int i = threadIdx.x; i < 256; i += kTkThreads) sh.hist[i] = 0u;
      __syncthreads();
      row_pass(row, L, [&](int, uint32_t key) {
        if ((key >> 8) == prefix) atomicAdd(&sh.hist[key & 0xffu], 1u);
      });
      __syncthreads();
      find_threshold(sh, 256, need, &T, &above);
      need -= above;
      prefix = (prefix << 8) | (uint32_t)T;
      shift = 0;
    }
  }
  // Selection: (key >> shift) > prefix, plus the `need` lowest positions
  // with (key >> shift) == prefix.
  const uint32_t n_eq_take = need;

  uint32_t base_gt = 0, base_eq = 0;
  for (int c0 = 0; c0 < L; c0 += kTkChunk) {
    __syncthreads();
    {
      float v[kTkV];
#pragma unroll
      for (int i = 0; i < kTkV; i++) {
        const int p = c0 + i * kTkThreads + (int)threadIdx.x;  // coalesced
        v[i] = (p < L) ? row[p] : 0.f;
      }
#pragma unroll
      for (int i = 0; i < kTkV; i++) {
        const int q = i * kTkThreads + threadIdx.x;
        sh.chunk[q + q / kTkV] = v[i];
      }
    }
    __syncthreads();
    const int my0 = threadIdx.x * kTkV;
    uint32_t gt_mask = 0, eq_mask = 0;
    for (int i = 0; i < kTkV; i++) {
      const int q = my0 + i;
      if (c0 + q < L) {
        const uint32_t k = mono_key(sh.chunk[q + q / kTkV]) >> shift;
        if (k > prefix) gt_mask |= 1u << i;
        else if (k == prefix) eq_mask |= 1u << i;
      }
    }
    const uint32_t packed =
        (uint32_t)__popc(gt_mask) | ((uint32_t)__popc(eq_mask) << 16);
    uint32_t tot;
    const uint32_t ex = block_excl_scan(packed, sh.wsum, &tot);
    const uint32_t G = base_gt + (ex & 0xffffu);
    uint32_t E = base_eq + (ex >> 16);
    uint32_t o = G + (E < n_eq_take ? E : n_eq_take);
    for (int i = 0; i < kTkV; i++) {
      const bool gt = (gt_mask >> i) & 1u;
      const bool eq = (eq_mask >> i) & 1u;
      // o < K always holds by construction; the bound keeps a logic error
      // from ever writing outside the row
      if (gt) {
        if (o < (uint32_t)K) out[o] = c0 + my0 + i;
        o++;
      } else if (eq) {
        if (E < n_eq_take) {
          if (o < (uint32_t)K) out[o] = c0 + my0 + i;
          o++;
        }
        E++;
      }
    }
    base_gt += tot & 0xffffu;
    base_eq += tot >> 16;
  }
  // Exactly K positions were written (L > K); nothing to pad.
}

template <bool HAVE_HIST>
__global__ void __launch_bounds__(kTkThreads) topk_row_kernel(
    const float* __restrict__ score, int64_t row_stride,
    const int32_t* __restrict__ seq_lens, const uint32_t* __restrict__ hist_in,
    int32_t* __restrict__ idx, int K) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  TopkShared& sh = *reinterpret_cast<TopkShared*>(smem_raw);
  const int r = blockIdx.x;
  const float* row = score + (int64_t)r * row_stride;
  int32_t* out = idx + (int64_t)r * K;
  int L = seq_lens[r];
  if (L > row_stride) L = (int)row_stride;
  if (L < 0) L = 0;
  if (L <= K) {
    for (int p = threadIdx.x; p < K; p += kTkThreads) out[p] = (p < L) ? p : -1;
    return;
  }
  topk_row_select(sh, row, L, K, out, HAVE_HIST ? hist_in + (int64_t)r * kTopkBins : nullptr);
}

template <bool HAVE_HIST>
static int launch_topk(const float* score, int n_rows, int64_t row_stride,
                       const int32_t* seq_lens, const uint32_t* hist, int32_t* idx,
                       int K, hipStream_t st) {
  const size_t smem = sizeof(TopkShared);
  const int rc = reserve_lds(reinterpret_cast<const void*>(topk_row_kernel<HAVE_HIST>), smem, "topk");
  if (rc) return rc;
  topk_row_kernel<HAVE_HIST><<<n_rows, kTkThreads, smem, st>>>(score, row_stride, seq_lens,
                                                              hist, idx, K);
  return check_launch("topk");
}

// ===========================================================================
// Whole-row top-k in two reads of the row (persistent_topk, and decode calls
// with more rows than the two-kernel path takes):
//  * read 1 builds the 12-bit level-1 histogram (skipped when the caller's
//    histogram counts exactly L keys).  Its threshold bin leaves `und` keys
//    undecided; while they exceed the LDS list, one more read of the row
//    builds the next 10-bit histogram among them (only heavily tied rows).
//  * read 2 marks every key above the undecided prefix in an LDS bitmap of
//    positions (one wave ballot covers 64 positions, two whole words) and
//    appends the undecided keys, with their positions, to an LDS list.
//  * The remaining 10-bit digits are selected on the list in LDS; list keys
//    above the exact k-th key tau join the bitmap, keys equal to tau go to
//    a second bitmap.  When the row reads already reached tau, read 2 fills
//    the second bitmap directly.
//  * One block scan over the two bitmaps' popcounts gives each thread its
//    output offset; it writes the positions of its words in ascending order,
//    taking the lowest positions among the ties at tau.
// LDS: the 16 KB histogram, two bitmaps of row_stride bits and the list,
// sized on the host so two workgroups share a CU at the C4 row width.
// ===========================================================================
struct Tk2Head {
  uint32_t hist[kTopkBins];
  uint32_t wsum[kTkWaves + 1];
  uint64_t wsum64[kTkWaves + 1];
  int T;
  uint32_t above;
  uint32_t n_list;
};
// loads in flight per thread in the row reads (8 keeps 64 VGPRs, two
// 1024-thread workgroups per CU)
constexpr int kTk2U = 8;
constexpr int kTk2HeadBytes = (int)((sizeof(Tk2Head) + 15) / 16 * 16);

// find_threshold by wave 0 alone; the other waves wait at one barrier.  Lane
// l sums bins [l per, l per + per) with 16-byte LDS reads, a suffix scan
// over the lanes finds the lane whose bins hold the threshold, and a second
// scan over that lane's bins, one per lane, finds the bin: the bin T with
// above(T) < need <= above(T) + hist[T], as find_threshold returns.  nbins
// is 1024 or 4096; requires 1 <= need <= total.  It ends without a barrier:
// a caller that writes hist next puts one first.
__device__ void find_threshold_w0(Tk2Head& sh, int nbins, uint32_t need, int* T,
                                  uint32_t* above) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int per = nbins >> 6;  // 16 or 64 bins per lane
    const u32x4* h4 = reinterpret_cast<const u32x4*>(sh.hist) + lane * (per >> 2);
    uint32_t cs = 0;
    for (int i = 0; i < (per >> 2); i++) {
      const u32x4 q = h4[i];
      cs += q[0] + q[1] + q[2] + q[3];
    }
    const uint32_t incl = wave_incl_scan(cs);
    const uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
    const uint32_t a = total - incl;  // keys in the bins of the lanes above
    const uint64_t hit = __ballot((a < need) & (a + cs >= need));
    const int L = hit != 0ull ? (int)__builtin_ctzll(hit) : 0;
    const uint32_t aL = (uint32_t)__builtin_amdgcn_readlane((int)a, L);
    const uint32_t hv = lane < per ? sh.hist[L * per + lane] : 0u;
    const uint32_t incl2 = wave_incl_scan(hv);
    const uint32_t a2 = aL + ((uint32_t)__builtin_amdgcn_readlane((int)incl2, 63) - incl2);
    const uint64_t hit2 = __ballot((lane < per) & (a2 < need) & (a2 + hv >= need));
    const int j = hit2 != 0ull ? (int)__builtin_ctzll(hit2) : 0;
    const uint32_t aj = (uint32_t)__builtin_amdgcn_readlane((int)a2, j);
    if (lane == 0) {
      sh.T = L * per + j;
      sh.above = aj;
    }
  }
  __syncthreads();
  *T = sh.T;
  *above = sh.above;
}

// wave_incl_scan of two packed 32-bit counts whose sums stay below 2^32.
__device__ __forceinline__ uint64_t wave_incl_scan64(uint64_t x) {
  const uint32_t lo = wave_incl_scan((uint32_t)x);
  const uint32_t hi = wave_incl_scan((uint32_t)(x >> 32));
  return (uint64_t)lo | ((uint64_t)hi << 32);
}

// Block-wide exclusive prefix sum of 64-bit values (two 32-bit counts
// packed, neither of which can carry into the other).
__device__ uint64_t block_excl_scan64(uint64_t v, uint64_t* wsum, uint64_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t x = wave_incl_scan64(v);
  if (lane == 63) wsum[wave] = x;
  __syncthreads();
  if (wave == 0) {
    const uint64_t t = lane < kTkWaves ? wsum[lane] : 0ull;
    const uint64_t y = wave_incl_scan64(t);
    if (lane < kTkWaves) wsum[lane] = y - t;
    if (lane == kTkWaves - 1) wsum[kTkWaves] = y;
  }
  __syncthreads();
  const uint64_t res = wsum[wave] + x - v;
  *total = wsum[kTkWaves];
  __syncthreads();
  return res;
}

// Appends (key, p) of the lanes with `take` to the LDS list with one LDS
// atomic per wave; *n_list counts every append, also those past cap.
__device__ __forceinline__ void list_append(bool take, uint32_t key, int p, uint32_t* n_list,
                                            uint32_t* lkey, int32_t* lpos, int cap) {
  const uint64_t m = __ballot(take);
  if (m == 0ull) return;
  const int lane = threadIdx.x & 63;
  uint32_t b0 = 0;
  if (lane == 0) b0 = atomicAdd(n_list, (uint32_t)__popcll(m));
  b0 = __shfl(b0, 0, 64);
  if (take) {
    const uint32_t j = b0 + (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
    if (j < (uint32_t)cap) {
      lkey[j] = key;
      lpos[j] = p;
    }
  }
}

// Read-1 layout of one step of kTk2U values per lane over kTkThreads *
// kTk2U positions: with V4 each lane loads 16-byte groups of 4 consecutive
// positions (rows 16-byte aligned, stride a multiple of 4 floats), else
// single floats; both are coalesced per wave.
template <bool V4>
__device__ __forceinline__ int r1_pos(int base, int e) {
  return V4 ? base + (((e >> 2) * kTkThreads + (int)threadIdx.x) << 2) + (e & 3)
            : base + e * kTkThreads + (int)threadIdx.x;
}

// Loads one step.  The loads are unconditional: a position >= L reads the
// row's last group (V4; a group that starts below L <= row_stride lies
// wholly inside the row) or element, and every use tests p < L.  Loads
// under a branch would make the compiler's wait before a step's first use
// vmcnt(0), draining the next step's prefetch as well.
template <bool V4>
__device__ __forceinline__ void r1_load(const float* __restrict__ row, int base, int L,
                                        float (&v)[kTk2U]) {
  if (V4) {
    const int last = (L - 1) & ~3;
#pragma unroll
    for (int u = 0; u < kTk2U / 4; u++) {
      const int p = min(r1_pos<true>(base, 4 * u), last);
      const float4 x = *reinterpret_cast<const float4*>(row + p);
      v[4 * u] = x.x;
      v[4 * u + 1] = x.y;
      v[4 * u + 2] = x.z;
      v[4 * u + 3] = x.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < kTk2U; e++) v[e] = row[min(r1_pos<false>(base, e), L - 1)];
  }
}

// nw2 = bitmap words (2 * ceil(row_stride / 64)); cap = list entries.
template <bool HAVE_HIST, bool V4>
__global__ void __launch_bounds__(kTkThreads) __attribute__((amdgpu_waves_per_eu(8))) topk_row2_kernel(
    const float* __restrict__ score, int64_t row_stride,
    const int32_t* __restrict__ seq_lens, const uint32_t* __restrict__ hist_in,
    int32_t* __restrict__ idx, int K, int nw2, int cap) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  Tk2Head& sh = *reinterpret_cast<Tk2Head*>(smem_raw);
  uint32_t* gtm = reinterpret_cast<uint32_t*>(smem_raw + kTk2HeadBytes);
  uint32_t* eqm = gtm + nw2;
  uint32_t* lkey = eqm + nw2;
  int32_t* lpos = reinterpret_cast<int32_t*>(lkey + cap);
  const int tid = threadIdx.x, lane = tid & 63;
  const int r = blockIdx.x;
  const float* row = score + (int64_t)r * row_stride;
  int32_t* out = idx + (int64_t)r * K;
  int L = seq_lens[r];
  if (L > row_stride) L = (int)row_stride;
  if (L < 0) L = 0;
  if (L <= K) {
    for (int p = tid; p < K; p += kTkThreads) out[p] = (p < L) ? p : -1;
    return;
  }
  // ---- read 1: level-1 histogram, bits [20,32) ----
  bool rebuild = !HAVE_HIST;
  if (HAVE_HIST) {
    const uint32_t* h = hist_in + (int64_t)r * kTopkBins;
    uint32_t part = 0;
    for (int i = tid; i < kTopkBins; i += kTkThreads) {
      sh.hist[i] = h[i];
      part += h[i];
    }
    uint32_t total;
    block_excl_scan(part, sh.wsum, &total);
    rebuild = (total != (uint32_t)L);
  }
  // A rebuilding read 1 lists the keys of level-1 bin >= te, with te taken
  // from a histogram of every fourth key of the first step (elements 0 and
  // 4 of each thread's eight) so that about 1.5 k keys of a row with
  // stationary scores qualify; past the first step it builds no histogram.  When at least k and at most cap keys were listed, the list
  // holds every key of the bins from te up, so the threshold bin (>= te)
  // and its neighbours' counts come from a histogram of the list, and the
  // second read is skipped.  Otherwise a histogram read of the row follows
  // and the second read runs.
  bool spec = false;
  uint32_t te = 0;
  if (rebuild) {
    constexpr int kS0 = kTkThreads * kTk2U;  // positions per step
    for (int i = tid; i < kTopkBins; i += kTkThreads) sh.hist[i] = 0u;
    if (tid == 0) sh.n_list = 0u;
    __syncthreads();
    // Double buffered: the next step's loads are in flight while this one
    // is tested and listed.  The first step builds the histogram that sets
    // te; every step then lists its keys of bin >= te.  The test is one
    // float compare: for a non-NaN v, mono_key(v) >= te << 20 exactly when
    // v >= fte, the smallest float of bin te, except v = -0 against
    // fte = +0 (te = 0x800), which the bit test excl removes; bins below
    // mono_key(-inf) hold only NaNs, so there fte = -inf.  The list holds
    // the raw float bits until read 1 ends.
    float v[kTk2U], w[kTk2U];
    r1_load<V4>(row, 0, L, v);
    r1_load<V4>(row, kS0, L, w);  // past the row: re-reads its last group, unused
#pragma unroll
    for (int e = 0; e < kTk2U; e += 4)
      if (r1_pos<V4>(0, e) < L) atomicAdd(&sh.hist[mono_key(v[e]) >> 20], 1u);
    __syncthreads();
    {
      // sampled positions below L: 4t and 4t + 4096 (V4), t and t + 1024 (else)
      const int S = V4 ? (min(L, kS0) + 3) / 4
                       : min(L, kTkThreads) + min(max(L - 4 * kTkThreads, 0), kTkThreads);
      uint64_t tgt = (3ull * (uint64_t)K * S + 2ull * L - 1) / (2ull * L);
      tgt = tgt < 1 ? 1 : (tgt > (uint64_t)S ? (uint64_t)S : tgt);
      int Te;
      uint32_t ab;
      find_threshold_w0(sh, kTopkBins, (uint32_t)tgt, &Te, &ab);
      te = (uint32_t)Te;
    }
    const uint32_t tkey = te << 20;
    const float fte = tkey <= 0x007fffffu
                          ? -INFINITY
                          : __uint_as_float((tkey & 0x80000000u) ? (tkey & 0x7fffffffu) : ~tkey);
    const uint32_t excl = tkey == 0x80000000u ? 0x80000000u : 0xffffffffu;  // 0xffffffff: a NaN
    const int lp0 = V4 ? 4 * tid : tid;  // this lane's position offset within a step
    // lists the keys of bin >= te among vals (positions base + ...); the
    // tag says whether the step reaches past L (conditions combined with &,
    // not &&, so that no branch splits the tests)
    auto step = [&](const float (&vals)[kTk2U], int base, auto check_tag) {
      constexpr bool check = decltype(check_tag)::value;
      bool tk[kTk2U];
      uint64_t m[kTk2U];
      uint32_t cnt = 0;
#pragma unroll
      for (int e = 0; e < kTk2U; e++) {
        tk[e] = (vals[e] >= fte) & (__float_as_uint(vals[e]) != excl);
        if constexpr (check)
          tk[e] = tk[e] & (base + lp0 + (V4 ? (e >> 2) * (4 * kTkThreads) + (e & 3) : e * kTkThreads) < L);
        m[e] = __builtin_amdgcn_ballot_w64(tk[e]);
        cnt += (uint32_t)__popcll(m[e]);
      }
      if (cnt == 0u) return;
      uint32_t b0 = 0;
      if (lane == 0) b0 = atomicAdd(&sh.n_list, cnt);
      b0 = __builtin_amdgcn_readlane(b0, 0);
#pragma unroll
      for (int e = 0; e < kTk2U; e++) {
        if (tk[e]) {
          // rank among the wave's taking lanes below this one
          const uint32_t j = b0 + __builtin_amdgcn_mbcnt_hi(
                                      (uint32_t)(m[e] >> 32),
                                      __builtin_amdgcn_mbcnt_lo((uint32_t)m[e], 0u));
          if (j < (uint32_t)cap) {
            lkey[j] = __float_as_uint(vals[e]);
            lpos[j] = base + lp0 + (V4 ? (e >> 2) * (4 * kTkThreads) + (e & 3) : e * kTkThreads);
          }
        }
        b0 += (uint32_t)__popcll(m[e]);
      }
    };
    // steps alternate between the two buffers; a step wholly below L skips
    // the position test
    int base = 0;
    while (true) {
      if (base + kS0 > L) {
        step(v, base, std::true_type{});
        break;
      }
      step(v, base, std::false_type{});
      base += kS0;
      if (base >= L) break;
      r1_load<V4>(row, base + kS0, L, v);
      if (base + kS0 > L) {
        step(w, base, std::true_type{});
        break;
      }
      step(w, base, std::false_type{});
      base += kS0;
      if (base >= L) break;
      r1_load<V4>(row, base + kS0, L, w);
    }
    __syncthreads();
    const uint32_t n_list = sh.n_list;
    spec = n_list >= (uint32_t)K && n_list <= (uint32_t)cap;
    __syncthreads();  // every thread has read n_list and the first-step histogram
    for (int i = tid; i < kTopkBins; i += kTkThreads) sh.hist[i] = 0u;
    __syncthreads();
    if (spec) {  // the list's keys as monotone keys, and their level-1 histogram
      for (int i = tid; i < (int)n_list; i += kTkThreads) {
        const uint32_t k = mono_key(__uint_as_float(lkey[i]));
        lkey[i] = k;
        atomicAdd(&sh.hist[k >> 20], 1u);
      }
    } else {     // the estimate missed: level-1 histogram of the whole row
      row_pass<kTk2U>(row, L, [&](int, uint32_t key) { atomicAdd(&sh.hist[key >> 20], 1u); });
    }
    __syncthreads();
  }
  int T;
  uint32_t above;
  find_threshold_w0(sh, kTopkBins, (uint32_t)K, &T, &above);
  uint32_t need = (uint32_t)K - above;   // keys still to take among the undecided
  uint32_t prefix = (uint32_t)T;         // undecided: (key >> shift) == prefix
  int shift = 20;
  uint32_t und = sh.hist[T];
  const int nwl = 2 * ((L + 63) >> 6);  // words covering [0, L) in whole wave steps
  bool list_mode;
  if (spec) {
    // T >= te: every key of bin >= T is on the list (so und <= cap)
    for (int i = tid; i < nwl; i += kTkThreads) {
      gtm[i] = 0u;
      eqm[i] = 0u;
    }
    __syncthreads();
    list_mode = true;
  } else {
    // ---- narrow on the row while the undecided keys overflow the list ----
    while (und > (uint32_t)cap && und != need && shift > 0) {
      const int s2 = shift - 10;
      __syncthreads();
      for (int i = tid; i < 1024; i += kTkThreads) sh.hist[i] = 0u;
      __syncthreads();
      row_pass<kTk2U>(row, L, [&](int, uint32_t key) {
        if ((key >> shift) == prefix) atomicAdd(&sh.hist[(key >> s2) & 1023u], 1u);
      });
      __syncthreads();
      find_threshold_w0(sh, 1024, need, &T, &above);
      need -= above;
      prefix = (prefix << 10) | (uint32_t)T;
      shift = s2;
      und = sh.hist[T];
    }
    // ---- read 2: bitmap of the keys above the prefix; list of the undecided ----
    // undecided keys that are all taken need no list: they go to the tie bitmap
    list_mode = shift > 0 && und != need;
    __syncthreads();
    if (list_mode)
      for (int i = tid; i < nwl; i += kTkThreads) eqm[i] = 0u;
    if (tid == 0) sh.n_list = 0u;
    __syncthreads();
    for (int base = 0; base < L; base += kTkThreads * kTk2U) {
      float v[kTk2U];
#pragma unroll
      for (int u = 0; u < kTk2U; u++) {
        const int p = base + u * kTkThreads + tid;
        v[u] = (p < L) ? row[p] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kTk2U; u++) {
        const int p = base + u * kTkThreads + tid;
        const int p0 = p - lane;  // first position of this wave step, a multiple of 64
        const uint32_t key = mono_key(v[u]);
        const uint32_t hi = key >> shift;
        const bool gt = p < L && hi > prefix;
        const bool un = p < L && hi == prefix;
        const uint64_t mg = __ballot(gt);
        const uint64_t mu = __ballot(un);
        if (p0 < L && lane == 0) {
          gtm[p0 >> 5] = (uint32_t)mg;
          gtm[(p0 >> 5) + 1] = (uint32_t)(mg >> 32);
          if (!list_mode) {
            eqm[p0 >> 5] = (uint32_t)mu;
            eqm[(p0 >> 5) + 1] = (uint32_t)(mu >> 32);
          }
        }
        if (list_mode) list_append(un, key, p, &sh.n_list, lkey, lpos, cap);
      }
    }
    __syncthreads();
  }
  // ---- remaining digits on the list, in LDS ----
  if (list_mode) {
    const int n_list = min((int)sh.n_list, cap);
    // a bin holding exactly the keys still needed is taken whole
    while (shift > 0 && und != need) {
      const int s2 = shift - 10;
      __syncthreads();  // every thread has read und
      for (int i = tid; i < 1024; i += kTkThreads) sh.hist[i] = 0u;
      __syncthreads();
      for (int i = tid; i < n_list; i += kTkThreads) {
        const uint32_t k = lkey[i];
        if ((k >> shift) == prefix) atomicAdd(&sh.hist[(k >> s2) & 1023u], 1u);
      }
      __syncthreads();
      find_threshold_w0(sh, 1024, need, &T, &above);
      need -= above;
      prefix = (prefix << 10) | (uint32_t)T;
      shift = s2;
      und = sh.hist[T];
    }
    // keys above the final prefix are taken; those equal to it are the ties
    for (int i = tid; i < n_list; i += kTkThreads) {
      const uint32_t k = lkey[i] >> shift;
      const int p = lpos[i];
      if (k > prefix) atomicOr(&gtm[p >> 5], 1u << (p & 31));
      else if (k == prefix) atomicOr(&eqm[p >> 5], 1u << (p & 31));
    }
    __syncthreads();
  }
  // ---- output: positions ascending, the lowest `need` positions of the tau ties ----
  const uint32_t take_eq = need;
  const int nwu = (L + 31) >> 5;
  const int per = (nwu + kTkThreads - 1) / kTkThreads;
  const int w0 = tid * per, w1 = min(w0 + per, nwu);
  uint64_t cnt = 0;
  for (int w = w0; w < w1; w++)
    cnt += (uint64_t)__popc(gtm[w]) | ((uint64_t)__popc(eqm[w]) << 32);
  uint64_t tot;
  const uint64_t ex = block_excl_scan64(cnt, sh.wsum64, &tot);
  uint32_t g = (uint32_t)ex, e = (uint32_t)(ex >> 32);
  for (int w = w0; w < w1; w++) {
    const uint32_t gw = gtm[w], ew = eqm[w];
    uint32_t m = gw | ew;
    while (m != 0u) {
      const int bit = __ffs(m) - 1;
      m &= m - 1u;
      const int pos = (w << 5) + bit;
      if ((gw >> bit) & 1u) {
        // o < K always holds by construction; the bound keeps a logic error
        // from ever writing outside the row
        const uint32_t o = g + (e < take_eq ? e : take_eq);
        if (o < (uint32_t)K) out[o] = pos;
        g++;
      } else {
        if (e < take_eq && g + e < (uint32_t)K) out[g + e] = pos;
        e++;
      }
    }
  }
}

// LDS plan of topk_row2_kernel for a row width: bitmap words and list
// capacity.  Returns false when the bitmaps leave no room for a list of k
// entries (then the three-read kernel runs).
static bool topk_row2_plan(int64_t row_stride, int k, int* nw2, int* cap, size_t* smem) {
  constexpr size_t kLdsMax = 160 * 1024;
  constexpr size_t kLdsHalf = 80 * 1024;  // two workgroups per CU
  const int64_t words = 2 * ((row_stride + 63) / 64);
  const size_t fixed = (size_t)kTk2HeadBytes + (size_t)words * 2 * sizeof(uint32_t);
  // prefer two workgroups per CU when the list still holds 2k entries
  size_t budget = kLdsHalf;
  if (fixed + (size_t)2 * k * 8 > budget) budget = kLdsMax;
  if (fixed + (size_t)k * 8 > budget) return false;
  *nw2 = (int)words;
  *cap = (int)((budget - fixed) / 8);
  *smem = fixed + (size_t)(*cap) * 8;
  return true;
}

template <bool HAVE_HIST, bool V4>
static int launch_topk_row2_v(const float* score, int n_rows, int64_t row_stride,
                              const int32_t* seq_lens, const uint32_t* hist, int32_t* idx, int K,
                              int nw2, int cap, size_t smem, hipStream_t st) {
  auto kern = topk_row2_kernel<HAVE_HIST, V4>;
  const int rc = reserve_lds(reinterpret_cast<const void*>(kern), 160 * 1024, "topk row2");
  if (rc) return rc;
  kern<<<n_rows, kTkThreads, smem, st>>>(score, row_stride, seq_lens, hist, idx, K, nw2, cap);
  return check_launch("topk row2");
}

template <bool HAVE_HIST>
static int launch_topk_row2(const float* score, int n_rows, int64_t row_stride,
                            const int32_t* seq_lens, const uint32_t* hist, int32_t* idx, int K,
                            hipStream_t st) {
  int nw2 = 0, cap = 0;
  size_t smem = 0;
  if (!topk_row2_plan(row_stride, K, &nw2, &cap, &smem))
    return launch_topk<HAVE_HIST>(score, n_rows, row_stride, seq_lens, hist, idx, K, st);
  if (row_stride % 4 == 0 && aligned_to(score, 16))
    return launch_topk_row2_v<HAVE_HIST, true>(score, n_rows, row_stride, seq_lens, hist, idx, K,
                                               nw2, cap, smem, st);
  return launch_topk_row2_v<HAVE_HIST, false>(score, n_rows, row_stride, seq_lens, hist, idx, K,
                                              nw2, cap, smem, st);
}

// ===========================================================================
// Decode top-k from the indexer histogram, in two kernels (no inter-
// workgroup synchronisation):
//  * topk_scan_kernel, grid (tiles of 1024 positions, rows): every workgroup
//    derives the level-1 threshold bin T1 from the row's histogram (bins
//    above T1 hold fewer than K keys, bins >= T1 at least K), then writes
//    its candidates -- positions with bin >= T1 -- with their keys, in
//    position order, and their count.
//  * topk_select_kernel, one workgroup per row: the candidates (about K plus
//    the keys sharing bin T1) are gathered into LDS, the exact threshold key
//    among the T1 keys is found by a two-level radix select on their low 20
//    bits, and one packed scan over the candidates in position order writes
//    the K positions, ascending.
// A histogram that does not count exactly L keys, or a candidate set larger
// than kTkCandCap, falls back to the whole-row selection in the select
// kernel.  Workspace per row: 4 meta words, the tile counts and
// 1024 (key, position) candidate slots per tile.
// ===========================================================================
constexpr int kScanTile = 1024;
constexpr int kScanThreads = 256;
constexpr int kTkCandCap = 14336;
constexpr int kSelBins = 1024;

struct ScanShared {
  float v[kScanTile];
  uint32_t wsum[2 * (kScanThreads / 64)];
  int T;
};

struct TopkWs {
  int32_t* meta;     // [B][4]: T1, keys above T1, status (0 ok, 1 bad histogram)
  int32_t* counts;   // [B][n_tiles]
  uint32_t* ckey;    // [B][n_tiles][kScanTile]
  int32_t* cpos;     // [B][n_tiles][kScanTile]
};

__host__ __device__ inline TopkWs topk_ws(void* base, int B, int n_tiles) {
  TopkWs w;
  char* p = reinterpret_cast<char*>(base);
  w.meta = reinterpret_cast<int32_t*>(p);
  p += (size_t)B * 4 * sizeof(int32_t);
  w.counts = reinterpret_cast<int32_t*>(p);
  p += ((size_t)B * n_tiles * sizeof(int32_t) + 15) / 16 * 16;
  w.ckey = reinterpret_cast<uint32_t*>(p);
  p += (size_t)B * n_tiles * kScanTile * sizeof(uint32_t);
  w.cpos = reinterpret_cast<int32_t*>(p);
  return w;
}

static size_t topk_ws_bytes(int B, int n_tiles) {
  return (size_t)B * 4 * sizeof(int32_t) + ((size_t)B * n_tiles * sizeof(int32_t) + 15) / 16 * 16 +
         (size_t)B * n_tiles * kScanTile * (sizeof(uint32_t) + sizeof(int32_t));
}

__global__ void __launch_bounds__(kScanThreads) topk_scan_kernel(
    const float* __restrict__ score, int max_kv, const int32_t* __restrict__ seq_lens,
    const uint32_t* __restrict__ hist, int K, TopkWs ws) {
  __shared__ ScanShared sh;
  const int b = blockIdx.y, tile = blockIdx.x, n_tiles = gridDim.x;
  const int p0 = tile * kScanTile;
  int L = seq_lens[b];
  L = L < 0 ? 0 : (L > max_kv ? max_kv : L);
  if (L <= K) return;  // the select kernel takes every position
  int32_t* cnt = ws.counts + (int64_t)b * n_tiles + tile;
  if (p0 >= L) {
    if (threadIdx.x == 0) *cnt = 0;
    return;
  }
  // positions of the tile, coalesced, staged in LDS; the loads are
  // unconditional (clamped to L - 1, the value then dropped) so all four are
  // in flight at once rather than one wait each
  const float* row = score + (int64_t)b * max_kv;
  constexpr int kPer = kScanTile / kScanThreads;
  float sv[kPer];
#pragma unroll
  for (int e = 0; e < kPer; e++) sv[e] = row[min(p0 + e * kScanThreads + (int)threadIdx.x, L - 1)];
#pragma unroll
  for (int e = 0; e < kPer; e++) {
    const int p = p0 + e * kScanThreads + (int)threadIdx.x;
    sh.v[e * kScanThreads + threadIdx.x] = (p < L) ? sv[e] : 0.f;
  }
  // ---- T1 from the histogram: thread t owns bins [16t, 16t+16) ----
  const uint32_t* h = hist + (int64_t)b * kTopkBins;
  constexpr int PER = kTopkBins / kScanThreads;
  uint32_t hb[PER], cs = 0;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    hb[i] = h[PER * threadIdx.x + i];
    cs += hb[i];
  }
  if (threadIdx.x == 0) sh.T = -1;  // before the scan's barrier
  uint32_t total;
  const uint32_t excl = block_excl_scan1<kScanThreads>(cs, sh.wsum, 0, &total);
  if (total != (uint32_t)L) {  // the histogram does not count the row's L keys
    if (tile == 0 && threadIdx.x == 0) ws.meta[(int64_t)b * 4 + 2] = 1;
    return;
  }
  {
    uint32_t a = total - excl - cs;  // keys in bins above this thread's bins
    for (int i = PER - 1; i >= 0; i--) {
      if (a < (uint32_t)K && a + hb[i] >= (uint32_t)K) {
        sh.T = PER * threadIdx.x + i;
        if (tile == 0) {
          ws.meta[(int64_t)b * 4 + 0] = sh.T;
          ws.meta[(int64_t)b * 4 + 1] = (int)a;
          ws.meta[(int64_t)b * 4 + 2] = 0;
        }
      }
      a += hb[i];
    }
  }
  __syncthreads();
  const uint32_t T1 = (uint32_t)sh.T;
  // ---- candidates of 4 consecutive positions per thread, position order ----
  uint32_t key[4];
  uint32_t n = 0;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const int p = p0 + 4 * threadIdx.x + e;
    key[e] = mono_key(sh.v[4 * threadIdx.x + e]);
    const bool cand = p < L && (key[e] >> 20) >= T1;
    n += cand ? 1u : 0u;
  }
  uint32_t tot;
  uint32_t off = block_excl_scan1<kScanThreads>(n, sh.wsum, 1, &tot);
  const int64_t slot0 = ((int64_t)b * n_tiles + tile) * kScanTile;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const int p = p0 + 4 * threadIdx.x + e;
    if (p < L && (key[e] >> 20) >= T1) {
      ws.ckey[slot0 + off] = key[e];
      ws.cpos[slot0 + off] = p;
      off++;
    }
  }
  if (threadIdx.x == 0) *cnt = (int)tot;
}

struct SelShared {
  union {
    TopkShared full;
    struct {
      uint32_t ckey[kTkCandCap];
      int32_t cpos[kTkCandCap];
      uint32_t hist[kSelBins];
      int32_t toff[1024 + 1];
    } c;
  } u;
  uint32_t wsum[2 * kTkWaves];
  int T[2];
  uint32_t above[2];
  int n_cand;
};

// Bin T of an nbins (<= 1024) LDS histogram with above(T) < need <=
// above(T) + hist[T]; one bin per thread.  par: the parity of this block
// scan (block_excl_scan1); it also selects the broadcast slot, so two calls
// of one parity are separated by the barriers of the call between them.
__device__ void sel_threshold(SelShared& sh, const uint32_t* hist, int nbins, uint32_t need,
                              int par, int* T, uint32_t* above) {
  const uint32_t hv = (int)threadIdx.x < nbins ? hist[threadIdx.x] : 0u;
  uint32_t total;
  const uint32_t excl = block_excl_scan1<kTkThreads>(hv, sh.wsum, par, &total);
  const uint32_t a = total - excl - hv;  // keys in higher bins
  if ((int)threadIdx.x < nbins && a < need && a + hv >= need) {
    sh.T[par] = threadIdx.x;
    sh.above[par] = a;
  }
  __syncthreads();
  *T = sh.T[par];
  *above = sh.above[par];
}

template <int TILE, bool AGENT>
__device__ void topk_select_body(SelShared& sh, const float* __restrict__ row, int L, int K,
                                 int32_t* __restrict__ out, const uint32_t* hrow, int n_tiles,
                                 const TopkWs& ws, int b, int status, int T1, uint32_t above1,
                                 uint32_t cnt_own);

// Row b of the select (every return is workgroup-uniform).
__device__ __forceinline__ void topk_select_row(
    SelShared& sh, const float* __restrict__ score, int max_kv,
    const int32_t* __restrict__ seq_lens, const uint32_t* hist,
    int32_t* __restrict__ idx, int K, int n_tiles, const TopkWs& ws, int b) {
  int32_t* out = idx + (int64_t)b * K;
  // The row's length, its scan metadata and thread t's tile count (this
  // path has n_tiles <= 1024) do not depend on each other: they are loaded
  // together, one memory round trip, before any of them is tested.
  const uint32_t cnt_own =
      (uint32_t)ws.counts[(int64_t)b * n_tiles + min((int)threadIdx.x, n_tiles - 1)];
  const int status = ws.meta[(int64_t)b * 4 + 2];
  const uint32_t above1 = (uint32_t)ws.meta[(int64_t)b * 4 + 1];
  const int T1 = ws.meta[(int64_t)b * 4 + 0];
  int L = seq_lens[b];
  asm volatile("" ::"v"(cnt_own), "v"(status), "v"(above1), "v"(T1), "v"(L));
  L = L < 0 ? 0 : (L > max_kv ? max_kv : L);
  if (L <= K) {
    for (int p = threadIdx.x; p < K; p += kTkThreads) out[p] = (p < L) ? p : -1;
    return;
  }
  topk_select_body<kScanTile, false>(sh, score + (int64_t)b * max_kv, L, K, out,
                                     hist + (int64_t)b * kTopkBins, n_tiles, ws, b, status, T1,
                                     above1, cnt_own);
}

// Loads of the candidate lists and counts: agent-scope (coherent across
// XCDs) where the lists were written in the same launch.
template <bool AGENT, class T>
__device__ __forceinline__ T ws_load(const T* p) {
  if constexpr (AGENT)
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    return *p;
}

// The select of one row (L > K) from the level-1 threshold bin T1, the keys
// above it (above1) and the candidate lists of TILE-position tiles; cnt_own
// is thread t's tile count (t < used tiles).  status != 0: the histogram
// was inconsistent with L, and the row is selected whole.
template <int TILE, bool AGENT>
__device__ void topk_select_body(SelShared& sh, const float* __restrict__ row, int L, int K,
                                 int32_t* __restrict__ out, const uint32_t* hrow, int n_tiles,
                                 const TopkWs& ws, int b, int status, int T1, uint32_t above1,
                                 uint32_t cnt_own) {
  if (status != 0) {  // histogram inconsistent with L: rebuild from the row
    topk_row_select(sh.u.full, row, L, K, out, nullptr);
    return;
  }
  const int used_tiles = (L + TILE - 1) / TILE;  // <= n_tiles <= 1024
  // the second-level histogram starts zero (the scan's barrier orders this
  // before the gather's counts)
  for (int i = threadIdx.x; i < kSelBins; i += kTkThreads) sh.u.c.hist[i] = 0u;
  // ---- tile offsets of the candidate lists ----
  int total_c;
  {
    const int t = threadIdx.x;
    const uint32_t n = t < used_tiles ? cnt_own : 0u;
    uint32_t tot;
    const uint32_t ex = block_excl_scan1<kTkThreads>(n, sh.wsum, 0, &tot);
    if (t < used_tiles) sh.u.c.toff[t] = (int)ex;
    total_c = (int)tot;
  }
  if (total_c > kTkCandCap || used_tiles > 1024) {
    __syncthreads();
    topk_row_select(sh.u.full, row, L, K, out, hrow);
    return;
  }
  if (threadIdx.x == 0) sh.u.c.toff[used_tiles] = total_c;
  __syncthreads();
  // ---- gather the candidates into LDS (tile lists are position ordered);
  // the keys of bin T1 are counted by their next 10 bits on the way ----
  // Flat over the candidate index: candidate i lives in the tile t with
  // toff[t] <= i < toff[t+1] (binary search in LDS), so every thread's loads
  // are independent and kGatherU of them are in flight at once.
  constexpr int kGatherU = 4;
  for (int i0 = threadIdx.x; i0 < total_c; i0 += kGatherU * kTkThreads) {
    uint32_t kk[kGatherU];
    int32_t pp[kGatherU];
#pragma unroll
    for (int u = 0; u < kGatherU; u++) {
      const int i = i0 + u * kTkThreads;
      if (i < total_c) {
        int lo = 0, hi = used_tiles;  // invariant: toff[lo] <= i < toff[hi]
        while (hi - lo > 1) {
          const int mid = (lo + hi) >> 1;
          if (sh.u.c.toff[mid] <= i) lo = mid; else hi = mid;
        }
        const int64_t src = ((int64_t)b * n_tiles + lo) * TILE + (i - sh.u.c.toff[lo]);
        kk[u] = ws_load<AGENT>(ws.ckey + src);
        pp[u] = ws_load<AGENT>(ws.cpos + src);
      }
    }
#pragma unroll
    for (int u = 0; u < kGatherU; u++) {
      const int i = i0 + u * kTkThreads;
      if (i < total_c) {
        sh.u.c.ckey[i] = kk[u];
        sh.u.c.cpos[i] = pp[u];
        if ((int)(kk[u] >> 20) == T1) atomicAdd(&sh.u.c.hist[(kk[u] >> 10) & 1023], 1u);
      }
    }
  }
  __syncthreads();
  // ---- exact threshold among the T1 keys: bits [10,20), then [0,10) ----
  const uint32_t need1 = (uint32_t)K - above1;  // keys to take from bin T1
  int T2;
  uint32_t above2;
  sel_threshold(sh, sh.u.c.hist, kSelBins, need1, 1, &T2, &above2);
  const uint32_t need2 = need1 - above2;
  const uint32_t pre2 = ((uint32_t)T1 << 10) | (uint32_t)T2;  // top 22 bits
  // The T1 keys (a few hundred) spread over 1024 second-level bins, so bin T2
  // is usually taken whole: then the threshold is pre2 at 22-bit precision,
  // every key of that bin is taken and the third level is skipped.
  const bool whole = sh.u.c.hist[T2] == need2;
  uint32_t tau, take_eq;
  int sh_bits;  // keys compare as k >> sh_bits against tau
  int par = 0;  // parity of the compaction's block scan
  if (whole) {
    tau = pre2;
    take_eq = need2;
    sh_bits = 10;
  } else {
    __syncthreads();  // every thread has read hist[T2]
    for (int i = threadIdx.x; i < kSelBins; i += kTkThreads) sh.u.c.hist[i] = 0u;
    __syncthreads();
    for (int i = threadIdx.x; i < total_c; i += kTkThreads) {
      const uint32_t k = sh.u.c.ckey[i];
      if ((k >> 10) == pre2) atomicAdd(&sh.u.c.hist[k & 1023], 1u);
    }
    __syncthreads();
    int T3;
    uint32_t above3;
    sel_threshold(sh, sh.u.c.hist, kSelBins, need2, 0, &T3, &above3);
    par = 1;
    tau = (pre2 << 10) | (uint32_t)T3;
    take_eq = need2 - above3;  // keys equal to tau to take, lowest positions
    sh_bits = 0;
  }
  // ---- ordered compaction over the candidates: packed (gt | eq << 16) scan ----
  const int per = (total_c + kTkThreads - 1) / kTkThreads;
  const int i0 = threadIdx.x * per, i1 = min(i0 + per, total_c);
  uint32_t packed = 0;
  for (int i = i0; i < i1; i++) {
    const uint32_t k = sh.u.c.ckey[i] >> sh_bits;
    packed += (k > tau ? 1u : 0u) + (k == tau ? (1u << 16) : 0u);
  }
  uint32_t tot;
  const uint32_t ex = block_excl_scan1<kTkThreads>(packed, sh.wsum, par, &tot);
  uint32_t gt = ex & 0xFFFFu, eq = ex >> 16;
  for (int i = i0; i < i1; i++) {
    const uint32_t k = sh.u.c.ckey[i] >> sh_bits;
    if (k > tau) {
      const uint32_t o = gt + (eq < take_eq ? eq : take_eq);
      if (o < (uint32_t)K) out[o] = sh.u.c.cpos[i];
      gt++;
    } else if (k == tau) {
      if (eq < take_eq) {
        const uint32_t o = gt + eq;
        if (o < (uint32_t)K) out[o] = sh.u.c.cpos[i];
      }
      eq++;
    }
  }
}


__global__ void __launch_bounds__(256) zero_u32x4_kernel(u32x4* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = (u32x4){0u, 0u, 0u, 0u};
}

// A decode layer step's q_nope -> latent projection, run beside the select:
// workgroups n_rows.. of the launch each take four 256-thread blocks of the
// decode-shaped projection (head_proj_block<4, 1>, which has no barrier).
// The select's B workgroups leave the rest of the chip idle.
struct SelProj {
  HpArgs hp;
  int gx;   // projection blocks per token chunk
  int wgs;  // projection blocks
};

// clear_hist (null or the histogram itself): the consuming variant, which
// leaves the row's histogram zero for the next step's logits launch once the
// row is selected.  PROJ: workgroups from n_rows on run the projection.
template <bool PROJ>
__global__ void __launch_bounds__(kTkThreads) topk_select_kernel(
    const float* __restrict__ score, int max_kv, const int32_t* __restrict__ seq_lens,
    const uint32_t* hist, int32_t* __restrict__ idx, int K, int n_tiles, TopkWs ws,
    uint32_t* clear_hist, int n_rows, SelProj proj) {
  if constexpr (PROJ) {
    if ((int)blockIdx.x >= n_rows) {
      const int vb = ((int)blockIdx.x - n_rows) * 4 + (int)(threadIdx.x >> 8);
      if (vb < proj.wgs) head_proj_block<4, 1>(proj.hp, vb % proj.gx, vb / proj.gx, threadIdx.x & 255);
      return;
    }
  }
  extern __shared__ __align__(16) unsigned char smem_raw[];
  SelShared& sh = *reinterpret_cast<SelShared*>(smem_raw);
  const int b = blockIdx.x;
  topk_select_row(sh, score, max_kv, seq_lens, hist, idx, K, n_tiles, ws, b);
  if (clear_hist != nullptr) {
    __syncthreads();  // every read of the row's histogram is done
    u32x4* h = reinterpret_cast<u32x4*>(clear_hist + (int64_t)b * kTopkBins);
    for (int i = threadIdx.x; i < kTopkBins / 4; i += kTkThreads) h[i] = (u32x4){0u, 0u, 0u, 0u};
  }
}

// ===========================================================================
// Decode top-k in one launch, for calls whose scan is one round of
// workgroups (rows x groups <= 256, one workgroup per CU).  Workgroup (b, g)
// of 1024 threads scans positions [4096 g, 4096 g + 4096) of row b as
// topk_scan_kernel does -- T1 from the row's histogram, then the keys of bin
// >= T1 in position order -- and writes its list and count with agent-scope
// stores (written through the XCD's L2 to memory).  After s_waitcnt
// vmcnt(0) -- every such store acknowledged -- it counts itself in on the
// row's arrival counter (one device atomic add); the workgroup that
// completes the count resets the counter to zero and selects the row
// (topk_select_body), reading the lists with agent-scope loads, which do
// not take stale lines from its own L2.  No workgroup waits on another.
// The counters come from the library's pool (arrive_slot); when it is
// spent, calls take the two-kernel path.
// ===========================================================================
constexpr int kFTile = 4 * kTkThreads;  // positions per workgroup
constexpr int kFusedMaxWgs = 256;

struct FusedShared {
  SelShared sel;
  uint32_t wsum[2 * kTkWaves];
  int T1;
  uint32_t above1;
  int last;
};

template <bool PROJ>
__global__ void __launch_bounds__(kTkThreads) topk_fused_kernel(
    const float* __restrict__ score, int max_kv, const int32_t* __restrict__ seq_lens,
    const uint32_t* hist, int32_t* __restrict__ idx, int K, int n_groups, TopkWs ws,
    uint32_t* arrive, uint32_t* clear_hist, int n_rows, SelProj proj) {
  const int id = blockIdx.x;
  if constexpr (PROJ) {
    if (id >= n_rows * n_groups) {
      const int vb = (id - n_rows * n_groups) * 4 + (int)(threadIdx.x >> 8);
      if (vb < proj.wgs) head_proj_block<4, 1>(proj.hp, vb % proj.gx, vb / proj.gx, threadIdx.x & 255);
      return;
    }
  }
  extern __shared__ __align__(16) unsigned char smem_raw[];
  FusedShared& sh = *reinterpret_cast<FusedShared*>(smem_raw);
  const int tid = threadIdx.x;
  const int b = id / n_groups, g = id - b * n_groups;
  int32_t* out = idx + (int64_t)b * K;
  const float* row = score + (int64_t)b * max_kv;
  const uint32_t* hrow = hist + (int64_t)b * kTopkBins;
  int L = seq_lens[b];
  L = L < 0 ? 0 : (L > max_kv ? max_kv : L);
  if (L <= K) {  // every position, -1 padded: workgroup 0 of the row
    if (g == 0) {
      for (int p = tid; p < K; p += kTkThreads) out[p] = (p < L) ? p : -1;
      if (clear_hist != nullptr) {
        u32x4* h = reinterpret_cast<u32x4*>(clear_hist + (int64_t)b * kTopkBins);
        for (int i = tid; i < kTopkBins / 4; i += kTkThreads) h[i] = (u32x4){0u, 0u, 0u, 0u};
      }
    }
    return;
  }
  const int ng = (L + kFTile - 1) / kFTile;  // the row's workgroups
  if (g >= ng) return;
  // ---- scan: thread t's 4 positions and 4 histogram bins, loaded together ----
  const int p0 = g * kFTile + 4 * tid;
  float v[4];
  uint32_t hb[4], cs = 0;
#pragma unroll
  for (int e = 0; e < 4; e++) v[e] = row[min(p0 + e, L - 1)];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    hb[i] = hrow[4 * tid + i];
    cs += hb[i];
  }
  uint32_t total;
  const uint32_t excl = block_excl_scan1<kTkThreads>(cs, sh.wsum, 0, &total);
  const bool bad = total != (uint32_t)L;  // the histogram does not count the row's L keys
  if (!bad) {
    uint32_t a = total - excl - cs;  // keys in bins above this thread's bins
#pragma unroll
    for (int i = 3; i >= 0; i--) {
      if (a < (uint32_t)K && a + hb[i] >= (uint32_t)K) {
        sh.T1 = 4 * tid + i;
        sh.above1 = a;
      }
      a += hb[i];
    }
  }
  __syncthreads();
  const int T1 = bad ? 0 : sh.T1;
  const uint32_t above1 = bad ? 0u : sh.above1;
  if (!bad) {  // the candidates, in position order
    uint32_t key[4], n = 0;
    bool cand[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      key[e] = mono_key(v[e]);
      cand[e] = p0 + e < L && (int)(key[e] >> 20) >= T1;
      n += cand[e] ? 1u : 0u;
    }
    uint32_t tot;
    uint32_t off = block_excl_scan1<kTkThreads>(n, sh.wsum, 1, &tot);
    const int64_t slot0 = ((int64_t)b * n_groups + g) * kFTile;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      if (cand[e]) {
        __hip_atomic_store(ws.ckey + slot0 + off, key[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(ws.cpos + slot0 + off, p0 + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        off++;
      }
    }
    if (tid == 0)
      __hip_atomic_store(ws.counts + (int64_t)b * n_groups + g, (int32_t)tot, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  // ---- arrival: every wave's list stores are complete before the count moves ----
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const uint32_t before =
        __hip_atomic_fetch_add(arrive + b, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = before + 1u == (uint32_t)ng;
    if (last) __hip_atomic_store(arrive + b, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sh.last = last ? 1 : 0;
  }
  __syncthreads();
  if (sh.last == 0) return;
  // ---- the row's select, by the workgroup that completed the count ----
  const uint32_t cnt_own = (uint32_t)ws_load<true>(ws.counts + (int64_t)b * n_groups +
                                                   min(tid, n_groups - 1));
  topk_select_body<kFTile, true>(sh.sel, row, L, K, out, hrow, n_groups, ws, b, bad ? 1 : 0, T1,
                                 above1, cnt_own);
  if (clear_hist != nullptr) {
    __syncthreads();  // every read of the row's histogram is done
    u32x4* h = reinterpret_cast<u32x4*>(clear_hist + (int64_t)b * kTopkBins);
    for (int i = tid; i < kTopkBins / 4; i += kTkThreads) h[i] = (u32x4){0u, 0u, 0u, 0u};
  }
}

}  // namespace mi355dsa

using namespace mi355dsa;

// Rows per call up to which the two-kernel path is used: it needs fewer
// launches' worth of parallelism than one workgroup per row provides.
constexpr int kTwoKernelMaxRows = 64;
static_assert(kArriveRows >= kTwoKernelMaxRows, "an arrival slot covers every row of a call");

static bool two_kernel_topk(int B, int max_kv, int k) {
  return B <= kTwoKernelMaxRows && max_kv > k && (max_kv + kScanTile - 1) / kScanTile <= 1024;
}

// The one-launch path: the scan is at most one round of workgroups.
static bool fused_topk(int B, int max_kv, int k) {
  return two_kernel_topk(B, max_kv, k) &&
         (int64_t)B * ((max_kv + kFTile - 1) / kFTile) <= kFusedMaxWgs;
}

// One-launch workspace: the group counts, then the 4096 (key, position)
// candidate slots per group.
static size_t fused_ws_bytes(int B, int ng) {
  return ((size_t)B * ng * sizeof(int32_t) + 15) / 16 * 16 +
         (size_t)B * ng * kFTile * (sizeof(uint32_t) + sizeof(int32_t));
}

static void fused_ws(void* base, int B, int ng, TopkWs* ws) {
  char* p = reinterpret_cast<char*>(base);
  ws->meta = nullptr;
  ws->counts = reinterpret_cast<int32_t*>(p);
  p += ((size_t)B * ng * sizeof(int32_t) + 15) / 16 * 16;
  ws->ckey = reinterpret_cast<uint32_t*>(p);
  p += (size_t)B * ng * kFTile * sizeof(uint32_t);
  ws->cpos = reinterpret_cast<int32_t*>(p);
}

extern "C" size_t mi355_dsa_decode_topk_workspace_size(int B, int max_kv, int k) {
  if (B <= 0 || max_kv <= 0 || !two_kernel_topk(B, max_kv, k)) return 0;
  const size_t two = topk_ws_bytes(B, (max_kv + kScanTile - 1) / kScanTile);
  if (!fused_topk(B, max_kv, k)) return two;
  // the one-launch layout, or the two-kernel one should the arrival pool be spent
  const size_t one = fused_ws_bytes(B, (max_kv + kFTile - 1) / kFTile);
  return one > two ? one : two;
}

// Shared by mi355_dsa_decode_topk and the layer step's variant.  clear: the
// histogram is left zero.  proj (non-null): the projection runs inside the
// select launch when the two-kernel path is taken (*proj_done set).
static int decode_topk_impl(int32_t* idx, const float* score, const int32_t* seq_lens,
                            int32_t* hist, int B, int max_kv, int k, void* workspace,
                            size_t workspace_bytes, bool clear, const SelProj* proj,
                            bool* proj_done, void* stream) {
  if (proj_done) *proj_done = false;
  DSA_CHECK(k >= 1, "k must be >= 1");
  DSA_CHECK(B >= 0 && max_kv >= 0, "B and max_kv must be >= 0");
  DSA_CHECK(k <= (1 << 16) - 1, "k too large");
  if (B == 0) return MI355_DSA_OK;
  DSA_CHECK(idx && score && seq_lens && hist, "null pointer argument");
  DSA_CHECK(!clear || aligned_to(hist, 16), "hist must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
  uint32_t* h = reinterpret_cast<uint32_t*>(hist);
  uint32_t* arrive = nullptr;
  if (fused_topk(B, max_kv, k)) arrive = arrive_slot(st);
  if (arrive != nullptr) {
    const int ng = (max_kv + kFTile - 1) / kFTile;
    const size_t need = fused_ws_bytes(B, ng);
    DSA_CHECK(workspace && workspace_bytes >= need,
              "workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    DSA_CHECK(aligned_to(workspace, 16), "workspace must be 16-byte aligned");
    TopkWs ws;
    fused_ws(workspace, B, ng, &ws);
    uint32_t* ch = clear ? h : nullptr;
    int rc;
    if (proj != nullptr) {
      rc = reserve_lds(reinterpret_cast<const void*>(topk_fused_kernel<true>), sizeof(FusedShared),
                       "decode_topk");
      if (rc) return rc;
      const int64_t grid = (int64_t)B * ng + (proj->wgs + 3) / 4;
      DSA_CHECK(grid < ((int64_t)1 << 31), "decode_topk: grid too large");
      topk_fused_kernel<true><<<(unsigned)grid, kTkThreads, sizeof(FusedShared), st>>>(
          score, max_kv, seq_lens, h, idx, k, ng, ws, arrive, ch, B, *proj);
      if (proj_done) *proj_done = true;
    } else {
      rc = reserve_lds(reinterpret_cast<const void*>(topk_fused_kernel<false>), sizeof(FusedShared),
                       "decode_topk");
      if (rc) return rc;
      topk_fused_kernel<false><<<(unsigned)(B * ng), kTkThreads, sizeof(FusedShared), st>>>(
          score, max_kv, seq_lens, h, idx, k, ng, ws, arrive, ch, B, SelProj{});
    }
    return check_launch("decode_topk fused");
  }
  if (two_kernel_topk(B, max_kv, k)) {
    const int n_tiles = (max_kv + kScanTile - 1) / kScanTile;
    const size_t need = topk_ws_bytes(B, n_tiles);
    DSA_CHECK(workspace && workspace_bytes >= need,
              "workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    DSA_CHECK(aligned_to(workspace, 16), "workspace must be 16-byte aligned");
    const TopkWs ws = topk_ws(workspace, B, n_tiles);
    topk_scan_kernel<<<dim3(n_tiles, B), kScanThreads, 0, st>>>(score, max_kv, seq_lens, h, k, ws);
    int rc = check_launch("decode_topk scan");
    if (rc) return rc;
    uint32_t* ch = clear ? h : nullptr;
    if (proj != nullptr) {
      rc = reserve_lds(reinterpret_cast<const void*>(topk_select_kernel<true>), sizeof(SelShared),
                       "decode_topk");
      if (rc) return rc;
      const int grid = B + (proj->wgs + 3) / 4;
      topk_select_kernel<true><<<grid, kTkThreads, sizeof(SelShared), st>>>(
          score, max_kv, seq_lens, h, idx, k, n_tiles, ws, ch, B, *proj);
      if (proj_done) *proj_done = true;
    } else {
      rc = reserve_lds(reinterpret_cast<const void*>(topk_select_kernel<false>), sizeof(SelShared),
                       "decode_topk");
      if (rc) return rc;
      topk_select_kernel<false><<<B, kTkThreads, sizeof(SelShared), st>>>(
          score, max_kv, seq_lens, h, idx, k, n_tiles, ws, ch, B, SelProj{});
    }
    return check_launch("decode_topk select");
  }
  int rc = launch_topk_row2<true>(score, B, max_kv, seq_lens, h, idx, k, st);
  if (rc || !clear) return rc;
  const int64_t n_vec = (int64_t)B * kTopkBins / 4;
  zero_u32x4_kernel<<<dim3((unsigned)((n_vec + 255) / 256)), 256, 0, st>>>(
      reinterpret_cast<u32x4*>(hist), n_vec);
  return check_launch("decode_topk clear");
}

extern "C" int mi355_dsa_decode_topk(int32_t* idx, const float* score,
                                     const int32_t* seq_lens, const int32_t* hist,
                                     int B, int max_kv, int k, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  clear_error();
  return decode_topk_impl(idx, score, seq_lens, const_cast<int32_t*>(hist), B, max_kv, k,
                          workspace, workspace_bytes, false, nullptr, nullptr, stream);
}

extern "C" int mi355_dsa_decode_layer_topk(
    int32_t* idx, const float* score, const int32_t* seq_lens, int32_t* hist, int B, int max_kv,
    int k, void* workspace, size_t workspace_bytes, void* q_lat, int64_t ql_tok_stride,
    int64_t ql_head_stride, const void* q, int64_t q_tok_stride, int64_t q_head_stride,
    const void* wt_uk, int T, int H, int N, int K, int tail, void* stream) {
  clear_error();
  SelProj proj{};
  int kw = 0;
  int64_t wgs = 0;
  int rc = hp_decode_setup(proj.hp, kw, proj.gx, wgs, "decode_layer_topk", q_lat, ql_tok_stride,
                           ql_head_stride, q, q_tok_stride, q_head_stride, wt_uk, T, H, N, K,
                           tail);
  if (rc) return rc;
  DSA_CHECK(wgs < ((int64_t)1 << 30), "decode_layer_topk: projection grid too large");
  proj.wgs = (int)wgs;
  bool done = false;
  rc = decode_topk_impl(idx, score, seq_lens, hist, B, max_kv, k, workspace, workspace_bytes,
                        true, kw == 1 ? &proj : nullptr, &done, stream);
  if (rc || done) return rc;
  // the projection as its own launch (whole-row top-k path, or K >= 256)
  return mi355_dsa_head_proj(q_lat, ql_tok_stride, ql_head_stride, q, q_tok_stride,
                             q_head_stride, wt_uk, T, H, N, K, tail, stream);
}

extern "C" size_t mi355_dsa_persistent_topk_workspace_size(int n_rows, int row_stride,
                                                           int k) {
  (void)n_rows;
  (void)row_stride;
  (void)k;
  return 0;
}

extern "C" int mi355_dsa_persistent_topk(const float* score, int n_rows, int row_stride,
                                         const int32_t* seq_lens, int32_t* idx, int k,
                                         int max_seq_len, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  clear_error();
  (void)workspace;
  (void)workspace_bytes;
  DSA_CHECK(k >= 1, "k must be >= 1");
  DSA_CHECK(k <= (1 << 16) - 1, "k too large");
  DSA_CHECK(n_rows >= 0 && row_stride >= 0, "n_rows and row_stride must be >= 0");
  DSA_CHECK(max_seq_len >= 0, "max_seq_len must be >= 0");
  if (n_rows == 0) return MI355_DSA_OK;
  DSA_CHECK(idx && score && seq_lens, "null pointer argument");
  return launch_topk_row2<false>(score, n_rows, row_stride, seq_lens, nullptr, idx, k,
                                 as_stream(stream));
}
