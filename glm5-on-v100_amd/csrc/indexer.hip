// DSA lightning-indexer logits on gfx950 MFMA.
//
//   score[b,p] = sum_{h<32} relu(q[b,h,:] . K[row(b,p),:]) * w[b,h]
//
// Two kernels, one per reference entry point:
//  * indexer_logits_kernel  -- mi355_dsa_indexer_logits (decode and generic
//    path; reference sm70_indexer_logits, csrc/attention/sm70_mla_decode.cu:
//    150-329 / host :2626-2764).  HBM-bound scan: a wave scores 16 keys per
//    MFMA group (S = Q . K^T, M = 16 heads x 2 tiles, N = 16 keys, K = 128),
//    keys are loaded straight from HBM into B-operand registers (no LDS),
//    double buffered.  The fused top-k histogram is built in LDS and flushed
//    once per workgroup (nonzero bins only).
//  * indexer_logits_packed_kernel -- mi355_dsa_indexer_logits_packed
//    (prefill; reference sm70_indexer_logits_packed, :542-653 / :2771-2836).
//    MFMA-bound: a 512-thread workgroup owns 64 queries x 256 keys; each wave
//    keeps 64 keys resident in A-operand registers for all 32 heads and
//    scores them against 32 of the queries, whose packed Q streams through
//    an LDS ring filled by LDS-DMA; the relu * w head-sum stays in registers.
//
// fp8 (132-byte) indexer rows: the decode kernel multiplies the exact
// e4m3 dot by the row scale before the relu (reference :309-313); the packed
// kernel dequantises keys to fp16 first (reference idxk_fp8_load4 + half
// store, :567-583).
#include <float.h>

#include "capi_internal.h"
#include "dsa_common.h"
#include "indexer_decode.h"

namespace mi355dsa {

// ===========================================================================
// decode / generic kernel: the workgroup body is indexer_logits_block
// (indexer_decode.h), shared with the fused decode-layer launch.
// A workgroup of 4 waves owns 1024 positions of one token row; a wave scores
// 16 keys per MFMA group (S = Q . K^T, M = 16 heads x 2 tiles, N = 16 keys,
// K = 128), keys loaded straight from HBM into B-operand registers (no LDS),
// double buffered.
// ===========================================================================
template <bool KFP8>
__global__ void __launch_bounds__(kIdxWaves * 64) indexer_logits_kernel(
    const f16* __restrict__ Q, const void* __restrict__ Kv, const f16* __restrict__ W,
    const int32_t* __restrict__ block_table, const int32_t* __restrict__ seq_lens,
    float* __restrict__ score, uint32_t* __restrict__ hist, int64_t n_kv_rows, int max_blocks,
    int page_shift, int max_kv, int hist8, int span) {
  const IdxDecArgs a{Q, Kv, W, block_table, seq_lens, score, hist, n_kv_rows, max_blocks,
                     page_shift, max_kv, hist8, span};
  const IdxNewKeys none{};
  indexer_logits_block<KFP8, false>(a, blockIdx.x, blockIdx.y, none);
}

// ===========================================================================
// packed (prefill) kernel
//
// Full tile = 64 queries (4 x 16) x 256 keys, 8 waves.  The tile balances
// two limits: it is small enough that the caller's 128-row sub-chunks launch
// ~256 workgroups at average causal reach, and wide enough in keys (256 FLOP
// per byte of streamed Q) that the L2 -> CU stream of Q stays below what one
// CU can ingest.
//
// Wave w owns keys [64 (w & 3), +64) and QB query blocks of 16 (QB = 2 in a
// full tile): its 64 keys (4 blocks x 128 dims, fp16) stay resident as MFMA
// A operands for all 32 heads, and per head it reads only its queries' Q
// from LDS.  The packed Q of each head (16 KB for 64 queries, contiguous in
// the packed layout) streams through an 8-slot LDS ring filled by LDS-DMA
// three head pairs ahead, the DMA rounds spread over the MFMA steps.
// relu(S) * w is summed over heads in registers, the epilogue of head h - 1
// interleaved with the MFMAs of head h.
//
// A launch holds W full tiles.  A workgroup takes one full tile, or half of
// one (QB = 1: 32 queries x 256 keys, same per-wave key set and the same
// MFMA : LDS-read ratio, half the MFMAs): when W <= 128 every tile is split
// in two so that the launch fills more CUs, and when W > 256 the last
// W mod 256 tiles (if at most 128) are split so that the final partial round
// of workgroups takes half as long.  Full tiles come first in launch order.
// ===========================================================================
constexpr int kPkWaves = 8;
constexpr int kPkThreads = kPkWaves * 64;
constexpr int kPkKT = 256;                 // keys per workgroup
constexpr int kPkWaveKeys = 64;            // keys per wave (4 blocks of 16)
constexpr int kPkRing = 8;                 // Q ring slots (heads): 4 pairs
constexpr int kPkSlot = 4 * 2048;          // halves per ring slot (one head, 64 queries)
constexpr int kPkMaxQT = 64;               // queries of a full tile
constexpr int kPkHalfMax = 128;            // at most this many tiles are split per launch
constexpr int kPkCUs = 256;                // workgroups of one full round (one per CU)

__device__ const __align__(16) f16 kIdxZeroPiece[8] = {};  // source of unmapped key rows

// LDS of a workgroup whose tiles hold at most QTMAX queries: the Q ring
// (one head of QTMAX queries per slot), the head weights, the causal lengths
// (64 entries: wave 0 writes one per lane).
template <int QTMAX>
struct PkSmemT {
  f16 q[kPkRing][QTMAX * kIdxHeadDim];
  float w[kIdxHeads][QTMAX];
  int32_t sl[64];
  int maxsl;
};
using PkSmem = PkSmemT<kPkMaxQT>;
static_assert(kPkMaxQT * kIdxHeadDim == kPkSlot, "ring slot = one head of a full tile");

// relu in one instruction (v_med3_f32 clamp to [0, FLT_MAX]; fmaxf would
// first canonicalise its input under IEEE mode)
__device__ __forceinline__ float relu1(float x) { return __builtin_amdgcn_fmed3f(x, 0.f, FLT_MAX); }

// at most k head pairs of Q (R LDS-DMA rounds per head) still in flight
template <int R>
__device__ __forceinline__ void pk_wait(int k) {
  switch (k) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * R) : "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * R) : "memory"); break;
  }
}

struct PkArgs {
  const f16* Qp;
  const void* Kv;
  const f16* W;
  const int32_t* block_table;
  const int32_t* seq_lens;
  float* score;
  int B;
  int64_t n_kv_rows;
  int max_blocks, page_shift, max_kv;
  int n_kt;    // key tiles per query tile
  int n_full;  // workgroups that take a whole tile
};

// One workgroup tile of NW waves: queries [q_base, q_base + QT) x keys
// [p_base, +256).  HS = 1: QT = 16 QB NW / 4 (wave w: keys 64 (w & 3), query
// blocks QB (w >> 2) .. +QB, all 32 heads).  HS = 2 (NW = 8, small launches):
// QT = 16 QB, and wave w takes keys 64 (w & 3) of every query for heads
// [16 (w >> 2), +16), so that each wave's head loop is half as long; ring
// slot h then holds heads h and h + 16, and the two halves' relu * w sums
// are added through LDS at the end (head sum = heads 0-15, then + heads
// 16-31).
template <bool KFP8, int QB, int NW, int HS, typename SM>
__device__ __forceinline__ void pk_tile(const PkArgs& a, SM& sh, int q_base, int p_base) {
  static_assert(HS == 1 || (HS == 2 && NW == 8), "head split: 8 waves");
  constexpr int NT = 64 * NW;
  constexpr int QT = 16 * QB * (NW / 4 / HS);     // queries of the tile
  constexpr int NHP = kIdxHeads / 2 / HS;         // head pairs per wave
  constexpr int QROUNDS = HS * QT * 256 / 16 / NT;  // LDS-DMA ops per thread per ring slot
  constexpr int SLOT = sizeof(sh.q[0]) / sizeof(f16);
  // fp16 key rows (64 KB) are staged in ring slots KSLOT0 .. : slots 2..5 of
  // 16 KB slots (slots 0, 1 stay free for the first head pair), or the whole
  // ring of 8 KB slots
  constexpr int KSLOT0 = SLOT * 2 >= 16384 ? 2 : 0;
  static_assert(HS * QT * kIdxHeadDim <= SLOT, "ring slot too small for the tile");
  static_assert((kPkRing - KSLOT0) * SLOT * 2 >= kPkKT * kIdxHeadDim * 2, "keys do not fit the ring");
  const f16* __restrict__ Qp = a.Qp;
  const int B = a.B, max_kv = a.max_kv, page_shift = a.page_shift, max_blocks = a.max_blocks;
  const int n_qt = (B + 15) >> 4;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int half = HS == 1 ? wave >> 2 : 0;  // query-block group
  const int hh = HS == 1 ? 0 : wave >> 2;    // head half (HS = 2)
  const int hoff = (kIdxHeads / HS) * hh;    // its first head
  const int c = lane & 15, g = lane >> 4;

  // Q ring: head h of the tile's 2 QB query tiles [qt0, qt0 + 2 QB) is
  // contiguous in the packed layout ([kt 8][row 16][dims 16] per tile);
  // tiles past the last one read tile 0 (their score columns are never
  // written).  In LDS the 16-byte pieces are reordered to the MFMA B-operand
  // order: unit (tile, step st, lane c + 16g) holds row c, dims 32st + 8g ..
  // +8, so that each B read of a wave is 1 KB contiguous (no bank
  // conflicts).  The 64 pieces of one DMA instruction still come from 1 KB
  // of global memory.  Round u of a head moves query tiles qt0 + 2u and
  // qt0 + 2u + 1.
  const int qt0 = q_base >> 4;
  const bool qfull = qt0 + QT / 16 <= n_qt;
  auto issue_q_round = [&](int h, int u) {
    const int i = threadIdx.x + u * NT;  // LDS 16-byte unit
    // HS = 2: units [0, 16 QT) hold head h, [16 QT, 32 QT) head h + 16
    const int hsel = HS == 1 ? 0 : i / (16 * QT);
    const int ii = i - 16 * QT * hsel;
    const int qt = qt0 + (ii >> 8);              // 256 units per tile
    const int st = (ii >> 6) & 3, gg = (ii >> 4) & 3, cc = ii & 15;
    const int piece = (2 * st + (gg >> 1)) * 32 + cc * 2 + (gg & 1);
    const int hq = h + (kIdxHeads / HS) * hsel;
    const int64_t src = ((int64_t)hq * n_qt + ((qfull || qt < n_qt) ? qt : 0)) * 2048 + piece * 8;
    dma16(Qp + src, &sh.q[h % kPkRing][(u * NT + 64 * wave) * 8]);
  };
  auto issue_q = [&](int h) {
#pragma unroll
    for (int u = 0; u < QROUNDS; u++) issue_q_round(h, u);
  };
  constexpr int kAhead = kPkRing / 2 - 1;  // head pairs issued ahead

  // ---- prologue ----
  // fp16 keys: the tile's 256 key rows (64 KB) are copied by LDS-DMA into
  // ring slots 2..5 before any Q is requested, each 256-B row stored with
  // its 16-byte pieces XOR-swizzled by the key's low 4 bits so that the
  // A-operand reads below are free of bank conflicts; the first head pair
  // follows, and pairs 1 and 2 go out once every wave has its keys in
  // registers.  fp8 keys are converted on the way to registers instead.
  // Keys are gathered with the block-table row of the tile's first query
  // (all rows of a call share one table).
  const int key0 = p_base + kPkWaveKeys * (wave & 3);  // this wave's 64 keys
  const int qb0 = QB * half;                           // its first query block
  const int32_t* bt_row = a.block_table + (int64_t)q_base * max_blocks;
  const int page = 1 << page_shift;
  constexpr int kKRounds = kPkKT * kIdxHeadDim * 2 / 16 / NT;  // 8
  int32_t kbt[KFP8 ? 4 : kKRounds];
  if constexpr (!KFP8) {
#pragma unroll
    for (int u = 0; u < kKRounds; u++) {
      const int p = p_base + ((threadIdx.x + u * NT) >> 4);
      const int pg = p >> page_shift;
      kbt[u] = (p < max_kv && pg < max_blocks) ? bt_row[pg] : -1;
    }
  } else {
    for (int h = 0; h < 2 * kAhead; h++) issue_q(h);
#pragma unroll
    for (int kb = 0; kb < 4; kb++) {
      const int p = key0 + 16 * kb + c;
      const int pg = p >> page_shift;
      kbt[kb] = (p < max_kv && pg < max_blocks) ? bt_row[pg] : -1;
    }
  }
  // Causal lengths and head weights: loaded unconditionally from clamped
  // query indices (queries past B are zeroed where the values reach LDS),
  // so the loads are in flight together and do not hold up the key DMAs
  // below behind one wait each.
  const int sl_raw = a.seq_lens[min(q_base + (int)(threadIdx.x & 63), B - 1)];  // wave 0's lanes
  constexpr int WPT = kIdxHeads * QT / NT;
  f16 wv[WPT];
#pragma unroll
  for (int u = 0; u < WPT; u++) {
    const int i = threadIdx.x + u * NT;
    const int h = i / QT, q = q_base + i % QT;
    wv[u] = a.W[(int64_t)min(q, B - 1) * kIdxHeads + h];
  }
  // A operands: this wave's keys (4 blocks of 16), dims 32s + 8g .. +8 for
  // the 4 x32 steps.
  f16x8 ka[4][4];
  f16* const kl = sh.q[KSLOT0];  // fp16 key rows
  if constexpr (!KFP8) {
#pragma unroll
    for (int u = 0; u < kKRounds; u++) {
      const int i = threadIdx.x + u * NT;  // LDS 16-byte unit
      const int key = i >> 4;
      const int p = p_base + key;
      const int64_t r = ((int64_t)kbt[u] << page_shift) + (p & (page - 1));
      const f16* src = (kbt[u] >= 0 && r < a.n_kv_rows)
                           ? reinterpret_cast<const f16*>(a.Kv) + r * kIdxHeadDim +
                                 (((i & 15) ^ (key & 15)) << 3)
                           : kIdxZeroPiece;
      dma16(src, &kl[(u * NT + 64 * wave) * 8]);
    }
    if constexpr (KSLOT0 > 0) {
      issue_q(0);
      issue_q(1);
    }
  } else {
#pragma unroll
    for (int kb = 0; kb < 4; kb++) {
      const int p = key0 + 16 * kb + c;
      const int64_t r = ((int64_t)kbt[kb] << page_shift) + (p & (page - 1));
      const int64_t row = (kbt[kb] >= 0 && r < a.n_kv_rows) ? r : -1;
#pragma unroll
      for (int s = 0; s < 4; s++) {
        if (row < 0) {
          ka[kb][s] = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
        } else {
          const uint8_t* rp = reinterpret_cast<const uint8_t*>(a.Kv) +
                              row * (int64_t)kIdxkFp8RowBytes;
          const u32x2 raw =
              *reinterpret_cast<const u32x2*>(rp + 32 * s + 8 * g);  // 4-B aligned
          const float sc = *reinterpret_cast<const float*>(rp + 128);
          const f16x4 k0 = e4m3x4_to_f16x4(raw[0]), k1 = e4m3x4_to_f16x4(raw[1]);
          const f16x8 k8 = {k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3]};
          f16x8 h;
#pragma unroll
          for (int e = 0; e < 8; e++) h[e] = (f16)((float)k8[e] * sc);
          ka[kb][s] = h;
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < WPT; u++) {
    const int i = threadIdx.x + u * NT;
    sh.w[i / QT][i % QT] = (q_base + i % QT < B) ? (float)wv[u] : 0.f;
  }
  if (wave == 0) {
    const int sl_v = (lane < QT && q_base + lane < B) ? sl_raw : 0;  // query q_base + lane
    sh.sl[lane] = sl_v;
    int m = sl_v;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = max(m, __shfl_xor(m, o, 64));
    if (lane == 0) sh.maxsl = m;
  }
  if constexpr (!KFP8) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // keys, pair 0
  __syncthreads();

  if (p_base >= sh.maxsl) {
    // no query of this tile reaches these keys: -inf padding only
    for (int e = threadIdx.x; e < QT * kPkKT; e += blockDim.x) {
      const int qi = e / kPkKT, p = p_base + e % kPkKT;
      const int q = q_base + qi;
      if (q < B && p < max_kv) a.score[(int64_t)q * max_kv + p] = -INFINITY;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no LDS-DMA may outlive the LDS
    return;
  }

  if constexpr (!KFP8) {
#pragma unroll
    for (int kb = 0; kb < 4; kb++) {
      const int key = kPkWaveKeys * (wave & 3) + 16 * kb + c;  // key & 15 == c
#pragma unroll
      for (int s2 = 0; s2 < 4; s2++)
        ka[kb][s2] = *reinterpret_cast<const f16x8*>(&kl[(key * 16 + ((4 * s2 + g) ^ c)) * 8]);
    }
    lds_barrier();  // every wave holds its keys: the key slots are free for Q
#pragma unroll
    for (int h = KSLOT0 > 0 ? 2 : 0; h < 2 * kAhead; h++) issue_q(h);
  }

  // Heads alternate between two accumulator sets: while the MFMAs of head h
  // fill one, the relu * w epilogue of head h - 1 drains the other, a
  // quarter (one key block) per x32 step.  The B operands of step st + 1 are
  // read from LDS during step st, so no MFMA waits on an LDS read except the
  // first of a pair (right after the barrier).
  f32x4 sacc[4][QB];  // [key block][query block], relu*w summed over heads
  f32x4 accA[4][QB], accB[4][QB];
#pragma unroll
  for (int kb = 0; kb < 4; kb++)
#pragma unroll
    for (int qb = 0; qb < QB; qb++) {
      sacc[kb][qb] = (f32x4){0.f, 0.f, 0.f, 0.f};
      accB[kb][qb] = (f32x4){0.f, 0.f, 0.f, 0.f};
    }
  // B operand: query column c of tile qb0 + qb, dims 32st + 8g .. +8, at LDS
  // unit (tile, st, lane)
  const int boff = hh * (QT * kIdxHeadDim) + qb0 * 2048 + lane * 8;
  auto load_b = [&](const f16* qs, int st, f16x8 (&b)[QB]) {
#pragma unroll
    for (int qb = 0; qb < QB; qb++)
      b[qb] = *reinterpret_cast<const f16x8*>(&qs[boff + qb * 2048 + st * 512]);
  };
  // load_w: the weights of head h for this lane's query columns
  auto load_w = [&](int h, float (&w2)[QB]) {
#pragma unroll
    for (int qb = 0; qb < QB; qb++) w2[qb] = sh.w[hoff + h][16 * (qb0 + qb) + c];
  };
  // head h: MFMAs into acc, epilogue of head h - 1 (prev, weights wn); with
  // next_in_pair, its last step also reads head h + 1's first B operands and
  // the weights of head h into bn / wn
  auto head = [&](int h, f32x4 (&acc)[4][QB], f32x4 (&prev)[4][QB], f16x8 (&bn)[QB],
                  float (&wn)[QB], bool next_in_pair, bool dma) {
    const f16* qs = sh.q[h % kPkRing];
    const f16* qs1 = sh.q[(h + 1) % kPkRing];
    float wq[QB];
#pragma unroll
    for (int qb = 0; qb < QB; qb++) wq[qb] = wn[qb];
#pragma unroll
    for (int st = 0; st < 4; st++) {
      f16x8 bc[QB];
#pragma unroll
      for (int qb = 0; qb < QB; qb++) bc[qb] = bn[qb];
      if (st < 3) {
        load_b(qs, st + 1, bn);
      } else if (next_in_pair) {
        load_b(qs1, 0, bn);
        load_w(h, wn);
      }
      if (dma && (st & 1) == 0 && (st >> 1) < QROUNDS) issue_q_round(h + 2 * kAhead, st >> 1);
#pragma unroll
      for (int qb = 0; qb < QB; qb++)
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
          acc[kb][qb] = mfma16x16x32(ka[kb][st], bc[qb],
                                     st == 0 ? (f32x4){0.f, 0.f, 0.f, 0.f} : acc[kb][qb]);
#pragma unroll
      for (int qb = 0; qb < QB; qb++)
#pragma unroll
        for (int r = 0; r < 4; r++) sacc[st][qb][r] += relu1(prev[st][qb][r]) * wq[qb];
      // the next step's LDS reads first, then one MFMA and two VALU, repeated
      if (st < 3) __builtin_amdgcn_sched_group_barrier(0x100, QB, 0);
      else if (next_in_pair) __builtin_amdgcn_sched_group_barrier(0x100, 2 * QB, 0);
#pragma unroll
      for (int i = 0; i < 4 * QB; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
      }
      __builtin_amdgcn_sched_barrier(0);  // steps do not mix
    }
  };

  // Pair j (heads 2j, 2j + 1): the two heads of pair j + kAhead are loaded
  // during it.  The refilling and the draining pairs are separate loops so
  // that neither has a branch inside its MFMA sequence.
  auto pair = [&](int j, bool refill) {
    const int h0 = 2 * j;
    pk_wait<QROUNDS>(min(NHP - 1 - j, kAhead - 1));
    lds_barrier();  // pair j landed; every wave is done with pair j - 1
    f16x8 bn[QB];
    float wn[QB];
#pragma unroll
    for (int qb = 0; qb < QB; qb++) wn[qb] = 0.f;
    load_b(sh.q[h0 % kPkRing], 0, bn);
    if (h0 > 0) load_w(h0 - 1, wn);
    head(h0, accA, accB, bn, wn, true, refill);
    head(h0 + 1, accB, accA, bn, wn, false, refill);
  };
#pragma nounroll
  for (int j = 0; j < NHP - kAhead; j++) pair(j, true);
#pragma nounroll
  for (int j = NHP - kAhead; j < NHP; j++) pair(j, false);
#pragma unroll
  for (int qb = 0; qb < QB; qb++) {
    const float wl = sh.w[hoff + 2 * NHP - 1][16 * (qb0 + qb) + c];
#pragma unroll
    for (int kb = 0; kb < 4; kb++)
#pragma unroll
      for (int r = 0; r < 4; r++) sacc[kb][qb][r] += relu1(accB[kb][qb][r]) * wl;
  }
  if constexpr (HS == 2) {
    // heads 16-31 of each key group meet heads 0-15 in LDS (the ring is free:
    // the last pair waited for every DMA, and the barrier for every read)
    __syncthreads();
    float* red = reinterpret_cast<float*>(&sh.q[0][0]);
    const int kg = wave & 3;
    static_assert(4 * 4 * QB * 256 * 4 <= sizeof(sh.q), "reduction buffer");
    if (hh == 1) {
#pragma unroll
      for (int kb = 0; kb < 4; kb++)
#pragma unroll
        for (int qb = 0; qb < QB; qb++)
          *reinterpret_cast<f32x4*>(&red[((kg * 4 + kb) * QB + qb) * 256 + lane * 4]) =
              sacc[kb][qb];
    }
    __syncthreads();
    if (hh == 1) return;
#pragma unroll
    for (int kb = 0; kb < 4; kb++)
#pragma unroll
      for (int qb = 0; qb < QB; qb++)
        sacc[kb][qb] += *reinterpret_cast<const f32x4*>(
            &red[((kg * 4 + kb) * QB + qb) * 256 + lane * 4]);
  }

  // D layout: lane (query col c, key rows 4g+r) -> 4 consecutive keys.
#pragma unroll
  for (int qb = 0; qb < QB; qb++) {
    const int qi = 16 * (qb0 + qb) + c;
    const int q = q_base + qi;
    if (q >= B) continue;
    const int sl = sh.sl[qi];
    float* srow = a.score + (int64_t)q * max_kv;
#pragma unroll
    for (int kb = 0; kb < 4; kb++) {
      const int p0 = key0 + 16 * kb + 4 * g;
      f32x4 v;
#pragma unroll
      for (int r = 0; r < 4; r++) v[r] = (p0 + r < sl) ? sacc[kb][qb][r] : -INFINITY;
      if (p0 + 3 < max_kv && (max_kv & 3) == 0) {
        *reinterpret_cast<f32x4*>(srow + p0) = v;
      } else {
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (p0 + r < max_kv) srow[p0 + r] = v[r];
      }
    }
  }
}

// Workgroups [0, n_full) take full tiles t = blockIdx.x (key tile t % n_kt
// of 64-query tile t / n_kt); the rest take halves of tiles n_full, ...
// (two consecutive workgroups per tile, 32 queries each).
template <bool KFP8>
__global__ void __launch_bounds__(kPkThreads) indexer_logits_packed_kernel(PkArgs a) {
  __shared__ PkSmem sh;
  const int id = blockIdx.x;
  if (id < a.n_full) {
    pk_tile<KFP8, 2, kPkWaves, 1>(a, sh, (id / a.n_kt) * kPkMaxQT, (id % a.n_kt) * kPkKT);
  } else {
    const int j = id - a.n_full;
    const int t = a.n_full + (j >> 1);
    const int q_base = (t / a.n_kt) * kPkMaxQT + 32 * (j & 1);
    if (q_base >= a.B) return;  // a half tile past the last query (no DMA issued yet)
    pk_tile<KFP8, 1, kPkWaves, 1>(a, sh, q_base, (t % a.n_kt) * kPkKT);
  }
}

// Four-wave workgroups over 32 queries x 256 keys (each wave: 64 keys x the
// 32 queries, as a full tile's wave), ~68 KB of LDS with 8 KB ring slots,
// so that two workgroups share a CU and one's prologue (64 KB of keys, the
// first Q pairs) and epilogue (its score stores) run beside the other's
// MFMAs.  Used for launches of more than one round (kPkhMinTiles full
// tiles and up): 4-5 % faster at 384 tiles and up, 0.5-1 us per launch
// faster at 257-383, ~1 % slower on launches of a round or less.
constexpr int kPkhWaves = 4;
constexpr int kPkhQT = 32;
constexpr int64_t kPkhMinTiles = kPkCUs + 1;
using PkSmemH = PkSmemT<kPkhQT>;

template <bool KFP8>
__global__ void __launch_bounds__(kPkhWaves * 64, 2) indexer_logits_packed_h_kernel(PkArgs a) {
  __shared__ PkSmemH sh;
  const int id = blockIdx.x;
  const int q_base = (id / a.n_kt) * kPkhQT;
  if (q_base >= a.B) return;
  pk_tile<KFP8, 2, kPkhWaves, 1>(a, sh, q_base, (id % a.n_kt) * kPkKT);
}

// Launches of more than one round of four-wave workgroups whose last round
// holds at most half a round (R = workgroups mod 512, 0 < R <= 256): the
// first n_full workgroups are four-wave 32-query workgroups as in
// indexer_logits_packed_h_kernel, and the last R of them run as 2R quarter
// tiles (16 queries each, at most one round), so that the last round takes
// a quarter tile's time instead of a 32-query workgroup's.
template <bool KFP8>
__global__ void __launch_bounds__(kPkhWaves * 64, 2) indexer_logits_packed_hq_kernel(PkArgs a) {
  __shared__ PkSmemH sh;
  const int id = blockIdx.x;
  if (id < a.n_full) {
    const int q_base = (id / a.n_kt) * kPkhQT;
    if (q_base >= a.B) return;
    pk_tile<KFP8, 2, kPkhWaves, 1>(a, sh, q_base, (id % a.n_kt) * kPkKT);
  } else {
    const int j = id - a.n_full;
    const int hq = a.n_full + (j >> 1);  // the 32-query workgroup this quarter is half of
    const int q_base = (hq / a.n_kt) * kPkhQT + 16 * (j & 1);
    if (q_base >= a.B) return;
    pk_tile<KFP8, 1, kPkhWaves, 1>(a, sh, q_base, (hq % a.n_kt) * kPkKT);
  }
}

// Quarter tiles for launches of at most kPkqMaxTiles full tiles (one piece
// per CU): 8 waves over 16 queries x 256 keys, the 32 heads split over two
// wave groups (each wave: 64 keys x the 16 queries x 16 heads), so that two
// waves per SIMD share the piece's MFMAs and hide each other's epilogue and
// barrier waits.  Per launch (128-row sub-chunks of a causal prefill):
// 10.4-11.8 us, against 11.7-12.8 us for four-wave quarters with all 32
// heads per wave and 15.6-16.4 us for half tiles.  Larger launches gain
// nothing from quarters: two sharing a CU take as long as one half tile
// alone; and the head split over 32-query pieces (65-128 tiles) measured
// level with the 8-wave half tiles, which already run two waves per SIMD.
constexpr int kPkqQT = 16;
constexpr int64_t kPkqMaxTiles = kPkCUs / 4;

template <bool KFP8>
__global__ void __launch_bounds__(kPkThreads) indexer_logits_packed_qs_kernel(PkArgs a) {
  __shared__ PkSmemT<2 * kPkqQT> sh;  // ring slots of two heads
  const int id = blockIdx.x;
  const int q_base = (id / a.n_kt) * kPkqQT;
  if (q_base >= a.B) return;
  pk_tile<KFP8, 1, kPkWaves, 2>(a, sh, q_base, (id % a.n_kt) * kPkKT);
}

// Tiles of a launch with W full tiles that run as two half tiles: all of
// them up to kPkHalfMax tiles (launches of more than one round take the
// four-wave kernel instead).
static int pk_split_tiles(int64_t W) { return W <= kPkHalfMax ? (int)W : 0; }

}  // namespace mi355dsa

using namespace mi355dsa;

static int check_indexer_args(int B, int max_kv, const void* k_cache,
                              int64_t n_kv_rows, int page_size,
                              const void* weights, const int32_t* block_table,
                              int max_blocks, const int32_t* seq_lens) {
  DSA_CHECK(B >= 0 && max_kv >= 0, "B and max_kv must be >= 0");
  DSA_CHECK(k_cache && weights && block_table && seq_lens, "null pointer argument");
  DSA_CHECK(page_size > 0 && (page_size & (page_size - 1)) == 0,
            "indexer cache page size must be a power of two");
  DSA_CHECK(n_kv_rows >= 0 && max_blocks >= 0, "bad cache / block-table size");
  return MI355_DSA_OK;
}

extern "C" int mi355_dsa_indexer_logits(
    float* score, int B, int max_kv, const void* q, int n_ihead, int head_dim,
    const void* k_cache, int k_fp8, int64_t n_kv_rows, int page_size,
    const void* weights, const int32_t* block_table, int max_blocks,
    const int32_t* seq_lens, int32_t* hist, void* stream) {
  clear_error();
  DSA_CHECK(head_dim == 128, "indexer head_dim must be 128");
  DSA_CHECK(n_ihead == 32, "kernel specialized for 32 indexer heads");
  int rc = check_indexer_args(B, max_kv, k_cache, n_kv_rows, page_size, weights,
                              block_table, max_blocks, seq_lens);
  if (rc) return rc;
  if (B == 0 || max_kv == 0) return MI355_DSA_OK;
  DSA_CHECK(score && q, "null pointer argument");
  DSA_CHECK(aligned_to(q, 16), "q must be 16-byte aligned");
  DSA_CHECK(k_fp8 ? aligned_to(k_cache, 4) : aligned_to(k_cache, 16),
            "k_cache is misaligned");
  DSA_CHECK(B <= 65535, "B too large");
  const dim3 grid((max_kv + kIdxPPB - 1) / kIdxPPB, B);
  const int shift = ilog2_pow2(page_size);
  hipStream_t st = as_stream(stream);
  uint32_t* h = reinterpret_cast<uint32_t*>(hist);
  const int hist8 = aligned_to(hist, 8) ? 1 : 0;
  IdxDecArgs a{};
  a.Q = reinterpret_cast<const f16*>(q);
  a.Kv = k_cache;
  a.W = reinterpret_cast<const f16*>(weights);
  a.block_table = block_table;
  a.seq_lens = seq_lens;
  a.score = score;
  a.hist = h;
  a.n_kv_rows = n_kv_rows;
  a.max_blocks = max_blocks;
  a.page_shift = shift;
  a.max_kv = max_kv;
  a.hist8 = hist8;
  a.span = idx_span_launch(k_fp8, B, max_kv);
  if (k_fp8)
    indexer_logits_kernel<true><<<grid, kIdxWaves * 64, 0, st>>>(
        a.Q, a.Kv, a.W, a.block_table, a.seq_lens, a.score, a.hist, a.n_kv_rows, a.max_blocks,
        a.page_shift, a.max_kv, a.hist8, a.span);
  else
    indexer_logits_kernel<false><<<grid, kIdxWaves * 64, 0, st>>>(
        a.Q, a.Kv, a.W, a.block_table, a.seq_lens, a.score, a.hist, a.n_kv_rows, a.max_blocks,
        a.page_shift, a.max_kv, a.hist8, a.span);
  DSA_LAUNCH_CHECK("indexer_logits");
  return MI355_DSA_OK;
}

extern "C" int mi355_dsa_indexer_logits_packed(
    float* score, int B, int max_kv, const void* q_packed, const void* k_cache,
    int k_fp8, int64_t n_kv_rows, int page_size, const void* weights,
    const int32_t* block_table, int max_blocks, const int32_t* seq_lens,
    void* stream) {
  clear_error();
  int rc = check_indexer_args(B, max_kv, k_cache, n_kv_rows, page_size, weights,
                              block_table, max_blocks, seq_lens);
  if (rc) return rc;
  if (B == 0 || max_kv == 0) return MI355_DSA_OK;
  DSA_CHECK(score && q_packed, "null pointer argument");
  DSA_CHECK(aligned_to(q_packed, 16), "q_packed must be 16-byte aligned");
  DSA_CHECK(k_fp8 ? aligned_to(k_cache, 4) : aligned_to(k_cache, 16),
            "k_cache is misaligned");
  DSA_CHECK(aligned_to(score, 16), "score must be 16-byte aligned");
  const int64_t n_kt = (max_kv + kPkKT - 1) / kPkKT;
  const int64_t W = n_kt * ((B + kPkMaxQT - 1) / kPkMaxQT);
  const int split = pk_split_tiles(W);
  const int64_t grid = W + split;
  DSA_CHECK(grid <= INT32_MAX, "B x max_kv too large");
  PkArgs a;
  a.Qp = reinterpret_cast<const f16*>(q_packed);
  a.Kv = k_cache;
  a.W = reinterpret_cast<const f16*>(weights);
  a.block_table = block_table;
  a.seq_lens = seq_lens;
  a.score = score;
  a.B = B;
  a.n_kv_rows = n_kv_rows;
  a.max_blocks = max_blocks;
  a.page_shift = ilog2_pow2(page_size);
  a.max_kv = max_kv;
  a.n_kt = (int)n_kt;
  a.n_full = (int)(W - split);
  hipStream_t st = as_stream(stream);
  if (W <= kPkqMaxTiles) {
    // small launches: 16-query head-split pieces, up to one per CU
    const int64_t gq = n_kt * ((B + kPkqQT - 1) / kPkqQT);
    if (k_fp8)
      indexer_logits_packed_qs_kernel<true><<<dim3((unsigned)gq), kPkThreads, 0, st>>>(a);
    else
      indexer_logits_packed_qs_kernel<false><<<dim3((unsigned)gq), kPkThreads, 0, st>>>(a);
  } else if (W >= kPkhMinTiles) {
    // large launches: four-wave 32-query workgroups, two per CU; a last
    // round of at most half a round runs as quarter tiles
    const int64_t gh = n_kt * ((B + kPkhQT - 1) / kPkhQT);
    DSA_CHECK(gh + kPkCUs <= INT32_MAX, "B x max_kv too large");
    const int64_t R = gh % (2 * kPkCUs);
    if (R > 0 && R <= kPkCUs) {
      a.n_full = (int)(gh - R);
      const unsigned grid_hq = (unsigned)(gh + R);
      if (k_fp8)
        indexer_logits_packed_hq_kernel<true><<<dim3(grid_hq), kPkhWaves * 64, 0, st>>>(a);
      else
        indexer_logits_packed_hq_kernel<false><<<dim3(grid_hq), kPkhWaves * 64, 0, st>>>(a);
    } else if (k_fp8) {
      indexer_logits_packed_h_kernel<true><<<dim3((unsigned)gh), kPkhWaves * 64, 0, st>>>(a);
    } else {
      indexer_logits_packed_h_kernel<false><<<dim3((unsigned)gh), kPkhWaves * 64, 0, st>>>(a);
    }
  } else if (k_fp8) {
    indexer_logits_packed_kernel<true><<<dim3((unsigned)grid), kPkThreads, 0, st>>>(a);
  } else {
    indexer_logits_packed_kernel<false><<<dim3((unsigned)grid), kPkThreads, 0, st>>>(a);
  }
  DSA_LAUNCH_CHECK("indexer_logits_packed");
  return MI355_DSA_OK;
}
