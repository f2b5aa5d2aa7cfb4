// Decode-shaped indexer logits workgroup (see indexer.hip for the design):
// shared by mi355_dsa_indexer_logits's kernel and the fused decode-layer
// launch (dsa_layer.hip).
#pragma once

#include <float.h>

#include "cache_write.h"
#include "dsa_common.h"

namespace mi355dsa {

// ===========================================================================
// decode / generic kernel
// ===========================================================================
constexpr int kIdxWaves = 4;
constexpr int kIdxPPB = 1024;             // positions per workgroup
constexpr int kIdxBlocksPerWave = kIdxPPB / 16 / kIdxWaves;  // 16
constexpr int kIdxGroup = 2;              // 16-key blocks per pipeline stage
// LDS slot of one staged fp8 block: 16 rows x 132 bytes, then the padding
// that the last DMA's lanes 16-63 fill
constexpr int kIdxSpanSlot = 2048 + 256;

// Key-row fragment of one 16-key block for one lane (key c, group g).
// fp16 rows: dims 32s + 8g .. +8 for steps s = 0..3, four 16-byte loads of
// which load s of the four lanes of a key covers 64 contiguous bytes of its
// row (one half cache line per key and instruction).  fp8 rows: dims
// [o_g, o_g + 16) and [o_g + 32, o_g + 48) with o_g = idx_fp8_piece(g)
// (0, 64, 16, 80): lanes g and g ^ 1 read 64 bytes apart, which keeps the
// LDS reads of the staged 132-byte rows (lanes c, g of a half wave) on
// distinct banks.
struct KeyFrag {
  u32x4 v[4];
  float scale;  // fp8: row scale; fp16: 1
};

__device__ __forceinline__ int idx_fp8_piece(int g) { return 64 * (g & 1) + 16 * (g >> 1); }

template <bool KFP8>
__device__ __forceinline__ void load_key_frag(KeyFrag& f, const void* kv,
                                              int64_t row) {
  if (row < 0) {
#pragma unroll
    for (int i = 0; i < 4; i++) f.v[i] = (u32x4){0u, 0u, 0u, 0u};
    f.scale = 0.f;
    return;
  }
  const int g = (threadIdx.x & 63) >> 4;
  if constexpr (KFP8) {
    const uint8_t* rp = reinterpret_cast<const uint8_t*>(kv) +
                        row * (int64_t)kIdxkFp8RowBytes + idx_fp8_piece(g);
    f.v[0] = *reinterpret_cast<const u32x4_a4*>(rp);
    f.v[1] = *reinterpret_cast<const u32x4_a4*>(rp + 32);
    f.scale = *reinterpret_cast<const float*>(rp - idx_fp8_piece(g) + 128);
  } else {
    const u32x4* p = reinterpret_cast<const u32x4*>(
        reinterpret_cast<const f16*>(kv) + row * kIdxHeadDim + 8 * g);
#pragma unroll
    for (int i = 0; i < 4; i++) f.v[i] = p[4 * i];
    f.scale = 1.f;
  }
}

// load_key_frag without branches, for workgroups inside the row: an
// unmapped row (row < 0) loads row 0 of the cache instead (n_kv_rows >= 1)
// and the caller replaces that key's score by the zero key's score, 0.  Its
// bytes reach only that key's MFMA column.  Every lane then issues the same
// global loads, so the compiler can count the memory operations in flight
// (vmcnt, which also counts stores) and waits for exactly the ones needed.
template <bool KFP8>
__device__ __forceinline__ void load_key_frag_nb(KeyFrag& f, const void* kv, int64_t row) {
  const int g = (threadIdx.x & 63) >> 4;
  const int64_t r = row < 0 ? 0 : row;
  if constexpr (KFP8) {
    const uint8_t* rp = reinterpret_cast<const uint8_t*>(kv) + r * (int64_t)kIdxkFp8RowBytes;
    f.v[0] = *reinterpret_cast<const u32x4_a4*>(rp + idx_fp8_piece(g));
    f.v[1] = *reinterpret_cast<const u32x4_a4*>(rp + idx_fp8_piece(g) + 32);
    f.scale = *reinterpret_cast<const float*>(rp + 128);
  } else {
    const u32x4* p = reinterpret_cast<const u32x4*>(reinterpret_cast<const f16*>(kv) +
                                                    r * kIdxHeadDim + 8 * g);
#pragma unroll
    for (int i = 0; i < 4; i++) f.v[i] = p[4 * i];
    f.scale = 1.f;
  }
}

// B operand for step s from a key fragment (dims 32s + 8g .. +8 for fp16
// rows, idx_fp8_piece(g) + 32 (s >> 1) + 8 (s & 1) .. +8 for fp8 rows).
template <bool KFP8>
__device__ __forceinline__ f16x8 key_operand(const KeyFrag& f, int s) {
  if constexpr (KFP8) {
    const f16x4 a = e4m3x4_to_f16x4(f.v[s >> 1][2 * (s & 1)]);
    const f16x4 b = e4m3x4_to_f16x4(f.v[s >> 1][2 * (s & 1) + 1]);
    return (f16x8){a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  } else {
    return __builtin_bit_cast(f16x8, f.v[s]);
  }
}

// Arguments of the decode logits (score rows of B tokens over max_kv
// positions; hist: the [B, 4096] level-1 histogram to add into, or null).
struct IdxDecArgs {
  const f16* Q;
  const void* Kv;
  const f16* W;
  const int32_t* block_table;
  const int32_t* seq_lens;
  float* score;
  uint32_t* hist;
  int64_t n_kv_rows;
  int max_blocks;
  int page_shift;
  int max_kv;
  int hist8;  // hist is 8-byte aligned: two bins per 64-bit atomic
  int span;   // fp8 keys: stage 16-key spans through LDS where the cache allows
};

// The launch's workgroups per CU above which the fp8 span path pays: with
// two or more resident per CU the staged spans (fewer, whole-line requests)
// raise the streaming rate; a launch of one workgroup per CU is bound by each
// wave's load-to-use latency, which the LDS staging lengthens.
constexpr int kIdxSpanMinWorkgroups = 512;
__host__ __device__ inline int idx_span_launch(int k_fp8, int B, int max_kv) {
  return k_fp8 && (int64_t)B * ((max_kv + kIdxPPB - 1) / kIdxPPB) >= kIdxSpanMinWorkgroups;
}

// The step's new index keys, for a launch that also writes them to the
// cache (the fused decode-layer launch): fp16 rows [T, 128] and their slots.
constexpr int kIdxMaxNew = 64;
struct IdxNewKeys {
  const u32x4* ik;      // [T][16] 16-byte chunks
  const int32_t* slot;  // [T]; slots < 0 or >= n_kv_rows are not written
  int T;                // <= kIdxMaxNew
  void* dst;            // the index-key cache they are written to: the memory
                        // the launch also reads keys from (Kv)
};

// One indexer-K row written as the cache's store kernel writes it: 16 lanes
// (sub = 0..15, one DPP row, all active) per row, lane sub holding dims
// 8 sub .. +8 of the fp16 key in raw.  dst null: nothing stored (the lanes
// still take part in the fp8 row maximum).
template <bool KFP8>
__device__ __forceinline__ void idx_key_row_store(const u32x4 raw, void* dst, int sub) {
  if constexpr (KFP8) {
    k_fp8_row_store(raw, reinterpret_cast<uint8_t*>(dst), sub);
  } else {
    if (dst != nullptr) reinterpret_cast<u32x4*>(dst)[sub] = raw;
  }
}

// Workgroup (tile, b) of the decode logits: positions [1024 tile, +1024) of
// token row b.  With NEWK, positions whose cache row is the slot of one of
// the step's new keys get that key written to the row first, by this
// workgroup, so that it reads exactly what a separate store launch before it
// would have left there.  The standalone kernel (NEWK = false) runs the same
// code without that step.
// (The pointers are restrict parameters of this function, not fields read
// from a struct, so that the compiler keeps knowing that the score stores
// do not alias the key loads.  Kv is not restrict: with NEWK the same rows
// are written through nk.dst, and read after the workgroup barrier.)
template <bool KFP8, bool NEWK>
__device__ __forceinline__ void indexer_logits_body(
    const f16* __restrict__ Q, const void* Kv, const f16* __restrict__ W,
    const int32_t* __restrict__ block_table, const int32_t* __restrict__ seq_lens,
    float* __restrict__ score, uint32_t* __restrict__ hist, int64_t n_kv_rows, int max_blocks,
    int page_shift, int max_kv, int hist8, int span, int tile, int b, const IdxNewKeys& nk) {
  const int p_lo = tile * kIdxPPB;
  const int p_hi = min(p_lo + kIdxPPB, max_kv);
  // The block-table entries of the tile's pages are loaded beside seq_len
  // (one round trip instead of two before the first key load); a tile past
  // the context reads them for nothing.
  constexpr int kNT = kIdxWaves * 64;
  constexpr int kBtRegs = (kIdxPPB + 2 + kNT - 1) / kNT;
  const int pg0 = p_lo >> page_shift;
  const int npg = ((p_hi - 1) >> page_shift) - pg0 + 1;
  const int32_t* bt_row = block_table + (int64_t)b * max_blocks;
  int32_t btv[kBtRegs];
#pragma unroll
  for (int k = 0; k < kBtRegs; k++) {
    const int i = (int)threadIdx.x + kNT * k;
    btv[k] = (i < npg && pg0 + i < max_blocks) ? bt_row[pg0 + i] : -1;
  }
  const int seq_len = seq_lens[b];
  float* srow = score + (int64_t)b * max_kv;

  // tiles wholly past the context only need the -inf padding
  if (p_lo >= seq_len) {
    for (int i = p_lo + threadIdx.x; i < p_hi; i += blockDim.x) srow[i] = -INFINITY;
    return;
  }

  __shared__ int32_t s_bt[kIdxPPB + 2];
  // level-1 counts of this workgroup's keys, two 16-bit bins per word (a
  // workgroup counts at most 1024 keys)
  __shared__ uint32_t s_hist[kTopkBins / 2];
  // fp8 span path: per wave, two stages of kIdxGroup staged blocks
  __shared__ __align__(16) uint8_t s_span[KFP8 ? kIdxWaves * 2 * kIdxGroup * kIdxSpanSlot : 16];
  __shared__ int32_t s_new[NEWK ? 2 * kIdxMaxNew : 1];  // slots, then "this workgroup reads it"
  const int page = 1 << page_shift;
#pragma unroll
  for (int k = 0; k < kBtRegs; k++) {
    const int i = (int)threadIdx.x + kNT * k;
    if (i < npg) s_bt[i] = btv[k];
  }
  if (hist != nullptr)
    for (int i = threadIdx.x; i < kTopkBins / 2; i += blockDim.x) s_hist[i] = 0u;
  if constexpr (NEWK) {
    for (int i = threadIdx.x; i < nk.T; i += blockDim.x) {
      s_new[i] = nk.slot[i];
      s_new[kIdxMaxNew + i] = 0;
    }
  }
  __syncthreads();
  if constexpr (NEWK) {
    // Which new keys land on a row this workgroup reads: slot s is read at
    // position p = (page of s in the table) + (s mod page) when p lies in
    // [p_lo, min(p_hi, seq_len)).
    const int lim = min(p_hi, seq_len);
    int found = 0;
    for (int i = threadIdx.x; i < nk.T * npg; i += blockDim.x) {
      const int t = i / npg, j = i - t * npg;
      const int32_t s = s_new[t];
      if (s >= 0 && s < n_kv_rows && s_bt[j] == (s >> page_shift)) {
        const int p = ((pg0 + j) << page_shift) | (s & ((1 << page_shift) - 1));
        if (p >= p_lo && p < lim) {
          s_new[kIdxMaxNew + t] = 1;
          found = 1;
        }
      }
    }
    // Most workgroups read none of the new rows: for them this one barrier
    // is the whole cost.
    if (__syncthreads_or(found)) {
      // 16 lanes per key, 16 keys per pass; a 16-lane group is wholly active
      // or wholly idle
      for (int t0 = 0; t0 < nk.T; t0 += 16) {
        const int t = t0 + (int)(threadIdx.x >> 4);
        if (t < nk.T && s_new[kIdxMaxNew + t]) {
          const int sub = threadIdx.x & 15;
          const int64_t row = s_new[t];
          void* dst = KFP8 ? (void*)(reinterpret_cast<uint8_t*>(nk.dst) +
                                     row * (int64_t)kIdxkFp8RowBytes)
                           : (void*)(reinterpret_cast<f16*>(nk.dst) + row * kIdxHeadDim);
          idx_key_row_store<KFP8>(nk.ik[(int64_t)t * 16 + sub], dst, sub);
        }
      }
      // the rows written above are read by every wave of this workgroup: the
      // barrier's workgroup-scope fence orders the stores before those loads
      __syncthreads();
    }
  }

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;

  // A operands: q rows (heads c and 16 + c), with the keys' k-slot mapping:
  // step s, group g, slot e -> dim 32s + 8g + e (fp16 keys) or
  // idx_fp8_piece(g) + 32 (s >> 1) + 8 (s & 1) + e (fp8 keys, whose two
  // 16-byte pieces per lane start at idx_fp8_piece(g) and 32 bytes later).
  f16x8 qa[2][4];
  const f16* qb = Q + (int64_t)b * kIdxHeads * kIdxHeadDim;
#pragma unroll
  for (int t = 0; t < 2; t++)
#pragma unroll
    for (int s = 0; s < 4; s++)
      qa[t][s] = *reinterpret_cast<const f16x8*>(
          qb + (16 * t + c) * kIdxHeadDim +
          (KFP8 ? idx_fp8_piece(g) + 32 * (s >> 1) + 8 * (s & 1) : 32 * s + 8 * g));
  // head weights of this lane's D rows: heads 4g + r and 16 + 4g + r
  float wv[2][4];
#pragma unroll
  for (int t = 0; t < 2; t++)
#pragma unroll
    for (int r = 0; r < 4; r++)
      wv[t][r] = (float)W[(int64_t)b * kIdxHeads + 16 * t + 4 * g + r];

  // Row of the key this lane loads for block `blk` (-1: zero key).
  auto key_row = [&](int blk) -> int64_t {
    const int p = p_lo + 16 * blk + c;
    if (p >= p_hi || p >= seq_len) return -1;
    const int32_t pb = s_bt[(p >> page_shift) - pg0];
    const int64_t row = ((int64_t)pb << page_shift) + (p & (page - 1));
    return (pb < 0 || row >= n_kv_rows) ? -1 : row;
  };

  KeyFrag cur[kIdxGroup], nxt[kIdxGroup];
  constexpr int n_groups = kIdxBlocksPerWave / kIdxGroup;
  static_assert(n_groups >= 2, "the span path's vmcnt waits assume two stages or more");
  // wave w owns blocks w, w+4, w+8, ... ; stage i covers its blocks
  // [i*kIdxGroup, (i+1)*kIdxGroup) in that order.
  auto blk_of = [&](int stage, int j) { return (stage * kIdxGroup + j) * kIdxWaves + wave; };

  // Score of one 16-key block for this lane's key (the same sum in the four
  // lanes g of a key: the butterfly only reorders commutative additions).
  auto block_score = [&](const KeyFrag& f) {
    float v = 0.f;
#pragma unroll
    for (int t = 0; t < 2; t++) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; s++) acc = mfma16x16x32(qa[t][s], key_operand<KFP8>(f, s), acc);
#pragma unroll
      for (int r = 0; r < 4; r++) {
        float d = acc[r];
        if constexpr (KFP8) d *= f.scale;
        v += relu_mfma(d) * wv[t][r];
      }
    }
    v = xor16_sum(v);
    v = xor32_sum(v);
    return v;
  };

  // one key into the level-1 count of bin key >> 20
  auto hist_count = [&](uint32_t key) {
    atomicAdd(&s_hist[key >> 21], 1u << ((key >> 16) & 16));
  };

  // fp8 rows, in a launch that asks for it (idx_span_launch), in pages of
  // >= 16 rows that the cache holds whole (its row count
  // a multiple of the page), 16-byte aligned: the 16 keys of a block are 16
  // consecutive rows, one 2112-byte span.
  const bool span_ok = KFP8 && span && page_shift >= 4 && n_kv_rows > 0 &&
                       (n_kv_rows & (page - 1)) == 0 &&
                       ((uintptr_t)Kv & 15) == 0;
  if (KFP8 && span_ok && p_lo + kIdxPPB <= max_kv) {
    // Whole workgroup inside the row.  Each block's span goes to LDS by
    // LDS-DMA in three instructions: bytes [0, 1024) and [1024, 2048), 16
    // per lane, and [2048, 2112), 4 per lane from lanes 0-15 (lanes 16-63
    // repeat them into the slot's padding).  A wave then reads its operands
    // from the staged rows.  Two stages (2 x kIdxGroup slots) per wave: the
    // next stage's spans are in flight while this one is scored.  A block of
    // an unmapped page (table entry < 0 or past the cache) fetches rows 0-15
    // instead and scores its keys as the zero key, 0.
    uint8_t* ring = s_span + wave * (2 * kIdxGroup * kIdxSpanSlot);
    const uint8_t* kb = reinterpret_cast<const uint8_t*>(Kv);
    auto issue = [&](int st, bool (&ok)[kIdxGroup]) {
#pragma unroll
      for (int j = 0; j < kIdxGroup; j++) {
        const int p0 = p_lo + 16 * blk_of(st, j);
        // one page per block: its table entry is wave-uniform
        const int32_t pb = __builtin_amdgcn_readfirstlane(s_bt[(p0 >> page_shift) - pg0]);
        ok[j] = pb >= 0 && ((int64_t)pb << page_shift) < n_kv_rows;
        const int64_t r0 = ok[j] ? ((int64_t)pb << page_shift) + (p0 & (page - 1)) : 0;
        const uint8_t* src = kb + r0 * kIdxkFp8RowBytes;
        uint8_t* slot = ring + ((st & 1) * kIdxGroup + j) * kIdxSpanSlot;
        dma16_at<0>(src + 16 * lane, slot);
        dma16_at<1024>(src + 16 * lane, slot + 1024);
        dma4_at<2048>(src + 4 * (lane & 15), slot + 2048);
      }
    };
    bool okc[kIdxGroup], okn[kIdxGroup];
    issue(0, okc);
#pragma unroll
    for (int st = 0; st < n_groups; st++) {
      if (st + 1 < n_groups) {
        // this wave's reads of the slots about to be refilled (stage st - 1)
        // are complete before their DMAs go out
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        issue(st + 1, okn);
      }
      // stage st landed: after its 3 kIdxGroup DMAs come the previous
      // stage's kIdxGroup score stores and the next stage's DMAs
      if (st == 0)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * kIdxGroup) : "memory");
      else if (st + 1 < n_groups)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * kIdxGroup) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kIdxGroup) : "memory");
#pragma unroll
      for (int j = 0; j < kIdxGroup; j++) {
        const uint8_t* rw = ring + ((st & 1) * kIdxGroup + j) * kIdxSpanSlot +
                            kIdxkFp8RowBytes * c;
        KeyFrag f;
        f.v[0] = *reinterpret_cast<const u32x4_a4*>(rw + idx_fp8_piece(g));
        f.v[1] = *reinterpret_cast<const u32x4_a4*>(rw + idx_fp8_piece(g) + 32);
        f.v[2] = f.v[3] = (u32x4){0u, 0u, 0u, 0u};
        f.scale = *reinterpret_cast<const float*>(rw + 128);
        float v = block_score(f);
        if (!okc[j]) v = 0.f;
        const int p = p_lo + 16 * blk_of(st, j) + c;
        const bool live = p < seq_len;
        srow[p] = live ? v : -INFINITY;
        if (hist != nullptr && g == 0 && live) hist_count(mono_key(v));
      }
      if (st + 1 < n_groups) {
#pragma unroll
        for (int j = 0; j < kIdxGroup; j++) okc[j] = okn[j];
      }
    }
  } else if (p_lo + kIdxPPB <= max_kv && n_kv_rows > 0) {
    // Whole workgroup inside the row: no branch around any global load or
    // store.  Every lane stores its key's score (the four lanes of a key
    // write the same bits), so the waits before a stage's MFMAs count
    // exactly the operations issued after its keys and never drain the next
    // stage's loads or the score stores.
    auto row_nb = [&](int blk) -> int64_t {  // key_row without branches
      const int p = p_lo + 16 * blk + c;
      const int32_t pb = s_bt[(p >> page_shift) - pg0];
      const int64_t row = ((int64_t)pb << page_shift) + (p & (page - 1));
      return (p >= seq_len || pb < 0 || row >= n_kv_rows) ? -1 : row;
    };
    int64_t rcur[kIdxGroup], rnxt[kIdxGroup];
#pragma unroll
    for (int j = 0; j < kIdxGroup; j++) {
      rcur[j] = row_nb(blk_of(0, j));
      load_key_frag_nb<KFP8>(cur[j], Kv, rcur[j]);
    }
#pragma unroll
    for (int st = 0; st < n_groups; st++) {
      if (st + 1 < n_groups) {
#pragma unroll
        for (int j = 0; j < kIdxGroup; j++) {
          rnxt[j] = row_nb(blk_of(st + 1, j));
          load_key_frag_nb<KFP8>(nxt[j], Kv, rnxt[j]);
        }
      }
#pragma unroll
      for (int j = 0; j < kIdxGroup; j++) {
        float v = block_score(cur[j]);
        if (rcur[j] < 0) v = 0.f;  // unmapped row: the zero key's score
        const int p = p_lo + 16 * blk_of(st, j) + c;
        const bool live = p < seq_len;
        srow[p] = live ? v : -INFINITY;
        if (hist != nullptr && g == 0 && live) hist_count(mono_key(v));
      }
      if (st + 1 < n_groups) {
#pragma unroll
        for (int j = 0; j < kIdxGroup; j++) {
          cur[j] = nxt[j];
          rcur[j] = rnxt[j];
        }
      }
    }
  } else {
    // the row's last workgroup: blocks past p_hi are skipped
#pragma unroll
    for (int j = 0; j < kIdxGroup; j++) load_key_frag<KFP8>(cur[j], Kv, key_row(blk_of(0, j)));
#pragma unroll
    for (int st = 0; st < n_groups; st++) {
      if (16 * blk_of(st, 0) + p_lo >= p_hi) break;
      if (st + 1 < n_groups) {
#pragma unroll
        for (int j = 0; j < kIdxGroup; j++)
          load_key_frag<KFP8>(nxt[j], Kv, key_row(blk_of(st + 1, j)));
      }
#pragma unroll
      for (int j = 0; j < kIdxGroup; j++) {
        const int p0 = p_lo + 16 * blk_of(st, j);
        if (p0 < p_hi) {
          const float v = block_score(cur[j]);
          const int p = p0 + c;
          if (g == 0 && p < p_hi) {
            if (p < seq_len) {
              srow[p] = v;
              if (hist != nullptr) hist_count(mono_key(v));
            } else {
              srow[p] = -INFINITY;
            }
          }
        }
      }
      if (st + 1 < n_groups) {
#pragma unroll
        for (int j = 0; j < kIdxGroup; j++) cur[j] = nxt[j];
      }
    }
  }

  if (hist != nullptr) {
    __syncthreads();
    // Flush: the workgroups of a row all add into the same few hot bins at
    // the end, so the device-scope atomics queue on those addresses.  Two
    // adjacent bins go in one 64-bit atomic (half the atomics); no carry
    // crosses from the low count into the high one, since a row's counts
    // stay below 2^32.
    if (hist8) {
      unsigned long long* hrow2 =
          reinterpret_cast<unsigned long long*>(hist + (int64_t)b * kTopkBins);
      for (int i = threadIdx.x; i < kTopkBins / 2; i += blockDim.x) {
        const uint32_t w2 = s_hist[i];
        const unsigned long long lo = w2 & 0xffffu, hi = w2 >> 16;
        if (w2) atomicAdd(hrow2 + i, lo | (hi << 32));
      }
    } else {  // a hist base that is not 8-byte aligned: one bin per atomic
      uint32_t* hrow = hist + (int64_t)b * kTopkBins;
      for (int i = threadIdx.x; i < kTopkBins; i += blockDim.x) {
        const uint32_t n = (s_hist[i >> 1] >> (16 * (i & 1))) & 0xffffu;
        if (n) atomicAdd(&hrow[i], n);
      }
    }
  }
}

template <bool KFP8, bool NEWK>
__device__ __forceinline__ void indexer_logits_block(const IdxDecArgs& a, int tile, int b,
                                                     const IdxNewKeys& nk) {
  indexer_logits_body<KFP8, NEWK>(a.Q, a.Kv, a.W, a.block_table, a.seq_lens, a.score, a.hist,
                                  a.n_kv_rows, a.max_blocks, a.page_shift, a.max_kv, a.hist8,
                                  a.span, tile, b, nk);
}

}  // namespace mi355dsa
