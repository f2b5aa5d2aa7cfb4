// Sparse (top-k) MLA attention over the paged latent cache, decode and
// prefill, on gfx950 MFMA.  Semantics follow sm70_sparse_mla_decode
// (reference csrc/attention/sm70_mla_decode.cu:918-1184, host :2457-2616):
//   * key j = idx[b,i] is used iff 0 <= j < seq_len[b] and its paged row
//     resolves inside the cache (:977-992);
//   * q is pre-multiplied by fp16(scale) and rounded to fp16 (:1016-1018);
//   * online softmax with m initialised to -1e30, masked scores -inf (:961,
//     :1047-1067); P is rounded to fp16 for the PV product (:1068), the
//     running sum uses the fp32 p;
//   * o = PV / l in fp16, lse = m + ln l, or o = 0 and lse = empty_lse when
//     no key is valid: -inf on the reference's split-decode path (merge
//     convention, :1175-1183) and -1e30 (= m_init + ln 1, :1789-1793) for the
//     shapes the reference sends to its prefill kernel (B >= 32 and
//     n_head <= 16, :2511).
//
// MFMA formulation (one wave owns 16 heads):
//   S^T[key][head] = K[key][:] . Qs[head][:]      v_mfma_f32_16x16x32_f16
//   O^T[dim][head] += V^T[dim][key] . P^T[key][head]
// S^T's accumulator layout (lane c = head, rows 4g..4g+3 = keys) is the
// B-operand layout of the PV step, so P never leaves registers and the
// softmax reductions over keys are two lane shuffles.  V^T operands come
// straight from the row-major key tile with ds_read_b64_tr_b16 (in a 16-lane
// group, lane j element k = lane (4k + j/4)'s element j%4), one LDS
// instruction per MFMA operand.  O^T lives in 32 accumulator tiles.
//
// fp8_ds_mla rows: the 512 e4m3 NoPE bytes become exact fp16 values with
// v_cvt_scalef32_pk_f16_fp8 at scale 1 (2 values per instruction) and the
// four fp32 tile scales are applied where they are linear: QK keeps one
// accumulator per 128-dim scale tile (plus RoPE) and combines them with the
// row's scales, PV multiplies P by the row's tile scale (one P^T operand per
// scale tile).  Products are therefore exact; the reference instead rounds
// e4m3*scale to fp16 before the dot (dsmla_load4 + half store), which the
// tolerance of the parity tests covers.
//
// Memory pipeline: every workgroup first resolves idx -> block table ->
// cache row for all its keys in one batched pass (rows kept in LDS), then
// streams key tiles with the global loads of tile t+1 held in registers
// while tile t is computed.
//
// Launch configurations of one kernel template:
//  * decode (HW=1, KW=4, NB=1): workgroup = (split, 16-head group, token);
//    its 4 waves take interleaved 16-key tiles of the split's range, each in
//    its own LDS tile, and are merged in LDS; splits write unnormalised
//    partials combined by sparse_mla_merge_kernel (flash-decode reduction,
//    :1138-1184).  Workgroups of one (token, split) differ by a multiple of 8
//    in launch order, so they share an XCD and its L2 for the gathered rows.
//  * prefill (HW=4, KW=1, NB=2): workgroup = token x 64 heads; 4 waves share
//    every gathered 32-key tile; consecutive tokens map to the same XCD so
//    their overlapping top-k sets hit in L2.
#include <float.h>

#include <mutex>

#include "capi_internal.h"
#include "dsa_common.h"

namespace mi355dsa {

constexpr int kPitch = kLatentDim + 8;   // LDS row pitch (halves) of Q / key tiles
constexpr int kOTiles = kValueDim / 16;  // 32 O^T accumulator tiles
constexpr int kSegKeys = 2048;           // keys resolved per segment

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

struct MlaParams {
  const f16* q;
  const void* kv;
  const int32_t* idx;
  const int32_t* bt;
  const int32_t* seq_lens;
  f16* o;
  float* lse;
  // [B, H, S, 512] per-split normalised outputs o_s (S > 1); inside each 512,
  // dim d = 64 w + 16 t + 4 g + r (w, t, g, r: 8, 4, 4, 4) is stored at
  // 64 w + 16 g + 4 t + r, so the lane holding the four MFMA tiles of a wave's
  // dims writes 32 contiguous bytes
  f16* part_o;
  float* part_ml;  // [B, H, S, 2]   per-split (m_s, l_s)
  int B, n_head, topk, max_blocks, page_size, n_splits;
  int page_shift;  // log2(page_size) when it is a power of two, else -1
  int64_t n_kv_rows;
  float scale_h;    // fp16-rounded softmax scale
  float empty_lse;  // lse of a (token, head) with no valid key
  // 1: a key in range whose row does not resolve is a zero key with score 0
  // (row code -2); 0: such a key is masked (-1)
  int zero_unresolved;
  int xcd_map;  // decode workgroup order (grid a multiple of 8): 0 plain; 1 a (token,
                // split)'s head groups share an XCD
};

template <int HW, int KW, int NB>
struct MlaSmem {
  static constexpr int TN = 16 * NB;  // keys per tile per key-wave group
  struct Main {
    f16 q[HW * 16 * kPitch];
    f16 k[KW * TN * kPitch];
    float sc[KW * TN * 4];  // fp8 tile scales of the tile's rows
  };
  // key-wave merge: wave w owns dims [128w, 128w+128) (8 O^T tiles) and
  // receives the other waves' tiles of that quarter: [quarter][source][tile][lane]
  static constexpr int XSRC = KW > 1 ? KW - 1 : 1;
  union {
    Main main;
    f32x4 xbuf[KW > 1 ? KW : 1][XSRC][kOTiles / (KW > 1 ? KW : 1)][64];
  } u;
  int32_t rows[kSegKeys];
  float m[KW * 16];
  float l[KW * 16];
};

// Per-thread register stage of one tile's global loads.  Chunks of invalid
// rows are loaded from row 0 and zeroed only when stored to LDS (bit u of
// `bad`), so issuing the loads never waits for them.
template <bool KVFP8, int TN, int GT>
struct TileStage {
  static constexpr int NCH = KVFP8 ? 41 : kLatentDim / 8;  // 16-B chunks per row
  static constexpr int PER = (TN * NCH + GT - 1) / GT;
  u32x4 v[PER];
  uint32_t bad;
};

// Writes the staged chunks into the LDS key tile (and fp8 scales).
template <bool KVFP8, int TN, int GT>
__device__ __forceinline__ void tile_store(const TileStage<KVFP8, TN, GT>& st, f16* ktile,
                                           float* sc, int t0) {
  constexpr int NCH = TileStage<KVFP8, TN, GT>::NCH;
  constexpr int PER = TileStage<KVFP8, TN, GT>::PER;
#pragma unroll
  for (int u = 0; u < PER; u++) {
    const int i = t0 + u * GT;
    if (i >= TN * NCH) continue;
    const int r = i / NCH, ch = i - r * NCH;
    f16* d = ktile + r * kPitch;
    const u32x4 val = ((st.bad >> u) & 1u) ? (u32x4){0u, 0u, 0u, 0u} : st.v[u];
    if constexpr (KVFP8) {
      if (ch < 32) {
        // 16 e4m3 bytes -> 16 exact fp16 values (dims 16ch .. 16ch+15)
        u32x4 h0, h1;
#pragma unroll
        for (int w = 0; w < 4; w++) {
          const f16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)val[w], 1.0f, false);
          const f16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)val[w], 1.0f, true);
          const uint32_t a = __builtin_bit_cast(uint32_t, lo);
          const uint32_t b = __builtin_bit_cast(uint32_t, hi);
          if (w < 2) {
            h0[2 * w] = a;
            h0[2 * w + 1] = b;
          } else {
            h1[2 * (w - 2)] = a;
            h1[2 * (w - 2) + 1] = b;
          }
        }
        *reinterpret_cast<u32x4*>(d + 16 * ch) = h0;
        *reinterpret_cast<u32x4*>(d + 16 * ch + 8) = h1;
      } else if (ch == 32) {
        *reinterpret_cast<u32x4*>(sc + 4 * r) = val;  // 4 fp32 tile scales
      } else {
        *reinterpret_cast<u32x4*>(d + 512 + 8 * (ch - 33)) = val;  // RoPE fp16
      }
    } else {
      *reinterpret_cast<u32x4*>(d + 8 * ch) = val;
    }
  }
}

// Resolves idx -> block table -> cache row for keys [j0, j0+n) of token b
// into rows[0..n).  Work is done in batches of NT*8 keys; each batch issues
// its eight idx loads per thread together, then the eight block-table loads.
// resolve_idx / resolve_finish split one batch so that independent work (Q
// staging) can run while the idx loads are in flight.
constexpr int kResU = 8;

template <int NT>
__device__ __forceinline__ void resolve_idx(const MlaParams& p, int b, int j0, int n, int base,
                                            int pos[kResU]) {
  if (p.idx == nullptr) {  // dense: key j is position j
#pragma unroll
    for (int u = 0; u < kResU; u++) {
      const int j = base + u * NT + (int)threadIdx.x;
      pos[u] = (j < n) ? j0 + j : -1;
    }
    return;
  }
  const int32_t* idx_row = p.idx + (int64_t)b * p.topk + j0;
#pragma unroll
  for (int u = 0; u < kResU; u++) {
    const int j = base + u * NT + (int)threadIdx.x;
    pos[u] = (j < n) ? idx_row[j] : -1;
  }
}

template <int NT>
__device__ __forceinline__ void resolve_bt(const MlaParams& p, int b, int seq_len,
                                           const int pos[kResU], int pg[kResU], int blk[kResU]) {
  const int32_t* bt_row = p.bt + (int64_t)b * p.max_blocks;
#pragma unroll
  for (int u = 0; u < kResU; u++) {
    pg[u] = (pos[u] >= 0) ? pos[u] / p.page_size : 0;
    const bool ok = pos[u] >= 0 && pos[u] < seq_len && pg[u] < p.max_blocks;
    blk[u] = ok ? bt_row[pg[u]] : -1;
  }
}

// Row codes: >= 0 a cache row; -1 a masked key; -2 a position below seq_len
// (and inside the block table) whose row does not resolve, when
// p.zero_unresolved is set -- it reads as a zero row and stays in the
// softmax with score 0, as the reference's dense kernel (sm70_mla_decode.cu:
// 762-771) and split-decode kernel (:970-992, :1047-1053) do.
template <int NT>
__device__ __forceinline__ void resolve_store(const MlaParams& p, int n, int base, int seq_len,
                                              const int pos[kResU], const int pg[kResU],
                                              const int blk[kResU], int32_t* rows) {
#pragma unroll
  for (int u = 0; u < kResU; u++) {
    const int j = base + u * NT + (int)threadIdx.x;
    if (j < n) {
      const int64_t row = (int64_t)blk[u] * p.page_size + (pos[u] - pg[u] * p.page_size);
      const bool bad = blk[u] < 0 || row >= p.n_kv_rows;
      const bool in_range = pos[u] >= 0 && pos[u] < seq_len && pg[u] < p.max_blocks;
      rows[j] = bad ? ((p.zero_unresolved && in_range) ? -2 : -1) : (int32_t)row;
    }
  }
}

template <bool KVFP8, int HW, int KW, int NB>
__global__ void __launch_bounds__(HW * KW * 64) sparse_mla_kernel(MlaParams p) {
  using Smem = MlaSmem<HW, KW, NB>;
  constexpr int TN = Smem::TN;
  constexpr int NT = HW * KW * 64;
  constexpr int GT = HW * 64;  // gather team = the HW waves of a key-wave group
  constexpr int NACC = KVFP8 ? 5 : 1;  // QK accumulators: 4 scale tiles + RoPE
  extern __shared__ __align__(16) unsigned char smem_raw[];
  Smem& sh = *reinterpret_cast<Smem*>(smem_raw);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int hw = wave % HW, kw = wave / HW;
  const int c = lane & 15, g = lane >> 4;

  // ---- work item ----
  int b, h0, split;
  if constexpr (KW == 1) {
    // prefill: XCD-aware token order (consecutive tokens share an XCD)
    const int nx = gridDim.x, bid = blockIdx.x;
    const int xcd = bid & 7, j = bid >> 3;
    const int per = nx >> 3, rem = nx & 7;
    b = xcd * per + (xcd < rem ? xcd : rem) + j;
    h0 = blockIdx.y * (16 * HW);
    split = 0;
  } else {
    split = blockIdx.x;
    h0 = blockIdx.y * (16 * HW);
    b = blockIdx.z;
  }
  const int seq_len = p.seq_lens[b];

  // ---- this workgroup's key range (tiles of TN) ----
  // Dense mode (idx == nullptr) attends to positions [0, seq_len): the
  // token's own length is split, not the table's width.
  const int n_keys = p.idx ? p.topk : max(0, min(p.topk, seq_len));
  const int n_tiles_all = (n_keys + TN - 1) / TN;
  const int tps = (n_tiles_all + p.n_splits - 1) / p.n_splits;  // tiles per split
  const int tile_lo = split * tps;
  const int tile_hi = min(tile_lo + tps, n_tiles_all);
  constexpr int SEG_TILES = kSegKeys / TN;

  // first index batch in flight while Q is staged
  int pos0[kResU];
  const int nkeys0 = tile_lo < tile_hi ? min(min(tile_lo + SEG_TILES, tile_hi) * TN, n_keys) - tile_lo * TN : 0;
  resolve_idx<NT>(p, b, tile_lo * TN, nkeys0, 0, pos0);

  // ---- scaled Q of this workgroup's heads into LDS; the block-table loads
  // of the first index batch are issued between the Q loads and the Q
  // stores so both latencies overlap ----
  int pg0[kResU], blk0[kResU];
  {
    constexpr int QCH = HW * 16 * (kLatentDim / 8);
    constexpr int QPER = (QCH + NT - 1) / NT;
    const f16* qb = p.q + ((int64_t)b * p.n_head) * kLatentDim;
    f16x8 raw[QPER];
#pragma unroll
    for (int u = 0; u < QPER; u++) {
      const int i = threadIdx.x + u * NT;
      const int hh = i / (kLatentDim / 8), ch = i - hh * (kLatentDim / 8);
      raw[u] = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
      if (i < QCH && h0 + hh < p.n_head)
        raw[u] = *reinterpret_cast<const f16x8*>(qb + (int64_t)(h0 + hh) * kLatentDim + 8 * ch);
    }
    resolve_bt<NT>(p, b, seq_len, pos0, pg0, blk0);
#pragma unroll
    for (int u = 0; u < QPER; u++) {
      const int i = threadIdx.x + u * NT;
      if (i < QCH) {
        const int hh = i / (kLatentDim / 8), ch = i - hh * (kLatentDim / 8);
        f16x8 v;
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = (f16)((float)raw[u][e] * p.scale_h);
        *reinterpret_cast<f16x8*>(&sh.u.main.q[hh * kPitch + 8 * ch]) = v;
      }
    }
  }

  f32x4 oacc[kOTiles];
#pragma unroll
  for (int t = 0; t < kOTiles; t++) oacc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float m_run = -1e30f, l_run = 0.f;

  f16* ktile = &sh.u.main.k[kw * TN * kPitch];
  float* ksc = &sh.u.main.sc[kw * TN * 4];
  const int gt = threadIdx.x - kw * GT;  // thread index inside the gather team
  const f16* qrow = &sh.u.main.q[(16 * hw + c) * kPitch + 8 * g];

  for (int seg_lo = tile_lo; seg_lo < tile_hi; seg_lo += SEG_TILES) {
    const int seg_hi = min(seg_lo + SEG_TILES, tile_hi);
    const int j0 = seg_lo * TN;
    const int nkeys = min(seg_hi * TN, n_keys) - j0;
    __syncthreads();  // previous segment done with sh.rows
    for (int base = 0; base < nkeys; base += NT * kResU) {
      if (seg_lo == tile_lo && base == 0) {
        resolve_store<NT>(p, nkeys, base, seq_len, pos0, pg0, blk0, sh.rows);
      } else {
        int pos[kResU], pg[kResU], blk[kResU];
        resolve_idx<NT>(p, b, j0, nkeys, base, pos);
        resolve_bt<NT>(p, b, seq_len, pos, pg, blk);
        resolve_store<NT>(p, nkeys, base, seq_len, pos, pg, blk, sh.rows);
      }
    }
    __syncthreads();
    const int rounds = (seg_hi - seg_lo + KW - 1) / KW;
    // The tile of round rd for this key-wave group is seg_lo + rd*KW + kw;
    // its rows start at sh.rows[(rd*KW + kw) * TN].  Keys past the segment
    // (or past nkeys) read as row -1.
    auto tile_valid = [&](int rd) { return seg_lo + rd * KW + kw < seg_hi; };
    TileStage<KVFP8, TN, GT> stage;
    auto row_of = [&](int rd, int r) -> int {
      const int kidx = (rd * KW + kw) * TN + r;
      const int v = sh.rows[kidx < nkeys ? kidx : 0];  // unconditional LDS read
      return (tile_valid(rd) && kidx < nkeys) ? v : -1;
    };
    // global loads of round rd's tile into the register stage
    auto issue = [&](int rd) {
      constexpr int NCH = TileStage<KVFP8, TN, GT>::NCH;
      constexpr int PER = TileStage<KVFP8, TN, GT>::PER;
      constexpr int RB = KVFP8 ? kDsmlaRowBytes : kLatentDim * 2;
      int rowu[PER];
#pragma unroll
      for (int u = 0; u < PER; u++) {
        const int i = gt + u * GT;
        const int r = i / NCH;
        rowu[u] = (i < TN * NCH && p.n_kv_rows > 0) ? row_of(rd, r < TN ? r : 0) : -1;
      }
      // Every lane loads (row 0 stands in for an invalid row, so no branch
      // guards the load) and invalid rows are zeroed afterwards: masked keys
      // then carry finite zeros whatever the cache holds in unused pages.
      if (p.n_kv_rows > 0) {  // uniform: an empty cache is never read
#pragma unroll
        for (int u = 0; u < PER; u++) {
          const int i = gt + u * GT;
          const int ch = i - (i / NCH) * NCH;
          const int row = rowu[u] >= 0 ? rowu[u] : 0;
          stage.v[u] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint8_t*>(p.kv) +
                                                      (int64_t)row * RB + 16 * ch);
        }
      }
      stage.bad = 0u;
#pragma unroll
      for (int u = 0; u < PER; u++) stage.bad |= (rowu[u] < 0 ? 1u : 0u) << u;
    };
    issue(0);
    for (int rd = 0; rd < rounds; rd++) {
      tile_store<KVFP8, TN, GT>(stage, ktile, ksc, gt);
      // validity of this tile's keys (before the rows array can change)
      bool valid[NB][4];
#pragma unroll
      for (int nb = 0; nb < NB; nb++)
#pragma unroll
        for (int r = 0; r < 4; r++) valid[nb][r] = row_of(rd, 16 * nb + 4 * g + r) != -1;
      if (rd + 1 < rounds) issue(rd + 1);
      __syncthreads();

      // ---- S^T blocks ----
      f32x4 sacc[NB];
      float mt = -INFINITY;
#pragma unroll
      for (int nb = 0; nb < NB; nb++) {
        f32x4 acc[NACC];
#pragma unroll
        for (int a = 0; a < NACC; a++) acc[a] = (f32x4){0.f, 0.f, 0.f, 0.f};
        const f16* krow = ktile + (16 * nb + c) * kPitch + 8 * g;
#pragma unroll
        for (int s = 0; s < kLatentDim / 32; s++) {
          const int a = KVFP8 ? (s < 16 ? s / 4 : 4) : 0;
          acc[a] = mfma16x16x32(*reinterpret_cast<const f16x8*>(krow + 32 * s),
                                *reinterpret_cast<const f16x8*>(qrow + 32 * s), acc[a]);
        }
        f32x4 sv;
        if constexpr (KVFP8) {
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const f32x4 s4 = *reinterpret_cast<const f32x4*>(&ksc[4 * (16 * nb + 4 * g + r)]);
            sv[r] = acc[4][r] + s4[0] * acc[0][r] + s4[1] * acc[1][r] + s4[2] * acc[2][r] +
                    s4[3] * acc[3][r];
          }
        } else {
          sv = acc[0];
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
          sv[r] = valid[nb][r] ? sv[r] : -INFINITY;
          mt = fmaxf(mt, sv[r]);
        }
        sacc[nb] = sv;
      }
      mt = fmaxf(mt, shfl_xor_f(mt, 16));
      mt = fmaxf(mt, shfl_xor_f(mt, 32));
      const float m_new = fmaxf(m_run, mt);
      const float alpha = expf(m_run - m_new);
      float ls = 0.f;
      float pr[NB][4];
#pragma unroll
      for (int nb = 0; nb < NB; nb++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          pr[nb][r] = valid[nb][r] ? expf(sacc[nb][r] - m_new) : 0.f;
          ls += pr[nb][r];
        }
      ls += shfl_xor_f(ls, 16);
      ls += shfl_xor_f(ls, 32);
      l_run = l_run * alpha + ls;
      m_run = m_new;
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int t = 0; t < kOTiles; t++)
#pragma unroll
          for (int r = 0; r < 4; r++) oacc[t][r] *= alpha;
      }

      // ---- O^T += V^T P^T ----
      // P^T operands, one per fp8 scale tile (dims 128*st .. 128*st+127)
      constexpr int NST = KVFP8 ? 4 : 1;
      f16x4 pb[NST][NB];
#pragma unroll
      for (int st = 0; st < NST; st++)
#pragma unroll
        for (int nb = 0; nb < NB; nb++)
#pragma unroll
          for (int r = 0; r < 4; r++) {
            float v = pr[nb][r];
            if constexpr (KVFP8) v *= ksc[4 * (16 * nb + 4 * g + r) + st];
            pb[st][nb][r] = (f16)v;
          }
      // transpose-read source: lane i of its 16-lane group supplies row
      // (4g + i/4) (+16 per block), dims 16t + 4(i%4) .. +3
      const f16* vsrc = ktile + (4 * g + (c >> 2)) * kPitch + 4 * (c & 3);
#pragma unroll
      for (int t = 0; t < kOTiles; t++) {
        const int st = KVFP8 ? t / 8 : 0;
        if constexpr (NB == 1) {
          const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4*)(vsrc + 16 * t));
          oacc[t] = mfma16x16x16(__builtin_bit_cast(f16x4, a), pb[st][0], oacc[t]);
        } else {
          const s16x4 a0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4*)(vsrc + 16 * t));
          const s16x4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4*)(vsrc + 16 * kPitch + 16 * t));
          const f16x4 x0 = __builtin_bit_cast(f16x4, a0), x1 = __builtin_bit_cast(f16x4, a1);
          const f16x8 av = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
          const f16x8 bv = {pb[st][0][0], pb[st][0][1], pb[st][0][2], pb[st][0][3],
                            pb[st][1][0], pb[st][1][1], pb[st][1][2], pb[st][1][3]};
          oacc[t] = mfma16x16x32(av, bv, oacc[t]);
        }
      }
      __syncthreads();
    }
  }

  // ---- finalize ----
  if constexpr (KW == 1) {
    const int h = h0 + 16 * hw + c;
    if (h < p.n_head) {
      if (g == 0)
        p.lse[(int64_t)b * p.n_head + h] = (l_run > 0.f) ? (m_run + logf(l_run)) : p.empty_lse;
      const float inv = (l_run > 0.f) ? 1.f / l_run : 0.f;
      f16* orow = p.o + ((int64_t)b * p.n_head + h) * kValueDim;
#pragma unroll
      for (int t = 0; t < kOTiles; t++) {
        f16x4 v;
#pragma unroll
        for (int r = 0; r < 4; r++) v[r] = (f16)(oacc[t][r] * inv);
        *reinterpret_cast<f16x4*>(orow + 16 * t + 4 * g) = v;
      }
    }
  } else {
    // Merge the KW key-waves (HW == 1: all waves hold the same 16 heads).
    // Wave w owns O^T tiles [8w, 8w+8) (dims 128w .. 128w+127): every wave
    // scales its accumulators by exp(m_w - M), writes the tiles of the other
    // quarters to LDS, then adds the three received copies of its own
    // quarter and stores it straight from registers.
    constexpr int QT = kOTiles / KW;  // tiles per quarter
    __syncthreads();
    if (g == 0) {
      sh.m[kw * 16 + c] = m_run;
      sh.l[kw * 16 + c] = l_run;
    }
    __syncthreads();
    float M = -1e30f;
#pragma unroll
    for (int k2 = 0; k2 < KW; k2++) M = fmaxf(M, sh.m[k2 * 16 + c]);
    float L = 0.f;
#pragma unroll
    for (int k2 = 0; k2 < KW; k2++) {
      const float lk = sh.l[k2 * 16 + c];
      L += (lk > 0.f) ? lk * expf(sh.m[k2 * 16 + c] - M) : 0.f;
    }
    const float wgt = (l_run > 0.f) ? expf(m_run - M) : 0.f;
#pragma unroll
    for (int t = 0; t < kOTiles; t++) {
      const int qd = t / QT;
      if (qd != kw) {
        const int slot = kw < qd ? kw : kw - 1;
        sh.u.xbuf[qd][slot][t % QT][lane] = oacc[t] * wgt;
      }
    }
    __syncthreads();
    const bool final_out = (p.n_splits == 1);
    const int h = h0 + c;
    const int64_t bh = (int64_t)b * p.n_head + h;
    const float inv = (L > 0.f) ? 1.f / L : 0.f;
#pragma unroll
    for (int t = 0; t < kOTiles; t++) {
      if (t / QT == kw) {
        f32x4 v = oacc[t] * wgt;
#pragma unroll
        for (int sl = 0; sl < KW - 1; sl++) v += sh.u.xbuf[kw][sl][t % QT][lane];
        if (h < p.n_head) {
          if (final_out) {
            f16x4 o4;
#pragma unroll
            for (int r = 0; r < 4; r++) o4[r] = (f16)(v[r] * inv);
            *reinterpret_cast<f16x4*>(p.o + bh * kValueDim + 16 * t + 4 * g) = o4;
          } else {
            // split partial stored normalised (|o_s| <= max|V|) in fp16
            const int64_t ps = bh * p.n_splits + split;
            f16x4 o4;
#pragma unroll
            for (int r = 0; r < 4; r++) o4[r] = (f16)(v[r] * inv);
            *reinterpret_cast<f16x4*>(p.part_o + ps * kValueDim + 64 * (t / 4) + 16 * g +
                                      4 * (t % 4)) = o4;
          }
        }
      }
    }
    if (kw == 0 && g == 0 && h < p.n_head) {
      if (final_out) {
        p.lse[bh] = (L > 0.f) ? (M + logf(L)) : p.empty_lse;
      } else {
        const int64_t ps = bh * p.n_splits + split;
        p.part_ml[ps * 2 + 0] = M;
        p.part_ml[ps * 2 + 1] = L;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// fp8_ds_mla split decode with LDS-DMA gathers.
//
// Workgroup = (token, split, 16-head group), 8 waves, at most 128 keys per
// split.  A small decode batch is a latency chain (idx -> block table ->
// rows -> QK -> softmax -> PV -> partials, then the merge launch), so every
// step is shortened:
//  * each wave owns 16 keys of the split end to end: its lanes 0..15 load
//    their idx entry, then that key's block-table entry (two small dependent
//    loads; no table row is staged), and the wave gathers its own 16 raw
//    656-B rows into its LDS region with global_load_lds_dwordx4; masked
//    keys read a static zero row, so they carry finite zeros;
//  * Q rows are fetched by LDS-DMA after the block-table loads are issued,
//    so they overlap the row gathers instead of delaying the table lookup;
//  * a wave starts its QK as soon as its own rows have landed (no barrier);
//    the e4m3 bytes become exact fp16 at operand load;
//  * softmax statistics are per wave (max and sum over its 16 keys); after
//    the one barrier each wave rescales by exp(m_w - M) inside PV, where
//    P^T already takes the key's tile scale;
//  * wave w computes O^T for value dims [64w, 64w+64) over all 128 keys
//    (ds_read_b64_tr_b8 transpose reads, v_mfma_f32_16x16x32_f16), so the
//    waves' outputs are disjoint; the loop has no branch (absent keys are
//    zero rows with P = 0).
// Splits write fp16 normalised partials plus (m, l) with streaming stores;
// sparse_mla_merge_kernel combines them.  Launch order is XCD-aware when the
// grid is a multiple of 8: the head groups of a (token, split) share an XCD
// and its L2 for the gathered rows, and a token's splits stay on few XCDs so
// its Q is fetched by few L2s.
// Barriers that must not wait for in-flight gathers are raw s_barrier with
// an explicit LDS wait (__syncthreads would also drain the LDS-DMA queue).
// ---------------------------------------------------------------------------
constexpr int kDmaWaves = 8;
constexpr int kDmaThreads = 64 * kDmaWaves;
constexpr int kDecWaveKeys = 16;                                         // keys per wave
constexpr int kDmaSplitKeys = kDecWaveKeys * kDmaWaves;                  // keys per split (max)
constexpr int kDecWavePieces = kDecWaveKeys * (kDsmlaRowBytes / 16);    // 656 16-B pieces
constexpr int kDecWaveRounds = (kDecWavePieces + 63) / 64;               // 11 LDS-DMA ops
constexpr int kDecWaveBytes = kDecWaveKeys * kDsmlaRowBytes;            // 10496 B
constexpr int kQPitchPieces = kLatentDim / 8 + 1;                        // 73 x 16 B: padded Q row
constexpr int kQRounds = (16 * kQPitchPieces + kDmaThreads - 1) / kDmaThreads;  // 3
constexpr int kPPitch = kDmaSplitKeys;                                   // fp32 P row pitch (floats)
// P[head c][key] at row c, 4-key chunk (key / 4) XOR c: the stores (16 heads x
// 4 chunks per instruction) and the PV reads are then free of LDS bank
// conflicts (measured; a padded 132-float row conflicted two-way on both)
__device__ __forceinline__ int dpt_at(int c, int key) {  // key % 4 == 0
  return c * kPPitch + ((((key >> 2) ^ c) & (kDmaSplitKeys / 4 - 1)) << 2);
}
constexpr int kDimsPerWave = kValueDim / kDmaWaves;                      // 64
constexpr int kTilesPerWave = kDimsPerWave / 16;                         // 4

__device__ __align__(16) const uint8_t kZeroRow[kDsmlaRowBytes] = {};

struct DmaSmem {
  uint8_t rows[kDmaWaves][kDecWaveBytes];  // raw rows: wave w's keys 16w .. 16w+15
  uint8_t q[kQRounds * kDmaThreads * 16];  // 16 Q rows (fp16, pitch 73 x 16 B)
  float pt[16 * kPPitch];                  // P[head][key] of the split, exp(s - m_wave)
  float m[kDmaWaves * 16];
  float l[kDmaWaves * 16];
};

typedef int s32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) s32x2 lds_s32x2;
typedef __attribute__((address_space(3))) void lds_void;

// Global load of one dword issued as inline asm: the compiler does not count
// it, so the caller's explicit s_waitcnt (which takes the value as an
// operand) is the only wait, and LDS-DMA issued after it is not drained.
__device__ __forceinline__ int load_dword_async(const int32_t* ptr) {
  int v;
  asm volatile("global_load_dword %0, %1, off" : "=v"(v) : "v"(ptr) : "memory");
  return v;
}

// QK of one wave's 16 keys of raw fp8_ds_mla rows at cb: returns the scores
// of keys 4g + r (r = 0..3, accumulator rows) for head c, -inf where
// valid[r] is false.
__device__ __forceinline__ f32x4 dma_qk(const uint8_t* cb, const f16x8 (&qf)[18],
                                        const bool (&valid)[4]) {
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  // All LDS operands are read first (in-order returns let each MFMA wait only
  // for its own operand).
  const uint8_t* krow = cb + c * kDsmlaRowBytes;
  u32x4 kraw[8];
  f16x8 krope[2];
  f32x4 ksc[4];
#pragma unroll
  for (int s2 = 0; s2 < 8; s2++) kraw[s2] = *reinterpret_cast<const u32x4*>(krow + 64 * s2 + 16 * g);
#pragma unroll
  for (int s3 = 0; s3 < 2; s3++)
    krope[s3] = *reinterpret_cast<const f16x8*>(krow + 528 + 64 * s3 + 16 * g);
#pragma unroll
  for (int r = 0; r < 4; r++)
    ksc[r] = *reinterpret_cast<const f32x4*>(cb + (4 * g + r) * kDsmlaRowBytes + 512);
  __builtin_amdgcn_sched_barrier(0);
  f32x4 acc[5];
#pragma unroll
  for (int a = 0; a < 5; a++) acc[a] = (f32x4){0.f, 0.f, 0.f, 0.f};
  // step order interleaves the accumulators (consecutive MFMAs independent):
  // read pair s2 holds steps 2s2, 2s2+1 of scale tile s2/2
#pragma unroll
  for (int j = 0; j < 2; j++) {
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const int s2 = 2 * t + j;
      const f16x4 a0 = e4m3x4_to_f16x4(kraw[s2][0]), a1 = e4m3x4_to_f16x4(kraw[s2][1]);
      const f16x4 a2 = e4m3x4_to_f16x4(kraw[s2][2]), a3 = e4m3x4_to_f16x4(kraw[s2][3]);
      const f16x8 k0 = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
      const f16x8 k1 = {a2[0], a2[1], a2[2], a2[3], a3[0], a3[1], a3[2], a3[3]};
      acc[t] = mfma16x16x32(k0, qf[2 * s2], acc[t]);
      acc[4] = (j == 0 && t == 1) ? mfma16x16x32(krope[0], qf[16], acc[4])
             : (j == 1 && t == 1) ? mfma16x16x32(krope[1], qf[17], acc[4]) : acc[4];
      acc[t] = mfma16x16x32(k1, qf[2 * s2 + 1], acc[t]);
    }
  }
  f32x4 sv;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const float v = acc[4][r] + ksc[r][0] * acc[0][r] + ksc[r][1] * acc[1][r] +
                    ksc[r][2] * acc[2][r] + ksc[r][3] * acc[3][r];
    sv[r] = valid[r] ? v : -INFINITY;
  }
  return sv;
}

__global__ void __launch_bounds__(kDmaThreads) sparse_mla_decode_dma_kernel(MlaParams p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  DmaSmem& sh = *reinterpret_cast<DmaSmem*>(smem_raw);
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  // work item: head group fastest, then split, then token; with xcd_map,
  // consecutive items share an XCD (workgroup i runs on XCD i % 8), so the
  // head groups that gather the same rows share that XCD's L2
  const int G = (p.n_head + 15) / 16;
  const int nwg = (int)gridDim.x;
  const int item = p.xcd_map ? ((int)blockIdx.x % 8) * (nwg / 8) + (int)blockIdx.x / 8
                             : (int)blockIdx.x;
  const int h0 = (item % G) * 16;
  const int split = (item / G) % p.n_splits;
  const int b = item / (G * p.n_splits);
  const uint8_t* kv = reinterpret_cast<const uint8_t*>(p.kv);
  const int seq_len = p.seq_lens[b];

  // this split's key range: a multiple of 16 keys, at most kDmaSplitKeys
  // (host-guaranteed), and this wave's 16 of them
  const int kps = ((p.topk + 15) / 16 + p.n_splits - 1) / p.n_splits * 16;
  const int key_lo = min(split * kps, p.topk);
  const int nkeys = min(key_lo + kps, p.topk) - key_lo;
  const int nk_w = min(max(nkeys - kDecWaveKeys * w, 0), kDecWaveKeys);

  // ---- idx -> block table -> cache row for this wave's key of lane jl ----
  const int jl = lane & 15;
  const bool kval = jl < nk_w;
  const int32_t* ip = p.idx + (int64_t)b * p.topk + (kval ? key_lo + kDecWaveKeys * w + jl : 0);
  int pos = load_dword_async(ip);
  asm volatile("s_waitcnt vmcnt(0)" : "+v"(pos)::"memory");
  pos = kval ? pos : -1;
  const bool in_range = pos >= 0 && pos < seq_len;
  const int pg = in_range ? (p.page_shift >= 0 ? pos >> p.page_shift : pos / p.page_size) : 0;
  const bool in_table = in_range && pg < p.max_blocks;
  // a key outside the table re-reads its own idx entry (a valid address)
  int blk = load_dword_async(in_table ? p.bt + (int64_t)b * p.max_blocks + pg : ip);

  // ---- Q rows (LDS-DMA), issued behind the block-table load ----
  {
    const uint8_t* qb = reinterpret_cast<const uint8_t*>(p.q + (int64_t)b * p.n_head * kLatentDim);
#pragma unroll
    for (int u = 0; u < kQRounds; u++) {
      const int q = kDmaThreads * u + 64 * w + lane;
      const int r = q / kQPitchPieces, ch = q - r * kQPitchPieces;
      const int hq = (r < 16 && h0 + r < p.n_head) ? h0 + r : h0;
      const int chq = (r < 16 && ch < kLatentDim / 8) ? ch : 0;
      dma16(qb + (int64_t)hq * kLatentDim * 2 + 16 * chq, sh.q + 16 * (kDmaThreads * u + 64 * w));
    }
  }
  asm volatile("s_waitcnt vmcnt(%1)" : "+v"(blk) : "n"(kQRounds) : "memory");  // table entry landed
  blk = in_table ? blk : -1;
  const int64_t row = (int64_t)blk * p.page_size + (pos - pg * p.page_size);
  const int code = (blk >= 0 && row < p.n_kv_rows) ? (int)row
                                                   : ((in_table && p.zero_unresolved) ? -2 : -1);

  // ---- this wave's 16 raw rows into its LDS region: piece q = 64u + lane
  // is key q / 41, 16-byte chunk q % 41 (the last round has 16 pieces) ----
  // The piece sources come first, all eleven cross-lane reads of the row
  // codes in flight together; interleaved with the DMAs, each read waited
  // for its own LDS round trip before the next gather went out.
  uint8_t* reg = sh.rows[w];
  int rcv[kDecWaveRounds];
#pragma unroll
  for (int u = 0; u < kDecWaveRounds; u++) {
    const int q = 64 * u + lane;
    rcv[u] = __shfl(code, (q < kDecWavePieces ? q : 0) / 41, 64);
  }
  __builtin_amdgcn_sched_barrier(0);  // every shuffle is issued before the first is used
#pragma unroll
  for (int u = 0; u < kDecWaveRounds; u++) {
    const int q = 64 * u + lane;
    const int r = (q < kDecWavePieces ? q : 0) / 41, ch = q - r * 41;
    const uint8_t* src = rcv[u] >= 0 ? kv + (int64_t)rcv[u] * kDsmlaRowBytes + 16 * ch
                                     : kZeroRow + 16 * (q < kDecWavePieces ? ch : 0);
    if (u + 1 < kDecWaveRounds || lane < kDecWavePieces - 64 * (kDecWaveRounds - 1))
      dma16(src, reg + 1024 * u);
  }
  // validity of keys 4g + r (the accumulator rows of this lane)
  bool valid[4];
#pragma unroll
  for (int r = 0; r < 4; r++) valid[r] = __shfl(code, 4 * g + r, 64) != -1;

  // ---- Q fragments (B operand of S^T = K Q^T), scaled in fp16 ----
  // step 2s'+e2 (s' < 8): lane group g holds dims 64s' + 16g + 8e2 .. +7
  // step 16+s'':          lane group g holds dims 512 + 32s'' + 8g .. +7
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kDecWaveRounds) : "memory");  // this wave's Q pieces
  lds_barrier();                                                          // everyone's
  f16x8 qf[18];
  {
    const f16* qr = reinterpret_cast<const f16*>(sh.q + c * kQPitchPieces * 16);
    const f16 sc = (f16)p.scale_h;
    const f16x8 sc8 = {sc, sc, sc, sc, sc, sc, sc, sc};
#pragma unroll
    for (int s2 = 0; s2 < 8; s2++) {
      qf[2 * s2] = *reinterpret_cast<const f16x8*>(qr + 64 * s2 + 16 * g) * sc8;
      qf[2 * s2 + 1] = *reinterpret_cast<const f16x8*>(qr + 64 * s2 + 16 * g + 8) * sc8;
    }
#pragma unroll
    for (int s3 = 0; s3 < 2; s3++)
      qf[16 + s3] = *reinterpret_cast<const f16x8*>(qr + 512 + 32 * s3 + 8 * g) * sc8;
  }

  // ---- S for this wave's keys, as soon as its own rows have landed ----
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const f32x4 sv = dma_qk(reg, qf, valid);

  // ---- per-wave softmax statistics (per head c) ----
  float mt = -1e30f;
#pragma unroll
  for (int r = 0; r < 4; r++) mt = fmaxf(mt, sv[r]);
  mt = fmaxf(mt, shfl_xor_f(mt, 16));
  mt = fmaxf(mt, shfl_xor_f(mt, 32));
  f32x4 pr;
  float ls = 0.f;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    pr[r] = (sv[r] > -INFINITY) ? __expf(sv[r] - mt) : 0.f;
    ls += pr[r];
  }
  ls += shfl_xor_f(ls, 16);
  ls += shfl_xor_f(ls, 32);
  if (g == 0) {
    sh.m[w * 16 + c] = mt;
    sh.l[w * 16 + c] = ls;
  }
  // P[head c][key]: keys 16w + 4g + r
  *reinterpret_cast<f32x4*>(&sh.pt[dpt_at(c, kDecWaveKeys * w + 4 * g)]) = pr;
  lds_barrier();
  float M = -1e30f;
#pragma unroll
  for (int w2 = 0; w2 < kDmaWaves; w2++) M = fmaxf(M, sh.m[w2 * 16 + c]);
  float L = 0.f;
#pragma unroll
  for (int w2 = 0; w2 < kDmaWaves; w2++) L += __expf(sh.m[w2 * 16 + c] - M) * sh.l[w2 * 16 + c];

  // ---- O^T[dims 64w .. +64][head] over the split's keys ----
  const int st = (kDimsPerWave * w) / 128;  // fp8 scale tile of these dims
  f32x4 oacc[kTilesPerWave];
#pragma unroll
  for (int t = 0; t < kTilesPerWave; t++) oacc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < kDmaSplitKeys / 32; kb++) {
    // keys 32kb + 8g .. +7 are rows 8(g & 1) .. +7 of wave region 2kb + g/2
    const int src_w = 2 * kb + (g >> 1);
    const uint8_t* cb = sh.rows[src_w] + 8 * (g & 1) * kDsmlaRowBytes;
    // P^T operand: keys 32kb + 8g + e of head c, times the key's scale of
    // tile st and the source wave's rescale factor
    const f32x4 pa = *reinterpret_cast<const f32x4*>(&sh.pt[dpt_at(c, 32 * kb + 8 * g)]);
    const f32x4 pc = *reinterpret_cast<const f32x4*>(&sh.pt[dpt_at(c, 32 * kb + 8 * g + 4)]);
    const float alpha = __expf(sh.m[src_w * 16 + c] - M);  // the source wave's rescale factor
    float ks[8];
#pragma unroll
    for (int e = 0; e < 8; e++)
      ks[e] = *reinterpret_cast<const float*>(cb + e * kDsmlaRowBytes + 512 + 4 * st) * alpha;
    // V^T transpose reads: lane i of a 16-lane group points at key 8g + i/2
    // of the block, dims 64w + 16t + 8(i%2); lane j receives the 8 keys
    // 8g .. +7 at dim 64w + 16t + j
    const uint8_t* vsrc = cb + (c >> 1) * kDsmlaRowBytes + kDimsPerWave * w + 8 * (c & 1);
    s32x2 vt[kTilesPerWave];
#pragma unroll
    for (int t = 0; t < kTilesPerWave; t++)
      vt[t] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_s32x2*)(vsrc + 16 * t));
    f16x8 pb;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      pb[e] = (f16)(pa[e] * ks[e]);
      pb[4 + e] = (f16)(pc[e] * ks[4 + e]);
    }
#pragma unroll
    for (int t = 0; t < kTilesPerWave; t++) {
      const f16x4 lo = e4m3x4_to_f16x4((uint32_t)vt[t][0]);
      const f16x4 hi = e4m3x4_to_f16x4((uint32_t)vt[t][1]);
      const f16x8 av = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      oacc[t] = mfma16x16x32(av, pb, oacc[t]);
    }
  }

  // ---- outputs: rows 4g + r of tile t are dims 64w + 16t + 4g + r ----
  const bool final_out = (p.n_splits == 1);
  const int h = h0 + c;
  const int64_t bh = (int64_t)b * p.n_head + h;
  const float inv = (L > 0.f) ? 1.f / L : 0.f;
  if (h < p.n_head) {
    if (final_out) {
#pragma unroll
      for (int t = 0; t < kTilesPerWave; t++) {
        f16x4 o4;
#pragma unroll
        for (int r = 0; r < 4; r++) o4[r] = (f16)(oacc[t][r] * inv);
        *reinterpret_cast<f16x4*>(p.o + bh * kValueDim + kDimsPerWave * w + 16 * t + 4 * g) = o4;
      }
    } else {
      // the lane's 16 values are contiguous in the partial layout: two 16-byte
      // streaming stores (the partials are read once, by the merge kernel)
      f16x8 o8[2];
#pragma unroll
      for (int t = 0; t < kTilesPerWave; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) o8[t >> 1][4 * (t & 1) + r] = (f16)(oacc[t][r] * inv);
      u32x4* dst = reinterpret_cast<u32x4*>(p.part_o + (bh * p.n_splits + split) * kValueDim +
                                            kDimsPerWave * w + 16 * g);
      __builtin_nontemporal_store(__builtin_bit_cast(u32x4, o8[0]), dst);
      __builtin_nontemporal_store(__builtin_bit_cast(u32x4, o8[1]), dst + 1);
    }
    if (w == 0 && g == 0) {
      if (final_out) {
        p.lse[bh] = (L > 0.f) ? (M + logf(L)) : p.empty_lse;
      } else {
        const int64_t ps = bh * p.n_splits + split;
        p.part_ml[ps * 2 + 0] = M;
        p.part_ml[ps * 2 + 1] = L;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 64-head attention kernels (fp8_ds_mla and fp16 latent rows): shared
// constants.  Keys stream through LDS in 32-key tiles.  The running softmax
// max is lazy: O and l are rescaled only when a head's tile max exceeds the
// running max by more than kPfLazyMax, so p = exp(s - m) <= e^8 (well inside
// fp16) and rescales are rare; o = O / l and lse = m + ln l are unchanged by
// the choice of m.
// ---------------------------------------------------------------------------
constexpr int kPfWaves = 8;
constexpr int kPfThreads = 64 * kPfWaves;
constexpr int kPfTileKeys = 32;
constexpr float kPfLazyMax = 8.0f;

constexpr int kP3Ring = 3;  // tile slots of the fp16-row kernel
// S partials and the P table: one unpadded row of 32 keys per head, the key
// chunks (4 floats of S, 8 halves of P) permuted by an XOR with bits of the
// head.  Measured with SQ_LDS_BANK_CONFLICT on gfx950, these orders make the
// QK stores of S (16 heads x 4 chunks per instruction), the softmax reads of
// S and stores of P, and the PV reads of P conflict-free; the padded rows
// they replace (36 floats, 40 halves) cost two cycles per access.
constexpr int kP3SPitch = 32;  // floats per (dim part, head) row of S partials
constexpr int kP3PPitch = 32;  // halves per (scale tile, head) row of P
__device__ __forceinline__ int sp_at(int head, int key) {  // key % 4 == 0
  return head * kP3SPitch + ((((key >> 2) ^ head) & 7) << 2);
}
__device__ __forceinline__ int pt_at(int head, int key) {  // key % 4 == 0
  return head * kP3PPitch + ((((key >> 3) ^ (2 * ((head >> 3) & 1))) & 3) << 3) + (key & 4);
}

// reductions over aligned groups of 8 lanes (the result is bitwise equal in
// all 8 lanes: every step combines a value with its partner symmetrically)
__device__ __forceinline__ float max8(float v) {
  v = fmaxf(v, dppf<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dppf<0x4E>(v));   // quad_perm [2,3,0,1]
  return fmaxf(v, dppf<0x141>(v));  // row_half_mirror: quad 0 <-> quad 1
}
__device__ __forceinline__ float sum8(float v) {
  v += dppf<0xB1>(v);
  v += dppf<0x4E>(v);
  return v + dppf<0x141>(v);
}

// ---------------------------------------------------------------------------
// fp8_ds_mla 64-head attention (the prefill configuration, and decode batches
// of >= 8 64-head units split over keys), laid out so that MFMA work and VALU
// work run in different waves of each SIMD.  Every e4m3 byte of a tile is
// converted to fp16 once per workgroup; products with the fp16 Q and P are
// exact, and each tile scale multiplies in fp32 (QK) or into P (PV).
//
// Workgroup = one token x 64 heads (x one key split), 12 waves, three per
// SIMD (<= 168 VGPRs each):
//   * waves 0-3, QK: wave qd holds Q of all 64 heads for NoPE dims
//     [128 qd, +128) (one fp8 scale tile) and RoPE dims [512 + 16 qd, +16),
//     and computes that dim part of S^T for all 32 keys of a tile.
//   * waves 4-7, PV: wave pw owns O^T of value dims [128 pw, +128) (scale
//     tile pw) for all 64 heads.  After its PV of a tile it refills that
//     tile's slot with its own dim quarter of the tile three ahead.
//   * waves 8-11, softmax: thread t owns head t / 4 and keys 8 (t % 4) .. +7
//     of a tile; these waves also fetch each tile's scales and RoPE dims.
// A tile slot holds, for its 32 keys: four NoPE blocks (one per dim quarter),
// the scales (tile-major: tile t of key r at 128 t + 4 r) and the RoPE dims.
// The NoPE and RoPE blocks
// are chunk-major: 16-B chunk j of key r at 512 j + 16 r, so the QK operand
// reads and the PV transpose reads of 16 keys are contiguous (free of LDS
// bank conflicts) and every DMA instruction fills 1 KB (two chunks of all 32
// keys).
// A 4-slot ring, one S partial buffer and two P buffers.  Each role runs its
// own copy of the tile loop (Q and O stay in registers only in the waves that
// use them); all copies take the same barriers:
//   iteration s (s = -1 .. ntiles - 1):
//     phase 1: QK(s+1) into registers | softmax(s) -> P[s & 1], DMA of tile
//              s+3's scales and RoPE | PV(s-1), then DMA of tile s+3's dim
//              quarter into the same slot
//     barrier
//     phase 2: QK(s+1) partials -> LDS | DMA waves wait for tile s+2
//     barrier
//   then PV(ntiles - 1) and a barrier.
// ---------------------------------------------------------------------------
constexpr int kWsWaves = 12;
constexpr int kWsThreads = 64 * kWsWaves;
constexpr int kWsRing = 4;
constexpr int kWsSubBytes = kPfTileKeys * 128;                // one NoPE dim quarter
constexpr int kWsScaleOff = 4 * kWsSubBytes;                   // 16384
constexpr int kWsRopeOff = kWsScaleOff + kPfTileKeys * 16;     // 16896
constexpr int kWsSlotBytes = kWsRopeOff + kPfTileKeys * 128;   // 20992
static_assert(kWsSlotBytes == kPfTileKeys * kDsmlaRowBytes, "a slot holds whole rows");

struct WsSmem {
  uint8_t ring[kWsRing][kWsSlotBytes];
  int32_t rows[kSegKeys];
  float sp[4][64 * kP3SPitch];   // [dim quarter][head][key]
  f16 pt[2][4][64 * kP3PPitch];  // [tile parity][scale tile][head][key]: fp16(p * scale)
  f32x4 alpha[2][16];            // [tile parity][head % 16][head / 16]
  f32x4 lsum[16];
  int rescale[2];
  int tmask[kSegKeys / kPfTileKeys];  // tile of the segment holds a masked key (row -1)
};
static_assert(sizeof(WsSmem) <= 160 * 1024, "one workgroup per CU");

// The PV wave pw's part of a tile's DMA: NoPE bytes [128 pw, +128) of the 32
// keys, four instructions; lane l of instruction i fetches chunk 2 i + l / 32
// of key l % 32.  Masked keys (row < 0) read zeros.
__device__ __forceinline__ void ws_dma_nope(const uint8_t* __restrict__ kv, const int32_t* trows,
                                            uint8_t* slot, int pw, int lane) {
  const int row = trows[lane & 31];
  const uint8_t* src = (row >= 0 ? kv + (int64_t)row * kDsmlaRowBytes : kZeroRow) + 128 * pw +
                       16 * (lane >> 5);
  uint8_t* dst = slot + pw * kWsSubBytes;
  dma16_at<0>(src, dst);
  dma16_at<32>(src, dst + 1024);
  dma16_at<64>(src, dst + 2048);
  dma16_at<96>(src, dst + 3072);
}

// The softmax wave sw's part: RoPE chunks 2 sw and 2 sw + 1 of the 32 keys
// (one instruction), and for wave 0 the four scales of every key, tile-major
// (scale of tile t of key r at 128 t + 4 r; two 4-byte instructions, lane l
// taking tile l / 32 (then + 2) of key l % 32).  Per tile wave 0 issues 3 DMA
// instructions, waves 1-3 issue 1.
__device__ __forceinline__ void ws_dma_tail(const uint8_t* __restrict__ kv, const int32_t* trows,
                                            uint8_t* slot, int sw, int lane) {
  const int row = trows[lane & 31];
  const uint8_t* base = row >= 0 ? kv + (int64_t)row * kDsmlaRowBytes : kZeroRow;
  dma16(base + (kDsmlaRowBytes - 128) + 16 * (2 * sw + (lane >> 5)), slot + kWsRopeOff + 1024 * sw);
  if (sw == 0) {
    dma4(base + 512 + 4 * (lane >> 5), slot + kWsScaleOff);
    dma4(base + 520 + 4 * (lane >> 5), slot + kWsScaleOff + 256);
  }
}

// vmcnt waits of the DMA waves: at most one tile's DMAs of this wave still in
// flight (one = true), or none.
__device__ __forceinline__ void ws_wait_pv(bool one) {
  if (one) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
__device__ __forceinline__ void ws_wait_sm(bool one, int sw) {
  if (!one) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else if (sw == 0) asm volatile("s_waitcnt vmcnt(3)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(1)" ::: "memory");
}

// The workgroup's token / head base / split and key range.
struct WsCtx {
  int b, hbase, split, seq_len, k_lo, k_hi;
};

__device__ __forceinline__ WsCtx ws_ctx(const MlaParams& p) {
  WsCtx x;
  const int nx = gridDim.x, bid = blockIdx.x;
  const int xcd = bid & 7, j = bid >> 3;
  const int per = nx >> 3, rem = nx & 7;
  x.b = xcd * per + (xcd < rem ? xcd : rem) + j;  // consecutive tokens share an XCD
  x.hbase = blockIdx.y * 64;
  x.split = blockIdx.z;
  x.seq_len = p.seq_lens[x.b];
  const int kps = ((p.topk + p.n_splits - 1) / p.n_splits + kPfTileKeys - 1) / kPfTileKeys *
                  kPfTileKeys;
  x.k_lo = min(x.split * kps, p.topk);
  x.k_hi = min(x.k_lo + kps, p.topk);
  return x;
}

// idx -> block table -> row of the segment's keys, by all 768 threads, then
// a barrier.  The caller's previous barrier ended every use of rows and ring.
__device__ __forceinline__ void ws_resolve(const MlaParams& p, const WsCtx& x, int seg_lo,
                                           int nkeys, int ntiles, int32_t* rows) {
  for (int base = 0; base < ntiles * kPfTileKeys; base += kWsThreads * kResU) {
    int pos[kResU], pg[kResU], blk[kResU];
#pragma unroll
    for (int u = 0; u < kResU; u++) {
      const int j = base + u * kWsThreads + (int)threadIdx.x;
      pos[u] = (j < nkeys) ? p.idx[(int64_t)x.b * p.topk + seg_lo + j] : -1;
    }
    resolve_bt<kWsThreads>(p, x.b, x.seq_len, pos, pg, blk);
#pragma unroll
    for (int u = 0; u < kResU; u++) {
      const int j = base + u * kWsThreads + (int)threadIdx.x;
      if (j < ntiles * kPfTileKeys) {
        const int64_t row = (int64_t)blk[u] * p.page_size + (pos[u] - pg[u] * p.page_size);
        const bool in_range = pos[u] >= 0 && pos[u] < x.seq_len && pg[u] < p.max_blocks;
        rows[j] = (blk[u] < 0 || row >= p.n_kv_rows)
                      ? ((in_range && p.zero_unresolved) ? -2 : -1) : (int32_t)row;
      }
    }
  }
  lds_barrier();
}

// ---- QK waves ----
__device__ __forceinline__ void ws_qk_role(const MlaParams& p, const WsCtx& x, WsSmem& sh) {
  const int lane = threadIdx.x & 63, qd = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  // NoPE step s: lane (head c of group hg, g) holds dims 128 qd + 32 g + 8 s .. +8;
  // RoPE: dims 512 + 16 qd + 4 g .. +4 (Q scaled in fp16)
  f16x8 qn[4][4];
  f16x4 qr[4];
  {
    const f16 sc = (f16)p.scale_h;
    const f16x8 sc8 = {sc, sc, sc, sc, sc, sc, sc, sc};
    const f16x4 sc4 = {sc, sc, sc, sc};
#pragma unroll
    for (int hg = 0; hg < 4; hg++) {
      const int h = x.hbase + 16 * hg + c;
      const f16* qrow = p.q + ((int64_t)x.b * p.n_head + (h < p.n_head ? h : 0)) * kLatentDim;
#pragma unroll
      for (int s = 0; s < 4; s++)
        qn[hg][s] = *reinterpret_cast<const f16x8*>(qrow + 128 * qd + 32 * g + 8 * s) * sc8;
      qr[hg] = *reinterpret_cast<const f16x4*>(qrow + 512 + 16 * qd + 4 * g) * sc4;
    }
  }
  // S^T partial of key block kb of the tile in slot cb: keys 16 kb + 4 g + r x head 16 hg + c
  auto qk = [&](const uint8_t* cb, int kb, f32x4 (&v)[4]) {
    const int r = 16 * kb + c;
    const uint8_t* krow = cb + qd * kWsSubBytes + 16 * r;
    const u32x4 k0 = *reinterpret_cast<const u32x4*>(krow + 512 * (2 * g));
    const u32x4 k1 = *reinterpret_cast<const u32x4*>(krow + 512 * (2 * g + 1));
    const f16x4 kr = *reinterpret_cast<const f16x4*>(cb + kWsRopeOff + 512 * (2 * qd + (g >> 1)) +
                                                     16 * r + 8 * (g & 1));
    // tile qd's scales of keys 16 kb + 4 g .. +3
    const f32x4 ksc = *reinterpret_cast<const f32x4*>(cb + kWsScaleOff + 128 * qd + 4 * (16 * kb + 4 * g));
    f32x4 accn[4], accr[4];
#pragma unroll
    for (int hg = 0; hg < 4; hg++) {
      accn[hg] = (f32x4){0.f, 0.f, 0.f, 0.f};
      accr[hg] = mfma16x16x16(kr, qr[hg], (f32x4){0.f, 0.f, 0.f, 0.f});
    }
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const uint32_t d0 = s < 2 ? k0[2 * s] : k1[2 * (s - 2)];
      const uint32_t d1 = s < 2 ? k0[2 * s + 1] : k1[2 * (s - 2) + 1];
      const f16x4 a0 = e4m3x4_to_f16x4(d0), a1 = e4m3x4_to_f16x4(d1);
      const f16x8 kf = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
#pragma unroll
      for (int hg = 0; hg < 4; hg++) accn[hg] = mfma16x16x32(kf, qn[hg][s], accn[hg]);
    }
#pragma unroll
    for (int hg = 0; hg < 4; hg++)
#pragma unroll
      for (int i = 0; i < 4; i++) v[hg][i] = accr[hg][i] + ksc[i] * accn[hg][i];
  };
  for (int seg_lo = x.k_lo; seg_lo < x.k_hi; seg_lo += kSegKeys) {
    const int nkeys = min(x.k_hi - seg_lo, kSegKeys);
    const int ntiles = (nkeys + kPfTileKeys - 1) / kPfTileKeys;
    ws_resolve(p, x, seg_lo, nkeys, ntiles, sh.rows);
    lds_barrier();  // tile 0 landed
    for (int s = -1; s < ntiles; s++) {
      f32x4 v[2][4];
      const bool work = s + 1 < ntiles;
      if (work) {
        const uint8_t* cb = sh.ring[(s + 1) % kWsRing];
        qk(cb, 0, v[0]);
        qk(cb, 1, v[1]);
      }
      lds_barrier();  // softmax(s) has read sp
      if (work) {
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
          for (int hg = 0; hg < 4; hg++)
            *reinterpret_cast<f32x4*>(&sh.sp[qd][sp_at(16 * hg + c, 16 * kb + 4 * g)]) = v[kb][hg];
      }
      lds_barrier();
    }
    lds_barrier();  // PV(ntiles - 1)
  }
  lds_barrier();  // l of every head in sh.lsum
}

// ---- PV waves ----
__device__ __forceinline__ void ws_pv_role(const MlaParams& p, const WsCtx& x, WsSmem& sh) {
  const int lane = threadIdx.x & 63, pw = (threadIdx.x >> 6) - 4;
  const int c = lane & 15, g = lane >> 4;
  const uint8_t* kv = reinterpret_cast<const uint8_t*>(p.kv);
  // PV and softmax waves issue ahead of the QK waves, which have the most slack
  __builtin_amdgcn_s_setprio(2);
  f32x4 oacc[8][4];  // [dim tile][head group]: O^T of dims 128 pw + 16 t + 4 g + r, head 16 hg + c
#pragma unroll
  for (int t = 0; t < 8; t++)
#pragma unroll
    for (int hg = 0; hg < 4; hg++) oacc[t][hg] = (f32x4){0.f, 0.f, 0.f, 0.f};
  auto pv = [&](int tile) {
    const uint8_t* cb = sh.ring[tile % kWsRing];
    if (sh.rescale[tile & 1] != 0) {
      const f32x4 al = sh.alpha[tile & 1][c];
#pragma unroll
      for (int t = 0; t < 8; t++)
#pragma unroll
        for (int hg = 0; hg < 4; hg++) oacc[t][hg] *= al[hg];
    }
    f16x8 pb[4];
#pragma unroll
    for (int hg = 0; hg < 4; hg++)
      pb[hg] = *reinterpret_cast<const f16x8*>(&sh.pt[tile & 1][pw][pt_at(16 * hg + c, 8 * g)]);
    // transpose source: lane i of a 16-lane group points at key 8g + i/2,
    // dims 128 pw + 16 t + 8 (i % 2) .. +8; lane j receives keys 8g .. 8g+7
    // at dim 128 pw + 16 t + j
    const uint8_t* vrow = cb + pw * kWsSubBytes + 16 * (8 * g + (c >> 1)) + 8 * (c & 1);
#pragma unroll
    for (int t = 0; t < 8; t++) {
      const s32x2 vt = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_s32x2*)(vrow + 512 * t));
      const f16x4 lo = e4m3x4_to_f16x4((uint32_t)vt[0]);
      const f16x4 hi = e4m3x4_to_f16x4((uint32_t)vt[1]);
      const f16x8 av = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
      for (int hg = 0; hg < 4; hg++) oacc[t][hg] = mfma16x16x32(av, pb[hg], oacc[t][hg]);
    }
  };
  for (int seg_lo = x.k_lo; seg_lo < x.k_hi; seg_lo += kSegKeys) {
    const int nkeys = min(x.k_hi - seg_lo, kSegKeys);
    const int ntiles = (nkeys + kPfTileKeys - 1) / kPfTileKeys;
    ws_resolve(p, x, seg_lo, nkeys, ntiles, sh.rows);
    ws_dma_nope(kv, sh.rows, sh.ring[0], pw, lane);
    if (ntiles > 1) ws_dma_nope(kv, sh.rows + kPfTileKeys, sh.ring[1], pw, lane);
    ws_wait_pv(ntiles > 1);
    lds_barrier();  // tile 0 landed
    for (int s = -1; s < ntiles; s++) {
      const bool dma = s + 3 < ntiles;
      if (s >= 1) pv(s - 1);
      if (dma) {
        // the slot of tile s - 1: this wave's own PV reads of it have returned
        // (and nothing of the refill is scheduled into the PV above, where
        // the O accumulators hold the registers)
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        ws_dma_nope(kv, sh.rows + (s + 3) * kPfTileKeys, sh.ring[(s + 3) % kWsRing], pw, lane);
      }
      lds_barrier();
      ws_wait_pv(dma);  // tile s + 2 landed (this wave's part)
      lds_barrier();
    }
    pv(ntiles - 1);
    lds_barrier();  // the ring and rows are free for the next segment
  }
  lds_barrier();  // l of every head in sh.lsum
  // ---- outputs: o = O / l, or the split's partial ----
  const f32x4 L = sh.lsum[c];
#pragma unroll
  for (int hg = 0; hg < 4; hg++) {
    const int h = x.hbase + 16 * hg + c;
    if (h >= p.n_head) continue;
    const int64_t bh = (int64_t)x.b * p.n_head + h;
    const float inv = (L[hg] > 0.f) ? 1.f / L[hg] : 0.f;
    if (p.n_splits == 1) {
      f16* orow = p.o + bh * kValueDim + 128 * pw;
#pragma unroll
      for (int t = 0; t < 8; t++) {
        f16x4 v;
#pragma unroll
        for (int r = 0; r < 4; r++) v[r] = (f16)(oacc[t][hg][r] * inv);
        *reinterpret_cast<f16x4*>(orow + 16 * t + 4 * g) = v;
      }
    } else {
      // the split merge's partial layout (merge_dim): per 64-dim chunk j,
      // lane g's 16 values (dims 64 j + 16 t + 4 g + r, t < 4) at 64 j + 16 g
#pragma unroll
      for (int j = 0; j < 2; j++) {
        f16x8 o8[2];
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
          for (int r = 0; r < 4; r++)
            o8[t >> 1][4 * (t & 1) + r] = (f16)(oacc[4 * j + t][hg][r] * inv);
        u32x4* dst = reinterpret_cast<u32x4*>(p.part_o + (bh * p.n_splits + x.split) * kValueDim +
                                              64 * (2 * pw + j) + 16 * g);
        dst[0] = __builtin_bit_cast(u32x4, o8[0]);
        dst[1] = __builtin_bit_cast(u32x4, o8[1]);
      }
    }
  }
}

// ---- softmax waves ----
__device__ __forceinline__ void ws_sm_role(const MlaParams& p, const WsCtx& x, WsSmem& sh) {
  const int lane = threadIdx.x & 63, sw = (threadIdx.x >> 6) - 8;
  const int ts = threadIdx.x - 512;
  const int hh = ts >> 2, kq = ts & 3;  // head, keys 8 kq .. +7
  const uint8_t* kv = reinterpret_cast<const uint8_t*>(p.kv);
  constexpr float kLog2e = 1.4426950408889634f;
  float m_run = -1e30f, l_run = 0.f;  // identical in the 4 threads of a head
  // these waves and the PV waves issue ahead of the QK waves (measured: QK
  // lowest gives 25.0 ms on the 64k prefill against 27-29 ms otherwise)
  __builtin_amdgcn_s_setprio(2);
  // softmax of tile `tile` from sh.sp -> sh.pt[tile & 1], alpha.  Its LDS reads
  // (S partials, key scales, the tile's flag) are all issued before any is
  // used; the row codes are read only for a tile that holds a masked key.
  auto softmax = [&](int tile) {
    const uint8_t* cb = sh.ring[tile % kWsRing];
    const int32_t* trows = sh.rows + tile * kPfTileKeys;
    f32x4 sq[4][2];
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int hf = 0; hf < 2; hf++)
        sq[q][hf] = *reinterpret_cast<const f32x4*>(&sh.sp[q][sp_at(hh, 8 * kq + 4 * hf)]);
    f32x4 ks[4][2];  // [scale tile][key half]: scales of keys 8 kq + 4 hf .. +3
#pragma unroll
    for (int st = 0; st < 4; st++)
#pragma unroll
      for (int hf = 0; hf < 2; hf++)
        ks[st][hf] = *reinterpret_cast<const f32x4*>(cb + kWsScaleOff + 128 * st + 4 * (8 * kq + 4 * hf));
    const int masked = sh.tmask[tile];
    __builtin_amdgcn_sched_barrier(0);
    f32x4 s4[2];
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
      s4[hf] = sq[0][hf];
#pragma unroll
      for (int q = 1; q < 4; q++) s4[hf] += sq[q][hf];
    }
    if (masked) {  // wave-uniform: most tiles hold no masked key
      const int4 vr0 = *reinterpret_cast<const int4*>(trows + 8 * kq);
      const int4 vr1 = *reinterpret_cast<const int4*>(trows + 8 * kq + 4);
      const int vv[8] = {vr0.x, vr0.y, vr0.z, vr0.w, vr1.x, vr1.y, vr1.z, vr1.w};
#pragma unroll
      for (int k = 0; k < 8; k++)  // -2: zero row, a valid key
        s4[k >> 2][k & 3] = vv[k] != -1 ? s4[k >> 2][k & 3] : -INFINITY;
    }
    float mt = -1e30f;
#pragma unroll
    for (int k = 0; k < 8; k++) mt = fmaxf(mt, s4[k >> 2][k & 3]);
    mt = fmaxf(mt, dppf<0xB1>(mt));  // quad_perm [1,0,3,2]
    mt = fmaxf(mt, dppf<0x4E>(mt));  // quad_perm [2,3,0,1]
    float alpha = 1.f;
    if (mt > m_run + kPfLazyMax) {
      const float m_new = fmaxf(m_run, mt);
      alpha = __expf(m_run - m_new);
      l_run *= alpha;
      m_run = m_new;
      sh.rescale[tile & 1] = 1;
    }
    if (kq == 0) reinterpret_cast<float*>(&sh.alpha[tile & 1][hh & 15])[hh >> 4] = alpha;
    // p = 2^(s log2 e - m log2 e): m_run is finite (it starts at -1e30), so a
    // masked key (s = -inf) gives exactly 0
    const float ml = m_run * kLog2e;
    float pr[8];
#pragma unroll
    for (int k = 0; k < 8; k++)
      pr[k] = __builtin_amdgcn_exp2f(__builtin_fmaf(s4[k >> 2][k & 3], kLog2e, -ml));
    // sum in the order of the 8-thread reduction over 4-key groups: each
    // group sequentially, the two groups of a thread, then across threads
    float la = 0.f, lb = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) la += pr[k];
#pragma unroll
    for (int k = 4; k < 8; k++) lb += pr[k];
    float ls = la + lb;
    ls += dppf<0xB1>(ls);
    ls += dppf<0x4E>(ls);
    l_run += ls;
#pragma unroll
    for (int st = 0; st < 4; st++) {
      f16x8 ph;
#pragma unroll
      for (int k = 0; k < 8; k++) ph[k] = (f16)(pr[k] * ks[st][k >> 2][k & 3]);
      *reinterpret_cast<f16x8*>(&sh.pt[tile & 1][st][pt_at(hh, 8 * kq)]) = ph;
    }
  };
  for (int seg_lo = x.k_lo; seg_lo < x.k_hi; seg_lo += kSegKeys) {
    const int nkeys = min(x.k_hi - seg_lo, kSegKeys);
    const int ntiles = (nkeys + kPfTileKeys - 1) / kPfTileKeys;
    ws_resolve(p, x, seg_lo, nkeys, ntiles, sh.rows);
    {  // which tiles hold a masked key: thread ts checks rows 8 ts .. +7 (tile ts / 4)
      const bool in = 8 * ts < ntiles * kPfTileKeys;
      int m = 0;
      if (in) {
        const int4 a = *reinterpret_cast<const int4*>(sh.rows + 8 * ts);
        const int4 b = *reinterpret_cast<const int4*>(sh.rows + 8 * ts + 4);
        m = (a.x == -1) | (a.y == -1) | (a.z == -1) | (a.w == -1) | (b.x == -1) | (b.y == -1) |
            (b.z == -1) | (b.w == -1);
      }
      const unsigned long long bal = __ballot(m);
      if (in && (ts & 3) == 0) sh.tmask[ts >> 2] = ((bal >> (lane & ~3)) & 0xfull) != 0;
    }
    // (the softmax waves read the flags after the barrier below)
    ws_dma_tail(kv, sh.rows, sh.ring[0], sw, lane);
    if (ntiles > 1) ws_dma_tail(kv, sh.rows + kPfTileKeys, sh.ring[1], sw, lane);
    ws_wait_sm(ntiles > 1, sw);
    lds_barrier();  // tile 0 landed
    for (int s = -1; s < ntiles; s++) {
      const bool dma = s + 3 < ntiles;
      // the scales and RoPE of the slot of tile s - 1 were last read by
      // softmax(s - 1) and QK(s - 1), both before the previous barrier
      if (dma) ws_dma_tail(kv, sh.rows + (s + 3) * kPfTileKeys, sh.ring[(s + 3) % kWsRing], sw, lane);
      if (s >= 0) softmax(s);
      lds_barrier();  // P(s) written; PV(s - 1) done
      if (ts == 0) sh.rescale[(s + 1) & 1] = 0;  // PV(s - 1) read it; softmax(s + 1) sets it
      ws_wait_sm(dma, sw);  // tile s + 2 landed (this wave's part)
      lds_barrier();
    }
    lds_barrier();  // PV(ntiles - 1)
  }
  // ---- l and lse ----
  if (kq == 0) {
    reinterpret_cast<float*>(&sh.lsum[hh & 15])[hh >> 4] = l_run;
    const int h = x.hbase + hh;
    if (h < p.n_head) {
      const int64_t bh = (int64_t)x.b * p.n_head + h;
      if (p.n_splits == 1) {
        p.lse[bh] = (l_run > 0.f) ? (m_run + logf(l_run)) : p.empty_lse;
      } else {
        const int64_t ps = bh * p.n_splits + x.split;
        p.part_ml[ps * 2 + 0] = m_run;
        p.part_ml[ps * 2 + 1] = l_run;
      }
    }
  }
  lds_barrier();  // l of every head in sh.lsum
}

__global__ void __launch_bounds__(kWsThreads) sparse_mla_prefill_fp8_ws_kernel(MlaParams p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  WsSmem& sh = *reinterpret_cast<WsSmem*>(smem_raw);
  const WsCtx x = ws_ctx(p);
  const int w = threadIdx.x >> 6;
  if (w < 4) ws_qk_role(p, x, sh);
  else if (w < 8) ws_pv_role(p, x, sh);
  else ws_sm_role(p, x, sh);
}

// ---------------------------------------------------------------------------
// fp16-row attention over 64 heads, software-pipelined over 32-key tiles:
// the fp16 (576-half) latent cache in the prefill configuration, and dense
// decode (idx == nullptr) split over the context.
//
// Workgroup = (token, 64 heads, split), 8 waves; tiles of raw 1152-byte rows
// stream through a 3-slot LDS ring by LDS-DMA, each row at a 1184-byte pitch
// (72 pieces + two zero pads, so that the QK operand reads of 16 rows are
// free of bank conflicts).
//   * QK: wave w = (key block kb = w & 1, dim half dh = (w >> 1) & 1, head
//     half hh = w >> 2) computes S^T for keys [16 kb, +16) x heads
//     [32 hh, +32) over dims [288 dh, +288), Q of its 32 heads for those dims
//     resident in registers.  The two dim halves meet in LDS and are summed
//     in a fixed order.
//   * softmax: thread t owns head t / 8 and keys 4 (t % 8) .. +3, lazy
//     running max, DPP reductions over the 8 threads of a head; P in fp16.
//   * PV: wave w owns value dims [64 w, +64) for all 64 heads; V^T operands
//     come from ds_read_b64_tr_b16 transpose reads (4 keys each).
// Two barrier-separated phases per tile: X = {PV(i), QK(i+1)} (independent
// MFMA streams that hide each other's LDS latency), then Y = {softmax(i+1),
// LDS-DMA of tile i+3, wait for tile i+2}.
// Split s of a token covers keys [s kps, (s+1) kps) of its key list (the
// top-k list, or positions [0, seq_len) in dense mode) and, with more than
// one split, writes its normalised partial for the merge kernel.
// ---------------------------------------------------------------------------
// Row pitch 74 pieces (two zero pads): with it the QK reads of 16 rows x 4
// adjacent pieces are free of LDS bank conflicts (measured; 73 pieces, a
// 1168-byte pitch, conflicted two-way).
constexpr int kHfPitchPieces = kLatentDim / 8 + 2;                       // 74
constexpr int kHfRowPitch = kHfPitchPieces * 16;                         // 1184 B
constexpr int kHfPieces = kPfTileKeys * kHfPitchPieces;                  // 2368
constexpr int kHfRounds = (kHfPieces + kPfThreads - 1) / kPfThreads;     // 5
constexpr int kHfSlotBytes = kHfRounds * kPfThreads * 16;                // 40960
constexpr int kHfSegKeys = 1024;
constexpr int kHfHalfDims = kLatentDim / 2;                              // 288
constexpr int kHfSteps = kHfHalfDims / 32;                               // 9

struct HfSmem {
  uint8_t ring[kP3Ring][kHfSlotBytes];
  int32_t rows[kHfSegKeys];
  float sp[2][64 * kP3SPitch];  // [dim half][head][key]
  f16 pt[64 * kP3PPitch];       // [head][key]
  f32x4 alpha[16];
  f32x4 lsum[16];
  int rescale[2];
};

__device__ __forceinline__ void hf_dma_tile(const uint8_t* __restrict__ kv, const int32_t* rows,
                                            uint8_t* slot) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int row[kHfRounds];
#pragma unroll
  for (int u = 0; u < kHfRounds; u++) {
    const int q = kPfThreads * u + 64 * wave + lane;
    const int r = q / kHfPitchPieces;
    row[u] = rows[r < kPfTileKeys ? r : 0];
  }
#pragma unroll
  for (int u = 0; u < kHfRounds; u++) {
    const int q = kPfThreads * u + 64 * wave + lane;
    const int r = q / kHfPitchPieces, ch = q - r * kHfPitchPieces;
    const bool ok = q < kHfPieces && ch < kLatentDim / 8 && row[u] >= 0;
    const uint8_t* src = ok ? kv + (int64_t)row[u] * (kLatentDim * 2) + 16 * ch : kZeroRow;
    dma16(src, slot + 16 * (kPfThreads * u + 64 * wave));
  }
}

__device__ __forceinline__ void hf_wait(int k) {  // at most k tiles still in flight
  if (k <= 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kHfRounds) : "memory");
}

__global__ void __launch_bounds__(kPfThreads) mla_attn_f16_kernel(MlaParams p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  HfSmem& sh = *reinterpret_cast<HfSmem*>(smem_raw);
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int kb = w & 1, dh = (w >> 1) & 1, hh = w >> 2;  // QK role
  int b;
  {
    // XCD-aware token order: consecutive tokens share an XCD
    const int nx = gridDim.x, bid = blockIdx.x;
    const int xcd = bid & 7, j = bid >> 3;
    const int per = nx >> 3, rem = nx & 7;
    b = xcd * per + (xcd < rem ? xcd : rem) + j;
  }
  const int hbase = blockIdx.y * 64;
  const int split = blockIdx.z;
  const uint8_t* kv = reinterpret_cast<const uint8_t*>(p.kv);
  const int seq_len = p.seq_lens[b];

  // ---- this workgroup's keys ----
  const int n_keys = p.idx ? p.topk : max(0, min(p.topk, seq_len));
  const int kps = ((n_keys + p.n_splits - 1) / p.n_splits + kPfTileKeys - 1) / kPfTileKeys *
                  kPfTileKeys;
  const int k_lo = min(split * kps, n_keys);
  const int k_hi = min(k_lo + kps, n_keys);

  // ---- Q of this wave's 32 heads over its 288 dims, scaled in fp16 ----
  // step s: lane (head c of group hg, g) holds dims 288 dh + 32 s + 8 g .. +8
  f16x8 qf[2][kHfSteps];
  {
    const f16 sc = (f16)p.scale_h;
    const f16x8 sc8 = {sc, sc, sc, sc, sc, sc, sc, sc};
#pragma unroll
    for (int hg = 0; hg < 2; hg++) {
      const int h = hbase + 32 * hh + 16 * hg + c;
      const f16* qrow = p.q + ((int64_t)b * p.n_head + (h < p.n_head ? h : 0)) * kLatentDim +
                        kHfHalfDims * dh + 8 * g;
#pragma unroll
      for (int st = 0; st < kHfSteps; st++)
        qf[hg][st] = *reinterpret_cast<const f16x8*>(qrow + 32 * st) * sc8;
    }
  }

  const int sm_h = threadIdx.x >> 3, sm_k = threadIdx.x & 7;  // softmax role
  float m_run = -1e30f, l_run = 0.f;
  f32x4 oacc[4][4];  // [dim tile][head group]: O^T of dims 64 w + 16 t + ..
#pragma unroll
  for (int t = 0; t < 4; t++)
#pragma unroll
    for (int hg = 0; hg < 4; hg++) oacc[t][hg] = (f32x4){0.f, 0.f, 0.f, 0.f};

  auto qk = [&](const uint8_t* cb) {
    const uint8_t* krow = cb + (16 * kb + c) * kHfRowPitch + 2 * (kHfHalfDims * dh + 8 * g);
    f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int st = 0; st < kHfSteps; st++) {
      const f16x8 kf = *reinterpret_cast<const f16x8*>(krow + 64 * st);
#pragma unroll
      for (int hg = 0; hg < 2; hg++) acc[hg] = mfma16x16x32(kf, qf[hg][st], acc[hg]);
    }
#pragma unroll
    for (int hg = 0; hg < 2; hg++)
      *reinterpret_cast<f32x4*>(&sh.sp[dh][sp_at(32 * hh + 16 * hg + c, 16 * kb + 4 * g)]) =
          acc[hg];
  };

  auto softmax = [&](const int32_t* trows, int* flag) {
    f32x4 s4 = *reinterpret_cast<const f32x4*>(&sh.sp[0][sp_at(sm_h, 4 * sm_k)]);
    s4 += *reinterpret_cast<const f32x4*>(&sh.sp[1][sp_at(sm_h, 4 * sm_k)]);
    const int4 vr = *reinterpret_cast<const int4*>(trows + 4 * sm_k);
    const int vv[4] = {vr.x, vr.y, vr.z, vr.w};
    float mt = -1e30f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      s4[r] = vv[r] != -1 ? s4[r] : -INFINITY;  // -2: dense zero row, a valid key
      mt = fmaxf(mt, s4[r]);
    }
    mt = max8(mt);
    float alpha = 1.f;
    if (mt > m_run + kPfLazyMax) {
      const float m_new = fmaxf(m_run, mt);
      alpha = __expf(m_run - m_new);
      l_run *= alpha;
      m_run = m_new;
      *flag = 1;
    }
    if (sm_k == 0) reinterpret_cast<float*>(&sh.alpha[sm_h & 15])[sm_h >> 4] = alpha;
    f16x4 ph;
    float ls = 0.f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float pr = (s4[r] > -INFINITY) ? __expf(s4[r] - m_run) : 0.f;
      ls += pr;
      ph[r] = (f16)pr;
    }
    l_run += sum8(ls);
    *reinterpret_cast<f16x4*>(&sh.pt[pt_at(sm_h, 4 * sm_k)]) = ph;
  };

  auto pv = [&](const uint8_t* cb, bool rescale) {
    if (rescale) {
      const f32x4 al = sh.alpha[c];
#pragma unroll
      for (int t = 0; t < 4; t++)
#pragma unroll
        for (int hg = 0; hg < 4; hg++) oacc[t][hg] *= al[hg];
    }
    f16x8 pb[4];
#pragma unroll
    for (int hg = 0; hg < 4; hg++)
      pb[hg] = *reinterpret_cast<const f16x8*>(&sh.pt[pt_at(16 * hg + c, 8 * g)]);
    // transpose reads: lane i of group g supplies key 8 g + i / 4 (+4 for the
    // second read), dims 64 w + 16 t + 4 (i % 4) .. +3; lane j receives keys
    // 8 g .. 8 g + 3 (then + 4 .. + 7) at dim 64 w + 16 t + j
    const uint8_t* vsrc = cb + (8 * g + (c >> 2)) * kHfRowPitch + 2 * (64 * w + 4 * (c & 3));
    s16x4 v0[4], v1[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      v0[t] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vsrc + 32 * t));
      v1[t] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vsrc + 4 * kHfRowPitch + 32 * t));
    }
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const f16x4 x0 = __builtin_bit_cast(f16x4, v0[t]), x1 = __builtin_bit_cast(f16x4, v1[t]);
      const f16x8 av = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
      for (int hg = 0; hg < 4; hg++) oacc[t][hg] = mfma16x16x32(av, pb[hg], oacc[t][hg]);
    }
  };

  for (int seg_lo = k_lo; seg_lo < k_hi; seg_lo += kHfSegKeys) {
    const int nkeys = min(k_hi - seg_lo, kHfSegKeys);
    const int ntiles = (nkeys + kPfTileKeys - 1) / kPfTileKeys;
    lds_barrier();  // previous segment done with rows and the ring
    for (int base = 0; base < ntiles * kPfTileKeys; base += kPfThreads * kResU) {
      int pos[kResU], pg[kResU], blk[kResU];
      resolve_idx<kPfThreads>(p, b, seg_lo, nkeys, base, pos);
      resolve_bt<kPfThreads>(p, b, seq_len, pos, pg, blk);
      resolve_store<kPfThreads>(p, ntiles * kPfTileKeys, base, seq_len, pos, pg, blk, sh.rows);
    }
    lds_barrier();
    hf_dma_tile(kv, sh.rows, sh.ring[0]);
    if (ntiles > 1) hf_dma_tile(kv, sh.rows + kPfTileKeys, sh.ring[1]);
    hf_wait(ntiles > 1 ? 1 : 0);
    if (threadIdx.x == 0) sh.rescale[0] = 0;
    lds_barrier();  // tile 0 landed
    qk(sh.ring[0]);
    lds_barrier();
    softmax(sh.rows, &sh.rescale[0]);
    if (ntiles > 2) hf_dma_tile(kv, sh.rows + 2 * kPfTileKeys, sh.ring[2]);
    hf_wait(ntiles > 2 ? 1 : 0);  // tile 1 landed (this wave's part)
    lds_barrier();

    for (int i = 0; i < ntiles; i++) {
      const bool rescale = sh.rescale[i & 1] != 0;
      if (threadIdx.x == 0) sh.rescale[(i + 1) & 1] = 0;
      pv(sh.ring[i % kP3Ring], rescale);
      if (i + 1 < ntiles) qk(sh.ring[(i + 1) % kP3Ring]);
      lds_barrier();
      if (i + 1 < ntiles) {
        softmax(sh.rows + (i + 1) * kPfTileKeys, &sh.rescale[(i + 1) & 1]);
        if (i + 3 < ntiles) hf_dma_tile(kv, sh.rows + (i + 3) * kPfTileKeys, sh.ring[i % kP3Ring]);
        hf_wait(i + 3 < ntiles ? 1 : 0);
        lds_barrier();
      }
    }
  }

  // ---- outputs: o = O / l and lse, or the split's partial ----
  const bool final_out = (p.n_splits == 1);
  if (sm_k == 0) {
    reinterpret_cast<float*>(&sh.lsum[sm_h & 15])[sm_h >> 4] = l_run;
    const int h = hbase + sm_h;
    if (h < p.n_head) {
      const int64_t bh = (int64_t)b * p.n_head + h;
      if (final_out) {
        p.lse[bh] = (l_run > 0.f) ? (m_run + logf(l_run)) : p.empty_lse;
      } else {
        const int64_t ps = bh * p.n_splits + split;
        p.part_ml[ps * 2 + 0] = m_run;
        p.part_ml[ps * 2 + 1] = l_run;
      }
    }
  }
  lds_barrier();
  const f32x4 L = sh.lsum[c];
#pragma unroll
  for (int hg = 0; hg < 4; hg++) {
    const int h = hbase + 16 * hg + c;
    if (h >= p.n_head) continue;
    const int64_t bh = (int64_t)b * p.n_head + h;
    const float inv = (L[hg] > 0.f) ? 1.f / L[hg] : 0.f;
    if (final_out) {
      f16* orow = p.o + bh * kValueDim + 64 * w;
#pragma unroll
      for (int t = 0; t < 4; t++) {
        f16x4 v;
#pragma unroll
        for (int r = 0; r < 4; r++) v[r] = (f16)(oacc[t][hg][r] * inv);
        *reinterpret_cast<f16x4*>(orow + 16 * t + 4 * g) = v;
      }
    } else {
      f16x8 o8[2];
#pragma unroll
      for (int t = 0; t < 4; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) o8[t >> 1][4 * (t & 1) + r] = (f16)(oacc[t][hg][r] * inv);
      u32x4* dst = reinterpret_cast<u32x4*>(p.part_o + (bh * p.n_splits + split) * kValueDim +
                                            64 * w + 16 * g);
      dst[0] = __builtin_bit_cast(u32x4, o8[0]);
      dst[1] = __builtin_bit_cast(u32x4, o8[1]);
    }
  }
}

// Flash-decode merge of S partial states (reference :1138-1184):
// m = max_s m_s, w_s = l_s > 0 ? exp(m_s - m) l_s : 0, o = sum w_s o_s / sum w_s
// (o_s is the split's own normalised output, stored in fp16).
// One workgroup per (token, head), 128 threads x 4 dims.  Splits are taken
// 16 at a time with every (m, l) pair and partial row of the batch loaded
// together (one memory latency per batch), combined online across batches.
constexpr int kMergeMaxSplits = 128;
constexpr int kMergeBatch = 16;

// Merged outputs of NU (token, head, position) units: unit j is (bh[j], i[j]),
// the 4 natural dims held by partial-layout position 4 i (i = 16 w + 4 g + t
// holds dims 64 w + 16 t + 4 g .. +3).  Returns them normalised in o4[j] and
// (m[j], l[j]) for the lse.  The loads of all NU units in a batch of splits
// are issued before any of them is combined; each unit's arithmetic is the
// same whatever NU is.
template <int NU>
__device__ __forceinline__ void merge_units(const f16* __restrict__ part_o,
                                            const float* __restrict__ part_ml,
                                            const int64_t (&bh)[NU], int n_splits,
                                            const int (&i)[NU], f16x4 (&o4)[NU], float (&m)[NU],
                                            float (&l)[NU]) {
  const f32x2* ml[NU];
  const f16* po[NU];
  f32x4 acc[NU];
#pragma unroll
  for (int j = 0; j < NU; j++) {
    ml[j] = reinterpret_cast<const f32x2*>(part_ml + bh[j] * n_splits * 2);
    po[j] = part_o + bh[j] * n_splits * kValueDim + 4 * i[j];
    m[j] = -1e30f;
    l[j] = 0.f;
    acc[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  }
  for (int s0 = 0; s0 < n_splits; s0 += kMergeBatch) {
    f32x2 mlv[NU][kMergeBatch];
    f16x4 hv[NU][kMergeBatch];
#pragma unroll
    for (int j = 0; j < NU; j++) {
#pragma unroll
      for (int u = 0; u < kMergeBatch; u++) {
        const int s = s0 + u;
        mlv[j][u] = (s < n_splits) ? ml[j][s] : (f32x2){-1e30f, 0.f};
        hv[j][u] = (s < n_splits) ? *reinterpret_cast<const f16x4*>(po[j] + (int64_t)s * kValueDim)
                                  : (f16x4){0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int j = 0; j < NU; j++) {
      f32x4 v[kMergeBatch];
#pragma unroll
      for (int u = 0; u < kMergeBatch; u++)
#pragma unroll
        for (int r = 0; r < 4; r++) v[u][r] = (float)hv[j][u][r];
      float mb = m[j];
#pragma unroll
      for (int u = 0; u < kMergeBatch; u++)
        if (mlv[j][u][1] > 0.f) mb = fmaxf(mb, mlv[j][u][0]);
      const float resc = (l[j] > 0.f) ? expf(m[j] - mb) : 0.f;
      l[j] *= resc;
      acc[j] *= resc;
#pragma unroll
      for (int u = 0; u < kMergeBatch; u++) {
        const float w = (mlv[j][u][1] > 0.f) ? expf(mlv[j][u][0] - mb) * mlv[j][u][1] : 0.f;
        l[j] += w;
        acc[j] += v[u] * w;
      }
      m[j] = mb;
    }
  }
#pragma unroll
  for (int j = 0; j < NU; j++) {
    const float inv = (l[j] > 0.f) ? 1.f / l[j] : 0.f;
#pragma unroll
    for (int r = 0; r < 4; r++) o4[j][r] = (f16)(acc[j][r] * inv);
  }
}

__device__ __forceinline__ int merge_dim(int i) {
  return 64 * (i >> 4) + 16 * (i & 3) + 4 * ((i >> 2) & 3);
}

// xpt > 0: the decode ran with its XCD order and each token's workgroups on
// xpt = 8 / B XCDs; workgroup i (on XCD x = i % 8) then merges a head of
// token x / xpt, the heads of a token split evenly over its XCDs.  The
// numbering is a permutation of (token, head), so the results do not depend
// on it.
__global__ void __launch_bounds__(128) sparse_mla_merge_kernel(
    const f16* __restrict__ part_o, const float* __restrict__ part_ml,
    f16* __restrict__ O, float* __restrict__ LSE, int n_splits, float empty_lse, int n_head,
    int xpt) {
  int64_t bh0 = blockIdx.x;
  if (xpt > 0) {
    const int x = (int)blockIdx.x % 8, k = (int)blockIdx.x / 8;
    bh0 = (int64_t)(x / xpt) * n_head + (x % xpt) * (n_head / xpt) + k;
  }
  const int64_t bh[1] = {bh0};
  const int i[1] = {(int)threadIdx.x};
  f16x4 o4[1];
  float m[1], l[1];
  merge_units<1>(part_o, part_ml, bh, n_splits, i, o4, m, l);
  *reinterpret_cast<f16x4*>(O + bh[0] * kValueDim + merge_dim(i[0])) = o4[0];
  if (threadIdx.x == 0) LSE[bh[0]] = (l[0] > 0.f) ? (m[0] + logf(l[0])) : empty_lse;
}

// Fused epilogue of a decode layer step: the split merge and the o @ W_UV
// projection in one launch.  Workgroup = (head h, 32 output columns), 8
// waves: wave w holds the k quarter [128 (w % 4), +128) of column tile w / 4
// (16 columns).  It loads its 32 KB slice of W_UV^T first, merges all B
// (<= 16) tokens of head h into LDS with merge_units (the merge kernel's
// arithmetic; NU units per thread, their loads issued together), then
// computes each column tile as head_proj_block<1, 4> does (four 16x16x32
// MFMAs per k quarter, the quarters' partial sums added in quarter order
// through LDS), so o, lse and out are bit-identical to
// sparse_mla_merge_kernel followed by mi355_dsa_head_proj.  The workgroups
// with cb == 0 also write o and lse.  Every workgroup of a head reads the
// same partials: with xcd_map the grid is numbered so that a head's
// workgroups share one XCD (dispatch goes round-robin over the 8 XCDs), and
// its partials one L2.
constexpr int kEpiMaxTok = 16;
constexpr int kEpiCols = 32;
constexpr int kEpiThreads = 512;

struct EpiArgs {
  const f16* part_o;
  const float* part_ml;
  int n_splits;
  int B, H, V;
  float empty_lse;
  const f16* uv_t;  // [H, V, 512]
  f16* out;         // out[b * out_st + h * V + n]
  int64_t out_st;
  f16* o;           // [B, H, 512]
  float* lse;       // [B, H]
  int xcd_map;      // grid size is a multiple of 8: group a head's workgroups per XCD
};

template <int NU>
__global__ void __launch_bounds__(kEpiThreads) decode_epilogue_kernel(EpiArgs a) {
  __shared__ __align__(16) f16 so[kEpiMaxTok][kValueDim + 8];
  __shared__ f32x4 red[3][2][64];
  const int n_cb = a.V / kEpiCols;
  const int bid = a.xcd_map ? (int)(blockIdx.x % 8) * (int)(gridDim.x / 8) + (int)(blockIdx.x / 8)
                            : (int)blockIdx.x;
  const int h = bid / n_cb, cb = bid % n_cb;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = wave >> 2, kq = wave & 3;
  const int g = lane >> 4, c = lane & 15;
  const int k0 = kq * 128 + 8 * g;
  // weight fragments: column n = 32 cb + 16 t + c, dims k0 + 32 i .. +8
  f16x8 bw[4];
  const f16* wrow = a.uv_t + ((int64_t)h * a.V + kEpiCols * cb + 16 * t + c) * kValueDim + k0;
#pragma unroll
  for (int i = 0; i < 4; i++) bw[i] = *reinterpret_cast<const f16x8*>(wrow + 32 * i);
  // merge: unit u = (token u / 128, position 4 (u % 128)); a thread takes
  // units u + 512 j, j < NU, together (those past the end repeat u and are
  // not stored)
  const int n_units = a.B * 128;
  for (int u = threadIdx.x; u < n_units; u += kEpiThreads * NU) {
    int uu[NU];
    int64_t bh[NU];
    int i[NU];
#pragma unroll
    for (int j = 0; j < NU; j++) {
      uu[j] = u + kEpiThreads * j < n_units ? u + kEpiThreads * j : u;
      bh[j] = (int64_t)(uu[j] >> 7) * a.H + h;
      i[j] = uu[j] & 127;
    }
    f16x4 o4[NU];
    float m[NU], l[NU];
    merge_units<NU>(a.part_o, a.part_ml, bh, a.n_splits, i, o4, m, l);
#pragma unroll
    for (int j = 0; j < NU; j++) {
      if (j > 0 && u + kEpiThreads * j >= n_units) break;
      const int d = merge_dim(i[j]);
      *reinterpret_cast<f16x4*>(&so[uu[j] >> 7][d]) = o4[j];
      if (cb == 0) {
        *reinterpret_cast<f16x4*>(a.o + bh[j] * kValueDim + d) = o4[j];
        if (i[j] == 0) a.lse[bh[j]] = (l[j] > 0.f) ? (m[j] + logf(l[j])) : a.empty_lse;
      }
    }
  }
  __syncthreads();
  // projection: D^T = W^T X^T, lane (c, g): token c, columns 4 g + r of the tile
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const f16x8 zero = {};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const f16x8 av = c < a.B ? *reinterpret_cast<const f16x8*>(&so[c][k0 + 32 * i]) : zero;
    acc = mfma16x16x32(bw[i], av, acc);
  }
  if (kq > 0) red[kq - 1][t][lane] = acc;
  __syncthreads();
  if (kq == 0 && c < a.B) {
#pragma unroll
    for (int j = 0; j < 3; ++j) acc += red[j][t][lane];
    f16* op = a.out + (int64_t)c * a.out_st + (int64_t)h * a.V + kEpiCols * cb + 16 * t + 4 * g;
    const f16x4 ov = {(f16)acc[0], (f16)acc[1], (f16)acc[2], (f16)acc[3]};
    *reinterpret_cast<f16x4*>(op) = ov;
  }
}

// ---------------------------------------------------------------------------
// launch configuration
// ---------------------------------------------------------------------------
constexpr int kDecKW = 4;        // decode: key-waves per workgroup
constexpr int kTargetWGs = 256;  // one wave of workgroups over 256 CUs

constexpr int kPipeMinUnits = 8;  // 64-head workgroups from which a batch of > 32 heads
                                  // takes the pipelined kernels with a key split

// fp8 decode with LDS-DMA gathers: every split holds at most 128 keys (16
// per wave), so the split count is raised to ceil(topk / 128) when needed.
static bool use_dma_decode(int topk) {
  return (topk + kDmaSplitKeys - 1) / kDmaSplitKeys <= kMergeMaxSplits;
}

static int dma_decode_splits(int B, int n_head, int topk) {
  const int hg = (n_head + 15) / 16;
  const int units = (topk + kDecWaveKeys - 1) / kDecWaveKeys;  // 16-key units
  int s = kTargetWGs / (B * hg > 0 ? B * hg : 1);
  if (s >= 8) s = s / 8 * 8;
  const int min_s = (topk + kDmaSplitKeys - 1) / kDmaSplitKeys;  // <= 128 keys per split
  if (s < min_s) s = min_s;
  if (s > units) s = units;
  if (s < 1) s = 1;
  return s;
}

static int decode_splits(int B, int n_head, int topk) {
  const int hg = (n_head + 15) / 16;
  const int tiles = (topk + 15) / 16;
  int s = kTargetWGs / (B * hg > 0 ? B * hg : 1);
  const int max_s = (tiles + kDecKW - 1) / kDecKW;  // >= one tile per key-wave
  if (s > max_s) s = max_s;
  if (s > kMergeMaxSplits) s = kMergeMaxSplits;
  if (s < 1) s = 1;
  if (s >= 8) s = s / 8 * 8;  // multiple of 8: a (token, split)'s head groups share an XCD
  return s;
}

// dense decode: splits of the context so that ~256 workgroups run, at least
// four 32-key tiles each (at short contexts the split partials, 1032 B per
// split, token and head, would otherwise rival the rows read: at 4k context,
// B = 4 x 64 heads, 32 splits measured 24.8 us against 27.5 us for 64)
static int dense_splits(int B, int n_head, int max_kv) {
  const int hg = (n_head + 63) / 64;
  int s = kTargetWGs / (B * hg > 0 ? B * hg : 1);
  const int max_s = (max_kv + 4 * kPfTileKeys - 1) / (4 * kPfTileKeys);
  if (s > max_s) s = max_s;
  if (s > kMergeMaxSplits) s = kMergeMaxSplits;
  if (s < 1) s = 1;
  return s;
}

static int launch_attn_f16(const MlaParams& prm, dim3 grid, hipStream_t st) {
  const int rc = reserve_lds(reinterpret_cast<const void*>(mla_attn_f16_kernel), sizeof(HfSmem),
                             "mla_attn_f16");
  if (rc) return rc;
  mla_attn_f16_kernel<<<grid, kPfThreads, sizeof(HfSmem), st>>>(prm);
  return check_launch("mla_attn_f16");
}

template <bool KVFP8, int HW, int KW, int NB>
static int launch_mla(const MlaParams& prm, dim3 grid, hipStream_t st) {
  using Smem = MlaSmem<HW, KW, NB>;
  auto kern = sparse_mla_kernel<KVFP8, HW, KW, NB>;
  const int rc = reserve_lds(reinterpret_cast<const void*>(kern), sizeof(Smem), "sparse_mla_decode");
  if (rc) return rc;
  kern<<<grid, HW * KW * 64, sizeof(Smem), st>>>(prm);
  return check_launch("sparse_mla_decode");
}

}  // namespace mi355dsa

using namespace mi355dsa;

// Which kernel runs a sparse attention call, and over how many key splits:
//  * kPipelined: the 64-head pipelined kernels (fp8:
//    sparse_mla_prefill_fp8_ws_kernel, fp16: mla_attn_f16_kernel), workgroup
//    = (token, 64 heads, key split), tiles streamed through an LDS ring.  Taken from 256 64-head
//    workgroups up (one split), and for > 32 heads from kPipeMinUnits up
//    with round(256 / units) splits of at least two 32-key tiles each;
//  * kSplitDma: fp8 split decode with per-wave LDS-DMA gathers (16 heads per
//    workgroup, at most 128 keys per split), for small batches;
//  * kSplitReg: the register-staged split decode (fp16 rows, or fp8 top-k
//    lists too long for kSplitDma).
enum DecodeKind { kPipelined, kSplitDma, kSplitReg };
struct DecodePlan {
  DecodeKind kind;
  int S;
};

static DecodePlan plan_decode(int B, int n_head, int topk, int kv_fp8) {
  const int64_t units = (int64_t)B * ((n_head + 63) / 64);
  if (units >= kTargetWGs) return {kPipelined, 1};
  if (n_head > 32 && units >= kPipeMinUnits) {
    int s = (int)((kTargetWGs + units / 2) / units);  // nearest: fewer partial second rounds
    const int max_s = (topk + 2 * kPfTileKeys - 1) / (2 * kPfTileKeys);  // >= 2 tiles per split
    if (s > max_s) s = max_s;
    if (s > kMergeMaxSplits) s = kMergeMaxSplits;
    if (s < 1) s = 1;
    return {kPipelined, s};
  }
  if (kv_fp8 && use_dma_decode(topk)) return {kSplitDma, dma_decode_splits(B, n_head, topk)};
  return {kSplitReg, decode_splits(B, n_head, topk)};
}

extern "C" size_t mi355_dsa_sparse_mla_workspace_size(int B, int n_head, int topk) {
  if (B <= 0 || n_head <= 0 || topk <= 0) return 0;
  // the larger of the fp16 and fp8 split counts, so one size serves both
  const int s16 = plan_decode(B, n_head, topk, 0).S, s8 = plan_decode(B, n_head, topk, 1).S;
  const int S = s16 > s8 ? s16 : s8;
  if (S <= 1) return 0;
  return (size_t)B * n_head * S * (kValueDim * sizeof(f16) + 2 * sizeof(float));
}

// Sparse (idx given, topk keys per token) and dense (idx == nullptr: the
// positions [0, seq_len) of each token, topk = the block table's width in
// keys) attention share the kernels below.
static int mla_decode_impl(
    void* o, float* lse, const void* q, int B, int n_head, const void* kv_cache,
    int kv_fp8, int64_t n_kv_rows, int page_size, const int32_t* idx, int topk,
    const int32_t* block_table, int max_blocks, const int32_t* seq_lens,
    float scale, void* workspace, size_t workspace_bytes, void* stream, bool dense,
    EpiArgs* epi = nullptr) {
  DSA_CHECK(B >= 0 && n_head > 0, "n_head must be > 0");
  DSA_CHECK(topk >= 0 && max_blocks >= 0 && n_kv_rows >= 0, "bad sizes");
  DSA_CHECK(page_size > 0, "page size must be > 0");
  DSA_CHECK(n_kv_rows < ((int64_t)1 << 31), "cache has too many rows");
  if (B == 0) return MI355_DSA_OK;
  DSA_CHECK(o && lse && q && kv_cache && seq_lens, "null pointer argument");
  DSA_CHECK(dense || topk == 0 || idx, "null idx");
  DSA_CHECK(max_blocks == 0 || block_table, "null block_table");
  DSA_CHECK(aligned_to(q, 16) && aligned_to(kv_cache, 16) && aligned_to(o, 8),
            "q / kv_cache / o misaligned");
  DSA_CHECK(B <= 65535 || dense || plan_decode(B, n_head, topk, kv_fp8).kind == kPipelined,
            "B too large");
  MlaParams prm;
  prm.q = reinterpret_cast<const f16*>(q);
  prm.kv = kv_cache;
  prm.idx = dense ? nullptr : idx;
  prm.bt = block_table;
  prm.seq_lens = seq_lens;
  prm.o = reinterpret_cast<f16*>(o);
  prm.lse = lse;
  prm.part_o = nullptr;
  prm.part_ml = nullptr;
  prm.B = B;
  prm.n_head = n_head;
  prm.topk = topk;
  prm.max_blocks = max_blocks;
  prm.page_size = page_size;
  prm.page_shift = (page_size & (page_size - 1)) == 0 ? ilog2_pow2(page_size) : -1;
  prm.n_kv_rows = n_kv_rows;
  prm.scale_h = (float)(f16)scale;
  // the reference's sparse prefill kernel (taken for B >= 32 && n_head <= 16,
  // sm70_mla_decode.cu:2511) leaves lse = -1e30 + ln 1 for an empty token;
  // its dense decode writes -inf (:891-894)
  prm.empty_lse = (!dense && B >= 32 && n_head <= 16) ? -1e30f : -INFINITY;
  // an in-range key whose row does not resolve: the reference's prefill
  // kernel masks it (:1617-1628, :1705), its split-decode and dense kernels
  // read a zero row that keeps score 0 (:970-992, :762-771)
  prm.zero_unresolved = (dense || !(B >= 32 && n_head <= 16)) ? 1 : 0;
  prm.xcd_map = 0;
  hipStream_t st = as_stream(stream);

  if (dense) {
    const int S = dense_splits(B, n_head, topk);
    prm.n_splits = S;
    if (S > 1) {
      const size_t need = mi355_dsa_mla_decode_workspace_size(B, n_head, topk);
      DSA_CHECK(workspace && workspace_bytes >= need,
                "workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
      DSA_CHECK(aligned_to(workspace, 16), "workspace must be 16-byte aligned");
      prm.part_o = reinterpret_cast<f16*>(workspace);
      prm.part_ml = reinterpret_cast<float*>(prm.part_o + (size_t)B * n_head * S * kValueDim);
    }
    int rc = launch_attn_f16(prm, dim3(B, (n_head + 63) / 64, S), st);
    if (rc != MI355_DSA_OK || S == 1) return rc;
    sparse_mla_merge_kernel<<<dim3((unsigned)((int64_t)B * n_head)), 128, 0, st>>>(
        prm.part_o, prm.part_ml, prm.o, prm.lse, S, prm.empty_lse, n_head, 0);
    return check_launch("sparse_mla_merge");
  }

  const DecodePlan plan = plan_decode(B, n_head, topk, kv_fp8);
  const int S = plan.S;
  prm.n_splits = S;
  if (S > 1) {
    const size_t need = mi355_dsa_sparse_mla_workspace_size(B, n_head, topk);
    DSA_CHECK(workspace && workspace_bytes >= need,
              "workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    DSA_CHECK(aligned_to(workspace, 16), "workspace must be 16-byte aligned");
    prm.part_o = reinterpret_cast<f16*>(workspace);
    prm.part_ml = reinterpret_cast<float*>(prm.part_o + (size_t)B * n_head * S * kValueDim);
  }
  const dim3 grid(S, (n_head + 15) / 16, B);
  int rc;
  if (plan.kind == kPipelined) {
    const dim3 pgrid(B, (n_head + 63) / 64, S);
    if (kv_fp8) {
      rc = reserve_lds(reinterpret_cast<const void*>(sparse_mla_prefill_fp8_ws_kernel),
                       sizeof(WsSmem), "sparse_mla_prefill_fp8");
      if (rc) return rc;
      sparse_mla_prefill_fp8_ws_kernel<<<pgrid, kWsThreads, sizeof(WsSmem), st>>>(prm);
      rc = check_launch("sparse_mla_decode");
    } else {
      rc = launch_attn_f16(prm, pgrid, st);
    }
  } else if (plan.kind == kSplitDma) {
    const int rc2 = reserve_lds(reinterpret_cast<const void*>(sparse_mla_decode_dma_kernel),
                                sizeof(DmaSmem), "sparse_mla_decode_dma");
    if (rc2) return rc2;
    const int64_t nwg = (int64_t)S * ((n_head + 15) / 16) * B;
    DSA_CHECK(nwg < ((int64_t)1 << 31), "sparse_mla_decode: grid too large");
    prm.xcd_map = (nwg % 8 == 0) ? 1 : 0;
    sparse_mla_decode_dma_kernel<<<dim3((unsigned)nwg), kDmaThreads, sizeof(DmaSmem), st>>>(prm);
    rc = check_launch("sparse_mla_decode");
  } else {
    rc = kv_fp8 ? launch_mla<true, 1, kDecKW, 1>(prm, grid, st)
                : launch_mla<false, 1, kDecKW, 1>(prm, grid, st);
  }
  if (rc != MI355_DSA_OK || S == 1) return rc;
  if (epi) {  // the fused merge + W_UV epilogue of a layer step
    epi->part_o = prm.part_o;
    epi->part_ml = prm.part_ml;
    epi->n_splits = S;
    epi->empty_lse = prm.empty_lse;
    const int nwg = n_head * (epi->V / kEpiCols);
    epi->xcd_map = (nwg % 8 == 0) ? 1 : 0;
    if (B * 128 <= kEpiThreads)
      decode_epilogue_kernel<1><<<dim3((unsigned)nwg), kEpiThreads, 0, st>>>(*epi);
    else
      decode_epilogue_kernel<2><<<dim3((unsigned)nwg), kEpiThreads, 0, st>>>(*epi);
    return check_launch("decode_epilogue");
  }
  // merge workgroups numbered onto the XCDs that ran their token's splits
  // (C3: 13.2 -> 12.6 us per layer)
  const int xpt = (plan.kind == kSplitDma && prm.xcd_map == 1 && 8 % B == 0 &&
                   n_head % (8 / B) == 0) ? 8 / B : 0;
  sparse_mla_merge_kernel<<<dim3((unsigned)((int64_t)B * n_head)), 128, 0, st>>>(
      prm.part_o, prm.part_ml, prm.o, prm.lse, S, prm.empty_lse, n_head, xpt);
  return check_launch("sparse_mla_merge");
}

extern "C" int mi355_dsa_sparse_mla_decode(
    void* o, float* lse, const void* q, int B, int n_head, const void* kv_cache,
    int kv_fp8, int64_t n_kv_rows, int page_size, const int32_t* idx, int topk,
    const int32_t* block_table, int max_blocks, const int32_t* seq_lens,
    float scale, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  return mla_decode_impl(o, lse, q, B, n_head, kv_cache, kv_fp8, n_kv_rows, page_size, idx,
                         topk, block_table, max_blocks, seq_lens, scale, workspace,
                         workspace_bytes, stream, false);
}

// Attention of one DSA decode layer step with its W_UV projection:
// mi355_dsa_sparse_mla_decode into o / lse, then out = o @ W_UV per head
// (mi355_dsa_head_proj with wt = uv_t [H, V, 512], K = 512, N = V).  When
// the decode splits the keys (workspace needed), B <= 16 and V is a multiple
// of 32, the merge and the projection run as one launch
// (decode_epilogue_kernel); the results are bit-identical either way.
extern "C" int mi355_dsa_decode_layer_attention(
    void* out, int64_t out_tok_stride, void* o, float* lse, const void* q, int B, int n_head,
    const void* kv_cache, int kv_fp8, int64_t n_kv_rows, int page_size, const int32_t* idx,
    int topk, const int32_t* block_table, int max_blocks, const int32_t* seq_lens, float scale,
    const void* uv_t, int V, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  DSA_CHECK(V > 0 && B >= 0 && n_head > 0, "decode_layer_attention: bad sizes");
  if (B == 0) return MI355_DSA_OK;
  DSA_CHECK(out && uv_t, "decode_layer_attention: null pointer argument");
  DSA_CHECK(out_tok_stride >= (int64_t)n_head * V,
            "decode_layer_attention: out rows must hold n_head * V values");
  DSA_CHECK(topk >= 0, "bad sizes");
  const DecodePlan plan = plan_decode(B, n_head, topk, kv_fp8);
  const bool fused = plan.S > 1 && B <= kEpiMaxTok && V % kEpiCols == 0 &&
                     (int64_t)n_head * (V / kEpiCols) < ((int64_t)1 << 31) &&
                     aligned_to(uv_t, 16) && aligned_to(out, 8) && out_tok_stride % 4 == 0;
  if (!fused) {
    int rc = mla_decode_impl(o, lse, q, B, n_head, kv_cache, kv_fp8, n_kv_rows, page_size, idx,
                             topk, block_table, max_blocks, seq_lens, scale, workspace,
                             workspace_bytes, stream, false);
    if (rc != MI355_DSA_OK) return rc;
    return mi355_dsa_head_proj(out, out_tok_stride, V, o, (int64_t)n_head * kValueDim, kValueDim,
                               uv_t, B, n_head, V, kValueDim, 0, stream);
  }
  EpiArgs epi{};
  epi.B = B;
  epi.H = n_head;
  epi.V = V;
  epi.uv_t = reinterpret_cast<const f16*>(uv_t);
  epi.out = reinterpret_cast<f16*>(out);
  epi.out_st = out_tok_stride;
  epi.o = reinterpret_cast<f16*>(o);
  epi.lse = lse;
  return mla_decode_impl(o, lse, q, B, n_head, kv_cache, kv_fp8, n_kv_rows, page_size, idx, topk,
                         block_table, max_blocks, seq_lens, scale, workspace, workspace_bytes,
                         stream, false, &epi);
}

// ---------------------------------------------------------------------------
// Allocation-free variant of mi355_dsa_sparse_mla_decode.  Its split partials
// live in a file-scope device array of kNoAllocScratchBytes instead of a
// caller workspace.  Host code never uses the array's name as an address:
// the device address comes from hipGetSymbolAddress, once per device, with
// that device current, on the entry point's first call there.  Every call on
// a device shares that device's array (the kernels write every partial they
// read, so nothing needs clearing between calls); calls that overlap on one
// device race on it.
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kNoAllocMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kNoAllocMaxDevices];  // zero-initialised: not yet looked up

static int noalloc_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0)
    return set_error(MI355_DSA_EHIP, "sparse_mla_decode_noalloc: no current HIP device");
  if (dev >= kNoAllocMaxDevices)
    return set_error(MI355_DSA_EINVAL, "sparse_mla_decode_noalloc: device %d >= %d", dev,
                     kNoAllocMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return set_error(MI355_DSA_EHIP, "sparse_mla_decode_noalloc: scratch lookup failed: %s",
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MI355_DSA_OK;
}

extern "C" size_t mi355_dsa_sparse_mla_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int mi355_dsa_sparse_mla_decode_noalloc(
    void* o, float* lse, const void* q, int B, int n_head, const void* kv_cache, int kv_fp8,
    int64_t n_kv_rows, int page_size, const int32_t* idx, int topk,
    const int32_t* block_table, int max_blocks, const int32_t* seq_lens, float scale,
    void* stream) {
  clear_error();
  const size_t need = mi355_dsa_sparse_mla_workspace_size(B, n_head, topk);
  DSA_CHECK(need <= kNoAllocScratchBytes,
            "sparse_mla_decode_noalloc: B=%d x n_head=%d x topk=%d needs %zu bytes of split "
            "scratch, more than its %zu-byte maximum; call mi355_dsa_sparse_mla_decode with a "
            "workspace instead",
            B, n_head, topk, need, kNoAllocScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    const int rc = noalloc_scratch(&ws);
    if (rc != MI355_DSA_OK) return rc;
  }
  return mla_decode_impl(o, lse, q, B, n_head, kv_cache, kv_fp8, n_kv_rows, page_size, idx,
                         topk, block_table, max_blocks, seq_lens, scale, ws, need, stream, false);
}

extern "C" size_t mi355_dsa_mla_decode_workspace_size(int B, int n_head, int max_kv) {
  if (B <= 0 || n_head <= 0 || max_kv <= 0) return 0;
  const int S = dense_splits(B, n_head, max_kv);
  if (S <= 1) return 0;
  return (size_t)B * n_head * S * (kValueDim * sizeof(f16) + 2 * sizeof(float));
}

extern "C" int mi355_dsa_mla_decode(void* o, float* lse, const void* q, int B, int n_head,
                                    const void* kv_cache, int64_t n_kv_rows, int page_size,
                                    const int32_t* block_table, int max_blocks,
                                    const int32_t* seq_lens, float scale, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  clear_error();
  DSA_CHECK(max_blocks >= 0 && page_size > 0 && (int64_t)max_blocks * page_size < (1 << 30),
            "mla_decode: block table too wide");
  const int max_kv = max_blocks * page_size;
  return mla_decode_impl(o, lse, q, B, n_head, kv_cache, 0, n_kv_rows, page_size, nullptr,
                         max_kv, block_table, max_blocks, seq_lens, scale, workspace,
                         workspace_bytes, stream, true);
}
