// Sparse (top-k) MLA attention over the paged latent cache, decode and
// prefill, on gfx950 MFMA.  Semantics follow sm70_sparse_mla_decode
// (reference csrc/attention/sm70_mla_decode.cu:918-1184, host :2457-2616):
//   * key j = idx[b,i] is used iff 0 <= j < seq_len[b] and its paged row
//     resolves inside the cache (:977-992);
//   * q is pre-multiplied by fp16(scale) and rounded to fp16 (:1016-1018);
//   * online softmax with m initialised to -1e30, masked scores -inf (:961,
//     :1047-1067); P is rounded to fp16 for the PV product (:1068), the
//     running sum uses the fp32 p;
//   * o = PV / l in fp16, lse = m + ln l, or o = 0 and lse = -inf when no
//     key is valid (merge convention, :1175-1183).
//
// MFMA formulation (one wave owns 16 heads):
//   S^T[key][head] = K[key][:] . Qs[head][:]   (v_mfma_f32_16x16x32_f16,
//                    18 steps over the 576 dims; D: lane = head, rows = keys)
//   O^T[dim][head] += V^T[dim][key] . P^T[key][head]  (v_mfma_f32_16x16x16_f16)
// S^T's accumulator layout (lane c = head, rows 4g..4g+3 = keys) is exactly
// the B-operand layout of the x16 PV step, so P never leaves registers; the
// softmax reductions over keys are two lane shuffles.  O^T lives in 32
// accumulator tiles (128 fp32 per lane).
//
// Two launch configurations of one kernel template:
//  * decode (HW=1, KW=4): workgroup = (split, 16-head group, token); its 4
//    waves take interleaved 16-key tiles of the split's key range, each into
//    its own LDS tile, and are merged in LDS at the end.  Splits write
//    unnormalised partials that sparse_mla_merge_kernel combines (the
//    flash-decode reduction of :1138-1184).  Workgroups sharing a (token,
//    split) differ by a multiple of 8 in launch order, so they land on the
//    same XCD and share its L2 for the gathered rows.
//  * prefill (HW=4, KW=1): workgroup = token x 64 heads; the 4 waves share
//    every gathered 32-key tile (each latent row crosses HBM/MALL once per
//    token), and consecutive tokens are mapped to the same XCD so their
//    overlapping top-k sets hit in L2.
#include <float.h>

#include "capi_internal.h"
#include "dsa_common.h"

namespace mi355dsa {

constexpr int kPitch = kLatentDim + 8;  // LDS row pitch (halves) of Q / key tiles
constexpr int kOTiles = kValueDim / 16;  // 32 O^T accumulator tiles

struct MlaParams {
  const f16* q;
  const void* kv;
  const int32_t* idx;
  const int32_t* bt;
  const int32_t* seq_lens;
  f16* o;
  float* lse;
  float* part_o;   // [B, H, S, 512] unnormalised partial outputs (S > 1)
  float* part_ml;  // [B, H, S, 2]   partial (m, l)
  int B, n_head, topk, max_blocks, page_size, n_splits;
  int64_t n_kv_rows;
  float scale_h;  // fp16-rounded softmax scale
};

template <int HW, int KW, int NB>
struct MlaSmem {
  static constexpr int TN = 16 * NB;  // keys per tile per key-wave group
  f16 q[HW * 16 * kPitch];
  f16 k[KW * TN * kPitch];
  int64_t row[KW * TN];
  float m[KW * 16];
  float l[KW * 16];
};

// Gathers one tile (TN rows) into LDS as fp16, dequantising fp8_ds_mla rows
// as fp16_rn(e4m3 * tile_scale).  Invalid rows become zeros.
template <bool KVFP8, int TN>
__device__ __forceinline__ void gather_tile(const void* kv, const int64_t* rows,
                                            f16* dst, int t0, int nthreads) {
  if constexpr (KVFP8) {
    constexpr int NCH = 40;  // 32 e4m3 chunks + 8 RoPE chunks of 16 bytes
    for (int i = t0; i < TN * NCH; i += nthreads) {
      const int r = i / NCH, ch = i - r * NCH;
      const int64_t row = rows[r];
      f16* d = dst + r * kPitch;
      if (ch < 32) {
        f16x8 h0 = (f16x8){0, 0, 0, 0, 0, 0, 0, 0}, h1 = h0;
        if (row >= 0) {
          const uint8_t* rp = reinterpret_cast<const uint8_t*>(kv) + row * (int64_t)kDsmlaRowBytes;
          const u32x4 raw = *reinterpret_cast<const u32x4*>(rp + 16 * ch);
          const float sc = *reinterpret_cast<const float*>(rp + 512 + 4 * (ch >> 3)) * 256.0f;
#pragma unroll
          for (int w = 0; w < 4; w++) {
            float v[4];
            e4m3x4_to_f32_div256(raw[w], v);
#pragma unroll
            for (int e = 0; e < 4; e++) {
              const f16 h = (f16)(v[e] * sc);
              if (w < 2) h0[4 * w + e] = h; else h1[4 * (w - 2) + e] = h;
            }
          }
        }
        *reinterpret_cast<f16x8*>(d + 16 * ch) = h0;
        *reinterpret_cast<f16x8*>(d + 16 * ch + 8) = h1;
      } else {
        const int cc = ch - 32;
        u32x4 raw = {0u, 0u, 0u, 0u};
        if (row >= 0)
          raw = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint8_t*>(kv) +
                                               row * (int64_t)kDsmlaRowBytes + 528 + 16 * cc);
        *reinterpret_cast<u32x4*>(d + 512 + 8 * cc) = raw;
      }
    }
  } else {
    constexpr int NCH = kLatentDim / 8;  // 72 chunks of 16 bytes
    for (int i = t0; i < TN * NCH; i += nthreads) {
      const int r = i / NCH, ch = i - r * NCH;
      const int64_t row = rows[r];
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (row >= 0)
        raw = *reinterpret_cast<const u32x4*>(reinterpret_cast<const f16*>(kv) +
                                             row * kLatentDim + 8 * ch);
      *reinterpret_cast<u32x4*>(dst + r * kPitch + 8 * ch) = raw;
    }
  }
}

// Resolves the cache row of top-k slot j of token b (-1 if not used).
__device__ __forceinline__ int64_t resolve_row(const MlaParams& p, int b, int j, int seq_len) {
  if (j >= p.topk) return -1;
  const int pos = p.idx[(int64_t)b * p.topk + j];
  if (pos < 0 || pos >= seq_len) return -1;
  const int pg = pos / p.page_size;
  if (pg >= p.max_blocks) return -1;
  const int blk = p.bt[(int64_t)b * p.max_blocks + pg];
  const int64_t row = (int64_t)blk * p.page_size + (pos - pg * p.page_size);
  return (blk < 0 || row >= p.n_kv_rows) ? -1 : row;
}

template <bool KVFP8, int HW, int KW, int NB>
__global__ void __launch_bounds__(HW * KW * 64) sparse_mla_kernel(MlaParams p) {
  using Smem = MlaSmem<HW, KW, NB>;
  constexpr int TN = Smem::TN;
  constexpr int NT = HW * KW * 64;
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

  // ---- scaled Q of this workgroup's heads into LDS, then registers ----
  {
    const f16* qb = p.q + ((int64_t)b * p.n_head) * kLatentDim;
    for (int i = threadIdx.x; i < HW * 16 * (kLatentDim / 8); i += NT) {
      const int hh = i / (kLatentDim / 8), ch = i - hh * (kLatentDim / 8);
      const int h = h0 + hh;
      f16x8 v = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
      if (h < p.n_head) {
        const f16x8 raw = *reinterpret_cast<const f16x8*>(qb + (int64_t)h * kLatentDim + 8 * ch);
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = (f16)((float)raw[e] * p.scale_h);
      }
      *reinterpret_cast<f16x8*>(&sh.q[hh * kPitch + 8 * ch]) = v;
    }
  }
  __syncthreads();
  // B operand of S^T: head column c of this wave, dims 32s + 8g .. +8
  f16x8 qreg[kLatentDim / 32];
#pragma unroll
  for (int s = 0; s < kLatentDim / 32; s++)
    qreg[s] = *reinterpret_cast<const f16x8*>(&sh.q[(16 * hw + c) * kPitch + 32 * s + 8 * g]);

  f32x4 oacc[kOTiles];
#pragma unroll
  for (int t = 0; t < kOTiles; t++) oacc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float m_run = -1e30f, l_run = 0.f;

  // ---- key tiles of this workgroup ----
  const int n_tiles_all = (p.topk + TN - 1) / TN;
  const int tps = (n_tiles_all + p.n_splits - 1) / p.n_splits;  // tiles per split
  const int tile_lo = split * tps;
  const int tile_hi = min(tile_lo + tps, n_tiles_all);
  const int rounds = (max(tile_hi - tile_lo, 0) + KW - 1) / KW;

  f16* ktile = &sh.k[kw * TN * kPitch];
  int64_t* krow = &sh.row[kw * TN];
  const int gt = threadIdx.x - kw * HW * 64;  // thread index inside the key-wave group

  for (int rd = 0; rd < rounds; rd++) {
    const int tile = tile_lo + rd * KW + kw;
    const bool have = tile < tile_hi;
    for (int r = gt; r < TN; r += HW * 64)
      krow[r] = have ? resolve_row(p, b, tile * TN + r, seq_len) : -1;
    __syncthreads();
    gather_tile<KVFP8, TN>(p.kv, krow, ktile, gt, HW * 64);
    __syncthreads();

    // S^T blocks
    f32x4 sacc[NB];
    bool valid[NB][4];
    float mt = -INFINITY;
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      const f16* krows = ktile + (16 * nb + c) * kPitch + 8 * g;
#pragma unroll
      for (int s = 0; s < kLatentDim / 32; s++)
        acc = mfma16x16x32(*reinterpret_cast<const f16x8*>(krows + 32 * s), qreg[s], acc);
#pragma unroll
      for (int r = 0; r < 4; r++) {
        valid[nb][r] = krow[16 * nb + 4 * g + r] >= 0;
        acc[r] = valid[nb][r] ? acc[r] : -INFINITY;
        mt = fmaxf(mt, acc[r]);
      }
      sacc[nb] = acc;
    }
    mt = fmaxf(mt, shfl_xor_f(mt, 16));
    mt = fmaxf(mt, shfl_xor_f(mt, 32));
    const float m_new = fmaxf(m_run, mt);
    const float alpha = expf(m_run - m_new);
    float ls = 0.f;
    f16x4 pb[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float pr = valid[nb][r] ? expf(sacc[nb][r] - m_new) : 0.f;
        ls += pr;
        pb[nb][r] = (f16)pr;
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
    // O^T += V^T P^T
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
      const f16* vk = ktile + (16 * nb + 4 * g) * kPitch + c;
#pragma unroll
      for (int t = 0; t < kOTiles; t++) {
        f16x4 a;
#pragma unroll
        for (int e = 0; e < 4; e++) a[e] = vk[e * kPitch + 16 * t];
        oacc[t] = mfma16x16x16(a, pb[nb], oacc[t]);
      }
    }
    __syncthreads();
  }

  // ---- finalize ----
  if constexpr (KW == 1) {
    const int h = h0 + 16 * hw + c;
    if (h < p.n_head && g == 0) {
      p.lse[(int64_t)b * p.n_head + h] = (l_run > 0.f) ? (m_run + logf(l_run)) : -INFINITY;
    }
    if (h < p.n_head) {
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
    // merge the KW key-waves in LDS (HW == 1: every wave holds the same 16 heads)
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
    float* acc = reinterpret_cast<float*>(sh.k);  // [16 heads][512] fp32 (32 KB)
    for (int k2 = 0; k2 < KW; k2++) {
      if (kw == k2) {
#pragma unroll
        for (int t = 0; t < kOTiles; t++)
#pragma unroll
          for (int r = 0; r < 4; r++) {
            float* dst = &acc[c * kValueDim + 16 * t + 4 * g + r];
            const float v = oacc[t][r] * wgt;
            *dst = (k2 == 0) ? v : (*dst + v);
          }
      }
      __syncthreads();
    }
    // write out: thread -> (head, 4 dims)
    const bool final_out = (p.n_splits == 1);
    for (int i = threadIdx.x; i < 16 * (kValueDim / 4); i += NT) {
      const int hh = i / (kValueDim / 4), d4 = i - hh * (kValueDim / 4);
      const int h = h0 + hh;
      if (h >= p.n_head) continue;
      const float Mh = [&] {
        float mm = -1e30f;
        for (int k2 = 0; k2 < KW; k2++) mm = fmaxf(mm, sh.m[k2 * 16 + hh]);
        return mm;
      }();
      float Lh = 0.f;
      for (int k2 = 0; k2 < KW; k2++) {
        const float lk = sh.l[k2 * 16 + hh];
        Lh += (lk > 0.f) ? lk * expf(sh.m[k2 * 16 + hh] - Mh) : 0.f;
      }
      const f32x4 v = *reinterpret_cast<const f32x4*>(&acc[hh * kValueDim + 4 * d4]);
      const int64_t bh = (int64_t)b * p.n_head + h;
      if (final_out) {
        const float inv = (Lh > 0.f) ? 1.f / Lh : 0.f;
        f16x4 o4;
#pragma unroll
        for (int r = 0; r < 4; r++) o4[r] = (f16)(v[r] * inv);
        *reinterpret_cast<f16x4*>(p.o + bh * kValueDim + 4 * d4) = o4;
        if (d4 == 0) p.lse[bh] = (Lh > 0.f) ? (Mh + logf(Lh)) : -INFINITY;
      } else {
        const int64_t ps = bh * p.n_splits + split;
        *reinterpret_cast<f32x4*>(p.part_o + ps * kValueDim + 4 * d4) = v;
        if (d4 == 0) {
          p.part_ml[ps * 2 + 0] = Mh;
          p.part_ml[ps * 2 + 1] = Lh;
        }
      }
    }
    (void)L;
  }
}

// Flash-decode merge of S partial states (reference :1138-1184):
// m = max_s m_s, w_s = l_s > 0 ? exp(m_s - m) : 0, o = sum w_s P_O_s / sum w_s l_s.
// One workgroup per (token, head), 128 threads x 4 dims.
__global__ void __launch_bounds__(128) sparse_mla_merge_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_ml,
    f16* __restrict__ O, float* __restrict__ LSE, int n_splits) {
  const int64_t bh = blockIdx.x;
  const float* ml = part_ml + bh * n_splits * 2;
  float m = -1e30f;
  for (int s = 0; s < n_splits; s++) m = fmaxf(m, ml[2 * s]);
  float l = 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const int d = 4 * threadIdx.x;
  for (int s = 0; s < n_splits; s++) {
    const float ls = ml[2 * s + 1];
    if (ls > 0.f) {
      const float w = expf(ml[2 * s] - m);
      l += ls * w;
      const f32x4 v = *reinterpret_cast<const f32x4*>(part_o + (bh * n_splits + s) * kValueDim + d);
#pragma unroll
      for (int r = 0; r < 4; r++) acc[r] += v[r] * w;
    }
  }
  const float inv = (l > 0.f) ? 1.f / l : 0.f;
  f16x4 o4;
#pragma unroll
  for (int r = 0; r < 4; r++) o4[r] = (f16)(acc[r] * inv);
  *reinterpret_cast<f16x4*>(O + bh * kValueDim + d) = o4;
  if (threadIdx.x == 0) LSE[bh] = (l > 0.f) ? (m + logf(l)) : -INFINITY;
}

// ---------------------------------------------------------------------------
// launch configuration
// ---------------------------------------------------------------------------
constexpr int kDecKW = 4;       // decode: key-waves per workgroup
constexpr int kTargetWGs = 256;  // one wave of workgroups over 256 CUs

static bool use_prefill_config(int B, int n_head) {
  return (int64_t)B * ((n_head + 63) / 64) >= kTargetWGs;
}

static int decode_splits(int B, int n_head, int topk) {
  const int hg = (n_head + 15) / 16;
  const int tiles = (topk + 15) / 16;
  int s = kTargetWGs / (B * hg > 0 ? B * hg : 1);
  const int max_s = (tiles + kDecKW - 1) / kDecKW;  // >= one tile per key-wave
  if (s > max_s) s = max_s;
  if (s < 1) s = 1;
  if (s >= 8) s = s / 8 * 8;  // multiple of 8: a (token, split)'s head groups share an XCD
  return s;
}

template <bool KVFP8, int HW, int KW, int NB>
static int launch_mla(const MlaParams& prm, dim3 grid, hipStream_t st) {
  using Smem = MlaSmem<HW, KW, NB>;
  auto kern = sparse_mla_kernel<KVFP8, HW, KW, NB>;
  static bool attr = false;
  if (!attr) {
    hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(Smem));
    attr = true;
  }
  kern<<<grid, HW * KW * 64, sizeof(Smem), st>>>(prm);
  return check_launch("sparse_mla_decode");
}

}  // namespace mi355dsa

using namespace mi355dsa;

extern "C" size_t mi355_dsa_sparse_mla_workspace_size(int B, int n_head, int topk) {
  if (B <= 0 || n_head <= 0 || topk <= 0) return 0;
  if (use_prefill_config(B, n_head)) return 0;
  const int S = decode_splits(B, n_head, topk);
  if (S <= 1) return 0;
  return (size_t)B * n_head * S * (kValueDim + 2) * sizeof(float);
}

extern "C" int mi355_dsa_sparse_mla_decode(
    void* o, float* lse, const void* q, int B, int n_head, const void* kv_cache,
    int kv_fp8, int64_t n_kv_rows, int page_size, const int32_t* idx, int topk,
    const int32_t* block_table, int max_blocks, const int32_t* seq_lens,
    float scale, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  DSA_CHECK(B >= 0 && n_head > 0, "n_head must be > 0");
  DSA_CHECK(topk >= 0 && max_blocks >= 0 && n_kv_rows >= 0, "bad sizes");
  DSA_CHECK(page_size > 0, "page size must be > 0");
  if (B == 0) return MI355_DSA_OK;
  DSA_CHECK(o && lse && q && kv_cache && seq_lens, "null pointer argument");
  DSA_CHECK(topk == 0 || idx, "null idx");
  DSA_CHECK(max_blocks == 0 || block_table, "null block_table");
  DSA_CHECK(aligned_to(q, 16) && aligned_to(kv_cache, 16) && aligned_to(o, 8),
            "q / kv_cache / o misaligned");
  DSA_CHECK(B <= 65535 || use_prefill_config(B, n_head), "B too large");
  MlaParams prm;
  prm.q = reinterpret_cast<const f16*>(q);
  prm.kv = kv_cache;
  prm.idx = idx;
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
  prm.n_kv_rows = n_kv_rows;
  prm.scale_h = (float)(f16)scale;
  hipStream_t st = as_stream(stream);

  if (use_prefill_config(B, n_head)) {
    prm.n_splits = 1;
    const dim3 grid(B, (n_head + 63) / 64);
    return kv_fp8 ? launch_mla<true, 4, 1, 2>(prm, grid, st)
                  : launch_mla<false, 4, 1, 2>(prm, grid, st);
  }
  const int S = decode_splits(B, n_head, topk);
  prm.n_splits = S;
  if (S > 1) {
    const size_t need = mi355_dsa_sparse_mla_workspace_size(B, n_head, topk);
    DSA_CHECK(workspace && workspace_bytes >= need,
              "workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    DSA_CHECK(aligned_to(workspace, 16), "workspace must be 16-byte aligned");
    prm.part_o = reinterpret_cast<float*>(workspace);
    prm.part_ml = prm.part_o + (size_t)B * n_head * S * kValueDim;
  }
  const dim3 grid(S, (n_head + 15) / 16, B);
  int rc = kv_fp8 ? launch_mla<true, 1, kDecKW, 1>(prm, grid, st)
                  : launch_mla<false, 1, kDecKW, 1>(prm, grid, st);
  if (rc != MI355_DSA_OK || S == 1) return rc;
  sparse_mla_merge_kernel<<<dim3((unsigned)((int64_t)B * n_head)), 128, 0, st>>>(
      prm.part_o, prm.part_ml, prm.o, prm.lse, S);
  return check_launch("sparse_mla_merge");
}
