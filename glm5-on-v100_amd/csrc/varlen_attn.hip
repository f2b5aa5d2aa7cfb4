// Dense varlen multi-head attention for MLA prefill (gfx950, wave64 MFMA):
//
//   out[t, h, :] = softmax(scale * q[t, h, :] . k[j, h, :]^T) v[j, h, :]
//
// over the keys j of token t's sequence (ragged batches given by
// cu_seqlens_q / cu_seqlens_k), causal with the diagonal aligned to the end
// of the key sequence (query i of a q_len-long sequence sees keys
// j <= i + k_len - q_len), or non-causal; lse[h, t] = natural-log
// log-sum-exp, -inf for a query with no key (its output is 0).  This is the
// attention that reference/vllm/v1/attention/backends/mla/prefill/
// sm70_triton.py:54-187 (_varlen_attention) computes per sequence in fp32.
//
// Workgroup = (query tile of 64 QB rows, sequence, head), 4 waves; wave w
// owns query rows [16 QB w, +16 QB).  Key tiles of KT keys stream through
// two LDS stages by LDS-DMA (K and V rows at padded pitches, so that the rows
// of an MFMA operand spread over the banks), the next tile in flight while
// the current one is used; two workgroups share a CU.  Per tile and wave:
//   * S^T = K Q^T (v_mfma_f32_16x16x32): keys are the A operand read from
//     LDS, the wave's queries the B operand resident in registers;
//   * online softmax per query column in exp2 with the scale folded in; the
//     tile maximum is the only cross-lane reduction (the row sums stay
//     per-lane partials until the end);
//   * O^T += V^T P^T: the S^T accumulator layout is the B-operand layout of
//     P^T (keys 4g..4g+3 of two 16-key blocks per lane), so P never leaves
//     registers; V^T comes from ds_read_b64_tr_b16 transpose reads in the
//     same key order.
// bf16 inputs use the bf16 MFMA; their P is split into two bf16 parts
// (p = hi + lo), so the PV product keeps ~16 bits of P.
#include <float.h>

#include "capi_internal.h"
#include "dsa_common.h"

namespace mi355dsa {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4v lds_s16x4v;

constexpr int kVaWaves = 4;
constexpr int kVaThreads = 64 * kVaWaves;

__device__ const __align__(16) uint16_t kVaZero[8] = {};

struct VaArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;  // [H, total_q] or null
  const int32_t* cu_q;
  const int32_t* cu_k;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh;  // element strides
  int H, total_q, n_qtiles, causal;
  float scale_log2;  // softmax scale * log2(e)
  float scale;
};

template <bool BF16>
__device__ __forceinline__ f32x4 mma(const u32x4& a, const u32x4& b, f32x4 c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <bool BF16>
__device__ __forceinline__ uint16_t to16(float x) {
  if constexpr (BF16) return __builtin_bit_cast(uint16_t, (__bf16)x);
  else return __builtin_bit_cast(uint16_t, (f16)x);
}
template <bool BF16>
__device__ __forceinline__ float from16(uint16_t x) {
  if constexpr (BF16) return (float)__builtin_bit_cast(__bf16, x);
  else return (float)__builtin_bit_cast(f16, x);
}

// K and V rows at a pitch of d / 8 + 2 pieces (two pads): the QK reads (16
// rows x 4 adjacent pieces per instruction) and the V^T transpose reads (8
// rows x 32 bytes per half-wave) are then free of LDS bank conflicts (both
// measured on gfx950; with one pad both conflicted two-way)
template <int DQK, int DV, int KT>
struct VaShape {
  static constexpr int PK = DQK / 8 + 2;  // K row pitch in 16-B pieces
  static constexpr int PV = DV / 8 + 2;
  static constexpr int RK = (KT * PK + kVaThreads - 1) / kVaThreads;  // DMA rounds
  static constexpr int RV = (KT * PV + kVaThreads - 1) / kVaThreads;
  static constexpr int KBYTES = RK * kVaThreads * 16;
  static constexpr int VBYTES = RV * kVaThreads * 16;
  static constexpr int STAGE = KBYTES + VBYTES;
};

template <int N>
__device__ __forceinline__ void va_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <bool BF16, int DQK, int DV, int QB, int KT, int MINB>
__global__ void __launch_bounds__(kVaThreads, MINB) varlen_attn_kernel(VaArgs a) {
  using Sh = VaShape<DQK, DV, KT>;
  constexpr int NKB = KT / 16;  // 16-key blocks per tile
  constexpr int NKH = KT / 32;  // 32-key PV steps per tile
  constexpr int QROWS = 16 * QB * kVaWaves;
  constexpr int NS = DQK / 32;  // QK k-steps
  constexpr int NDT = DV / 16;  // O^T dim tiles
  extern __shared__ __align__(16) unsigned char smem_raw[];

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int seq = blockIdx.y, h = blockIdx.z;
  const int qs = a.cu_q[seq], q_len = a.cu_q[seq + 1] - qs;
  const int ks = a.cu_k[seq], k_len = a.cu_k[seq + 1] - ks;
  // heaviest (latest) query tiles first under a causal mask
  const int tile = a.causal ? a.n_qtiles - 1 - (int)blockIdx.x : (int)blockIdx.x;
  const int q0 = tile * QROWS;
  if (q0 >= q_len) return;
  const int offset = a.causal ? k_len - q_len : 0;
  const int kend = a.causal ? max(0, min(k_len, q0 + QROWS + offset)) : k_len;
  const int n_kt = (kend + KT - 1) / KT;

  // ---- Q fragments (B operand): row q0 + 16(QB w + qb) + c, dims 32 s + 8 g ----
  u32x4 qf[QB][NS];
#pragma unroll
  for (int qb = 0; qb < QB; qb++) {
    const int i = q0 + 16 * (QB * w + qb) + c;
    const uint16_t* qrow = a.q + (int64_t)(qs + (i < q_len ? i : 0)) * a.q_st + (int64_t)h * a.q_sh +
                           8 * g;
    // rows past q_len read row 0 of the sequence: their MFMA columns and
    // softmax state are their own, and their outputs are not stored
#pragma unroll
    for (int s = 0; s < NS; s++) qf[qb][s] = *reinterpret_cast<const u32x4*>(qrow + 32 * s);
  }

  auto issue_tile = [&](int kt) {
    unsigned char* st = smem_raw + (kt & 1) * Sh::STAGE;
    const int k0 = kt * KT;
#pragma unroll
    for (int u = 0; u < Sh::RK; u++) {
      const int qq = kVaThreads * u + 64 * w + lane;
      const int r = qq / Sh::PK, ch = qq - r * Sh::PK;
      const bool ok = r < KT && ch < DQK / 8 && k0 + r < kend;
      const uint16_t* src = ok ? a.k + (int64_t)(ks + k0 + r) * a.k_st + (int64_t)h * a.k_sh + 8 * ch
                               : kVaZero;
      dma16(src, st + 16 * (kVaThreads * u + 64 * w));
    }
#pragma unroll
    for (int u = 0; u < Sh::RV; u++) {
      const int qq = kVaThreads * u + 64 * w + lane;
      const int r = qq / Sh::PV, ch = qq - r * Sh::PV;
      const bool ok = r < KT && ch < DV / 8 && k0 + r < kend;
      const uint16_t* src = ok ? a.v + (int64_t)(ks + k0 + r) * a.v_st + (int64_t)h * a.v_sh + 8 * ch
                               : kVaZero;
      dma16(src, st + Sh::KBYTES + 16 * (kVaThreads * u + 64 * w));
    }
  };

  f32x4 oacc[NDT][QB];
#pragma unroll
  for (int t = 0; t < NDT; t++)
#pragma unroll
    for (int qb = 0; qb < QB; qb++) oacc[t][qb] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float m_run[QB], l_part[QB];  // raw-score running max (same in the 4 lane groups), partial sums
#pragma unroll
  for (int qb = 0; qb < QB; qb++) {
    m_run[qb] = -1e30f;
    l_part[qb] = 0.f;
  }

  if (n_kt > 0) issue_tile(0);
  // Q completes here, together with tile 0 (one round trip).  The compiler
  // does not count the tile DMAs issued by inline asm, so a wait for Q left
  // to the loop would be vmcnt(0) on every step and drain the next tile.
#pragma unroll
  for (int qb = 0; qb < QB; qb++)
#pragma unroll
    for (int s = 0; s < NS; s++) asm volatile("" ::"v"(qf[qb][s]));
  for (int kt = 0; kt < n_kt; kt++) {
    if (kt + 1 < n_kt) {
      issue_tile(kt + 1);
      va_wait<Sh::RK + Sh::RV>();
    } else {
      va_wait<0>();
    }
    lds_barrier();  // tile kt landed for every wave
    const unsigned char* kst = smem_raw + (kt & 1) * Sh::STAGE;
    const unsigned char* vst = kst + Sh::KBYTES;
    const int k0 = kt * KT;

    // ---- S^T blocks: keys 16 kb + 4 g + r, query column c of block qb ----
    f32x4 sacc[NKB][QB];
#pragma unroll
    for (int kb = 0; kb < NKB; kb++)
#pragma unroll
      for (int qb = 0; qb < QB; qb++) sacc[kb][qb] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; s++) {
#pragma unroll
      for (int kb = 0; kb < NKB; kb++) {
        const u32x4 kf = *reinterpret_cast<const u32x4*>(kst + (16 * kb + c) * Sh::PK * 16 +
                                                         64 * s + 16 * g);
#pragma unroll
        for (int qb = 0; qb < QB; qb++) sacc[kb][qb] = mma<BF16>(kf, qf[qb][s], sacc[kb][qb]);
      }
    }

    // ---- masks and online softmax per query column ----
    u32x4 pb[NKH][QB], pl[NKH][QB];  // P^T operands per 32 keys (hi and, for bf16, lo parts)
#pragma unroll
    for (int qb = 0; qb < QB; qb++) {
      const int i = q0 + 16 * (QB * w + qb) + c;  // query row of this column
      const int jmax = a.causal ? min(kend, i + offset + 1) : kend;  // keys < jmax are valid
      float mt = -1e30f;
#pragma unroll
      for (int kb = 0; kb < NKB; kb++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int j = k0 + 16 * kb + 4 * g + r;
          if (j >= jmax) sacc[kb][qb][r] = -INFINITY;
          mt = fmaxf(mt, sacc[kb][qb][r]);
        }
      mt = fmaxf(mt, shfl_xor_f(mt, 16));
      mt = fmaxf(mt, shfl_xor_f(mt, 32));
      const float m_new = fmaxf(m_run[qb], mt);
      const float alpha = exp2f((m_run[qb] - m_new) * a.scale_log2);
      m_run[qb] = m_new;
      const float mb = m_new * a.scale_log2;
      float ls = 0.f;
      float pv[NKB][4];
#pragma unroll
      for (int kb = 0; kb < NKB; kb++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float sv = sacc[kb][qb][r];
          const float p = (sv > -INFINITY) ? exp2f(__builtin_fmaf(sv, a.scale_log2, -mb)) : 0.f;
          pv[kb][r] = p;
          ls += p;
        }
      l_part[qb] = l_part[qb] * alpha + ls;
#pragma unroll
      for (int t = 0; t < NDT; t++) oacc[t][qb] *= alpha;
#pragma unroll
      for (int kh = 0; kh < NKH; kh++) {
        uint16_t hi[8], lo[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const float p = pv[2 * kh + (e >> 2)][e & 3];
          hi[e] = to16<BF16>(p);
          lo[e] = BF16 ? to16<BF16>(p - from16<BF16>(hi[e])) : (uint16_t)0;
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
          pb[kh][qb][e] = (uint32_t)hi[2 * e] | ((uint32_t)hi[2 * e + 1] << 16);
          pl[kh][qb][e] = (uint32_t)lo[2 * e] | ((uint32_t)lo[2 * e + 1] << 16);
        }
      }
    }

    // ---- O^T += V^T P^T: keys 32 kh + {4g .. 4g+3, 16 + 4g .. 16 + 4g + 3} ----
    // transpose source: lane i of group g points at key 32 kh + 4 g + i / 4
    // (+16 for the second read), dims 16 t + 4 (i % 4) .. +3
    const unsigned char* vsrc = vst + (4 * g + (c >> 2)) * Sh::PV * 16 + 8 * (c & 3);
#pragma unroll
    for (int kh = 0; kh < NKH; kh++) {
#pragma unroll
      for (int t = 0; t < NDT; t++) {
        const s16x4v v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4v*)(vsrc + (32 * kh) * Sh::PV * 16 + 32 * t));
        const s16x4v v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4v*)(vsrc + (32 * kh + 16) * Sh::PV * 16 + 32 * t));
        const u32x2 x0 = __builtin_bit_cast(u32x2, v0), x1 = __builtin_bit_cast(u32x2, v1);
        const u32x4 av = {x0[0], x0[1], x1[0], x1[1]};
#pragma unroll
        for (int qb = 0; qb < QB; qb++) {
          oacc[t][qb] = mma<BF16>(av, pb[kh][qb], oacc[t][qb]);
          if constexpr (BF16) oacc[t][qb] = mma<BF16>(av, pl[kh][qb], oacc[t][qb]);
        }
      }
    }
    lds_barrier();  // every wave is done with this stage before it is refilled
  }

  // ---- outputs ----
#pragma unroll
  for (int qb = 0; qb < QB; qb++) {
    float l = l_part[qb];
    l += shfl_xor_f(l, 16);
    l += shfl_xor_f(l, 32);
    const int i = q0 + 16 * (QB * w + qb) + c;
    if (i >= q_len) continue;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    uint16_t* orow = a.o + (int64_t)(qs + i) * a.o_st + (int64_t)h * a.o_sh;
#pragma unroll
    for (int t = 0; t < NDT; t++) {
      u32x2 pk;
      pk[0] = (uint32_t)to16<BF16>(oacc[t][qb][0] * inv) |
              ((uint32_t)to16<BF16>(oacc[t][qb][1] * inv) << 16);
      pk[1] = (uint32_t)to16<BF16>(oacc[t][qb][2] * inv) |
              ((uint32_t)to16<BF16>(oacc[t][qb][3] * inv) << 16);
      *reinterpret_cast<u32x2*>(orow + 16 * t + 4 * g) = pk;
    }
    if (a.lse != nullptr && g == 0)
      a.lse[(int64_t)h * a.total_q + qs + i] =
          l > 0.f ? m_run[qb] * a.scale + logf(l) : -INFINITY;
  }
}

template <bool BF16, int DQK, int DV, int QB, int KT, int MINB>
int launch_va(const VaArgs& a0, int num_seqs, int max_q_len, hipStream_t st) {
  using Sh = VaShape<DQK, DV, KT>;
  constexpr int QROWS = 16 * QB * kVaWaves;
  auto kern = varlen_attn_kernel<BF16, DQK, DV, QB, KT, MINB>;
  const int rc = reserve_lds(reinterpret_cast<const void*>(kern), 2 * Sh::STAGE, "varlen_attention");
  if (rc) return rc;
  VaArgs a = a0;
  a.n_qtiles = (max_q_len + QROWS - 1) / QROWS;
  if (a.n_qtiles == 0) return MI355_DSA_OK;
  kern<<<dim3(a.n_qtiles, num_seqs, a.H), kVaThreads, 2 * Sh::STAGE, st>>>(a);
  return check_launch("varlen_attention");
}

template <bool BF16>
int dispatch_va(const VaArgs& a, int d_qk, int d_v, int num_seqs, int max_q_len, hipStream_t st) {
  // 32-key tiles and two workgroups per CU: two waves per SIMD, so one
  // wave's softmax overlaps the other's MFMAs (1.7x the 64-key tile at one
  // wave per SIMD on the (192, 128) causal prefill)
  if (d_qk == 192 && d_v == 128) return launch_va<BF16, 192, 128, 2, 32, 2>(a, num_seqs, max_q_len, st);
  if (d_qk == 128 && d_v == 128) return launch_va<BF16, 128, 128, 2, 32, 2>(a, num_seqs, max_q_len, st);
  if (d_qk == 64 && d_v == 64) return launch_va<BF16, 64, 64, 2, 32, 2>(a, num_seqs, max_q_len, st);
  if (d_qk == 256 && d_v == 256) return launch_va<BF16, 256, 256, 1, 32, 2>(a, num_seqs, max_q_len, st);
  return set_error(MI355_DSA_EINVAL,
                   "varlen_attention: head dims (%d, %d) not built; supported (qk, v): "
                   "(192, 128), (128, 128), (64, 64), (256, 256)", d_qk, d_v);
}

// ---------------------------------------------------------------------------
// fp32 inputs: the same attention in fp32 arithmetic throughout, on the fp32
// MFMA (v_mfma_f32_16x16x4_f32), as the reference computes fp32 inputs
// (sm70_triton.py:193 lists fp32; :54-187 runs it in fp32 torch).  Nothing
// is rounded to 16 bits, so the whole fp32 range is accepted.
//
// Workgroup = (query tile of 64 rows, sequence, head), 4 waves; wave w owns
// query rows [16 w, +16).  Key tiles of 32 keys stream through two LDS
// stages by LDS-DMA (rows at a pitch of d + 4 floats: 16 consecutive rows
// then cover all 64 banks).  Per tile and wave:
//   * S^T = K Q^T: K step j of dims 16 u .. 16 u + 15 takes dim 16 u + 4 g +
//     j from lane group g (one 16-byte LDS read per lane feeds 4 MFMAs); Q
//     is resident in registers in the same dim order;
//   * online softmax per query column (exp2, scale folded in), P kept fp32;
//   * O^T += V^T P^T: MFMA step r of a 16-key block takes key 4 g + r from
//     lane group g, which is element r of that lane's own S^T accumulator,
//     so P never moves; V^T[dim 16 t + c][key] is one fp32 LDS read.
// ---------------------------------------------------------------------------
template <int DQK, int DV>
struct VaShape32 {
  static constexpr int KT = 32;
  static constexpr int PK = DQK / 4 + 1;  // row pitch in 16-B pieces (4 floats), one pad
  static constexpr int PV = DV / 4 + 1;
  static constexpr int RK = (KT * PK + kVaThreads - 1) / kVaThreads;  // DMA rounds
  static constexpr int RV = (KT * PV + kVaThreads - 1) / kVaThreads;
  static constexpr int KBYTES = RK * kVaThreads * 16;
  static constexpr int VBYTES = RV * kVaThreads * 16;
  static constexpr int STAGE = KBYTES + VBYTES;
};

__device__ __forceinline__ f32x4 mma32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int DQK, int DV>
__global__ void __launch_bounds__(kVaThreads) varlen_attn_f32_kernel(VaArgs a) {
  using Sh = VaShape32<DQK, DV>;
  constexpr int KT = Sh::KT;
  constexpr int NKB = KT / 16;
  constexpr int QROWS = 16 * kVaWaves;
  constexpr int NU = DQK / 16;  // 16-dim groups of the QK product
  constexpr int NDT = DV / 16;  // O^T dim tiles
  constexpr int PKF = 4 * Sh::PK, PVF = 4 * Sh::PV;  // row pitches in floats
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const float* qg = reinterpret_cast<const float*>(a.q);
  const float* kg = reinterpret_cast<const float*>(a.k);
  const float* vg = reinterpret_cast<const float*>(a.v);
  float* og = reinterpret_cast<float*>(a.o);

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int seq = blockIdx.y, h = blockIdx.z;
  const int qs = a.cu_q[seq], q_len = a.cu_q[seq + 1] - qs;
  const int ks = a.cu_k[seq], k_len = a.cu_k[seq + 1] - ks;
  const int tile = a.causal ? a.n_qtiles - 1 - (int)blockIdx.x : (int)blockIdx.x;
  const int q0 = tile * QROWS;
  if (q0 >= q_len) return;
  const int offset = a.causal ? k_len - q_len : 0;
  const int kend = a.causal ? max(0, min(k_len, q0 + QROWS + offset)) : k_len;
  const int n_kt = (kend + KT - 1) / KT;

  // ---- Q (B operand): row q0 + 16 w + c, dims 16 u + 4 g .. +3 ----
  const int qi = q0 + 16 * w + c;
  f32x4 qf[NU];
  {
    const float* qrow = qg + (int64_t)(qs + (qi < q_len ? qi : 0)) * a.q_st + (int64_t)h * a.q_sh +
                        4 * g;
#pragma unroll
    for (int u = 0; u < NU; u++) qf[u] = *reinterpret_cast<const f32x4*>(qrow + 16 * u);
  }

  auto issue_tile = [&](int kt) {
    unsigned char* st = smem_raw + (kt & 1) * Sh::STAGE;
    const int k0 = kt * KT;
#pragma unroll
    for (int u = 0; u < Sh::RK; u++) {
      const int qq = kVaThreads * u + 64 * w + lane;
      const int r = qq / Sh::PK, ch = qq - r * Sh::PK;
      const bool ok = r < KT && ch < DQK / 4 && k0 + r < kend;
      const void* src = ok ? (const void*)(kg + (int64_t)(ks + k0 + r) * a.k_st +
                                           (int64_t)h * a.k_sh + 4 * ch)
                           : (const void*)kVaZero;
      dma16(src, st + 16 * (kVaThreads * u + 64 * w));
    }
#pragma unroll
    for (int u = 0; u < Sh::RV; u++) {
      const int qq = kVaThreads * u + 64 * w + lane;
      const int r = qq / Sh::PV, ch = qq - r * Sh::PV;
      const bool ok = r < KT && ch < DV / 4 && k0 + r < kend;
      const void* src = ok ? (const void*)(vg + (int64_t)(ks + k0 + r) * a.v_st +
                                           (int64_t)h * a.v_sh + 4 * ch)
                           : (const void*)kVaZero;
      dma16(src, st + Sh::KBYTES + 16 * (kVaThreads * u + 64 * w));
    }
  };

  f32x4 oacc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; t++) oacc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float m_run = -1e30f, l_part = 0.f;

  if (n_kt > 0) issue_tile(0);
#pragma unroll
  for (int u = 0; u < NU; u++) asm volatile("" ::"v"(qf[u]));  // Q lands with tile 0
  const int jmax_q = a.causal ? qi + offset + 1 : kend;  // keys < jmax of this column
  for (int kt = 0; kt < n_kt; kt++) {
    if (kt + 1 < n_kt) {
      issue_tile(kt + 1);
      va_wait<Sh::RK + Sh::RV>();
    } else {
      va_wait<0>();
    }
    lds_barrier();  // tile kt landed for every wave
    const float* kst = reinterpret_cast<const float*>(smem_raw + (kt & 1) * Sh::STAGE);
    const float* vst = reinterpret_cast<const float*>(smem_raw + (kt & 1) * Sh::STAGE + Sh::KBYTES);
    const int k0 = kt * KT;

    // ---- S^T blocks: keys 16 kb + 4 g + r, query column c ----
    f32x4 sacc[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; kb++) {
      sacc[kb] = (f32x4){0.f, 0.f, 0.f, 0.f};
      const float* krow = kst + (16 * kb + c) * PKF + 4 * g;
#pragma unroll
      for (int u = 0; u < NU; u++) {
        const f32x4 kf = *reinterpret_cast<const f32x4*>(krow + 16 * u);
#pragma unroll
        for (int j = 0; j < 4; j++) sacc[kb] = mma32(kf[j], qf[u][j], sacc[kb]);
      }
    }

    // ---- masks and online softmax of column c ----
    const int jmax = min(kend, jmax_q);
    float mt = -1e30f;
#pragma unroll
    for (int kb = 0; kb < NKB; kb++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        if (k0 + 16 * kb + 4 * g + r >= jmax) sacc[kb][r] = -INFINITY;
        mt = fmaxf(mt, sacc[kb][r]);
      }
    mt = fmaxf(mt, shfl_xor_f(mt, 16));
    mt = fmaxf(mt, shfl_xor_f(mt, 32));
    const float m_new = fmaxf(m_run, mt);
    const float alpha = exp2f((m_run - m_new) * a.scale_log2);
    m_run = m_new;
    const float mb = m_new * a.scale_log2;
    float ls = 0.f;
#pragma unroll
    for (int kb = 0; kb < NKB; kb++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float sv = sacc[kb][r];
        const float pr = (sv > -INFINITY) ? exp2f(__builtin_fmaf(sv, a.scale_log2, -mb)) : 0.f;
        sacc[kb][r] = pr;
        ls += pr;
      }
    l_part = l_part * alpha + ls;
#pragma unroll
    for (int t = 0; t < NDT; t++) oacc[t] *= alpha;

    // ---- O^T += V^T P^T ----
#pragma unroll
    for (int kb = 0; kb < NKB; kb++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float* vrow = vst + (16 * kb + 4 * g + r) * PVF + c;
#pragma unroll
        for (int t = 0; t < NDT; t++) oacc[t] = mma32(vrow[16 * t], sacc[kb][r], oacc[t]);
      }
    lds_barrier();  // every wave is done with this stage before it is refilled
  }

  // ---- outputs: O^T rows 4 g + r of tile t are dims 16 t + 4 g + r ----
  float l = l_part;
  l += shfl_xor_f(l, 16);
  l += shfl_xor_f(l, 32);
  if (qi >= q_len) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  float* orow = og + (int64_t)(qs + qi) * a.o_st + (int64_t)h * a.o_sh + 4 * g;
#pragma unroll
  for (int t = 0; t < NDT; t++) *reinterpret_cast<f32x4*>(orow + 16 * t) = oacc[t] * inv;
  if (a.lse != nullptr && g == 0)
    a.lse[(int64_t)h * a.total_q + qs + qi] = l > 0.f ? m_run * a.scale + logf(l) : -INFINITY;
}

template <int DQK, int DV>
int launch_va32(const VaArgs& a0, int num_seqs, int max_q_len, hipStream_t st) {
  using Sh = VaShape32<DQK, DV>;
  constexpr int QROWS = 16 * kVaWaves;
  auto kern = varlen_attn_f32_kernel<DQK, DV>;
  const int rc = reserve_lds(reinterpret_cast<const void*>(kern), 2 * Sh::STAGE,
                             "varlen_attention_f32");
  if (rc) return rc;
  VaArgs a = a0;
  a.n_qtiles = (max_q_len + QROWS - 1) / QROWS;
  if (a.n_qtiles == 0) return MI355_DSA_OK;
  kern<<<dim3(a.n_qtiles, num_seqs, a.H), kVaThreads, 2 * Sh::STAGE, st>>>(a);
  return check_launch("varlen_attention_f32");
}

int dispatch_va32(const VaArgs& a, int d_qk, int d_v, int num_seqs, int max_q_len,
                  hipStream_t st) {
  if (d_qk == 192 && d_v == 128) return launch_va32<192, 128>(a, num_seqs, max_q_len, st);
  if (d_qk == 128 && d_v == 128) return launch_va32<128, 128>(a, num_seqs, max_q_len, st);
  if (d_qk == 64 && d_v == 64) return launch_va32<64, 64>(a, num_seqs, max_q_len, st);
  if (d_qk == 256 && d_v == 256) return launch_va32<256, 256>(a, num_seqs, max_q_len, st);
  return set_error(MI355_DSA_EINVAL,
                   "varlen_attention: head dims (%d, %d) not built; supported (qk, v): "
                   "(192, 128), (128, 128), (64, 64), (256, 256)", d_qk, d_v);
}

}  // namespace
}  // namespace mi355dsa

using namespace mi355dsa;

extern "C" int mi355_dsa_varlen_attention(
    void* out, float* lse, const void* q, const void* k, const void* v, int dtype, int num_seqs,
    int n_head, int d_qk, int d_v, int64_t q_tok_stride, int64_t q_head_stride,
    int64_t k_tok_stride, int64_t k_head_stride, int64_t v_tok_stride, int64_t v_head_stride,
    int64_t o_tok_stride, int64_t o_head_stride, const int32_t* cu_seqlens_q,
    const int32_t* cu_seqlens_k, int max_q_len, int total_q, float softmax_scale, int causal,
    void* stream) {
  clear_error();
  DSA_CHECK(num_seqs >= 0 && n_head > 0 && max_q_len >= 0 && total_q >= 0, "varlen_attention: bad sizes");
  if (num_seqs == 0 || max_q_len == 0 || total_q == 0) return MI355_DSA_OK;
  DSA_CHECK(out && q && k && v && cu_seqlens_q && cu_seqlens_k, "varlen_attention: null pointer argument");
  DSA_CHECK(dtype >= 0 && dtype <= 2, "varlen_attention: dtype must be 0 (fp16), 1 (bf16) or 2 (fp32)");
  DSA_CHECK(num_seqs <= 65535 && n_head <= 65535, "varlen_attention: too many sequences or heads");
  const bool f32 = dtype == 2;
  DSA_CHECK(aligned_to(q, 16) && aligned_to(k, 16) && aligned_to(v, 16) &&
                aligned_to(out, f32 ? 16 : 8),
            "varlen_attention: q / k / v must be 16-byte and out %d-byte aligned", f32 ? 16 : 8);
  const int64_t sm = f32 ? 4 : 8;  // elements per 16-byte piece
  DSA_CHECK(q_tok_stride % sm == 0 && q_head_stride % sm == 0 && k_tok_stride % sm == 0 &&
                k_head_stride % sm == 0 && v_tok_stride % sm == 0 && v_head_stride % sm == 0 &&
                o_tok_stride % 4 == 0 && o_head_stride % 4 == 0,
            "varlen_attention: strides must be multiples of %d elements (out: 4)", (int)sm);
  VaArgs a{};
  a.q = reinterpret_cast<const uint16_t*>(q);
  a.k = reinterpret_cast<const uint16_t*>(k);
  a.v = reinterpret_cast<const uint16_t*>(v);
  a.o = reinterpret_cast<uint16_t*>(out);
  a.lse = lse;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.q_st = q_tok_stride;
  a.q_sh = q_head_stride;
  a.k_st = k_tok_stride;
  a.k_sh = k_head_stride;
  a.v_st = v_tok_stride;
  a.v_sh = v_head_stride;
  a.o_st = o_tok_stride;
  a.o_sh = o_head_stride;
  a.H = n_head;
  a.total_q = total_q;
  a.causal = causal ? 1 : 0;
  a.scale = softmax_scale;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  hipStream_t st = as_stream(stream);
  if (f32) return dispatch_va32(a, d_qk, d_v, num_seqs, max_q_len, st);
  return dtype == 1 ? dispatch_va<true>(a, d_qk, d_v, num_seqs, max_q_len, st)
                    : dispatch_va<false>(a, d_qk, d_v, num_seqs, max_q_len, st);
}
