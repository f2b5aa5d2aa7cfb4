// C-ABI plumbing: error reporting, version, and the device self-check that
// verifies the MFMA accumulator placement and the e4m3 decode the kernels
// rely on (the role of the reference's first-launch WMMA layout probe,
// csrc/attention/sm70_mla_decode.cu:511-540 and :2807-2818).
#include <string.h>

#include <map>
#include <mutex>
#include <string>
#include <utility>

#include "capi_internal.h"
#include "dsa_common.h"

namespace mi355dsa {

static thread_local std::string g_last_error;

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

void clear_error() { g_last_error.clear(); }

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(MI355_DSA_EHIP, "%s: HIP launch failed: %s", what,
                     hipGetErrorString(e));
  return MI355_DSA_OK;
}

int reserve_lds(const void* kernel, size_t bytes, const char* what) {
  // The dynamic-LDS limit is a per-device property of a kernel: it is set once
  // per (device, kernel) for the largest size asked so far, under a lock so
  // that concurrent first calls from several host threads are safe.
  static std::mutex mu;
  static std::map<std::pair<int, const void*>, size_t> done;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess)
    return set_error(MI355_DSA_EHIP, "%s: no current HIP device", what);
  std::lock_guard<std::mutex> lock(mu);
  auto it = done.find({dev, kernel});
  if (it != done.end() && it->second >= bytes) return MI355_DSA_OK;
  const hipError_t e =
      hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e != hipSuccess)
    return set_error(MI355_DSA_EHIP, "%s: cannot reserve %zu bytes of LDS: %s", what, bytes,
                     hipGetErrorString(e));
  done[{dev, kernel}] = bytes;
  return MI355_DSA_OK;
}

// out[0..63]  : x32 MFMA probe results, out[64..127]: x16 probe results,
// out[128..383]: bit-trick e4m3 decode of bytes 0..255 (value exactly),
// out[384..639]: hardware v_cvt_pk_f32_fp8 decode of bytes 0..255,
// out[640..895]: v_cvt_scalef32_pk_f16_fp8 (scale 1) decode of bytes 0..255,
// the conversion the sparse attention gathers use.
// mfma_bad bit 4: ds_read_b64_tr_b16 lane mapping differs from the one the
// sparse attention PV step assumes (lane j of a 16-lane group whose lane i
// points at row 4g + i/4, column 4(i%4) receives column j of rows 4g..4g+3).
// Probe p uses a single non-zero k-slot (g = p/KPL, e = p%KPL) in both A and
// B: A[row c] = c+1, B[col c] = c+101, so D[i][j] must be (i+1)(j+101) at
// lane (col j, rows 4g'..) whatever k that slot maps to.
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__global__ void selfcheck_kernel(float* out, int* mfma_bad) {
  const int lane = threadIdx.x;
  const int c = lane & 15, g = lane >> 4;
  int bad32 = 0, bad16 = 0, badtr = 0;
  // 16 x 16 fp16 tile with value 16*row + col (exact in fp16)
  __shared__ __align__(16) f16 tile[16 * 16];
  for (int i = lane; i < 256; i += 64) tile[i] = (f16)(float)i;
  __syncthreads();
  {
    const f16* src = tile + (4 * g + (c >> 2)) * 16 + 4 * (c & 3);
    const s16x4 t = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)src);
    const f16x4 h = __builtin_bit_cast(f16x4, t);
#pragma unroll
    for (int k = 0; k < 4; k++)
      if ((float)h[k] != (float)(16 * (4 * g + k) + c)) badtr++;
  }
  for (int p = 0; p < 32; p++) {
    f16x8 a, b;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const bool on = (g == p / 8) && (e == p % 8);
      a[e] = on ? (f16)(c + 1) : (f16)0;
      b[e] = on ? (f16)(c + 101) : (f16)0;
    }
    f32x4 d = {0.f, 0.f, 0.f, 0.f};
    d = mfma16x16x32(a, b, d);
#pragma unroll
    for (int r = 0; r < 4; r++)
      if (d[r] != (float)((4 * g + r + 1) * (c + 101))) bad32++;
    if (p == 0) out[lane] = d[0];
  }
  for (int p = 0; p < 16; p++) {
    f16x4 a, b;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const bool on = (g == p / 4) && (e == p % 4);
      a[e] = on ? (f16)(c + 1) : (f16)0;
      b[e] = on ? (f16)(c + 101) : (f16)0;
    }
    f32x4 d = {0.f, 0.f, 0.f, 0.f};
    d = mfma16x16x16(a, b, d);
#pragma unroll
    for (int r = 0; r < 4; r++)
      if (d[r] != (float)((4 * g + r + 1) * (c + 101))) bad16++;
    if (p == 0) out[64 + lane] = d[0];
  }
  if (bad32) atomicOr(mfma_bad, 1);
  if (bad16) atomicOr(mfma_bad, 2);
  if (badtr) atomicOr(mfma_bad, 4);
  // e4m3 decode of all 256 byte values, 4 per lane.
  const uint32_t w = (uint32_t)(4 * lane) | ((uint32_t)(4 * lane + 1) << 8) |
                     ((uint32_t)(4 * lane + 2) << 16) |
                     ((uint32_t)(4 * lane + 3) << 24);
  float v[4];
  e4m3x4_to_f32_div256(w, v);
  const f32x2 h0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const f32x2 h1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
#pragma unroll
  for (int i = 0; i < 4; i++) out[128 + 4 * lane + i] = v[i] * 256.0f;
  out[384 + 4 * lane + 0] = h0[0];
  out[384 + 4 * lane + 1] = h0[1];
  out[384 + 4 * lane + 2] = h1[0];
  out[384 + 4 * lane + 3] = h1[1];
  const f16x2 s0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w, 1.0f, false);
  const f16x2 s1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w, 1.0f, true);
  out[640 + 4 * lane + 0] = (float)s0[0];
  out[640 + 4 * lane + 1] = (float)s0[1];
  out[640 + 4 * lane + 2] = (float)s1[0];
  out[640 + 4 * lane + 3] = (float)s1[1];
}

// Exact OCP e4m3 value of a byte (0x7f / 0xff are NaN in e4m3fn; the
// bit-trick decode maps them to +-480, which no finite encoder emits).
static double e4m3_value(int b) {
  const int s = (b >> 7) & 1, e = (b >> 3) & 15, m = b & 7;
  const double mag = (e == 0) ? ldexp((double)m, -9) : ldexp(8.0 + m, e - 10);
  return s ? -mag : mag;
}

constexpr int kArriveSlots = 16384;
__device__ uint32_t g_arrive[kArriveSlots * kArriveRows];

uint32_t* arrive_slot(hipStream_t st) {
  static std::mutex mu;
  static std::map<int, uint32_t*> pool;                     // device -> pool base
  static std::map<int, int> used;                           // device -> slots handed out
  static std::map<std::pair<int, hipStream_t>, int> eager;  // (device, stream) -> slot
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  auto pit = pool.find(dev);
  if (pit == pool.end()) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_arrive)) != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      return nullptr;
    }
    pit = pool.emplace(dev, reinterpret_cast<uint32_t*>(p)).first;
  }
  int& n = used[dev];
  if (cs == hipStreamCaptureStatusNone) {
    const auto it = eager.find({dev, st});
    if (it != eager.end()) return pit->second + (size_t)it->second * kArriveRows;
    if (n >= kArriveSlots) return nullptr;
    eager.emplace(std::make_pair(dev, st), n);
  } else if (n >= kArriveSlots) {
    return nullptr;
  }
  return pit->second + (size_t)(n++) * kArriveRows;
}

}  // namespace mi355dsa

using namespace mi355dsa;

extern "C" const char* mi355_dsa_last_error(void) { return g_last_error.c_str(); }

extern "C" int mi355_dsa_abi_version(void) { return 1; }

extern "C" int mi355_dsa_selfcheck(void* stream) {
  clear_error();
  hipStream_t st = as_stream(stream);
  float* d_out = nullptr;
  int* d_bad = nullptr;
  const size_t nout = 896;
  if (hipMalloc(&d_out, nout * sizeof(float)) != hipSuccess ||
      hipMalloc(&d_bad, sizeof(int)) != hipSuccess) {
    if (d_out) hipFree(d_out);
    return set_error(MI355_DSA_EHIP, "selfcheck: hipMalloc failed");
  }
  int rc = MI355_DSA_OK;
  float h_out[896];
  int h_bad = 0;
  if (hipMemsetAsync(d_bad, 0, sizeof(int), st) != hipSuccess) {
    rc = set_error(MI355_DSA_EHIP, "selfcheck: memset failed");
  } else {
    selfcheck_kernel<<<1, 64, 0, st>>>(d_out, d_bad);
    rc = check_launch("selfcheck");
    if (rc == MI355_DSA_OK &&
        (hipMemcpyAsync(h_out, d_out, sizeof(h_out), hipMemcpyDeviceToHost,
                        st) != hipSuccess ||
         hipMemcpyAsync(&h_bad, d_bad, sizeof(int), hipMemcpyDeviceToHost,
                        st) != hipSuccess ||
         hipStreamSynchronize(st) != hipSuccess))
      rc = set_error(MI355_DSA_EHIP, "selfcheck: readback failed");
  }
  hipFree(d_out);
  hipFree(d_bad);
  if (rc != MI355_DSA_OK) return rc;
  if (h_bad & 3)
    return set_error(MI355_DSA_ECHECK,
                     "selfcheck: MFMA accumulator placement mismatch (mask %d)",
                     h_bad);
  if (h_bad & 4)
    return set_error(MI355_DSA_ECHECK, "selfcheck: ds_read_b64_tr_b16 lane mapping mismatch");
  int hw_ok = 1;
  for (int b = 0; b < 256; b++) {
    if ((b & 0x7f) == 0x7f) continue;  // NaN codes
    const double want = e4m3_value(b);
    if ((double)h_out[128 + b] != want)
      return set_error(MI355_DSA_ECHECK,
                       "selfcheck: e4m3 decode of 0x%02x gave %g, want %g", b,
                       (double)h_out[128 + b], want);
    if ((double)h_out[384 + b] != want) hw_ok = 0;
    if ((double)h_out[640 + b] != want)
      return set_error(MI355_DSA_ECHECK,
                       "selfcheck: scaled fp8->fp16 conversion of 0x%02x gave %g, want %g", b,
                       (double)h_out[640 + b], want);
  }
  // Informational: whether v_cvt_pk_f32_fp8 decodes OCP e4m3 on this device.
  set_error(MI355_DSA_OK, "selfcheck ok; hw_cvt_pk_f32_fp8_ocp=%d", hw_ok);
  return MI355_DSA_OK;
}
