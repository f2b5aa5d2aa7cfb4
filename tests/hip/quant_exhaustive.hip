// Test kit (not part of the product library): exhaustive check of the
// e4m3 quantizer the cache scatters use (e4m3_quant8 in dsa_common.h)
// against IEEE division and the integer SATFINITE encoder
// (f32_to_e4m3_satfinite), for every positive finite amax of a 16-bit type
// and every value v of that type with |v| <= amax, both signs, with
// scale = max(amax/448, FLT_MIN) as the kernels compute it.
#include <float.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../glm5-on-v100_amd/csrc/dsa_common.h"

using namespace mi355dsa;

template <bool BF16>
__global__ void quant_exhaustive_kernel(unsigned long long* bad, uint32_t* first) {
  const uint32_t ab = blockIdx.x + 1;  // amax bit pattern
  const float amax =
      BF16 ? __uint_as_float(ab << 16) : (float)__builtin_bit_cast(_Float16, (uint16_t)ab);
  const float s = fmaxf(amax / 448.0f, FLT_MIN);
  const uint32_t n = 2 * ab + 2;  // v bit patterns 0..ab, both signs
  for (uint32_t base = 0; base < n; base += 8 * blockDim.x) {
    float v[8];
    uint32_t want[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      uint32_t vv = base + 8 * threadIdx.x + i;
      if (vv >= n) vv = 0;
      const uint32_t vb = (vv >> 1) | ((vv & 1) << 15);
      v[i] = BF16 ? __uint_as_float(vb << 16) : (float)__builtin_bit_cast(_Float16, (uint16_t)vb);
      want[i] = f32_to_e4m3_satfinite(v[i] / s);
    }
    const u32x2 q = e4m3_quant8(v, amax, s);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t got = (q[i >> 2] >> (8 * (i & 3))) & 0xffu;
      if (got != want[i]) {
        if (atomicAdd(bad, 1ull) == 0) {
          first[0] = ab;
          first[1] = __float_as_uint(v[i]);
        }
      }
    }
  }
}

// Returns 0 and the mismatch count in *bad_host (first mismatch in first_host),
// or a negative HIP error step.
extern "C" int dsa_test_quant_exhaustive(int bf16, unsigned long long* bad_host,
                                         uint32_t* first_host) {
  unsigned long long* bad = nullptr;
  uint32_t* first = nullptr;
  if (hipMalloc(&bad, sizeof(*bad)) != hipSuccess) return -1;
  if (hipMalloc(&first, 2 * sizeof(*first)) != hipSuccess) return -2;
  if (hipMemset(bad, 0, sizeof(*bad)) != hipSuccess) return -3;
  if (hipMemset(first, 0, 2 * sizeof(*first)) != hipSuccess) return -3;
  if (bf16)
    quant_exhaustive_kernel<true><<<0x7f7f, 256>>>(bad, first);
  else
    quant_exhaustive_kernel<false><<<0x7bff, 256>>>(bad, first);
  if (hipGetLastError() != hipSuccess) return -4;
  if (hipMemcpy(bad_host, bad, sizeof(*bad), hipMemcpyDeviceToHost) != hipSuccess) return -5;
  if (hipMemcpy(first_host, first, 2 * sizeof(*first), hipMemcpyDeviceToHost) != hipSuccess)
    return -5;
  if (hipFree(bad) != hipSuccess || hipFree(first) != hipSuccess) return -6;
  return 0;
}
