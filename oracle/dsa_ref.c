/*
 * C restatement of the byte/integer parts of the DSA hot path --
 * TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Built by
 * oracle/Makefile into oracle/_build/liboracle_dsa.so and loaded by
 * oracle/cref.py.  Never linked into the product library.
 *
 *   oracle_e4m3_encode   fp32 -> e4m3 RNE + SATFINITE
 *                        (__nv_cvt_float_to_fp8, csrc/attention/sm70_mla_decode.cu:704)
 *   oracle_e4m3_decode   e4m3 -> fp32 (csrc/attention/sm70_attn_fp8.cu:16-20)
 *   oracle_topk_rows     exact top-k per row, lowest position wins ties,
 *                        ascending output, -1 padding (contract of
 *                        sm70_decode_topk, sm70_mla_decode.cu:1187-1212)
 *
 * The encoder is written from the number format (value grid and ties in
 * double precision), independently of the kernels' integer bit trick.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Value of e4m3 code c (0..126) as a double. */
static double e4m3_mag(int c) {
  const int e = c >> 3, m = c & 7;
  return e == 0 ? ldexp((double)m, -9) : ldexp(1.0 + m / 8.0, e - 7);
}

void oracle_e4m3_decode(const uint8_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    const int b = in[i];
    const int c = b & 0x7f;
    double v = (c == 0x7f) ? NAN : e4m3_mag(c);
    out[i] = (float)((b & 0x80) ? -v : v);
  }
}

/* Round |x| to the e4m3 grid: nearest magnitude, ties to the even code,
 * saturating at 448 (code 0x7e). */
static uint8_t encode_one(float xf) {
  if (isnan(xf)) return (uint8_t)(signbit(xf) ? 0xff : 0x7f);
  const int neg = signbit(xf) ? 1 : 0;
  const double a = fabs((double)xf);
  int code;
  if (a >= 448.0) {
    code = 0x7e;
  } else {
    /* binary search the largest code with magnitude <= a */
    int lo = 0, hi = 0x7e;
    while (lo < hi) {
      const int mid = (lo + hi + 1) / 2;
      if (e4m3_mag(mid) <= a) lo = mid; else hi = mid - 1;
    }
    code = lo;
    if (code < 0x7e) {
      const double below = e4m3_mag(code), above = e4m3_mag(code + 1);
      const double d0 = a - below, d1 = above - a;
      if (d1 < d0 || (d1 == d0 && (code & 1))) code += 1;
    }
  }
  return (uint8_t)(code | (neg ? 0x80 : 0));
}

void oracle_e4m3_encode(const float* in, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = encode_one(in[i]);
}

static uint32_t mono(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

typedef struct {
  uint32_t key;
  int32_t pos;
} kp_t;

static int cmp_desc_key_asc_pos(const void* a, const void* b) {
  const kp_t* x = (const kp_t*)a;
  const kp_t* y = (const kp_t*)b;
  if (x->key != y->key) return x->key > y->key ? -1 : 1;
  return x->pos < y->pos ? -1 : (x->pos > y->pos);
}

static int cmp_i32(const void* a, const void* b) {
  const int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
  return (x > y) - (x < y);
}

/* score: [n_rows, row_stride] fp32; seq_lens: [n_rows]; idx: [n_rows, k]. */
int oracle_topk_rows(const float* score, int64_t n_rows, int64_t row_stride,
                     const int32_t* seq_lens, int k, int32_t* idx) {
  kp_t* buf = (kp_t*)malloc(sizeof(kp_t) * (size_t)(row_stride > 0 ? row_stride : 1));
  if (!buf) return -1;
  for (int64_t r = 0; r < n_rows; r++) {
    int64_t L = seq_lens[r];
    if (L > row_stride) L = row_stride;
    if (L < 0) L = 0;
    const float* row = score + r * row_stride;
    for (int64_t p = 0; p < L; p++) {
      buf[p].key = mono(row[p]);
      buf[p].pos = (int32_t)p;
    }
    int32_t* out = idx + r * k;
    const int64_t take = L < k ? L : k;
    if (L > k) qsort(buf, (size_t)L, sizeof(kp_t), cmp_desc_key_asc_pos);
    for (int64_t i = 0; i < take; i++) out[i] = buf[i].pos;
    qsort(out, (size_t)take, sizeof(int32_t), cmp_i32);
    for (int64_t i = take; i < k; i++) out[i] = -1;
  }
  free(buf);
  return 0;
}
