/*
 * oracle.c — CPU restatement of the reference's quantized-storage Dense path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP library, never part of it.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Compile with -O2 -ffp-contract=off and without fast-math: every rounding
 * step below is meant literally.  Reference citations are file:line in the
 * reference checkout.  Casts from floating point to integers are written out
 * with the reference platform's (arm64) semantics: saturate, NaN -> 0.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ helpers */

static uint32_t f32bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bitsf32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint64_t f64bits(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
static double bitsf64(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

/* arm64 fcvtzs / fcvtzu: truncate toward zero, saturate, NaN -> 0 */
static int32_t cvt_i32(double v) {
  if (v != v) return 0;
  if (v >= 2147483648.0) return INT32_MAX;
  if (v <= -2147483649.0) return INT32_MIN;
  return (int32_t)v;
}
static int64_t cvt_i64(double v) {
  if (v != v) return 0;
  if (v >= 9223372036854775808.0) return INT64_MAX;
  if (v < -9223372036854775808.0) return INT64_MIN;
  return (int64_t)v;
}
static uint32_t cvt_u32(double v) {
  if (v != v || v <= -1.0) return 0;
  if (v >= 4294967296.0) return UINT32_MAX;
  return (uint32_t)v;
}
static uint64_t cvt_u64(double v) {
  if (v != v || v <= -1.0) return 0;
  if (v >= 18446744073709551616.0) return UINT64_MAX;
  return (uint64_t)v;
}

/* native_codec.cpp:42-48 (double) and ops_storage.metal:114-120 (float) */
static double clamp_d(double v, double lo, double hi) { return v < lo ? lo : (v > hi ? hi : v); }
static float clamp_f(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* native_codec.cpp:50-71: little-endian byte access */
static void put_u16(uint8_t *b, int64_t off, uint16_t v) { b[off] = (uint8_t)v; b[off + 1] = (uint8_t)(v >> 8); }
static void put_u32(uint8_t *b, int64_t off, uint32_t v) { for (int i = 0; i < 4; ++i) b[off + i] = (uint8_t)(v >> (8 * i)); }
static void put_u64(uint8_t *b, int64_t off, uint64_t v) { for (int i = 0; i < 8; ++i) b[off + i] = (uint8_t)(v >> (8 * i)); }
static uint16_t get_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t get_u32(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
static uint64_t get_u64(const uint8_t *p) { uint64_t v = 0; for (int i = 0; i < 8; ++i) v |= (uint64_t)p[i] << (8 * i); return v; }

/* native_codec.cpp:93-110 */
static const float kNf4[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};
/* float_codecs.cpp:184 */
static const float kFp4[16] = {0, 0.5f, 1, 1.5f, 2, 3, 4, 6, -0.0f, -0.5f, -1, -1.5f, -2, -3, -4, -6};

/* ------------------------------------------------------- scalar float codecs */

/* float_codecs.cpp:23-35 — truncating; exponent <= 0 -> signed zero; >= 31 -> Inf */
uint16_t or_f32_to_f16(float f) {
  const uint32_t b = f32bits(f);
  const uint16_t sign = (uint16_t)((b >> 16) & 0x8000);
  const int expo = (int)((b >> 23) & 0xff) - 127 + 15;
  const uint32_t mant = b & 0x7fffff;
  if (expo <= 0) return sign;
  if (expo >= 31) return (uint16_t)(sign | 0x7c00);
  return (uint16_t)(sign | (expo << 10) | (mant >> 13));
}

/* float_codecs.cpp:37-51 */
float or_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
  const uint32_t expo = (h >> 10) & 0x1f;
  const uint32_t mant = h & 0x3ff;
  if (expo == 0) {
    if (mant == 0) return bitsf32(sign);
    return bitsf32(sign | f32bits((float)mant / 1024.0f / 16384.0f));
  }
  if (expo == 31) return bitsf32(sign | 0x7f800000u | (mant << 13));
  return bitsf32(sign | ((expo - 15 + 127) << 23) | (mant << 13));
}

/* float_codecs.cpp:53-55 */
uint16_t or_f32_to_bf16(float f) { return (uint16_t)(f32bits(f) >> 16); }
float or_bf16_to_f32(uint16_t h) { return bitsf32((uint32_t)h << 16); }

/* float_codecs.cpp:57-97 — guard-bit rounding, saturating to 0x7e */
uint8_t or_f32_to_e4m3(float f) {
  if (f == 0.0f || isnan(f)) return 0;
  uint8_t sign = 0;
  if (f < 0) { sign = 0x80; f = -f; }
  if (f > 448.0f) return (uint8_t)(sign | 0x7e);
  const uint32_t bits = f32bits(f);
  const int ex = (int)((bits >> 23) & 0xff) - 127;
  uint32_t mant = bits & 0x7fffff;
  int e = ex + 7;
  if (e <= 0) {
    if (e < -2) return sign;
    mant |= 0x800000;
    const unsigned shift = (unsigned)(1 - e + 20);
    return (uint8_t)(sign | ((mant >> shift) & 0x7));
  }
  if (e >= 15) return (uint8_t)(sign | 0x7e);
  uint32_t m = (mant >> 20) & 0x7;
  if (mant & 0x80000) {
    m++;
    if (m == 8) {
      m = 0;
      e++;
      if (e >= 15) return (uint8_t)(sign | 0x7e);
    }
  }
  return (uint8_t)(sign | (e << 3) | m);
}

/* float_codecs.cpp:99-117 — subnormal codes decode to signed zero, 0x7f -> 448 */
float or_e4m3_to_f32(uint8_t b) {
  const uint32_t sign = (b & 0x80) ? 0x80000000u : 0u;
  const int e = (b >> 3) & 0xf;
  const int m = b & 0x7;
  if (e == 0) {
    if (m == 0) return bitsf32(sign);
    return bitsf32(sign) * (float)m / 8.0f / 64.0f;
  }
  if (e == 15 && m == 7) return bitsf32(sign | f32bits(448.0f));
  return bitsf32(sign | ((uint32_t)(e - 7 + 127) << 23) | ((uint32_t)m << 20));
}

/* float_codecs.cpp:119-158 */
uint8_t or_f32_to_e5m2(float f) {
  if (isnan(f)) return 0x7e;
  uint8_t sign = 0;
  if (f < 0 || signbit(f)) {
    sign = 0x80;
    if (f < 0) f = -f;
  }
  if (isinf(f)) return (uint8_t)(sign | 0x7c);
  if (f == 0.0f) return sign;
  const uint32_t bits = f32bits(f);
  const int ex = (int)((bits >> 23) & 0xff) - 127;
  const uint32_t mant = bits & 0x7fffff;
  int e = ex + 15;
  if (e <= 0) return sign;
  if (e >= 31) return (uint8_t)(sign | 0x7c);
  uint32_t m = (mant >> 21) & 0x3;
  if (mant & 0x100000) {
    m++;
    if (m == 4) {
      m = 0;
      e++;
      if (e >= 31) return (uint8_t)(sign | 0x7c);
    }
  }
  return (uint8_t)(sign | (e << 2) | m);
}

/* float_codecs.cpp:160-181 */
float or_e5m2_to_f32(uint8_t b) {
  const uint32_t sign = (b & 0x80) ? 0x80000000u : 0u;
  const int e = (b >> 2) & 0x1f;
  const int m = b & 0x3;
  if (e == 0) {
    if (m == 0) return bitsf32(sign);
    return bitsf32(sign) * (float)m / 4.0f / 16384.0f;
  }
  if (e == 31) return bitsf32(sign | (m == 0 ? 0x7f800000u : 0x7fc00000u));
  return bitsf32(sign | ((uint32_t)(e - 15 + 127) << 23) | ((uint32_t)m << 21));
}

/* float_codecs.cpp:187-200 — nearest table entry, first index wins ties */
uint8_t or_f32_to_fp4(float f) {
  uint8_t best = 0;
  float best_err = FLT_MAX;
  for (int c = 0; c < 16; ++c) {
    const float e = fabsf(f - kFp4[c]);
    if (e < best_err) { best_err = e; best = (uint8_t)c; }
  }
  return best;
}
float or_fp4_to_f32(uint8_t code) { return kFp4[code & 0xf]; }

/* ------------------------------------------------------------- native store */

/* byte sizes of each FormatNone payload (native_codec.cpp:189-560) */
int64_t or_native_bytes(int dt, int64_t n) {
  switch (dt) {
  case OR_FLOAT64: case OR_INT64: case OR_INT: case OR_COMPLEX64: return n * 8;
  case OR_FLOAT32: case OR_INT32: return n * 4;
  case OR_FLOAT16: case OR_BFLOAT16: case OR_INT16: return n * 2;
  case OR_FP8E4M3: case OR_FP8E5M2: case OR_INT8: return n;
  case OR_UINT64: case OR_UINT: case OR_UINTPTR: return 4 + n * 8;
  case OR_UINT32: return 4 + n * 4;
  case OR_UINT16: return 4 + n * 2;
  case OR_UINT8: return 4 + n;
  case OR_INT4: case OR_FP4: case OR_NF4: return (n + 1) / 2;
  case OR_UINT4: return 4 + (n + 1) / 2;
  case OR_INT2: case OR_TERNARY: return (n + 3) / 4;
  case OR_UINT2: return 4 + (n + 3) / 4;
  case OR_BINARY: return (n + 7) / 8;
  case OR_COMPLEX128: return n * 16;
  case OR_FP6: case OR_INT6: return (n * 6 + 7) / 8;
  case OR_UINT6: return 4 + (n * 6 + 7) / 8;
  case OR_INT5: return (n * 5 + 7) / 8;
  case OR_UINT5: return 4 + (n * 5 + 7) / 8;
  case OR_INT3: return (n * 3 + 7) / 8;
  case OR_UINT3: return 4 + (n * 3 + 7) / 8;
  }
  return -1;
}

/* native_codec.cpp:22-30 */
static float abs_max(const float *w, int64_t n) {
  float m = 0;
  for (int64_t i = 0; i < n; ++i) {
    const float a = fabsf(w[i]);
    if (a > m) m = a;
  }
  return m;
}

/* native_codec.cpp:32-40 */
static void min_max(const float *w, int64_t n, float *mn, float *mx) {
  *mn = *mx = w[0];
  for (int64_t i = 1; i < n; ++i) {
    if (w[i] < *mn) *mn = w[i];
    if (w[i] > *mx) *mx = w[i];
  }
}

/* native_codec.cpp:112-136 — LSB-first bitstream */
static void put_bits(uint8_t *b, int64_t i, int bits, uint64_t code) {
  const int64_t off = i * bits;
  for (int k = 0; k < bits; ++k) {
    const int64_t bit = off + k;
    if ((code >> k) & 1) b[bit / 8] |= (uint8_t)(1u << (bit % 8));
    else b[bit / 8] &= (uint8_t)~(1u << (bit % 8));
  }
}
static uint64_t get_bits(const uint8_t *raw, int64_t i, int bits) {
  const int64_t off = i * bits;
  uint64_t c = 0;
  for (int k = 0; k < bits; ++k)
    if (raw[(off + k) / 8] & (1u << ((off + k) % 8))) c |= (uint64_t)1 << k;
  return c;
}
/* native_codec.cpp:138-146 */
static int64_t sign_extend(uint64_t code, int bits) {
  const uint64_t sign_bit = (uint64_t)1 << (bits - 1);
  code &= ((uint64_t)1 << bits) - 1;
  if (code & sign_bit) return (int64_t)code - (int64_t)((uint64_t)1 << bits);
  return (int64_t)code;
}

/* native_codec.cpp:148-166 */
static void pack_signed_nbit(const float *w, int64_t n, int bits, uint8_t *out, float *scale) {
  const int max_q = (1 << (bits - 1)) - 1;
  const int min_q = -(1 << (bits - 1));
  float s = abs_max(w, n) / (float)max_q;
  if (s == 0) s = 1;
  memset(out, 0, (size_t)((n * bits + 7) / 8));
  for (int64_t i = 0; i < n; ++i) {
    int q = cvt_i32(roundf(w[i] / s));
    if (q > max_q) q = max_q;
    if (q < min_q) q = min_q;
    put_bits(out, i, bits, (uint64_t)((unsigned)q & ((1u << bits) - 1)));
  }
  *scale = s;
}

/* native_codec.cpp:168-187 */
static void pack_unsigned_nbit(const float *w, int64_t n, int bits, uint8_t *out, float *scale) {
  const int max_q = (1 << bits) - 1;
  float mn, mx;
  min_max(w, n, &mn, &mx);
  float span = mx - mn;
  if (span == 0) span = 1;
  memset(out, 0, (size_t)(4 + (n * bits + 7) / 8));
  put_u32(out, 0, f32bits(mn));
  for (int64_t i = 0; i < n; ++i) {
    const int q = cvt_i32(clamp_d(roundf((w[i] - mn) / span * (float)max_q), 0, max_q));
    put_bits(out + 4, i, bits, (uint64_t)q);
  }
  *scale = span / (float)max_q;
}

/* pack_native native_codec.cpp:189-560, plus the Float32 copy of
 * encode_format_none native_codec.cpp:819-833.  `out` holds or_native_bytes. */
int or_pack(int dt, const float *w, int64_t n, uint8_t *out, float *scale) {
  *scale = 1;
  if (n <= 0) return 1;
  switch (dt) {
  case OR_FLOAT32:
    for (int64_t i = 0; i < n; ++i) put_u32(out, i * 4, f32bits(w[i]));
    return 0;
  case OR_FLOAT64:
    for (int64_t i = 0; i < n; ++i) put_u64(out, i * 8, f64bits((double)w[i]));
    return 0;
  case OR_FLOAT16:
    for (int64_t i = 0; i < n; ++i) put_u16(out, i * 2, or_f32_to_f16(w[i]));
    return 0;
  case OR_BFLOAT16:
    for (int64_t i = 0; i < n; ++i) put_u16(out, i * 2, or_f32_to_bf16(w[i]));
    return 0;
  case OR_FP8E4M3:
    for (int64_t i = 0; i < n; ++i) out[i] = or_f32_to_e4m3(w[i]);
    return 0;
  case OR_FP8E5M2:
    for (int64_t i = 0; i < n; ++i) out[i] = or_f32_to_e5m2(w[i]);
    return 0;
  case OR_FP4: /* :223-233 */
    memset(out, 0, (size_t)((n + 1) / 2));
    for (int64_t i = 0; i < n; ++i) {
      const uint8_t code = or_f32_to_fp4(w[i]) & 0xF;
      if (i % 2 == 0) out[i / 2] = code;
      else out[i / 2] |= (uint8_t)(code << 4);
    }
    return 0;
  case OR_INT64: case OR_INT: { /* :234-247, :433-445 (LP64 host) */
    float s = abs_max(w, n);
    if (s == 0) s = 1;
    for (int64_t i = 0; i < n; ++i) {
      const float qf = w[i] / s * 1e6f;
      put_u64(out, i * 8, (uint64_t)cvt_i64(round((double)qf)));
    }
    *scale = s / 1e6f;
    return 0;
  }
  case OR_INT32: { /* :248-262 — the +absmax element is 2^31: saturates (arm64) */
    float s = abs_max(w, n);
    if (s == 0) s = 1;
    for (int64_t i = 0; i < n; ++i) {
      const float qf = w[i] / s * 2147483647.0f;
      put_u32(out, i * 4, (uint32_t)cvt_i32(round((double)qf)));
    }
    *scale = s / 2147483647.0f;
    return 0;
  }
  case OR_INT16: { /* :263-276 */
    float s = abs_max(w, n);
    if (s == 0) s = 1;
    for (int64_t i = 0; i < n; ++i) {
      const float qf = w[i] / s * 32767.0f;
      const int q = cvt_i32(clamp_d(round((double)qf), -32768, 32767));
      put_u16(out, i * 2, (uint16_t)(int16_t)q);
    }
    *scale = s / 32767.0f;
    return 0;
  }
  case OR_INT8: { /* :277-288 */
    float s = abs_max(w, n) / 127.0f;
    if (s == 0) s = 1;
    for (int64_t i = 0; i < n; ++i) {
      const int q = cvt_i32(clamp_d(roundf(w[i] / s), -128, 127));
      out[i] = (uint8_t)(int8_t)q;
    }
    *scale = s;
    return 0;
  }
  case OR_UINT8: case OR_UINT16: case OR_UINT32: case OR_UINT64: case OR_UINT: case OR_UINTPTR: {
    /* :289-341, :457-502 (LP64 host: Uint and Uintptr use the Uint64 layout) */
    float mn, mx;
    min_max(w, n, &mn, &mx);
    float span = mx - mn;
    if (span == 0) span = 1;
    put_u32(out, 0, f32bits(mn));
    if (dt == OR_UINT8) {
      for (int64_t i = 0; i < n; ++i) {
        const float qf = (w[i] - mn) / span * 255.0f;
        out[4 + i] = (uint8_t)cvt_u32(clamp_d(round((double)qf), 0, 255));
      }
      *scale = span / 255.0f;
    } else if (dt == OR_UINT16) {
      for (int64_t i = 0; i < n; ++i) {
        const float qf = (w[i] - mn) / span * 65535.0f;
        put_u16(out, 4 + i * 2, (uint16_t)cvt_u32(clamp_d(round((double)qf), 0, 65535)));
      }
      *scale = span / 65535.0f;
    } else if (dt == OR_UINT32) {
      const float maxu_f = (float)4294967295u;
      for (int64_t i = 0; i < n; ++i) {
        const float qf = (w[i] - mn) / span * maxu_f;
        put_u32(out, 4 + i * 4, cvt_u32(clamp_d(round((double)qf), 0, 4294967295.0)));
      }
      *scale = span / maxu_f;
    } else {
      for (int64_t i = 0; i < n; ++i) {
        const float qf = (w[i] - mn) / span * 1e15f;
        put_u64(out, 4 + i * 8, cvt_u64(clamp_d(round((double)qf), 0, 1e15)));
      }
      *scale = span / 1e15f;
    }
    return 0;
  }
  case OR_INT4: { /* :342-356 */
    float s = abs_max(w, n) / 7.0f;
    if (s == 0) s = 1;
    memset(out, 0, (size_t)((n + 1) / 2));
    for (int64_t i = 0; i < n; ++i) {
      const int q = cvt_i32(clamp_d(roundf(w[i] / s), -8, 7)) & 0xF;
      if (i % 2 == 0) out[i / 2] = (uint8_t)q;
      else out[i / 2] |= (uint8_t)(q << 4);
    }
    *scale = s;
    return 0;
  }
  case OR_UINT4: { /* :357-375 */
    float mn, mx;
    min_max(w, n, &mn, &mx);
    float span = mx - mn;
    if (span == 0) span = 1;
    memset(out, 0, (size_t)(4 + (n + 1) / 2));
    put_u32(out, 0, f32bits(mn));
    for (int64_t i = 0; i < n; ++i) {
      const float qf = (w[i] - mn) / span * 15.0f;
      const int q = cvt_i32(clamp_d(round((double)qf), 0, 15)) & 0xF;
      if (i % 2 == 0) out[4 + i / 2] = (uint8_t)q;
      else out[4 + i / 2] |= (uint8_t)(q << 4);
    }
    *scale = span / 15.0f;
    return 0;
  }
  case OR_INT2: { /* :376-388 */
    float s = abs_max(w, n);
    if (s == 0) s = 1;
    memset(out, 0, (size_t)((n + 3) / 4));
    for (int64_t i = 0; i < n; ++i) {
      const int q = cvt_i32(clamp_d(roundf(w[i] / s), -2, 1));
      out[i / 4] |= (uint8_t)(((q + 2) & 3) << ((i % 4) * 2));
    }
    *scale = s;
    return 0;
  }
  case OR_UINT2: { /* :389-403 — note the double 3.0 */
    float mn, mx;
    min_max(w, n, &mn, &mx);
    float span = mx - mn;
    if (span == 0) span = 1;
    memset(out, 0, (size_t)(4 + (n + 3) / 4));
    put_u32(out, 0, f32bits(mn));
    for (int64_t i = 0; i < n; ++i) {
      const int q = cvt_i32(clamp_d(round((double)((w[i] - mn) / span) * 3.0), 0, 3)) & 3;
      out[4 + i / 4] |= (uint8_t)(q << ((i % 4) * 2));
    }
    *scale = span / 3.0f;
    return 0;
  }
  case OR_TERNARY: { /* :404-420 */
    float s = abs_max(w, n);
    if (s == 0) s = 1;
    memset(out, 0, (size_t)((n + 3) / 4));
    for (int64_t i = 0; i < n; ++i) {
      const float r = w[i] / s;
      int code = 1;
      if (r > 0.5f) code = 2;
      else if (r < -0.5f) code = 0;
      out[i / 4] |= (uint8_t)(code << ((i % 4) * 2));
    }
    *scale = s;
    return 0;
  }
  case OR_BINARY: { /* :421-432 */
    float s = abs_max(w, n);
    if (s == 0) s = 1;
    memset(out, 0, (size_t)((n + 7) / 8));
    for (int64_t i = 0; i < n; ++i)
      if (w[i] >= 0) out[i / 8] |= (uint8_t)(1u << (i % 8));
    *scale = s;
    return 0;
  }
  case OR_COMPLEX64: /* :503-510 */
    for (int64_t i = 0; i < n; ++i) { put_u32(out, i * 8, f32bits(w[i])); put_u32(out, i * 8 + 4, 0); }
    return 0;
  case OR_COMPLEX128: /* :511-518 */
    for (int64_t i = 0; i < n; ++i) { put_u64(out, i * 16, f64bits((double)w[i])); put_u64(out, i * 16 + 8, 0); }
    return 0;
  case OR_NF4: { /* :519-542 — one per-tensor absmax scale */
    float s = abs_max(w, n);
    if (s == 0) s = 1;
    memset(out, 0, (size_t)((n + 1) / 2));
    for (int64_t i = 0; i < n; ++i) {
      const float r = w[i] / s;
      int best = 0;
      float best_err = FLT_MAX;
      for (int c = 0; c < 16; ++c) {
        const float e = fabsf(r - kNf4[c]);
        if (e < best_err) { best_err = e; best = c; }
      }
      if (i % 2 == 0) out[i / 2] = (uint8_t)(best & 0xF);
      else out[i / 2] |= (uint8_t)((best & 0xF) << 4);
    }
    *scale = s;
    return 0;
  }
  case OR_FP6: case OR_INT6: pack_signed_nbit(w, n, 6, out, scale); return 0; /* :543-545 */
  case OR_UINT6: pack_unsigned_nbit(w, n, 6, out, scale); return 0;
  case OR_INT5: pack_signed_nbit(w, n, 5, out, scale); return 0;
  case OR_UINT5: pack_unsigned_nbit(w, n, 5, out, scale); return 0;
  case OR_INT3: pack_signed_nbit(w, n, 3, out, scale); return 0;
  case OR_UINT3: pack_unsigned_nbit(w, n, 3, out, scale); return 0;
  }
  return 2;
}

/* weight_at native_codec.cpp:562-813: element i of n, as float.  Returns 1
 * when the payload is short, like the reference. */
static int weight_at(int dt, const uint8_t *raw, int64_t raw_n, float scale, int64_t i, int64_t n,
                     float *out) {
  if (scale == 0) scale = 1;
  const int64_t need = or_native_bytes(dt, n);
  if (need < 0) return 3;
  if (raw_n < need) return 1;
  switch (dt) {
  case OR_FLOAT32: return 1; /* :809-810 — Float32 lives in the f32 vector */
  case OR_FLOAT64: *out = (float)bitsf64(get_u64(raw + i * 8)); return 0;
  case OR_FLOAT16: *out = or_f16_to_f32(get_u16(raw + i * 2)); return 0;
  case OR_BFLOAT16: *out = or_bf16_to_f32(get_u16(raw + i * 2)); return 0;
  case OR_FP8E4M3: *out = or_e4m3_to_f32(raw[i]); return 0;
  case OR_FP8E5M2: *out = or_e5m2_to_f32(raw[i]); return 0;
  case OR_FP4: *out = or_fp4_to_f32((i % 2 == 0) ? (raw[i / 2] & 0xF) : (raw[i / 2] >> 4)); return 0;
  case OR_INT64: case OR_INT: *out = (float)(int64_t)get_u64(raw + i * 8) * scale; return 0;
  case OR_INT32: *out = (float)(int32_t)get_u32(raw + i * 4) * scale; return 0;
  case OR_INT16: *out = (float)(int16_t)get_u16(raw + i * 2) * scale; return 0;
  case OR_INT8: *out = (float)(int8_t)raw[i] * scale; return 0;
  case OR_UINT8: *out = (float)raw[4 + i] * scale + bitsf32(get_u32(raw)); return 0;
  case OR_UINT16: *out = (float)get_u16(raw + 4 + i * 2) * scale + bitsf32(get_u32(raw)); return 0;
  case OR_UINT32: *out = (float)get_u32(raw + 4 + i * 4) * scale + bitsf32(get_u32(raw)); return 0;
  case OR_UINT64: case OR_UINT: case OR_UINTPTR:
    *out = (float)get_u64(raw + 4 + i * 8) * scale + bitsf32(get_u32(raw)); return 0;
  case OR_INT4: {
    int q = (i % 2 == 0) ? (raw[i / 2] & 0xF) : (raw[i / 2] >> 4);
    if (q > 7) q -= 16;
    *out = (float)q * scale;
    return 0;
  }
  case OR_UINT4: {
    const uint8_t *body = raw + 4;
    const int q = (i % 2 == 0) ? (body[i / 2] & 0xF) : (body[i / 2] >> 4);
    *out = (float)q * scale + bitsf32(get_u32(raw));
    return 0;
  }
  case OR_INT2: *out = (float)(((raw[i / 4] >> ((i % 4) * 2)) & 3) - 2) * scale; return 0;
  case OR_UINT2:
    *out = (float)((raw[4 + i / 4] >> ((i % 4) * 2)) & 3) * scale + bitsf32(get_u32(raw)); return 0;
  case OR_TERNARY: {
    const int code = (raw[i / 4] >> ((i % 4) * 2)) & 3;
    *out = code == 0 ? -scale : (code == 2 ? scale : 0.0f);
    return 0;
  }
  case OR_BINARY: *out = (raw[i / 8] & (1u << (i % 8))) ? scale : -scale; return 0;
  case OR_COMPLEX64: *out = bitsf32(get_u32(raw + i * 8)); return 0;
  case OR_COMPLEX128: *out = (float)bitsf64(get_u64(raw + i * 16)); return 0;
  case OR_NF4: *out = kNf4[(i % 2 == 0) ? (raw[i / 2] & 0xF) : (raw[i / 2] >> 4)] * scale; return 0;
  case OR_FP6: case OR_INT6: *out = (float)sign_extend(get_bits(raw, i, 6), 6) * scale; return 0;
  case OR_INT5: *out = (float)sign_extend(get_bits(raw, i, 5), 5) * scale; return 0;
  case OR_INT3: *out = (float)sign_extend(get_bits(raw, i, 3), 3) * scale; return 0;
  case OR_UINT6: *out = (float)get_bits(raw + 4, i, 6) * scale + bitsf32(get_u32(raw)); return 0;
  case OR_UINT5: *out = (float)get_bits(raw + 4, i, 5) * scale + bitsf32(get_u32(raw)); return 0;
  case OR_UINT3: *out = (float)get_bits(raw + 4, i, 3) * scale + bitsf32(get_u32(raw)); return 0;
  }
  return 3;
}

/* decode_row_f64 native_codec.cpp:835-870 over the whole matrix: Float32 is
 * widened, Float64 keeps full precision, the rest widen the float decode. */
int or_decode_f64(int dt, const uint8_t *raw, int64_t raw_n, float scale, int64_t n, double *out) {
  if (dt == OR_FLOAT32) {
    if (raw_n < n * 4) return 1;
    for (int64_t i = 0; i < n; ++i) out[i] = (double)bitsf32(get_u32(raw + i * 4));
    return 0;
  }
  if (dt == OR_FLOAT64) {
    if (raw_n < n * 8) return 1;
    for (int64_t i = 0; i < n; ++i) out[i] = bitsf64(get_u64(raw + i * 8));
    return 0;
  }
  for (int64_t i = 0; i < n; ++i) {
    float v = 0;
    const int st = weight_at(dt, raw, raw_n, scale, i, n, &v);
    if (st) return st;
    out[i] = (double)v;
  }
  return 0;
}

/* export_f32 store.cpp:122-149 */
int or_decode(int dt, const uint8_t *raw, int64_t raw_n, float scale, int64_t n, float *out) {
  if (dt == OR_FLOAT32) {
    if (raw_n < n * 4) return 1;
    for (int64_t i = 0; i < n; ++i) out[i] = bitsf32(get_u32(raw + i * 4));
    return 0;
  }
  if (dt == OR_FLOAT64) {
    if (raw_n < n * 8) return 1;
    for (int64_t i = 0; i < n; ++i) out[i] = (float)bitsf64(get_u64(raw + i * 8));
    return 0;
  }
  for (int64_t i = 0; i < n; ++i) {
    const int st = weight_at(dt, raw, raw_n, scale, i, n, &out[i]);
    if (st) return st;
  }
  return 0;
}

/* ops_storage.metal:611-623 */
static void put_nibble(uint8_t *raw, int64_t i, uint8_t code) {
  code &= 0xF;
  if (i % 2 == 0) raw[i / 2] = (uint8_t)((raw[i / 2] & 0xF0) | code);
  else raw[i / 2] = (uint8_t)((raw[i / 2] & 0x0F) | (code << 4));
}
static void put_2bit(uint8_t *raw, int64_t i, uint8_t code) {
  const unsigned shift = (unsigned)(i % 4) * 2;
  raw[i / 4] = (uint8_t)((raw[i / 4] & ~(3u << shift)) | ((code & 3u) << shift));
}

/* ops_storage.metal:106-113 */
static uint64_t quant_u64(float v, float min_v, float scale) {
  const float q = roundf((v - min_v) / scale);
  if (q <= 0) return 0;
  if (q >= 1e15f) return 1000000000000000ull;
  return cvt_u64(q);
}

/* set_weight_at ops_storage.metal:655-921: fixed-scale in-place re-encode of
 * element i.  The float-format cases share the scalar codecs above; the
 * clamp bounds are float, so 2147483647.0 and 4294967295.0 become 2^31, 2^32
 * and the following integer conversion saturates. */
int or_set(int dt, uint8_t *raw, int64_t raw_n, float scale, int64_t i, int64_t n, float v) {
  if (scale == 0) scale = 1;
  const int64_t need = or_native_bytes(dt, n);
  if (need < 0 || dt == OR_FLOAT32 || dt == OR_FLOAT64) return 1;
  if (raw_n < need || i < 0 || i >= n) return 1;
  switch (dt) {
  case OR_FLOAT16: put_u16(raw, i * 2, or_f32_to_f16(v)); return 0;
  case OR_BFLOAT16: put_u16(raw, i * 2, or_f32_to_bf16(v)); return 0;
  case OR_FP8E4M3: raw[i] = or_f32_to_e4m3(v); return 0;
  case OR_FP8E5M2: raw[i] = or_f32_to_e5m2(v); return 0;
  case OR_FP4: put_nibble(raw, i, or_f32_to_fp4(v)); return 0;
  case OR_INT64: case OR_INT: put_u64(raw, i * 8, (uint64_t)cvt_i64(roundf(v / scale))); return 0;
  case OR_INT32:
    put_u32(raw, i * 4, (uint32_t)cvt_i32(clamp_f(roundf(v / scale), -2147483648.0f, 2147483648.0f)));
    return 0;
  case OR_INT16:
    put_u16(raw, i * 2, (uint16_t)(int16_t)cvt_i32(clamp_f(roundf(v / scale), -32768.0f, 32767.0f)));
    return 0;
  case OR_INT8: raw[i] = (uint8_t)(int8_t)cvt_i32(clamp_f(roundf(v / scale), -128.0f, 127.0f)); return 0;
  case OR_UINT8: {
    const float mn = bitsf32(get_u32(raw));
    raw[4 + i] = (uint8_t)cvt_u32(clamp_f(roundf((v - mn) / scale), 0.0f, 255.0f));
    return 0;
  }
  case OR_UINT16: {
    const float mn = bitsf32(get_u32(raw));
    put_u16(raw, 4 + i * 2, (uint16_t)cvt_u32(clamp_f(roundf((v - mn) / scale), 0.0f, 65535.0f)));
    return 0;
  }
  case OR_UINT32: {
    const float mn = bitsf32(get_u32(raw));
    put_u32(raw, 4 + i * 4, cvt_u32(clamp_f(roundf((v - mn) / scale), 0.0f, 4294967296.0f)));
    return 0;
  }
  case OR_UINT64: case OR_UINT: case OR_UINTPTR:
    put_u64(raw, 4 + i * 8, quant_u64(v, bitsf32(get_u32(raw)), scale));
    return 0;
  case OR_INT4: put_nibble(raw, i, (uint8_t)(cvt_i32(clamp_f(roundf(v / scale), -8.0f, 7.0f)) & 0xF)); return 0;
  case OR_UINT4: {
    const float mn = bitsf32(get_u32(raw));
    put_nibble(raw + 4, i, (uint8_t)(cvt_i32(clamp_f(roundf((v - mn) / scale), 0.0f, 15.0f)) & 0xF));
    return 0;
  }
  case OR_INT2: {
    const int q = cvt_i32(clamp_f(roundf(v / scale), -2.0f, 1.0f));
    put_2bit(raw, i, (uint8_t)((q + 2) & 3));
    return 0;
  }
  case OR_UINT2: {
    const float mn = bitsf32(get_u32(raw));
    put_2bit(raw + 4, i, (uint8_t)(cvt_i32(clamp_f(roundf((v - mn) / scale), 0.0f, 3.0f)) & 3));
    return 0;
  }
  case OR_TERNARY: {
    const float r = v / scale;
    uint8_t code = 1;
    if (r > 0.5f) code = 2;
    else if (r < -0.5f) code = 0;
    put_2bit(raw, i, code);
    return 0;
  }
  case OR_BINARY:
    if (v >= 0) raw[i / 8] |= (uint8_t)(1u << (i % 8));
    else raw[i / 8] &= (uint8_t)~(1u << (i % 8));
    return 0;
  case OR_COMPLEX64: put_u32(raw, i * 8, f32bits(v)); return 0;
  case OR_COMPLEX128: put_u64(raw, i * 16, f64bits((double)v)); return 0;
  case OR_NF4: {
    const float r = v / scale;
    int best = 0;
    float best_err = FLT_MAX;
    for (int c = 0; c < 16; ++c) {
      const float e = fabsf(r - kNf4[c]);
      if (e < best_err) { best_err = e; best = c; }
    }
    put_nibble(raw, i, (uint8_t)best);
    return 0;
  }
  case OR_FP6: case OR_INT6: case OR_INT5: case OR_INT3: { /* :636-646 */
    const int bits = (dt == OR_INT5) ? 5 : (dt == OR_INT3 ? 3 : 6);
    const int max_q = (1 << (bits - 1)) - 1, min_q = -(1 << (bits - 1));
    int q = cvt_i32(roundf(v / scale));
    if (q > max_q) q = max_q;
    if (q < min_q) q = min_q;
    put_bits(raw, i, bits, (uint64_t)((unsigned)q & ((1u << bits) - 1)));
    return 0;
  }
  case OR_UINT6: case OR_UINT5: case OR_UINT3: { /* :647-654 */
    const int bits = (dt == OR_UINT5) ? 5 : (dt == OR_UINT3 ? 3 : 6);
    const float mn = bitsf32(get_u32(raw));
    const int q = cvt_i32(clamp_f(roundf((v - mn) / scale), 0.0f, (float)((1 << bits) - 1)));
    put_bits(raw + 4, i, bits, (uint64_t)q);
    return 0;
  }
  }
  return 1;
}

/* ----------------------------------------------------------------- training */

/* WeightStore::apply_sgd native_codec.cpp:909-945 (native part) with the
 * kernel op_native_sgd ops_storage.metal:924-958: element 0 is decoded and
 * re-encoded once before the loop; each element then becomes
 * fl32(old - lr*g) and is re-encoded with the stored scale/min.  Float64
 * updates the f64 value directly.  dW arrives as f32 and widens exactly. */
int or_native_sgd(int dt, uint8_t *raw, int64_t raw_n, float scale, int64_t n, const float *dW,
                  double lr) {
  if (!dW || n <= 0 || !isfinite(lr)) return 1;
  if (dt == OR_FLOAT32) return 1;
  if (raw_n <= 0 || (dt == OR_FLOAT64 && raw_n != n * 8)) return 1;
  for (int64_t i = 0; i < n; ++i)
    if (!isfinite(dW[i])) return 1;
  if (dt == OR_FLOAT64) {
    for (int64_t i = 0; i < n; ++i) {
      const double old = bitsf64(get_u64(raw + i * 8));
      put_u64(raw, i * 8, f64bits(old - lr * (double)dW[i]));
    }
    return 0;
  }
  float v0 = 0;
  if (weight_at(dt, raw, raw_n, scale, 0, n, &v0) || or_set(dt, raw, raw_n, scale, 0, n, v0)) return 1;
  for (int64_t i = 0; i < n; ++i) {
    float old = 0;
    if (weight_at(dt, raw, raw_n, scale, i, n, &old)) return 1;
    const float value = (float)((double)old - lr * (double)dW[i]);
    if (or_set(dt, raw, raw_n, scale, i, n, value)) return 1;
  }
  return 0;
}

/* op_native_repack ops_storage.metal:971-1144 (the complete store
 * replacement behind WeightStore::set_from_f32_gpu, native_codec.cpp:872-907):
 * fresh statistics and scale, then every element re-encoded.
 *  - statistics: hi = max |a[i]|, mn / mx = min / max of a[i]; Metal's
 *    max/min return the other operand of a NaN, so NaN elements (element 0
 *    included) are skipped; with no number at all mn = mx = NaN.  Equal
 *    extremes keep the first element that attains them (the sign of a zero
 *    extreme is where Metal's min/max leave the choice open).
 *  - cam_div / cam_mul divide / multiply through double-float and round to
 *    f32: for two f32 operands that is the correctly rounded f32 quotient /
 *    product (the f64 result holds it exactly, or rounds innocuously), so
 *    they are f32 '/' and '*' here.
 *  - scale: base = hi (0 -> 1); Int64 / Int base / 1e6, Int32 base /
 *    2147483647 (= 2^31 as float), Int16 base / 32767, Int8 hi / 127 (0 -> 1),
 *    Int4 hi / 7 (0 -> 1), Int2 / Ternary / Binary / NF4 base, n-bit signed
 *    hi / (2^(bits-1) - 1) (0 -> 1), unsigned span / maxu with the f32 min
 *    as the 4-byte header; every other dtype 1.
 *  - codes as pack_native's, except Uint2 (q = round(fl32(fl32((v - mn) /
 *    span) * 3.0f)), an f32 multiply where pack rounds a double product) and
 *    the unsigned qf clamped below by max(0, qf) (NaN -> 0); the float
 *    formats, Binary and the complex types go through set_weight_at with
 *    the new scale (or_set).
 * Returns 0, or 1 for bad arguments. */
int or_repack(int dt, const float *a, int64_t n, uint8_t *raw, int64_t raw_n, float *scale_out) {
  if (n <= 0 || dt < 0 || dt >= OR_NUM_DTYPES) return 1;
  const int64_t bytes = or_native_bytes(dt, n);
  if (bytes < 0 || raw_n < bytes) return 1;
  memset(raw, 0, (size_t)bytes);
  float hi = 0, mn = NAN, mx = NAN;
  int have = 0;
  for (int64_t i = 0; i < n; ++i) {
    const float v = a[i];
    if (fabsf(v) > hi) hi = fabsf(v);
    if (v != v) continue;
    if (!have) {
      mn = mx = v;
      have = 1;
    } else {
      if (v < mn) mn = v;
      if (v > mx) mx = v;
    }
  }
  const float base = hi == 0 ? 1 : hi;
  float span = mx - mn;
  if (span == 0) span = 1;
  float scale = 1;
  const int uns = dt == OR_UINT64 || dt == OR_UINT32 || dt == OR_UINT16 || dt == OR_UINT8 ||
                  dt == OR_UINT4 || dt == OR_UINT2 || dt == OR_UINT || dt == OR_UINTPTR ||
                  dt == OR_UINT6 || dt == OR_UINT5 || dt == OR_UINT3;
  const int nbit = dt == OR_FP6 || dt == OR_INT6 ? 6 : dt == OR_INT5 ? 5 : dt == OR_INT3 ? 3 : 0;
  if (dt == OR_INT64 || dt == OR_INT) scale = base / 1e6f;
  if (dt == OR_INT32) scale = base / 2147483647.0f;
  if (dt == OR_INT16) scale = base / 32767.0f;
  if (dt == OR_INT8) {
    scale = hi / 127.0f;
    if (scale == 0) scale = 1;
  }
  if (dt == OR_INT4) {
    scale = hi / 7.0f;
    if (scale == 0) scale = 1;
  }
  if (dt == OR_INT2 || dt == OR_TERNARY || dt == OR_BINARY || dt == OR_NF4) scale = base;
  if (nbit) {
    scale = hi / (float)((1 << (nbit - 1)) - 1);
    if (scale == 0) scale = 1;
  }
  float maxu = 1;
  if (uns) {
    maxu = (dt == OR_UINT64 || dt == OR_UINT || dt == OR_UINTPTR) ? 1e15f
           : dt == OR_UINT32 ? 4294967295.0f
           : dt == OR_UINT16 ? 65535.0f
           : dt == OR_UINT8 ? 255.0f
           : dt == OR_UINT4 ? 15.0f
           : dt == OR_UINT2 ? 3.0f
           : (float)((1 << (dt == OR_UINT6 ? 6 : dt == OR_UINT5 ? 5 : 3)) - 1);
    scale = span / maxu;
    put_u32(raw, 0, f32bits(mn));
  }
  *scale_out = scale;
  for (int64_t i = 0; i < n; ++i) {
    const float v = a[i];
    switch (dt) {
    case OR_FLOAT32: put_u32(raw, i * 4, f32bits(v)); continue;
    case OR_FLOAT64: put_u64(raw, i * 8, f64bits((double)v)); continue;
    case OR_INT64: case OR_INT:
      put_u64(raw, i * 8, (uint64_t)cvt_i64(roundf(v / base * 1e6f)));
      continue;
    case OR_INT32: {
      int64_t q = cvt_i64(roundf(v / base * 2147483647.0f));
      q = q < -2147483648LL ? -2147483648LL : (q > 2147483647LL ? 2147483647LL : q);
      put_u32(raw, i * 4, (uint32_t)q);
      continue;
    }
    case OR_INT16: put_u16(raw, i * 2, (uint16_t)cvt_i64(roundf(v / base * 32767.0f))); continue;
    case OR_INT8: {
      int64_t q = cvt_i64(roundf(v / scale));
      q = q < -128 ? -128 : (q > 127 ? 127 : q);
      raw[i] = (uint8_t)q;
      continue;
    }
    case OR_INT4: {
      int q = cvt_i32(roundf(v / scale));
      q = q < -8 ? -8 : (q > 7 ? 7 : q);
      put_nibble(raw, i, (uint8_t)(q & 15));
      continue;
    }
    case OR_INT2: {
      int q = cvt_i32(roundf(v / scale));
      q = q < -2 ? -2 : (q > 1 ? 1 : q);
      put_2bit(raw, i, (uint8_t)((q + 2) & 3));
      continue;
    }
    case OR_TERNARY: {
      const float norm = v / scale;
      put_2bit(raw, i, norm > .5f ? 2 : norm < -.5f ? 0 : 1);
      continue;
    }
    case OR_NF4: {
      const float norm = v / scale;
      float err = FLT_MAX;
      int best = 0;
      for (int c = 0; c < 16; ++c) {
        const float d = fabsf(norm - kNf4[c]);
        if (d < err) {
          err = d;
          best = c;
        }
      }
      put_nibble(raw, i, (uint8_t)best);
      continue;
    }
    case OR_FP6: case OR_INT6: case OR_INT5: case OR_INT3: {
      const int lim = 1 << (nbit - 1);
      int q = cvt_i32(roundf(v / scale));
      q = q < -lim ? -lim : (q > lim - 1 ? lim - 1 : q);
      put_bits(raw, i, nbit, (uint64_t)((uint32_t)q & ((1u << nbit) - 1)));
      continue;
    }
    default: break;
    }
    if (uns) {
      float qf = roundf((v - mn) / span * maxu);
      qf = fmaxf(0.0f, qf);  /* Metal max: NaN -> 0 */
      uint64_t q = cvt_u64(qf);
      if (dt == OR_UINT32 && q > 4294967295ull) q = 4294967295ull;
      uint8_t *body = raw + 4;
      if (dt == OR_UINT64 || dt == OR_UINT || dt == OR_UINTPTR) put_u64(body, i * 8, q);
      else if (dt == OR_UINT32) put_u32(body, i * 4, (uint32_t)q);
      else if (dt == OR_UINT16) put_u16(body, i * 2, (uint16_t)q);
      else if (dt == OR_UINT8) body[i] = (uint8_t)q;
      else if (dt == OR_UINT4) put_nibble(body, i, (uint8_t)q);
      else if (dt == OR_UINT2) put_2bit(body, i, (uint8_t)q);
      else put_bits(body, i, dt == OR_UINT6 ? 6 : dt == OR_UINT5 ? 5 : 3, q);
      continue;
    }
    /* Float16, BFloat16, FP8, FP4, Binary, Complex64/128: set_weight_at */
    if (or_set(dt, raw, raw_n, scale, i, n, v)) return 1;
  }
  return 0;
}

/* welvet_sgd_f32_f64_grad welvet_dense.metal:263-281: the step is rounded to
 * f32 first, then subtracted in f32. */
void or_sgd_f32(float *w, const float *dW, int64_t n, double lr) {
  for (int64_t i = 0; i < n; ++i) {
    const float step = (float)(lr * (double)dW[i]);
    w[i] = w[i] - step;
  }
}

/* welvet_mse_loss welvet_dense.metal:193-205 (serial, element order) */
double or_mse(const float *pred, const float *target, int64_t n) {
  double sum = 0;
  for (int64_t i = 0; i < n; ++i) {
    const double d = (double)pred[i] - (double)target[i];
    sum += d * d;
  }
  return sum / (double)n;
}

/* welvet_mse_grad welvet_dense.metal:207-215 */
void or_mse_grad(const float *pred, const float *target, int64_t n, float *grad) {
  for (int64_t i = 0; i < n; ++i)
    grad[i] = (float)((((double)pred[i] - (double)target[i]) * 2.0) / (double)n);
}

/* -------------------------------------------------------------- activations */

static const double kGeluC = 0.044715;               /* ops_common.metal:93 (hi+lo) */
static const double kGeluK = 0.7978845608028654;     /* sqrt(2/pi), ops_common.metal:94 */

static double sigmoid64(double x) { return 1.0 / (1.0 + exp(-x)); }  /* ops_common.metal:64-66 */
static double tanh64(double x) {                                     /* ops_common.metal:67-74 */
  if (x > 18) return 1;
  if (x < -18) return -1;
  return tanh(x);
}

/* act_value ops_common.metal:83-105 */
float or_act(float v, int act) {
  const double x = (double)v;
  switch (act) {
  case 1: return (float)(x * sigmoid64(x));
  case 3: return (float)tanh64(x);
  case 4: return (float)sigmoid64(x);
  case 2: {
    const double cubic = ((x * x) * x) * kGeluC;
    const double u = (x + cubic) * kGeluK;
    return (float)((x * 0.5) * (1.0 + tanh64(u)));
  }
  case 0: return v > 0.0f ? v : 0.0f;
  case 6: return v < 0 ? 0.0f : v * v;
  case 5: return v < 0 ? (float)(x * 0.01) : v;
  }
  return v;
}

/* act_prime ops_common.metal:106-138 */
float or_act_prime(float v, int act) {
  const double x = (double)v;
  switch (act) {
  case 1: {
    const double z = sigmoid64(x);
    return (float)(z * (1.0 + x * (1.0 - z)));
  }
  case 2: {
    const double xx = x * x;
    const double u = kGeluK * (x + kGeluC * (xx * x));
    const double t = tanh64(u);
    const double du = kGeluK * (1.0 + (kGeluC * xx) * 3.0);
    return (float)((1.0 + t) * 0.5 + ((x * 0.5) * (1.0 - t * t)) * du);
  }
  case 3: {
    const double t = tanh64(x);
    return (float)(1.0 - t * t);
  }
  case 4: {
    const double z = sigmoid64(x);
    return (float)(z * (1.0 - z));
  }
  case 0: return v > 0 ? 1.0f : 0.0f;
  case 6: return v > 0 ? 2 * v : 0.0f;
  case 5: return v > 0 ? 1.0f : 0.01f;
  }
  return 1.0f;
}

/* -------------------------------------------------------------------- Dense */

/* welvet_dense_matvec_softdouble_batch welvet_dense.metal:54-85 pinned to the
 * Go contract pre = fl32(sum_k f64(W)*f64(x)) in k order, then
 * welvet_dense_bias_act :87-105: pre = fl32(f64(pre) + bias) for o < bias_len,
 * post = act(pre).  Wd is the decode_row_f64 matrix [out][in]. */
/* Outputs are independent and each keeps its k order, so splitting the
 * (b, o) pairs over OpenMP threads changes no bit of the result. */
void or_dense_forward(int batch, int in, int out, int act, const double *Wd, const double *bias,
                      int64_t bias_len, const float *x, float *pre, float *post) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < batch; ++b) {
    for (int o = 0; o < out; ++o) {
      double acc = 0;
      const double *row = Wd + (int64_t)o * in;
      const float *xb = x + (int64_t)b * in;
      for (int k = 0; k < in; ++k) acc += row[k] * (double)xb[k];
      float p = (float)acc;
      if (bias && o < bias_len) p = (float)((double)p + bias[o]);
      pre[(int64_t)b * out + o] = p;
      post[(int64_t)b * out + o] = or_act(p, act);
    }
  }
}

/* welvet_dense_act_deriv :107-119, welvet_dense_matvect_softdouble_batch
 * :121-153 (dX = fl32(sum_o W[o,i]*dpre[b,o]) in o order) and
 * welvet_dense_outer_batch :155-178 (dW[o,i] = sequential fp32 FMA over b). */
/* Each dX[b][i] is summed over o in ascending order and each dW[o][i] over b
 * in ascending order; the loops below keep those orders (the running sums of
 * a whole row advance together, one o or one b at a time), so the threads
 * and the row-wise traversal change no bit of the result. */
void or_dense_backward(int batch, int in, int out, int act, const double *Wd, const float *x,
                       const float *pre, const float *gy, float *dpre, float *dX, float *dW) {
  const int64_t ny = (int64_t)batch * out;
  for (int64_t j = 0; j < ny; ++j) dpre[j] = gy[j] * or_act_prime(pre[j], act);
#pragma omp parallel
  {
    double *acc = (double *)malloc(sizeof(double) * (size_t)in);
#pragma omp for schedule(static)
    for (int b = 0; b < batch; ++b) {
      for (int i = 0; i < in; ++i) acc[i] = 0;
      for (int o = 0; o < out; ++o) {
        const double g = (double)dpre[(int64_t)b * out + o];
        const double *row = Wd + (int64_t)o * in;
        for (int i = 0; i < in; ++i) acc[i] += row[i] * g;
      }
      for (int i = 0; i < in; ++i) dX[(int64_t)b * in + i] = (float)acc[i];
    }
    free(acc);
  }
#pragma omp parallel for schedule(static)
  for (int o = 0; o < out; ++o) {
    float *row = dW + (int64_t)o * in;
    for (int i = 0; i < in; ++i) row[i] = 0.0f;
    for (int b = 0; b < batch; ++b) {
      const float g = dpre[(int64_t)b * out + o];
      const float *xb = x + (int64_t)b * in;
      for (int i = 0; i < in; ++i) row[i] = fmaf(g, xb[i], row[i]);
    }
  }
}

/* welvet_dense_normalbp_f32 c_abi.cpp:142-207 with the checks of
 * WeightStore::apply_sgd native_codec.cpp:909-945 and the Float32 launcher
 * training.mm:71-128.  Status codes: 0 ok, 1 invalid, 2 unsupported. */
/* op_swiglu shaders/ops_common.metal:27-38.  c[1] == 0: d = act_value(a, SiLU) * b;
 * c[1] == 1: e = d * act_value(a, SiLU), f = (d * b) * act_prime(a, SiLU) with
 * d * b held in double-float (exact in f64) and one rounding to f32. */
void or_swiglu_h(const float *gate, const float *up, int64_t n, float *h) {
  for (int64_t i = 0; i < n; ++i) {
    const float s = or_act(gate[i], 1);
    h[i] = s * up[i];
  }
}

void or_swiglu_split(const float *gate, const float *up, const float *gh, int64_t n, float *d_up,
                     float *d_gate) {
  for (int64_t i = 0; i < n; ++i) {
    const float s = or_act(gate[i], 1);
    d_up[i] = gh[i] * s;
    d_gate[i] = (float)(((double)gh[i] * (double)up[i]) * (double)or_act_prime(gate[i], 1));
  }
}

int or_normalbp(int batch, int in, int out, int act, int dtype, const float *W_init,
                const double *bias, int64_t bias_len, const float *x, const float *grad_or_target,
                int use_target, double lr, float *pre, float *post, float *dX, float *dW,
                float *W_after, double *loss) {
  if (batch <= 0 || in <= 0 || out <= 0 || !W_init || !x || !grad_or_target || !pre || !post ||
      !dX || !dW || !W_after || !loss)
    return 1;
  if (dtype < 0 || dtype >= OR_NUM_DTYPES) return 1;
  const int64_t n = (int64_t)out * in, ny = (int64_t)batch * out, nx = (int64_t)batch * in;
  const int64_t nb = or_native_bytes(dtype, n);
  uint8_t *raw = (uint8_t *)calloc((size_t)nb, 1);
  double *Wd = (double *)malloc(sizeof(double) * (size_t)n);
  float *pre_t = (float *)malloc(sizeof(float) * (size_t)ny), *post_t = (float *)malloc(sizeof(float) * (size_t)ny);
  float *gy = (float *)malloc(sizeof(float) * (size_t)ny), *dpre = (float *)malloc(sizeof(float) * (size_t)ny);
  float *dx_t = (float *)malloc(sizeof(float) * (size_t)nx), *dw_t = (float *)malloc(sizeof(float) * (size_t)n);
  float scale = 1;
  int st = or_pack(dtype, W_init, n, raw, &scale);
  if (!st) st = or_decode_f64(dtype, raw, nb, scale, n, Wd);
  if (!st) {
    const int64_t bl = (bias && bias_len > 0) ? bias_len : 0;
    or_dense_forward(batch, in, out, act, Wd, bl ? bias : NULL, bl, x, pre_t, post_t);
    *loss = 0.0;
    memcpy(gy, grad_or_target, sizeof(float) * (size_t)ny);
    if (use_target) {
      *loss = or_mse(post_t, grad_or_target, ny);
      or_mse_grad(post_t, grad_or_target, ny, gy);
    }
    or_dense_backward(batch, in, out, act, Wd, x, pre_t, gy, dpre, dx_t, dw_t);
    if (lr != 0.0) {
      if (!isfinite(lr)) st = 1;
      else if (dtype == OR_FLOAT32) {
        for (int64_t i = 0; i < n && !st; ++i)
          if (!isfinite(dw_t[i])) st = 2;
        if (!st && (fabs(lr) > FLT_MAX || fabs(lr) < FLT_MIN)) st = 2;
        if (!st) {
          float *w = (float *)malloc(sizeof(float) * (size_t)n);
          for (int64_t i = 0; i < n; ++i) w[i] = bitsf32(get_u32(raw + i * 4));
          or_sgd_f32(w, dw_t, n, lr);
          for (int64_t i = 0; i < n; ++i) put_u32(raw, i * 4, f32bits(w[i]));
          free(w);
        }
      } else {
        st = or_native_sgd(dtype, raw, nb, scale, n, dw_t, lr);
      }
    }
    if (!st) st = or_decode(dtype, raw, nb, scale, n, W_after);
    if (!st) {
      memcpy(pre, pre_t, sizeof(float) * (size_t)ny);
      memcpy(post, post_t, sizeof(float) * (size_t)ny);
      memcpy(dX, dx_t, sizeof(float) * (size_t)nx);
      memcpy(dW, dw_t, sizeof(float) * (size_t)n);
    }
  }
  free(raw); free(Wd); free(pre_t); free(post_t); free(gy); free(dpre); free(dx_t); free(dw_t);
  return st;
}

/* CPU baseline: the reference's only host hot loop is the per-element
 * decode switch (decode_row_f64 native_codec.cpp:835-870); this decodes each
 * row that way and applies the f64 dot of the Go contract.  threads > 1 splits
 * output rows across OpenMP threads. */
void or_dense_forward_native(int batch, int in, int out, int act, int dtype, const uint8_t *raw,
                             int64_t raw_n, float scale, const double *bias, int64_t bias_len,
                             const float *x, float *pre, float *post, int threads) {
  const int64_t n = (int64_t)out * in;
#ifdef _OPENMP
  if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
#endif
  {
    double *row = (double *)malloc(sizeof(double) * (size_t)in);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
    for (int o = 0; o < out; ++o) {
      for (int k = 0; k < in; ++k) {
        const int64_t i = (int64_t)o * in + k;
        if (dtype == OR_FLOAT32) row[k] = (double)bitsf32(get_u32(raw + i * 4));
        else if (dtype == OR_FLOAT64) row[k] = bitsf64(get_u64(raw + i * 8));
        else {
          float v = 0;
          weight_at(dtype, raw, raw_n, scale, i, n, &v);
          row[k] = (double)v;
        }
      }
      for (int b = 0; b < batch; ++b) {
        double acc = 0;
        const float *xb = x + (int64_t)b * in;
        for (int k = 0; k < in; ++k) acc += row[k] * (double)xb[k];
        float p = (float)acc;
        if (bias && o < bias_len) p = (float)((double)p + bias[o]);
        pre[(int64_t)b * out + o] = p;
        post[(int64_t)b * out + o] = or_act(p, act);
      }
    }
    free(row);
  }
  (void)threads;
}

/* Bulk scalar-codec decode: kind 0 f16, 1 bf16, 2 e4m3, 3 e5m2, 4 fp4, into
 * an f32 array (memory keeps signaling-NaN payloads bit for bit). */
void or_decode_many(int kind, const uint32_t *codes, int64_t n, float *out) {
  for (int64_t i = 0; i < n; ++i) {
    switch (kind) {
    case 0: out[i] = or_f16_to_f32((uint16_t)codes[i]); break;
    case 1: out[i] = or_bf16_to_f32((uint16_t)codes[i]); break;
    case 2: out[i] = or_e4m3_to_f32((uint8_t)codes[i]); break;
    case 3: out[i] = or_e5m2_to_f32((uint8_t)codes[i]); break;
    default: out[i] = or_fp4_to_f32((uint8_t)codes[i]); break;
    }
  }
}

/* Bulk scalar-codec sweep for exhaustive checks: kind 0 f16, 1 bf16, 2 e4m3,
 * 3 e5m2, 4 fp4; uint16 output for kinds 0-1, uint8 otherwise. */
void or_encode_many(int kind, const float *in, int64_t n, void *out) {
  for (int64_t i = 0; i < n; ++i) {
    switch (kind) {
    case 0: ((uint16_t *)out)[i] = or_f32_to_f16(in[i]); break;
    case 1: ((uint16_t *)out)[i] = or_f32_to_bf16(in[i]); break;
    case 2: ((uint8_t *)out)[i] = or_f32_to_e4m3(in[i]); break;
    case 3: ((uint8_t *)out)[i] = or_f32_to_e5m2(in[i]); break;
    default: ((uint8_t *)out)[i] = or_f32_to_fp4(in[i]); break;
    }
  }
}
