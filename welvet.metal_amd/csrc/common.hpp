// common.hpp — dtype table, status codes and the device-side codec for the
// 34 FormatNone storage types.
//
// Storage layout in HBM (one weight matrix, rows = out, cols = in):
//   body   the reference's native payload with the 4-byte min header of the
//          unsigned types split off (header kept as `minv`), 256-byte aligned
//          by hipMalloc and padded so 16-byte chunk loads past the last row
//          stay inside the allocation.  Element i (= row*cols + col) sits at
//          bit i*bits, LSB first, exactly as native_codec.cpp:112-136 packs it.
//   scale  per-tensor f32 scale (weights.hpp:25); minv the unsigned header.
//
// Every arithmetic step of encode/decode is written out literally and the
// whole library is compiled with -ffp-contract=off: `q*s + min` must round
// twice (native_codec.cpp:634), never fuse.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wh {

// include/welvet/dtype.hpp:9-44
enum DType : int32_t {
  kFloat64 = 0, kFloat32 = 1, kFloat16 = 2, kBFloat16 = 3, kFP8E4M3 = 4, kFP8E5M2 = 5,
  kInt64 = 6, kInt32 = 7, kInt16 = 8, kInt8 = 9, kUint64 = 10, kUint32 = 11, kUint16 = 12,
  kUint8 = 13, kInt4 = 14, kUint4 = 15, kFP4 = 16, kInt2 = 17, kUint2 = 18, kTernary = 19,
  kBinary = 20, kInt = 21, kUint = 22, kUintptr = 23, kComplex64 = 24, kComplex128 = 25,
  kNF4 = 26, kFP6 = 27, kInt6 = 28, kUint6 = 29, kInt5 = 30, kUint5 = 31, kInt3 = 32,
  kUint3 = 33, kNumDTypes = 34
};

// include/welvet/status.hpp:8-14
enum Code : int32_t { kOk = 0, kInvalid = 1, kUnsupported = 2, kGap = 3, kInternal = 4 };

// include/welvet/activate.hpp:8-17
enum Act : int32_t { kLinear = -1, kReLU = 0, kSilu = 1, kGELU = 2, kTanh = 3, kSigmoid = 4,
                     kLeakyReLU = 5, kReLU2 = 6 };
// Epilogue of SwiGLU's Up projection (this library's, not a reference
// activation): post already holds the Gate projection g at each output, and
// the epilogue writes pre = u and post = fl32(silu(g)) * u there: op_swiglu's
// h (ops_common.metal:27-38) without a launch of its own.
constexpr int32_t kSwiGated = 100;

// Bits per element in the body (native_codec.cpp:189-560; LP64 host: Int,
// Uint and Uintptr are 64-bit).
__host__ __device__ constexpr int dtype_bits(int dt) {
  switch (dt) {
  case kFloat64: case kInt64: case kInt: case kComplex64: case kUint64: case kUint:
  case kUintptr: return 64;
  case kComplex128: return 128;
  case kFloat32: case kInt32: case kUint32: return 32;
  case kFloat16: case kBFloat16: case kInt16: case kUint16: return 16;
  case kFP8E4M3: case kFP8E5M2: case kInt8: case kUint8: return 8;
  case kInt4: case kUint4: case kFP4: case kNF4: return 4;
  case kInt2: case kUint2: case kTernary: return 2;
  case kBinary: return 1;
  case kFP6: case kInt6: case kUint6: return 6;
  case kInt5: case kUint5: return 5;
  case kInt3: case kUint3: return 3;
  }
  return 0;
}

// Unsigned formats carry the 4-byte f32 min header (native_codec.cpp:183, :300).
__host__ __device__ constexpr bool dtype_has_min(int dt) {
  return dt == kUint64 || dt == kUint32 || dt == kUint16 || dt == kUint8 || dt == kUint4 ||
         dt == kUint2 || dt == kUint || dt == kUintptr || dt == kUint6 || dt == kUint5 ||
         dt == kUint3;
}

// Formats decoded through a 2^bits-entry table of exact decoded values.
__host__ __device__ constexpr bool dtype_lut(int dt) { return dtype_bits(dt) <= 8; }

// Byte size of the reference payload including the header (native_codec.cpp:189-560).
__host__ __device__ inline int64_t native_bytes(int dt, int64_t n) {
  const int bits = dtype_bits(dt);
  return (n * bits + 7) / 8 + (dtype_has_min(dt) ? 4 : 0);
}

// ----------------------------------------------------------- bit utilities
__host__ __device__ inline uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ inline float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
__host__ __device__ inline uint64_t d2u(double d) { return __builtin_bit_cast(uint64_t, d); }
__host__ __device__ inline double u2d(uint64_t u) { return __builtin_bit_cast(double, u); }

// Float -> integer conversions of the reference platform (arm64 fcvtzs /
// fcvtzu): truncate, saturate, NaN -> 0.  Written out so the compiler cannot
// treat out-of-range conversions as undefined.
__device__ inline int32_t sat_i32(double v) {
  if (v != v) return 0;
  if (v >= 2147483648.0) return INT32_MAX;
  if (v <= -2147483649.0) return INT32_MIN;
  return (int32_t)v;
}
__device__ inline int64_t sat_i64(double v) {
  if (v != v) return 0;
  if (v >= 9223372036854775808.0) return INT64_MAX;
  if (v < -9223372036854775808.0) return INT64_MIN;
  return (int64_t)v;
}
__device__ inline uint32_t sat_u32(double v) {
  if (v != v || v <= -1.0) return 0;
  if (v >= 4294967296.0) return UINT32_MAX;
  return (uint32_t)v;
}
__device__ inline uint64_t sat_u64(double v) {
  if (v != v || v <= -1.0) return 0;
  if (v >= 18446744073709551616.0) return UINT64_MAX;
  return (uint64_t)v;
}
__device__ inline double clampd(double v, double lo, double hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}
__device__ inline float clampf_(float v, float lo, float hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// ----------------------------------------------------- scalar float codecs
// src/core/float_codecs.cpp:23-35 — truncating f16 encode
__device__ inline uint16_t enc_f16(float f) {
  const uint32_t b = f2u(f);
  const uint16_t sign = (uint16_t)((b >> 16) & 0x8000);
  const int expo = (int)((b >> 23) & 0xff) - 112;
  if (expo <= 0) return sign;
  if (expo >= 31) return (uint16_t)(sign | 0x7c00);
  return (uint16_t)(sign | (expo << 10) | ((b & 0x7fffff) >> 13));
}
// float_codecs.cpp:37-51 — IEEE half decode with the payload kept for NaN
__device__ inline float dec_f16(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16, expo = (h >> 10) & 0x1f, mant = h & 0x3ff;
  if (expo == 0) return u2f(sign | f2u((float)mant * 5.9604644775390625e-8f));  // mant * 2^-24
  if (expo == 31) return u2f(sign | 0x7f800000u | (mant << 13));
  return u2f(sign | ((expo + 112) << 23) | (mant << 13));
}
// float_codecs.cpp:53-55
__device__ inline uint16_t enc_bf16(float f) { return (uint16_t)(f2u(f) >> 16); }
__device__ inline float dec_bf16(uint32_t h) { return u2f(h << 16); }

// float_codecs.cpp:57-97 — guard-bit round-up (ties away), every |f| >= 248
// saturates to 0x7e, subnormal range truncates, 0 and NaN -> +0.  Written
// without branches (the SGD re-encode runs it per element): exponent and
// mantissa form one field e << 3 | m, so adding the guard bit carries a full
// mantissa into the exponent as the reference's m == 8 step does, and one
// compare against 15 << 3 covers both of its saturation tests; the subnormal
// range (biased exponent 118..120) keeps its truncating shift.  Identical to
// the reference's branches on all 2^32 inputs (checked exhaustively on the
// host against a transcription of them).
__device__ inline uint8_t enc_e4m3(float f) {
  const uint32_t u = f2u(f), b = u & 0x7fffffffu;
  const int e = (int)(b >> 23) - 120;
  const uint32_t mant = b & 0x7fffffu;
  const uint32_t nf = (uint32_t)((e << 3) | (int)((mant >> 20) & 7u)) + ((mant >> 19) & 1u);
  const uint32_t nrm = nf >= 120u ? 0x7eu : nf;
  const int sh = min(max(21 - e, 0), 31);
  const uint32_t sub = e < -2 ? 0u : ((mant | 0x800000u) >> sh) & 7u;
  uint32_t code = e <= 0 ? sub : nrm;
  code = u2f(b) > 448.0f ? 0x7eu : code;
  code |= (u >> 24) & 0x80u;
  return (f == 0.0f || f != f) ? (uint8_t)0 : (uint8_t)code;
}
// float_codecs.cpp:99-117 — subnormal codes -> signed zero, 0x7f -> 448
__device__ inline float dec_e4m3(uint32_t b) {
  const uint32_t sign = (b & 0x80u) << 24, e = (b >> 3) & 0xf, m = b & 7;
  if (e == 0) return u2f(sign);
  if (e == 15 && m == 7) return u2f(sign | 0x43e00000u);
  return u2f(sign | ((e + 120) << 23) | (m << 20));
}
// float_codecs.cpp:119-158
__device__ inline uint8_t enc_e5m2(float f) {
  if (f != f) return 0x7e;
  uint32_t b = f2u(f);
  const uint8_t sign = (uint8_t)((b >> 24) & 0x80);
  b &= 0x7fffffffu;
  if (b == 0x7f800000u) return sign | 0x7c;
  if (b == 0) return sign;
  int e = (int)(b >> 23) - 112;
  const uint32_t mant = b & 0x7fffff;
  if (e <= 0) return sign;
  if (e >= 31) return sign | 0x7c;
  uint32_t m = (mant >> 21) & 3;
  if (mant & 0x100000) {
    if (++m == 4) {
      m = 0;
      if (++e >= 31) return sign | 0x7c;
    }
  }
  return (uint8_t)(sign | (e << 2) | m);
}
// float_codecs.cpp:160-181
__device__ inline float dec_e5m2(uint32_t b) {
  const uint32_t sign = (b & 0x80u) << 24, e = (b >> 2) & 0x1f, m = b & 3;
  if (e == 0) return u2f(sign);
  if (e == 31) return u2f(sign | (m ? 0x7fc00000u : 0x7f800000u));
  return u2f(sign | ((e + 112) << 23) | (m << 21));
}

// float_codecs.cpp:184 and native_codec.cpp:93-110 as bit patterns
#define WH_FP4_VALUES 0.f, .5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f, -0.f, -.5f, -1.f, -1.5f, -2.f, -3.f, -4.f, -6.f
#define WH_NF4_VALUES                                                                            \
  -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f, -0.28444138169288635f, \
      -0.18477343022823334f, -0.09105003625154495f, 0.0f, 0.07958029955625534f, 0.16093020141124725f, \
      0.24611230194568634f, 0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f,       \
      0.7229568362236023f, 1.0f
__device__ __constant__ const float kFp4Tab[16] = {WH_FP4_VALUES};
__device__ __constant__ const float kNf4Tab[16] = {WH_NF4_VALUES};

// Nearest table entry, first index wins ties, NaN/Inf -> 0
// (float_codecs.cpp:187-198, native_codec.cpp:525-534).
__host__ __device__ inline uint32_t nearest16(const float *tab, float r) {
  uint32_t best = 0;
  float best_err = 3.402823466e38f;
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    const float e = fabsf(r - tab[c]);
    if (e < best_err) { best_err = e; best = (uint32_t)c; }
  }
  return best;
}

// nearest16 for FP4 and NF4 through a window of four candidates.  The NF4
// values are sorted; FP4 is searched on |r| over its eight magnitudes (code k
// for r >= 0, k + 8 for r < 0 and k > 0: the +0 code 0 ties the -0 code 8 at
// every r and wins on its index; a code of the other sign is never nearer).
// A bucket of r (1/16 wide over [-2, 2] for NF4, 1/4 over [0, 8] for the FP4
// magnitude) gives the window's first index: one before the last entry at or
// below the bucket's start, so a bucket misjudged by one rounding still holds
// the answer.  Within |r| <= 2 (NF4) or 64 (FP4) the f32 errors of entries
// outside the window are strictly larger (entries >= 0.079 apart, far above
// an ulp of the error), so the window's first-index minimum is nearest16's;
// elsewhere, and for NaN, the full search runs.  Checked against nearest16 on
// every f32 of both ranges (tests/native/nearest_check.cpp).
struct TabSearch {
  float val[16];      // nearest16's table (code order)
  float win[13][4];   // sorted values (NF4) / magnitudes (FP4) k0 .. k0 + 3
  uint8_t first[64];  // bucket -> k0
};
template <bool NF4>
__host__ __device__ constexpr TabSearch make_tab_search() {
  TabSearch t{};
  const float fp4[16] = {WH_FP4_VALUES}, nf4[16] = {WH_NF4_VALUES};
  float sorted[16] = {};
  const int n = NF4 ? 16 : 8, nb = NF4 ? 64 : 32, last = n - 4;
  for (int i = 0; i < 16; ++i) t.val[i] = NF4 ? nf4[i] : fp4[i];
  for (int i = 0; i < n; ++i) sorted[i] = NF4 ? nf4[i] : fp4[i];  // FP4 codes 0-7: the magnitudes
  for (int k = 0; k <= last; ++k)
    for (int j = 0; j < 4; ++j) t.win[k][j] = sorted[k + j];
  for (int b = 0; b < nb; ++b) {
    const float start = NF4 ? (float)b / 16.0f - 2.0f : (float)b / 4.0f;
    int lo = 0;
    for (int k = 0; k < n; ++k)
      if (sorted[k] <= start) lo = k;
    const int k0 = lo - 1 < 0 ? 0 : (lo - 1 > last ? last : lo - 1);
    t.first[b] = (uint8_t)k0;
  }
  return t;
}
__device__ __constant__ const TabSearch kFp4Search = make_tab_search<false>();
__device__ __constant__ const TabSearch kNf4Search = make_tab_search<true>();
// t: make_tab_search<NF4>() (a copy in LDS on the device)
template <bool NF4>
__host__ __device__ inline uint32_t nearest_window(const TabSearch &t, float r) {
  const float m = NF4 ? r : fabsf(r);
  if (!(fabsf(r) <= (NF4 ? 2.0f : 64.0f))) return nearest16(t.val, r);
  int b = NF4 ? (int)((r + 2.0f) * 16.0f) : (int)(m * 4.0f);
  const int nb = NF4 ? 64 : 32;
  b = b < 0 ? 0 : (b >= nb ? nb - 1 : b);
  const int k0 = t.first[b];
  const float *w = t.win[k0];
  uint32_t best = (uint32_t)k0;
  float be = fabsf(m - w[0]);
#pragma unroll
  for (int j = 1; j < 4; ++j) {
    const float e = fabsf(m - w[j]);
    if (e < be) { be = e; best = (uint32_t)(k0 + j); }
  }
  if (!NF4 && best > 0 && r < 0.0f) best += 8;
  return best;
}

// --------------------------------------------------- activations (f64 math)
// shaders/ops_common.metal:83-138 evaluated in f64 (the Go contract the
// soft-double code approximates); constants 0.044715 and sqrt(2/pi).
__device__ inline double sigmoid64(double x) { return 1.0 / (1.0 + exp(-x)); }
__device__ inline double tanh64(double x) { return x > 18 ? 1.0 : (x < -18 ? -1.0 : tanh(x)); }

// The activations that need exp/tanh, out of line: inlined into a
// grid-stride kernel their f64 constants would be hoisted into registers for
// the kernel's whole life.
static __device__ __attribute__((noinline)) float act_value_f64(float v, int act) {
  const double x = (double)v;
  switch (act) {
  case kSilu: return (float)(x * sigmoid64(x));
  case kTanh: return (float)tanh64(x);
  case kSigmoid: return (float)sigmoid64(x);
  case kGELU: {
    const double cubic = ((x * x) * x) * 0.044715;
    const double u = (x + cubic) * 0.7978845608028654;
    return (float)((x * 0.5) * (1.0 + tanh64(u)));
  }
  }
  return v;
}

__device__ inline float act_value(float v, int act) {
  switch (act) {
  case kSilu: case kTanh: case kSigmoid: case kGELU: return act_value_f64(v, act);
  case kReLU: return v > 0.0f ? v : 0.0f;
  case kReLU2: return v < 0 ? 0.0f : v * v;
  case kLeakyReLU: return v < 0 ? (float)((double)v * 0.01) : v;
  }
  return v;
}

// act_prime of the piecewise activations (ReLU, ReLU2, LeakyReLU; 1 for
// every other id): act_prime below returns these for those ids, so a kernel
// that applies one of them in its epilogue gives act_deriv_kernel's bits.
__host__ __device__ inline bool act_piecewise(int act) { return act == kReLU || act == kReLU2 || act == kLeakyReLU; }
__device__ inline float act_prime_piecewise(float v, int act) {
  switch (act) {
  case kReLU: return v > 0 ? 1.0f : 0.0f;
  case kReLU2: return v > 0 ? 2 * v : 0.0f;
  case kLeakyReLU: return v > 0 ? 1.0f : 0.01f;
  }
  return 1.0f;
}

__device__ inline float act_prime(float v, int act) {
  const double x = (double)v;
  switch (act) {
  case kSilu: {
    const double z = sigmoid64(x);
    return (float)(z * (1.0 + x * (1.0 - z)));
  }
  case kGELU: {
    const double xx = x * x;
    const double u = 0.7978845608028654 * (x + 0.044715 * (xx * x));
    const double t = tanh64(u);
    const double du = 0.7978845608028654 * (1.0 + (0.044715 * xx) * 3.0);
    return (float)((1.0 + t) * 0.5 + ((x * 0.5) * (1.0 - t * t)) * du);
  }
  case kTanh: {
    const double t = tanh64(x);
    return (float)(1.0 - t * t);
  }
  case kSigmoid: {
    const double z = sigmoid64(x);
    return (float)(z * (1.0 - z));
  }
  }
  return act_prime_piecewise(v, act);
}

// Forward epilogue (welvet_dense.metal:87-105): pre = fl32(sum); with a bias
// pre = fl32(f64(pre) + bias) (two roundings); post = act(pre).
__device__ inline void bias_act_store(double sum, int o, const double *bias, int bias_len, int act,
                                      float *pre, float *post, int64_t idx) {
  float p = (float)sum;
  if (bias != nullptr && o < bias_len) p = (float)((double)p + bias[o]);
  pre[idx] = p;
  post[idx] = act == kSwiGated ? act_value(post[idx], kSilu) * p : act_value(p, act);
}

}  // namespace wh
