// codec.hpp — per-dtype element codes: pack (fresh scale), decode, and the
// fixed-scale re-encode used by SGD.  All three are bit-exact restatements of
// the reference's scalar code; the kernels in codec.hip only arrange threads.
#pragma once

#include "common.hpp"

namespace wh {

// Quantisation parameters of one tensor, computed on the device by the
// statistics pass (native_codec.cpp:22-40, :148-560):
//   s      the divisor pack uses (absmax, absmax/max_q, or the unsigned span)
//   scale  the scale the store keeps (weights.hpp:25)
//   minv   the unsigned min header (native_codec.cpp:183)
struct Meta {
  float s;
  float scale;
  float minv;
  float pad;
};

// ---------------------------------------------------------------- decode
// weight_at native_codec.cpp:562-813 for one code of element width
// dtype_bits(DT).  `lo` holds the code (the low 64 bits for Complex128).
template <int DT>
__device__ inline float dec_code(uint64_t lo, float scale, float minv) {
  if (scale == 0.0f) scale = 1.0f;
  if constexpr (DT == kFloat32 || DT == kComplex64) return u2f((uint32_t)lo);
  else if constexpr (DT == kFloat64 || DT == kComplex128) return (float)u2d(lo);
  else if constexpr (DT == kFloat16) return dec_f16((uint32_t)lo);
  else if constexpr (DT == kBFloat16) return dec_bf16((uint32_t)lo);
  else if constexpr (DT == kFP8E4M3) return dec_e4m3((uint32_t)lo);
  else if constexpr (DT == kFP8E5M2) return dec_e5m2((uint32_t)lo);
  else if constexpr (DT == kFP4) return kFp4Tab[lo & 15];
  else if constexpr (DT == kNF4) return kNf4Tab[lo & 15] * scale;
  else if constexpr (DT == kInt64 || DT == kInt) return (float)(int64_t)lo * scale;
  else if constexpr (DT == kInt32) return (float)(int32_t)(uint32_t)lo * scale;
  else if constexpr (DT == kInt16) return (float)(int16_t)(uint16_t)lo * scale;
  else if constexpr (DT == kInt8) return (float)(int8_t)(uint8_t)lo * scale;
  else if constexpr (DT == kUint64 || DT == kUint || DT == kUintptr) return (float)lo * scale + minv;
  else if constexpr (DT == kUint32 || DT == kUint16 || DT == kUint8 || DT == kUint4 ||
                     DT == kUint2 || DT == kUint6 || DT == kUint5 || DT == kUint3)
    return (float)(uint32_t)lo * scale + minv;
  else if constexpr (DT == kInt4) return (float)((int)(lo & 15) - ((lo & 8) ? 16 : 0)) * scale;
  else if constexpr (DT == kInt2) return (float)((int)(lo & 3) - 2) * scale;
  else if constexpr (DT == kTernary) {
    const int c = (int)(lo & 3);
    return c == 0 ? -scale : (c == 2 ? scale : 0.0f);
  } else if constexpr (DT == kBinary) return (lo & 1) ? scale : -scale;
  else {  // Int6 / FP6 / Int5 / Int3: two's complement of `bits` bits
    constexpr int bits = dtype_bits(DT);
    const int q = (int)(lo & ((1u << bits) - 1));
    return (float)(q >= (1 << (bits - 1)) ? q - (1 << bits) : q) * scale;
  }
}

// ------------------------------------------------------------------ pack
// pack_native native_codec.cpp:189-560: the code of element value w under
// the tensor's fresh statistics.  Returns the low 64 bits of the code; the
// high half of Complex128 is always 0.
template <int DT>
__device__ inline uint64_t pack_code(float w, const Meta &m) {
  const float s = m.s;
  if constexpr (DT == kFloat32) return f2u(w);
  else if constexpr (DT == kFloat64 || DT == kComplex128) return d2u((double)w);
  else if constexpr (DT == kComplex64) return (uint64_t)f2u(w);
  else if constexpr (DT == kFloat16) return enc_f16(w);
  else if constexpr (DT == kBFloat16) return enc_bf16(w);
  else if constexpr (DT == kFP8E4M3) return enc_e4m3(w);
  else if constexpr (DT == kFP8E5M2) return enc_e5m2(w);
  else if constexpr (DT == kFP4) return nearest16(kFp4Tab, w);
  else if constexpr (DT == kNF4) return nearest16(kNf4Tab, w / s);
  else if constexpr (DT == kInt64 || DT == kInt) {  // :234-247
    const float qf = w / s * 1e6f;
    return (uint64_t)sat_i64(round((double)qf));
  } else if constexpr (DT == kInt32) {  // :248-262; +absmax saturates
    const float qf = w / s * 2147483647.0f;
    return (uint64_t)(uint32_t)sat_i32(round((double)qf));
  } else if constexpr (DT == kInt16) {  // :263-276
    const float qf = w / s * 32767.0f;
    return (uint16_t)(int16_t)sat_i32(clampd(round((double)qf), -32768.0, 32767.0));
  } else if constexpr (DT == kInt8) {  // :277-288
    return (uint8_t)(int8_t)sat_i32(clampd((double)roundf(w / s), -128.0, 127.0));
  } else if constexpr (DT == kUint8) {  // :298-306
    const float qf = (w - m.minv) / s * 255.0f;
    return sat_u32(clampd(round((double)qf), 0.0, 255.0));
  } else if constexpr (DT == kUint16) {
    const float qf = (w - m.minv) / s * 65535.0f;
    return sat_u32(clampd(round((double)qf), 0.0, 65535.0));
  } else if constexpr (DT == kUint32) {  // float(4294967295u) == 2^32
    const float qf = (w - m.minv) / s * 4294967296.0f;
    return sat_u32(clampd(round((double)qf), 0.0, 4294967295.0));
  } else if constexpr (DT == kUint64 || DT == kUint || DT == kUintptr) {
    const float qf = (w - m.minv) / s * 1e15f;
    return sat_u64(clampd(round((double)qf), 0.0, 1e15));
  } else if constexpr (DT == kInt4) {  // :342-356
    return (uint32_t)sat_i32(clampd((double)roundf(w / s), -8.0, 7.0)) & 15u;
  } else if constexpr (DT == kUint4) {  // :357-375
    const float qf = (w - m.minv) / s * 15.0f;
    return (uint32_t)sat_i32(clampd(round((double)qf), 0.0, 15.0)) & 15u;
  } else if constexpr (DT == kInt2) {  // :376-388
    const int q = sat_i32(clampd((double)roundf(w / s), -2.0, 1.0));
    return (uint32_t)(q + 2) & 3u;
  } else if constexpr (DT == kUint2) {  // :389-403 (double 3.0)
    return (uint32_t)sat_i32(clampd(round((double)((w - m.minv) / s) * 3.0), 0.0, 3.0)) & 3u;
  } else if constexpr (DT == kTernary) {  // :404-420
    const float r = w / s;
    return r > 0.5f ? 2u : (r < -0.5f ? 0u : 1u);
  } else if constexpr (DT == kBinary) {  // :421-432
    return w >= 0 ? 1u : 0u;
  } else if constexpr (DT == kInt6 || DT == kFP6 || DT == kInt5 || DT == kInt3) {  // :148-166
    constexpr int bits = dtype_bits(DT);
    constexpr int max_q = (1 << (bits - 1)) - 1, min_q = -(1 << (bits - 1));
    int q = sat_i32(roundf(w / s));
    q = q > max_q ? max_q : (q < min_q ? min_q : q);
    return (uint32_t)q & ((1u << bits) - 1);
  } else {  // Uint6 / Uint5 / Uint3 :168-187
    constexpr int bits = dtype_bits(DT);
    constexpr int max_q = (1 << bits) - 1;
    return (uint32_t)sat_i32(clampd((double)roundf((w - m.minv) / s * (float)max_q), 0.0, (double)max_q));
  }
}

// ----------------------------------------------------------------- repack
// op_native_repack ops_storage.metal:971-1144 (WeightStore::set_from_f32_gpu):
// the code of w under fresh statistics.  Its cam_div / cam_mul are the
// correctly rounded f32 '/' and '*', so every dtype's code is pack_code's
// except Uint2, whose product with 3 is an f32 multiply there
// (round(fl32(fl32((w - min) / span) * 3.0f))) where pack rounds a double
// product.  The statistics differ in their NaN rule (repack_finalize_kernel).
template <int DT>
__device__ inline uint64_t repack_code(float w, const Meta &m) {
  if constexpr (DT == kUint2) {
    const float qf = roundf((w - m.minv) / m.s * 3.0f);
    return (uint32_t)sat_i32(clampf_(qf, 0.0f, 3.0f)) & 3u;
  } else {
    return pack_code<DT>(w, m);
  }
}

// -------------------------------------------------------------- re-encode
// set_weight_at ops_storage.metal:655-921: the code of v under the stored
// scale and min.  The clamp bounds are float there, so the Int32 and Uint32
// upper bounds become 2^31 and 2^32 and the conversion saturates.
template <int DT>
__device__ inline uint64_t fix_code(float v, float scale, float minv) {
  if (scale == 0.0f) scale = 1.0f;
  if constexpr (DT == kFloat32) return f2u(v);
  else if constexpr (DT == kFloat64 || DT == kComplex128) return d2u((double)v);
  else if constexpr (DT == kComplex64) return (uint64_t)f2u(v);
  else if constexpr (DT == kFloat16) return enc_f16(v);
  else if constexpr (DT == kBFloat16) return enc_bf16(v);
  else if constexpr (DT == kFP8E4M3) return enc_e4m3(v);
  else if constexpr (DT == kFP8E5M2) return enc_e5m2(v);
  else if constexpr (DT == kFP4) return nearest16(kFp4Tab, v);
  else if constexpr (DT == kNF4) return nearest16(kNf4Tab, v / scale);
  else if constexpr (DT == kInt64 || DT == kInt) return (uint64_t)sat_i64((double)roundf(v / scale));
  else if constexpr (DT == kInt32)
    return (uint32_t)sat_i32(clampf_(roundf(v / scale), -2147483648.0f, 2147483648.0f));
  else if constexpr (DT == kInt16)
    return (uint16_t)(int16_t)sat_i32(clampf_(roundf(v / scale), -32768.0f, 32767.0f));
  else if constexpr (DT == kInt8)
    return (uint8_t)(int8_t)sat_i32(clampf_(roundf(v / scale), -128.0f, 127.0f));
  else if constexpr (DT == kUint8) return sat_u32(clampf_(roundf((v - minv) / scale), 0.0f, 255.0f));
  else if constexpr (DT == kUint16) return sat_u32(clampf_(roundf((v - minv) / scale), 0.0f, 65535.0f));
  else if constexpr (DT == kUint32)
    return sat_u32(clampf_(roundf((v - minv) / scale), 0.0f, 4294967296.0f));
  else if constexpr (DT == kUint64 || DT == kUint || DT == kUintptr) {  // quant_u64 :106-113
    const float q = roundf((v - minv) / scale);
    if (q <= 0) return 0;
    if (q >= 1e15f) return 1000000000000000ull;
    return sat_u64(q);
  } else if constexpr (DT == kInt4)
    return (uint32_t)sat_i32(clampf_(roundf(v / scale), -8.0f, 7.0f)) & 15u;
  else if constexpr (DT == kUint4)
    return (uint32_t)sat_i32(clampf_(roundf((v - minv) / scale), 0.0f, 15.0f)) & 15u;
  else if constexpr (DT == kInt2) {
    const int q = sat_i32(clampf_(roundf(v / scale), -2.0f, 1.0f));
    return (uint32_t)(q + 2) & 3u;
  } else if constexpr (DT == kUint2)
    return (uint32_t)sat_i32(clampf_(roundf((v - minv) / scale), 0.0f, 3.0f)) & 3u;
  else if constexpr (DT == kTernary) {
    const float r = v / scale;
    return r > 0.5f ? 2u : (r < -0.5f ? 0u : 1u);
  } else if constexpr (DT == kBinary) return v >= 0 ? 1u : 0u;
  else if constexpr (DT == kInt6 || DT == kFP6 || DT == kInt5 || DT == kInt3) {  // :636-646
    constexpr int bits = dtype_bits(DT);
    constexpr int max_q = (1 << (bits - 1)) - 1, min_q = -(1 << (bits - 1));
    int q = sat_i32(roundf(v / scale));
    q = q > max_q ? max_q : (q < min_q ? min_q : q);
    return (uint32_t)q & ((1u << bits) - 1);
  } else {  // Uint6 / Uint5 / Uint3 :647-654
    constexpr int bits = dtype_bits(DT);
    return (uint32_t)sat_i32(clampf_(roundf((v - minv) / scale), 0.0f, (float)((1 << bits) - 1)));
  }
}

// Bytes of the element written by set_weight_at: the complex formats only
// overwrite their real part (ops_storage.metal:851-862).
template <int DT>
__host__ __device__ constexpr int fix_bytes() {
  return DT == kComplex64 ? 4 : (DT == kComplex128 ? 8 : dtype_bits(DT) / 8);
}

// Elements per thread unit for the pack / re-encode kernels: one element for
// byte-sized formats, one byte for 1/2/4-bit, eight elements (= `bits` bytes)
// for 3/5/6-bit, so no two threads touch the same byte.
template <int DT>
__host__ __device__ constexpr int unit_elems() {
  constexpr int b = dtype_bits(DT);
  return b >= 8 ? 1 : (b == 1 || b == 2 || b == 4 ? 8 / b : 8);
}

// Decode-ready copy of an FP8 code: the byte the hardware converters
// (v_cvt_*_fp8 / _bf8, OCP formats) decode to exactly the reference's value.
// E4M3 (float_codecs.cpp:99-117): a zero exponent field decodes to signed
// zero, 0x7f / 0xff decode to +-448 (= 0x7e / 0xfe; OCP reads 0x7f as NaN).
// E5M2 (:160-181): a zero exponent field decodes to signed zero; Inf and NaN
// codes already agree.  Stores keep the reference bytes (export, SGD); kernels
// that decode FP8 through the converters read this copy.
template <int DT>
__host__ __device__ constexpr bool has_kcopy() {
  return DT == kFP8E4M3 || DT == kFP8E5M2;
}
template <int DT>
__host__ __device__ inline uint8_t kcode(uint32_t c) {
  if constexpr (DT == kFP8E4M3) {
    if ((c & 0x78u) == 0) return (uint8_t)(c & 0x80u);
    return (uint8_t)((c & 0x7fu) == 0x7fu ? c ^ 1u : c);
  } else {
    return (uint8_t)((c & 0x7cu) == 0 ? (c & 0x80u) : c);
  }
}

// Reads the code of element i of a packed body.
template <int DT>
__device__ inline uint64_t load_code(const uint8_t *body, int64_t i) {
  constexpr int bits = dtype_bits(DT);
  if constexpr (bits == 128 || bits == 64) {
    const uint8_t *p = body + i * (bits / 8);
    return (uint64_t)(*(const uint32_t *)p) | ((uint64_t)(*(const uint32_t *)(p + 4)) << 32);
  } else if constexpr (bits == 32) return *(const uint32_t *)(body + i * 4);
  else if constexpr (bits == 16) return *(const uint16_t *)(body + i * 2);
  else if constexpr (bits == 8) return body[i];
  else {
    const int64_t bit = i * bits;
    const int64_t byte = bit >> 3;
    uint32_t v = body[byte];
    if ((bit & 7) + bits > 8) v |= (uint32_t)body[byte + 1] << 8;
    return (v >> (bit & 7)) & ((1u << bits) - 1);
  }
}

}  // namespace wh
