// ref_shim.cpp — extern "C" access to the reference's own host codec, built
// from the reference sources into oracle/_ref/libwelvet_ref.so by
// oracle/Makefile.  TEST INFRASTRUCTURE ONLY: it checks the oracle's
// restatement; nothing in the product loads it.
//
// Entry points wrap the reference's public C++ API:
//   WeightStore::make / encode_format_none  include/welvet/weights.hpp:34-39
//   WeightStore::export_f32                 src/weights/store.cpp:32-59
//   WeightStore::decode_row_f64             src/weights/native_codec.cpp:835-870
//   scalar float codecs                     include/welvet/float_codecs.hpp
#include "welvet/float_codecs.hpp"
#include "welvet/weights.hpp"

#include <cstring>

#define REF_API extern "C" __attribute__((visibility("default")))

// Encodes n floats as one row; returns the payload size (or -code on error).
REF_API long ref_pack(int dtype, const float *w, int n, unsigned char *out, long cap, float *scale) {
  welvet::WeightStore s;
  auto st = welvet::WeightStore::make(1, n, static_cast<welvet::DType>(dtype), w, &s);
  if (!st.ok()) return -static_cast<long>(st.code);
  if (static_cast<welvet::DType>(dtype) == welvet::DType::Float32) {
    const long bytes = static_cast<long>(s.f32.size() * 4);
    if (bytes > cap) return -100;
    std::memcpy(out, s.f32.data(), static_cast<size_t>(bytes));
  } else {
    if (static_cast<long>(s.native.size()) > cap) return -100;
    std::memcpy(out, s.native.data(), s.native.size());
  }
  *scale = s.scale;
  return static_cast<long>(static_cast<welvet::DType>(dtype) == welvet::DType::Float32
                               ? s.f32.size() * 4 : s.native.size());
}

static void load_store(welvet::WeightStore *s, int dtype, const unsigned char *raw, long raw_n,
                       float scale, int n) {
  s->dtype = static_cast<welvet::DType>(dtype);
  s->rows = 1;
  s->cols = n;
  s->scale = scale;
  if (s->dtype == welvet::DType::Float32) {
    s->f32.resize(static_cast<size_t>(raw_n / 4));
    std::memcpy(s->f32.data(), raw, static_cast<size_t>(raw_n / 4) * 4);
  } else {
    s->native.assign(raw, raw + raw_n);
  }
}

// export_f32 of a one-row store; returns the status code.
REF_API int ref_decode(int dtype, const unsigned char *raw, long raw_n, float scale, int n, float *out) {
  welvet::WeightStore s;
  load_store(&s, dtype, raw, raw_n, scale, n);
  return static_cast<int>(s.export_f32(out).code);
}

// decode_row_f64 of a one-row store; returns the status code.
REF_API int ref_decode_f64(int dtype, const unsigned char *raw, long raw_n, float scale, int n, double *out) {
  welvet::WeightStore s;
  load_store(&s, dtype, raw, raw_n, scale, n);
  return static_cast<int>(s.decode_row_f64(0, out).code);
}

REF_API unsigned short ref_f32_to_f16(float f) { return welvet::float32_to_float16(f); }
REF_API float ref_f16_to_f32(unsigned short h) { return welvet::float16_to_float32(h); }
REF_API unsigned short ref_f32_to_bf16(float f) { return welvet::float32_to_bfloat16(f); }
REF_API float ref_bf16_to_f32(unsigned short h) { return welvet::bfloat16_to_float32(h); }
REF_API unsigned char ref_f32_to_e4m3(float f) { return welvet::float32_to_fp8e4m3(f); }
REF_API float ref_e4m3_to_f32(unsigned char b) { return welvet::fp8e4m3_to_float32(b); }
REF_API unsigned char ref_f32_to_e5m2(float f) { return welvet::float32_to_fp8e5m2(f); }
REF_API float ref_e5m2_to_f32(unsigned char b) { return welvet::fp8e5m2_to_float32(b); }
REF_API unsigned char ref_f32_to_fp4(float f) { return welvet::float32_to_fp4(f); }
REF_API float ref_fp4_to_f32(unsigned char c) { return welvet::fp4_to_float32(c); }

// Decodes n codes into an f32 array (kind as below).  Writing the result to
// memory keeps every bit, including signaling-NaN payloads, which a scalar
// float return converted to a double by a caller would quiet.
REF_API void ref_decode_many(int kind, const unsigned int *codes, long n, float *out) {
  for (long i = 0; i < n; ++i) {
    const unsigned int c = codes[i];
    switch (kind) {
    case 0: out[i] = welvet::float16_to_float32(static_cast<unsigned short>(c)); break;
    case 1: out[i] = welvet::bfloat16_to_float32(static_cast<unsigned short>(c)); break;
    case 2: out[i] = welvet::fp8e4m3_to_float32(static_cast<unsigned char>(c)); break;
    case 3: out[i] = welvet::fp8e5m2_to_float32(static_cast<unsigned char>(c)); break;
    default: out[i] = welvet::fp4_to_float32(static_cast<unsigned char>(c)); break;
    }
  }
}

// Bulk scalar-codec sweep for exhaustive checks: kind 0 f16, 1 bf16, 2 e4m3,
// 3 e5m2, 4 fp4; encodes n floats into out (uint16 for kinds 0-1, else uint8).
REF_API void ref_encode_many(int kind, const float *in, long n, void *out) {
  for (long i = 0; i < n; ++i) {
    switch (kind) {
    case 0: static_cast<unsigned short *>(out)[i] = welvet::float32_to_float16(in[i]); break;
    case 1: static_cast<unsigned short *>(out)[i] = welvet::float32_to_bfloat16(in[i]); break;
    case 2: static_cast<unsigned char *>(out)[i] = welvet::float32_to_fp8e4m3(in[i]); break;
    case 3: static_cast<unsigned char *>(out)[i] = welvet::float32_to_fp8e5m2(in[i]); break;
    default: static_cast<unsigned char *>(out)[i] = welvet::float32_to_fp4(in[i]); break;
    }
  }
}
