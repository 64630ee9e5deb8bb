// dense.hip — Dense forward / backward over packed native weights.
//
// Replaces the reference's float2 soft-double mirror kernels
// (welvet_dense.metal:54-178): weights stay packed in HBM and are decoded in
// registers (through LDS tables for formats of <= 8 bits) inside the product.
//
//   forward, batch 1      gemv_pf_kernel / gemv_loop_kernel: lanes stream
//                         16-byte chunks of a row (C per lane, all loads
//                         issued before any decode), R rows per block, x in
//                         registers; the loop form walks the row groups with a
//                         fixed grid.  Bias + activation fused in the store.
//   forward, batch 2-8    gemv_loopb_kernel where the batch's x fits in
//                         registers; gemv_kernel for other batch <= 4 shapes.
//   forward, batch > 4    split-x bf16 MFMA GEMM (x = three exact bf16 parts)
//                         for FP8 / Int8 / FP4 / NF4: gemm_bf3r_kernel without
//                         a k split, else gemm_bf3{,s,k}_kernel + sk_reduce;
//                         fp32 MFMA gemm_regr / gemm_regx (batch <= 16, no k
//                         split), gemm_reg / gemm_sk (+ sk_reduce) for the
//                         other formats.
//   dX, batch <= 2        dx_small_kernel: lanes own column chunks and walk a
//                         segment of rows (coalesced), ordered reduction.
//   dX, batch > 2         gemm_regt_kernel (batch <= 16), the split-x GEMM over
//                         the store's transposed copy, or gemm_sk through the
//                         transposed tile loader; the next layer's activation
//                         derivative fused in the store where it is piecewise.
//   dW                    dw_mfma_kernel / dw_batch_kernel: fp32 MFMA over the
//                         batch with the reference's per-element rounding
//                         (welvet_dense.metal:155-178).
//   unaligned rows        gemv_generic_kernel / dx_generic_kernel.
//
// Accumulation is fp32 inside a lane/tile and f64 across split-K / segment
// partials; outputs are fl32 of that, within the stated tolerance of the f64
// contract.  Float64 storage accumulates in f64 on the GEMV path.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "codec.hpp"
#include "kernels.hpp"

namespace wh {
namespace {

// Kernel formats: dtypes sharing a body layout and decode share a kernel.
// FL* decode through an LDS table of 2^bits exact values; FL4P is the 4-bit
// layout read through a 256-entry table of value pairs (one read per byte);
// FE4 / FE5 decode FP8 E4M3 / E5M2 with the hardware converts, reading the
// store's decode-ready copy (codec.hpp kcode: the reference's quirks applied
// at encode / SGD time); FI8 decodes Int8 by integer conversion; FF4 decodes
// FP4 E2M1 with the hardware converts (exact for all 16 codes, no scale).
enum Fmt {
  FL1, FL2, FL3, FL4, FL5, FL6, FL8, FH16, FB16, FI16, FU16, FF32, FI32, FU32, FI64, FU64, FC64,
  FC128, FF64, FE4, FE5, FI8, FL4P, FF4, kNumFmt
};

int fmt_of(int dt) {
  switch (dt) {
  case kFloat64: return FF64;
  case kFloat32: return FF32;
  case kFloat16: return FH16;
  case kBFloat16: return FB16;
  case kFP8E4M3: case kFP8E5M2: case kInt8: case kUint8: return FL8;
  case kInt64: case kInt: return FI64;
  case kInt32: return FI32;
  case kInt16: return FI16;
  case kUint64: case kUint: case kUintptr: return FU64;
  case kUint32: return FU32;
  case kUint16: return FU16;
  case kInt4: case kUint4: case kFP4: case kNF4: return FL4;
  case kInt2: case kUint2: case kTernary: return FL2;
  case kBinary: return FL1;
  case kComplex64: return FC64;
  case kComplex128: return FC128;
  case kFP6: case kInt6: case kUint6: return FL6;
  case kInt5: case kUint5: return FL5;
  case kInt3: case kUint3: return FL3;
  }
  return -1;
}

// Chunk = the unit one lane loads: kE elements in kW dwords.
template <int F>
struct FI {
  static constexpr int kBits = F == FL1 ? 1 : F == FL2 ? 2 : F == FL3 ? 3 : (F == FL4 || F == FL4P || F == FF4) ? 4
                             : F == FL5 ? 5 : F == FL6 ? 6 : (F == FL8 || F == FE4 || F == FE5 || F == FI8) ? 8
                             : (F == FH16 || F == FB16 || F == FI16 || F == FU16) ? 16
                             : (F == FF32 || F == FI32 || F == FU32) ? 32 : F == FC128 ? 128 : 64;
  static constexpr bool kLut = (kBits <= 8 && F != FE4 && F != FE5 && F != FI8 && F != FF4) || F == FL4P;
  static constexpr bool kPair = F == FL4P;
  // floats of LDS table: 2^bits values, or 256 value pairs
  static constexpr int kTable = kPair ? 512 : (kLut ? (1 << kBits) : 1);
  static constexpr int kE = kBits <= 6 ? 32 : 128 / kBits;
  static constexpr int kW = kBits <= 6 ? kBits : 4;
  using Acc = std::conditional_t<F == FF64, double, float>;
  // decodes that can be Inf or NaN (float codes; 8-bit tables include E5M2)
  static constexpr bool kMayBeNonFinite = F == FE5 || F == FL8 || F == FH16 || F == FB16 ||
                                          F == FF32 || F == FF64 || F == FC64 || F == FC128;
};

// Fills the block's LDS table from the store's 2^bits decoded values.
template <int F>
__device__ inline void fill_table(float *tab, const float *lut, int tid, int nthreads) {
  using I = FI<F>;
  if constexpr (I::kPair) {
    for (int b = tid; b < 256; b += nthreads) {
      tab[2 * b] = lut[b & 15];
      tab[2 * b + 1] = lut[b >> 4];
    }
  } else if constexpr (I::kLut) {
    for (int i = tid; i < (1 << I::kBits); i += nthreads) tab[i] = lut[i];
  }
}

int fmt_chunk_elems(int f) {
  switch (f) {
  case FL1: case FL2: case FL3: case FL4: case FL5: case FL6: return 32;
  case FL8: case FE4: case FE5: case FI8: return 16;
  case FL4P: case FF4: return 32;
  case FH16: case FB16: case FI16: case FU16: return 8;
  case FF32: case FI32: case FU32: return 4;
  case FC128: return 1;
  default: return 2;
  }
}
int fmt_chunk_bytes(int f) {
  switch (f) {
  case FL1: return 4;
  case FL2: return 8;
  case FL3: return 12;
  case FL5: return 20;
  case FL6: return 24;
  default: return 16;
  }
}

template <int W>
__device__ inline void load_words(const uint8_t *__restrict__ p, uint32_t (&w)[W]) {
  if constexpr (W == 4) {
    const uint4 v = *(const uint4 *)p;
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else if constexpr (W == 2) {
    const uint2 v = *(const uint2 *)p;
    w[0] = v.x; w[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < W; ++i) w[i] = ((const uint32_t *)p)[i];
  }
}

// Workgroup barrier for LDS hand-offs only: this wave's LDS operations are
// complete (lgkmcnt 0) and its global loads stay in flight, where
// __syncthreads' fence would also wait for every outstanding load (on this
// target one counter covers vector-memory loads and stores).  The empty asm
// statements keep the compiler from moving memory accesses across it.
__device__ inline void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt at their maxima
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// load_words with the non-temporal hint (streamed weights, read once).
template <int W>
__device__ inline void load_words_nt(const uint8_t *__restrict__ p, uint32_t (&w)[W]) {
  typedef uint32_t u4v __attribute__((ext_vector_type(4)));
  typedef uint32_t u2v __attribute__((ext_vector_type(2)));
  if constexpr (W == 4) {
    const u4v v = __builtin_nontemporal_load((const u4v *)p);
    w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
  } else if constexpr (W == 2) {
    const u2v v = __builtin_nontemporal_load((const u2v *)p);
    w[0] = v[0]; w[1] = v[1];
  } else {
#pragma unroll
    for (int i = 0; i < W; ++i) w[i] = __builtin_nontemporal_load((const uint32_t *)p + i);
  }
}

// Code of element e of a chunk (LSB-first bitstream over little-endian words).
template <int BITS, int W>
__device__ inline uint32_t chunk_code(const uint32_t (&w)[W], int e) {
  const int bit = e * BITS, word = bit >> 5, off = bit & 31;
  uint32_t v = w[word] >> off;
  if (off + BITS > 32) v |= w[word + 1] << (32 - off);
  return v & ((1u << BITS) - 1);
}

// Decoded value of element e (exact decode of the reference, widened later).
template <int F>
__device__ inline typename FI<F>::Acc chunk_value(const uint32_t (&w)[FI<F>::kW], int e,
                                                  const float *lut, float scale, float minv) {
  using I = FI<F>;
  typedef float f2 __attribute__((ext_vector_type(2)));
  if constexpr (F == FL4P) {
    const uint32_t b = (w[e >> 3] >> (8 * ((e >> 1) & 3))) & 0xffu;
    return lut[2 * b + (e & 1)];
  } else if constexpr (I::kLut) return lut[chunk_code<I::kBits, I::kW>(w, e)];
  else if constexpr (F == FF4) {
    const f2 p = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[e >> 3] >> (8 * ((e >> 1) & 3)), 1.0f, 0);
    return (e & 1) ? p[1] : p[0];
  } else if constexpr (F == FE4 || F == FE5) {
    const uint32_t q = w[e >> 2];
    f2 p;
    if (F == FE4) p = (e & 2) ? __builtin_amdgcn_cvt_pk_f32_fp8(q, true) : __builtin_amdgcn_cvt_pk_f32_fp8(q, false);
    else p = (e & 2) ? __builtin_amdgcn_cvt_pk_f32_bf8(q, true) : __builtin_amdgcn_cvt_pk_f32_bf8(q, false);
    return (e & 1) ? p[1] : p[0];
  } else if constexpr (F == FI8) return (float)(int8_t)(uint8_t)(w[e >> 2] >> (8 * (e & 3))) * scale;
  else if constexpr (F == FH16) {
    const uint16_t h = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
    return (float)__builtin_bit_cast(_Float16, h);
  } else if constexpr (F == FB16) return u2f((w[e >> 1] >> (16 * (e & 1))) << 16);
  else if constexpr (F == FI16) return (float)(int16_t)(uint16_t)(w[e >> 1] >> (16 * (e & 1))) * scale;
  else if constexpr (F == FU16) return (float)(w[e >> 1] >> (16 * (e & 1)) & 0xffffu) * scale + minv;
  else if constexpr (F == FF32) return u2f(w[e]);
  else if constexpr (F == FI32) return (float)(int32_t)w[e] * scale;
  else if constexpr (F == FU32) return (float)w[e] * scale + minv;
  else if constexpr (F == FI64) return (float)(int64_t)((uint64_t)w[2 * e] | ((uint64_t)w[2 * e + 1] << 32)) * scale;
  else if constexpr (F == FU64) return (float)((uint64_t)w[2 * e] | ((uint64_t)w[2 * e + 1] << 32)) * scale + minv;
  else if constexpr (F == FC64) return u2f(w[2 * e]);
  else if constexpr (F == FC128) return (float)u2d((uint64_t)w[0] | ((uint64_t)w[1] << 32));
  else return u2d((uint64_t)w[2 * e] | ((uint64_t)w[2 * e + 1] << 32));  // FF64
}

// All E values of a chunk, decoded before any of them is used so the table
// reads (or converts) of a chunk are independent and issue back to back.
template <int F>
__device__ inline void decode_chunk(const uint32_t (&w)[FI<F>::kW], typename FI<F>::Acc (&v)[FI<F>::kE],
                                    const float *tab, float scale, float minv) {
  using I = FI<F>;
  typedef float f2 __attribute__((ext_vector_type(2)));
  if constexpr (F == FE4 || F == FE5) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f2 lo, hi;
      if constexpr (F == FE4) {
        lo = __builtin_amdgcn_cvt_pk_f32_fp8(w[i], false);
        hi = __builtin_amdgcn_cvt_pk_f32_fp8(w[i], true);
      } else {
        lo = __builtin_amdgcn_cvt_pk_f32_bf8(w[i], false);
        hi = __builtin_amdgcn_cvt_pk_f32_bf8(w[i], true);
      }
      v[4 * i] = lo[0];
      v[4 * i + 1] = lo[1];
      v[4 * i + 2] = hi[0];
      v[4 * i + 3] = hi[1];
    }
  } else if constexpr (F == FL4P) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t b = (w[j >> 2] >> (8 * (j & 3))) & 0xffu;
      const f2 p = ((const f2 *)tab)[b];
      v[2 * j] = p[0];
      v[2 * j + 1] = p[1];
    }
  } else if constexpr (F == FF4) {
    // byte j of the chunk holds elements 2j (low nibble) and 2j + 1
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f2 p[4] = {__builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[i], 1.0f, 0),
                       __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[i], 1.0f, 1),
                       __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[i], 1.0f, 2),
                       __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[i], 1.0f, 3)};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[8 * i + 2 * j] = p[j][0];
        v[8 * i + 2 * j + 1] = p[j][1];
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < I::kE; ++e) v[e] = chunk_value<F>(w, e, tab, scale, minv);
  }
}

template <int E>
__device__ inline void load_x(const float *__restrict__ p, float (&v)[E]) {
  if constexpr (E >= 4) {
#pragma unroll
    for (int i = 0; i < E; i += 4) {
      const float4 q = *(const float4 *)(p + i);
      v[i] = q.x; v[i + 1] = q.y; v[i + 2] = q.z; v[i + 3] = q.w;
    }
  } else if constexpr (E == 2) {
    const float2 q = *(const float2 *)p;
    v[0] = q.x; v[1] = q.y;
  } else {
    v[0] = p[0];
  }
}

template <typename T>
__device__ inline T wave_sum(T v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

struct GemvArgs {
  const uint8_t *body;
  const float *lut;
  float scale, minv;
  const float *x;
  int K, N, nchunks;
  int64_t row_bytes;
  const double *bias;
  int bias_len, act;
  float *pre, *post;
};

// A GEMV block's LDS decode table, in two steps around the weight loads:
// load() before them (so the wait for the table covers no weight load) and
// store() + lds_barrier() after they are issued.  Thread t < 64 of the block
// copies float4 entries t and t + 64 of the store's table (the pair table for
// FL4P: 128 entries; other tables have at most 64); the loads read clamped
// in-range entries.  Two named registers, no array: an array here is placed
// in LDS by the compiler.
template <int F>
struct TabCopy {
  static constexpr int kFloats = FI<F>::kTable;
  static constexpr int kQ = (kFloats + 3) / 4;
  static_assert(kQ <= 128, "two float4 per thread cover the table");
  float4 q0, q1;
  __device__ void load(const float *lut, int tid) {
    const float4 *src = (const float4 *)(FI<F>::kPair ? lut + kPairLut : lut);
    q0 = src[min(tid & 63, kQ - 1)];
    if constexpr (kQ > 64) q1 = src[min((tid & 63) + 64, kQ - 1)];
  }
  __device__ void store(float *tab, int tid) const {
    if (tid < 64 && tid < kQ) put(tab, tid, q0);
    if constexpr (kQ > 64)
      if (tid < 64 && tid + 64 < kQ) put(tab, tid + 64, q1);
  }
  __device__ static void put(float *tab, int i, float4 v) {
    if constexpr (kFloats % 4 == 0) {
      ((float4 *)tab)[i] = v;
    } else {  // tables of 2 floats (1-bit formats)
      if (4 * i < kFloats) tab[4 * i] = v.x;
      if (4 * i + 1 < kFloats) tab[4 * i + 1] = v.y;
    }
  }
};

// ----------------------------------------------------------------- GEMV
template <int F, int B, int R>
__global__ void __launch_bounds__(256) gemv_kernel(GemvArgs a) {
  using I = FI<F>;
  using Acc = typename I::Acc;
  constexpr int E = I::kE, W = I::kW;
  __shared__ float lut_s[I::kTable];
  if constexpr (I::kLut) {
    fill_table<F>(lut_s, a.lut, threadIdx.x, 256);
    __syncthreads();
  }
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
  Acc acc[R][B];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < B; ++b) acc[r][b] = 0;
  for (int c = lane; c < a.nchunks; c += 64) {
    uint32_t w[R][W];
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (row0 + r < a.N) load_words<W>(a.body + (int64_t)(row0 + r) * a.row_bytes + (int64_t)c * (W * 4), w[r]);
    float xv[B][E];
#pragma unroll
    for (int b = 0; b < B; ++b) load_x<E>(a.x + (int64_t)b * a.K + (int64_t)c * E, xv[b]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (row0 + r < a.N) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const Acc wv = chunk_value<F>(w[r], e, lut_s, a.scale, a.minv);
#pragma unroll
          for (int b = 0; b < B; ++b) acc[r][b] = fma(wv, (Acc)xv[b][e], acc[r][b]);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < B; ++b) acc[r][b] = wave_sum(acc[r][b]);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = row0 + r;
      if (row < a.N) {
#pragma unroll
        for (int b = 0; b < B; ++b)
          bias_act_store((double)acc[r][b], row, a.bias, a.bias_len, a.act, a.pre, a.post,
                         (int64_t)b * a.N + row);
      }
    }
  }
}

// Lane exchanges without the LDS crossbar (f64 values as two dwords).
// swap32: a <- [a lanes 0-31, b lanes 0-31], b <- [a lanes 32-63, b lanes 32-63]
// (v_permlane32_swap); swap16: the same on 16-lane row pairs (rows 0/1, 2/3:
// v_permlane16_swap); dpp<CTRL>: the value of the DPP partner lane
// (0x140 row mirror i <-> 15 - i, 0x141 half-row mirror i <-> 7 - i, quad
// permutes 0xB1 = xor 1, 0x4E = xor 2).
typedef unsigned u32x2v __attribute__((ext_vector_type(2)));
__device__ inline void swap32(double &a, double &b) {
  const uint64_t ua = __builtin_bit_cast(uint64_t, a), ub = __builtin_bit_cast(uint64_t, b);
  const u32x2v lo = __builtin_amdgcn_permlane32_swap((unsigned)ua, (unsigned)ub, false, false);
  const u32x2v hi = __builtin_amdgcn_permlane32_swap((unsigned)(ua >> 32), (unsigned)(ub >> 32), false, false);
  a = __builtin_bit_cast(double, (uint64_t)lo[0] | ((uint64_t)hi[0] << 32));
  b = __builtin_bit_cast(double, (uint64_t)lo[1] | ((uint64_t)hi[1] << 32));
}
__device__ inline void swap16(double &a, double &b) {
  const uint64_t ua = __builtin_bit_cast(uint64_t, a), ub = __builtin_bit_cast(uint64_t, b);
  const u32x2v lo = __builtin_amdgcn_permlane16_swap((unsigned)ua, (unsigned)ub, false, false);
  const u32x2v hi = __builtin_amdgcn_permlane16_swap((unsigned)(ua >> 32), (unsigned)(ub >> 32), false, false);
  a = __builtin_bit_cast(double, (uint64_t)lo[0] | ((uint64_t)hi[0] << 32));
  b = __builtin_bit_cast(double, (uint64_t)lo[1] | ((uint64_t)hi[1] << 32));
}
template <int CTRL>
__device__ inline double dpp(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const unsigned lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)u, CTRL, 0xf, 0xf, false);
  const unsigned hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(u >> 32), CTRL, 0xf, 0xf, false);
  return __builtin_bit_cast(double, (uint64_t)lo | ((uint64_t)hi << 32));
}

// Reduction of the batch-1 GEMV: acc[r] holds this lane's partial of row r.
// log2(R) transposing steps (lane bit 5, 4, 3, 2: each lane keeps half of its
// rows and adds the other half's partner values), then a sum over the lanes
// left sharing a row.  Returns, on every lane l, the full sum of row
// l >> (6 - log2 R).  Any pairing that counts each lane once gives the sum:
// the mirrors pair lanes across the same bit boundary as an xor would.
template <int R>
__device__ inline double row_reduce(double (&acc)[R], int lane) {
  constexpr int LR = R == 1 ? 0 : R == 2 ? 1 : R == 4 ? 2 : R == 8 ? 3 : 4;
  static_assert((1 << LR) == R, "rows per block must be 1, 2, 4, 8 or 16");
  if constexpr (LR >= 1) {
#pragma unroll
    for (int i = 0; i < R / 2; ++i) {
      swap32(acc[i], acc[i + R / 2]);
      acc[i] += acc[i + R / 2];
    }
  }
  if constexpr (LR >= 2) {
#pragma unroll
    for (int i = 0; i < R / 4; ++i) {
      swap16(acc[i], acc[i + R / 4]);
      acc[i] += acc[i + R / 4];
    }
  }
  if constexpr (LR >= 3) {
    const bool hi = (lane >> 3) & 1;
#pragma unroll
    for (int i = 0; i < R / 8; ++i)
      acc[i] = (hi ? acc[i + R / 8] : acc[i]) + dpp<0x140>(hi ? acc[i] : acc[i + R / 8]);
  }
  if constexpr (LR >= 4) {
    const bool hi = (lane >> 2) & 1;
    acc[0] = (hi ? acc[1] : acc[0]) + dpp<0x141>(hi ? acc[0] : acc[1]);
  }
  double v = acc[0];
  if constexpr (LR == 0) {
    double w = v;
    swap32(v, w);
    v += w;
  }
  if constexpr (LR <= 1) {
    double w = v;
    swap16(v, w);
    v += w;
  }
  if constexpr (LR <= 2) v += dpp<0x140>(v);
  if constexpr (LR <= 3) v += dpp<0x141>(v);
  v += dpp<0x4E>(v);
  v += dpp<0xB1>(v);
  return v;
}

// row_reduce on fp32 values (one 32-bit exchange per value instead of two):
// the same pairing, so lane l ends with the full sum of row l >> (6 - log2 R)
// of the wave, added in fp32.
__device__ inline void swap32f(float &a, float &b) {
  const u32x2v r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ inline void swap16f(float &a, float &b) {
  const u32x2v r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
template <int CTRL>
__device__ inline float dppf(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int R>
__device__ inline float row_reduce_f32(float (&acc)[R], int lane) {
  constexpr int LR = R == 1 ? 0 : R == 2 ? 1 : R == 4 ? 2 : R == 8 ? 3 : 4;
  static_assert((1 << LR) == R, "rows per block must be 1, 2, 4, 8 or 16");
  if constexpr (LR >= 1) {
#pragma unroll
    for (int i = 0; i < R / 2; ++i) {
      swap32f(acc[i], acc[i + R / 2]);
      acc[i] += acc[i + R / 2];
    }
  }
  if constexpr (LR >= 2) {
#pragma unroll
    for (int i = 0; i < R / 4; ++i) {
      swap16f(acc[i], acc[i + R / 4]);
      acc[i] += acc[i + R / 4];
    }
  }
  if constexpr (LR >= 3) {
    const bool hi = (lane >> 3) & 1;
#pragma unroll
    for (int i = 0; i < R / 8; ++i)
      acc[i] = (hi ? acc[i + R / 8] : acc[i]) + dppf<0x140>(hi ? acc[i] : acc[i + R / 8]);
  }
  if constexpr (LR >= 4) {
    const bool hi = (lane >> 2) & 1;
    acc[0] = (hi ? acc[1] : acc[0]) + dppf<0x141>(hi ? acc[0] : acc[1]);
  }
  float v = acc[0];
  if constexpr (LR == 0) {
    float w = v;
    swap32f(v, w);
    v += w;
  }
  if constexpr (LR <= 1) {
    float w = v;
    swap16f(v, w);
    v += w;
  }
  if constexpr (LR <= 2) v += dppf<0x140>(v);
  if constexpr (LR <= 3) v += dppf<0x141>(v);
  v += dppf<0x4E>(v);
  v += dppf<0xB1>(v);
  return v;
}

// Batch-1 GEMV with every load of a lane in flight at once.  A block owns R
// rows; its S waves split the row into column slices of 64*C chunks (lane i
// of a wave reads chunk slice*64*C + cc*64 + i of each row: 1 KB contiguous
// per wave per (row, cc)).  The table load is issued first, then all R*C
// weight chunks and the C x chunks, so one memory latency covers the whole
// wave.  Per-lane fp32 FMA over its C*E products, then an f64 butterfly
// transpose-reduce over the R rows and an ordered f64 sum over the S slices.
template <int F, int C, int R>
__global__ void __launch_bounds__(512) gemv_pf_kernel(GemvArgs a) {
  using I = FI<F>;
  using Acc = std::conditional_t<F == FF64, double, float>;
  constexpr int E = I::kE, W = I::kW, NL = I::kTable;
  __shared__ __align__(16) float lut_s[NL];
  __shared__ double part[8][R];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  TabCopy<F> tab;
  if constexpr (I::kLut) {
    tab.load(a.lut, tid);
    __builtin_amdgcn_sched_barrier(0);  // issued before x and the weights
  }
  const int r0 = blockIdx.x * R;
  const int cbase = wave * 64 * C + lane;
  // issue order matters: vmcnt retires in order, so the table and x loads go
  // first and row r's arithmetic waits only for loads up to row r
  // Loads are unconditional, from clamped in-range addresses (lanes past the
  // row end or rows past N read a valid chunk whose products are never
  // used): straight-line loads let each row's arithmetic wait for exactly
  // the loads before it instead of for all of them.
  float xv[C][E];
#pragma unroll
  for (int cc = 0; cc < C; ++cc) {
    const int c = min(cbase + cc * 64, a.nchunks - 1);
    load_x<E>(a.x + (int64_t)c * E, xv[cc]);
  }
  uint32_t w[R][C][W];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t row = min(r0 + r, a.N - 1);
#pragma unroll
    for (int cc = 0; cc < C; ++cc) {
      const int c = min(cbase + cc * 64, a.nchunks - 1);
      load_words<W>(a.body + row * a.row_bytes + (int64_t)c * (W * 4), w[r][cc]);
    }
  }
  if constexpr (I::kLut) {
    tab.store(lut_s, tid);
    lds_barrier();
  }
  // A wave whose column slice runs past the row end zeroes, on its lanes
  // past the end (duplicate reads), x and — for formats with non-finite
  // codes — the weight words, so they add exact zeros.  The lane mask is
  // opaque to the compiler, which would otherwise move the loads under a
  // branch on it (and then wait for all of them at the join).
  if (__builtin_amdgcn_readfirstlane(wave) * 64 * C + 64 * C > a.nchunks) {
#pragma unroll
    for (int cc = 0; cc < C; ++cc) {
      uint32_t keep = cbase + cc * 64 < a.nchunks ? ~0u : 0u;
      asm volatile("" : "+v"(keep));
#pragma unroll
      for (int e = 0; e < E; ++e) xv[cc][e] = __uint_as_float(__float_as_uint(xv[cc][e]) & keep);
      if constexpr (FI<F>::kMayBeNonFinite) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int i = 0; i < W; ++i) w[r][cc][i] &= keep;
      }
    }
  }
  double acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    Acc s[4] = {0, 0, 0, 0};
#pragma unroll
    for (int cc = 0; cc < C; ++cc) {
      Acc v[E];
      decode_chunk<F>(w[r][cc], v, lut_s, a.scale, a.minv);
#pragma unroll
      for (int e = 0; e < E; ++e) s[e & 3] = fma(v[e], (Acc)xv[cc][e], s[e & 3]);
    }
    acc[r] = ((double)s[0] + (double)s[1]) + ((double)s[2] + (double)s[3]);
  }
  // lane l: the sum of row l >> (6 - log2 R) over the wave
  constexpr int LR = R == 1 ? 0 : R == 2 ? 1 : R == 4 ? 2 : R == 8 ? 3 : 4;
  const double v = row_reduce<R>(acc, lane);
  const int S = blockDim.x >> 6;
  if (S == 1) {
    if ((lane & ((64 >> LR) - 1)) == 0) {
      const int row = r0 + (lane >> (6 - LR));
      if (row < a.N) bias_act_store(v, row, a.bias, a.bias_len, a.act, a.pre, a.post, row);
    }
    return;
  }
  if ((lane & ((64 >> LR) - 1)) == 0) part[wave][lane >> (6 - LR)] = v;
  __syncthreads();
  if (tid < R && r0 + tid < a.N) {
    double s = 0;
    for (int g = 0; g < S; ++g) s += part[g][tid];
    bias_act_store(s, r0 + tid, a.bias, a.bias_len, a.act, a.pre, a.post, r0 + tid);
  }
}

// gemv_pf_kernel as a grid-stride loop: a fixed number of blocks walks the
// row groups, so x and the decode table are loaded once per block.  A row
// group is R rows; the block's S waves split each row into column slices of 64*C
// chunks (lane i of a wave reads chunk slice*64*C + cc*64 + i of each row:
// 1 KB contiguous per wave per (row, cc)).  Per row group the lane issues all
// R*C weight loads (non-temporal: the weights are streamed once) before any
// arithmetic, so one memory latency covers the group.  Per-lane fp32 FMA over
// its C*E products, then an fp32 butterfly transpose-reduce over the R rows
// and an ordered f64 sum over the S slices.  The block walks row groups
// blockIdx.x, blockIdx.x + gridDim.x, ...
template <int F, int C, int R>
__global__ void __launch_bounds__(512) gemv_loop_kernel(GemvArgs a) {
  using I = FI<F>;
  static_assert(F != FF64, "fp32 partial sums: not for Float64 weights");
  constexpr int E = I::kE, W = I::kW, NL = I::kTable;
  constexpr int LR = R == 1 ? 0 : R == 2 ? 1 : R == 4 ? 2 : R == 8 ? 3 : 4;
  static_assert((1 << LR) == R, "rows per block must be 1, 2, 4, 8 or 16");
  __shared__ __align__(16) float lut_s[NL];
  __shared__ double part[2][8][R];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int S = blockDim.x >> 6;
  const int ngroups = (a.N + R - 1) / R;
  TabCopy<F> tab;
  if constexpr (I::kLut) {
    tab.load(a.lut, tid);
    __builtin_amdgcn_sched_barrier(0);  // issued before x and the weights
  }
  const int cbase = wave * 64 * C + lane;
  // issue order matters: vmcnt retires in order, so the table and x loads go
  // first and row r's arithmetic waits only for loads up to row r
  // Loads are unconditional, from clamped in-range addresses (lanes past the
  // row end or rows past N read a valid chunk whose products are never
  // used): straight-line loads let each row's arithmetic wait for exactly
  // the loads before it instead of for all of them.
  float xv[C][E];
#pragma unroll
  for (int cc = 0; cc < C; ++cc) {
    const int c = min(cbase + cc * 64, a.nchunks - 1);
    load_x<E>(a.x + (int64_t)c * E, xv[cc]);
  }
  // A wave whose column slice runs past the row end zeroes, on its lanes
  // past the end (duplicate reads), x and — for formats with non-finite
  // codes — the weight words, so they add exact zeros.  The lane mask is
  // opaque to the compiler, which would otherwise move the loads under a
  // branch on it (and then wait for all of them at the join).
  const bool ragged = __builtin_amdgcn_readfirstlane(wave) * 64 * C + 64 * C > a.nchunks;
  uint32_t keep[C];
#pragma unroll
  for (int cc = 0; cc < C; ++cc) {
    keep[cc] = cbase + cc * 64 < a.nchunks ? ~0u : 0u;
    asm volatile("" : "+v"(keep[cc]));
  }
  // one row group: loads, decode + FMA, reductions, epilogue
  auto group = [&](int g, bool first, int buf) {
    const int r0 = g * R;
    uint32_t w[R][C][W];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t row = min(r0 + r, a.N - 1);
#pragma unroll
      for (int cc = 0; cc < C; ++cc) {
        const int c = min(cbase + cc * 64, a.nchunks - 1);
        const uint8_t *src = a.body + row * a.row_bytes + (int64_t)c * (W * 4);
        load_words_nt<W>(src, w[r][cc]);
      }
    }
    if (first) {
      if constexpr (I::kLut) {
        tab.store(lut_s, tid);
        lds_barrier();
      }
      if (ragged) {
#pragma unroll
        for (int cc = 0; cc < C; ++cc)
#pragma unroll
          for (int e = 0; e < E; ++e) xv[cc][e] = __uint_as_float(__float_as_uint(xv[cc][e]) & keep[cc]);
      }
    }
    if constexpr (FI<F>::kMayBeNonFinite) {
      if (ragged) {
#pragma unroll
        for (int cc = 0; cc < C; ++cc)
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < W; ++i) w[r][cc][i] &= keep[cc];
      }
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float sm[4] = {0, 0, 0, 0};
#pragma unroll
      for (int cc = 0; cc < C; ++cc) {
        float v[E];
        decode_chunk<F>(w[r][cc], v, lut_s, a.scale, a.minv);
#pragma unroll
        for (int e = 0; e < E; ++e) sm[e & 3] = fmaf(v[e], xv[cc][e], sm[e & 3]);
      }
      acc[r] = (sm[0] + sm[1]) + (sm[2] + sm[3]);
    }
    // lane l: the sum of row l >> (6 - log2 R) over the wave, in fp32
    const double v = (double)row_reduce_f32<R>(acc, lane);
    if (S == 1) {
      if ((lane & ((64 >> LR) - 1)) == 0) {
        const int row = r0 + (lane >> (6 - LR));
        if (row < a.N) bias_act_store(v, row, a.bias, a.bias_len, a.act, a.pre, a.post, row);
      }
      return;
    }
    // part is double-buffered: the next group's writes go to the other half,
    // and the barrier of that group orders them after this group's reads
    if ((lane & ((64 >> LR) - 1)) == 0) part[buf][wave][lane >> (6 - LR)] = v;
    __syncthreads();
    if (tid < R && r0 + tid < a.N) {
      double sum = 0;
      for (int q = 0; q < S; ++q) sum += part[buf][q][tid];
      bias_act_store(sum, r0 + tid, a.bias, a.bias_len, a.act, a.pre, a.post, r0 + tid);
    }
  };
  int buf = 0;
  for (int g = blockIdx.x; g < ngroups; g += gridDim.x, buf ^= 1) group(g, g == (int)blockIdx.x, buf);
}

// SwiGLU's Gate and Up projections at batch 1 in one launch (the
// loop GEMV's structure, one chunk per lane): a row group is R rows of Gate
// and the same R rows of Up (two stores of one format and shape; each its own
// decode table and scale), so x is loaded once per block for both and the
// epilogue has g and u of an output together: pre = g, pre2 = u, post = h =
// fl32(silu(g)) * u (op_swiglu's product, ops_common.metal:27-38).  The 2R
// sums take the fp32 butterfly as 2R rows (Gate's in rows 0..R-1, Up's in
// R..2R-1), then the ordered f64 sum over the S slices.
struct GemvPairArgs {
  GemvArgs a;  // Gate: body, lut, scale, minv; x, K, N, nchunks, row_bytes; pre = g, post = h
  const uint8_t *body2;  // Up
  const float *lut2;
  float scale2, minv2;
  float *pre2;  // u
};
template <int F, int R>
__global__ void __launch_bounds__(512) gemv_pair_kernel(GemvPairArgs pa) {
  using I = FI<F>;
  const GemvArgs &a = pa.a;
  constexpr int E = I::kE, W = I::kW, NL = I::kTable, R2 = 2 * R;
  constexpr int LR2 = R2 == 2 ? 1 : R2 == 4 ? 2 : R2 == 8 ? 3 : 4;
  static_assert((1 << LR2) == R2, "2R rows: 2, 4, 8 or 16");
  __shared__ __align__(16) float lut_s[2][NL];
  __shared__ double part[2][8][R2];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int S = blockDim.x >> 6;
  const int ngroups = (a.N + R - 1) / R;
  TabCopy<F> tab, tab2;
  if constexpr (I::kLut) {
    tab.load(a.lut, tid);
    tab2.load(pa.lut2, tid);
    __builtin_amdgcn_sched_barrier(0);
  }
  const int cbase = wave * 64 + lane;
  float xv[E];
  load_x<E>(a.x + (int64_t)min(cbase, a.nchunks - 1) * E, xv);
  const bool ragged = __builtin_amdgcn_readfirstlane(wave) * 64 + 64 > a.nchunks;
  uint32_t keep = cbase < a.nchunks ? ~0u : 0u;
  asm volatile("" : "+v"(keep));
  auto group = [&](int g, bool first, int buf) {
    const int r0 = g * R;
    uint32_t w[R2][W];
    const int c = min(cbase, a.nchunks - 1);
#pragma unroll
    for (int r = 0; r < R2; ++r) {
      const int64_t row = min(r0 + (r % R), a.N - 1);
      const uint8_t *src = (r < R ? a.body : pa.body2) + row * a.row_bytes + (int64_t)c * (W * 4);
      load_words_nt<W>(src, w[r]);
    }
    if (first) {
      if constexpr (I::kLut) {
        tab.store(lut_s[0], tid);
        tab2.store(lut_s[1], tid);
        lds_barrier();
      }
      if (ragged) {
#pragma unroll
        for (int e = 0; e < E; ++e) xv[e] = __uint_as_float(__float_as_uint(xv[e]) & keep);
      }
    }
    if constexpr (FI<F>::kMayBeNonFinite) {
      if (ragged) {
#pragma unroll
        for (int r = 0; r < R2; ++r)
#pragma unroll
          for (int i = 0; i < W; ++i) w[r][i] &= keep;
      }
    }
    float acc[R2];
#pragma unroll
    for (int r = 0; r < R2; ++r) {
      float sm[4] = {0, 0, 0, 0};
      float v[E];
      if (r < R) decode_chunk<F>(w[r], v, lut_s[0], a.scale, a.minv);
      else decode_chunk<F>(w[r], v, lut_s[1], pa.scale2, pa.minv2);
#pragma unroll
      for (int e = 0; e < E; ++e) sm[e & 3] = fmaf(v[e], xv[e], sm[e & 3]);
      acc[r] = (sm[0] + sm[1]) + (sm[2] + sm[3]);
    }
    // lane l: the sum of row l >> (6 - log2 2R); Up's row r sits 32 lanes
    // after Gate's
    const float v = row_reduce_f32<R2>(acc, lane);
    auto store = [&](double gs, double us, int row) {
      const float gv = (float)gs, uv = (float)us;
      a.pre[row] = gv;
      pa.pre2[row] = uv;
      a.post[row] = act_value(gv, kSilu) * uv;
    };
    if (S == 1) {
      const float u = __shfl(v, (lane + 32) & 63);
      if (lane < 32 && (lane & ((64 >> LR2) - 1)) == 0) {
        const int row = r0 + (lane >> (6 - LR2));
        if (row < a.N) store((double)v, (double)u, row);
      }
      return;
    }
    if ((lane & ((64 >> LR2) - 1)) == 0) part[buf][wave][lane >> (6 - LR2)] = (double)v;
    __syncthreads();
    if (tid < R && r0 + tid < a.N) {
      double gs = 0, us = 0;
      for (int q = 0; q < S; ++q) {
        gs += part[buf][q][tid];
        us += part[buf][q][R + tid];
      }
      store(gs, us, r0 + tid);
    }
  };
  int buf = 0;
  for (int g = blockIdx.x; g < ngroups; g += gridDim.x, buf ^= 1) group(g, g == (int)blockIdx.x, buf);
}

// gemv_loop_kernel for batch 2..B: the block holds the column slice of x of
// all B batch rows in registers, so each weight chunk is loaded and decoded
// once and feeds B products.  A row group is R rows; its R * B sums (one fp32
// FMA chain per row and batch row over the lane's C * E products) go through
// the butterfly as R * B rows, in fp32, then the ordered f64 sum over the S
// slices.
// Batch rows from `batch` to B - 1 read x row batch - 1 and are never stored.
template <int F, int C, int R, int B>
__global__ void __launch_bounds__(512) gemv_loopb_kernel(GemvArgs a, int batch) {
  using I = FI<F>;
  static_assert(F != FF64, "fp32 partial sums: not for Float64 weights");
  constexpr int E = I::kE, W = I::kW, NL = I::kTable, V = R * B;
  constexpr int LV = V == 2 ? 1 : V == 4 ? 2 : V == 8 ? 3 : 4;
  static_assert((1 << LV) == V, "rows per group times batch rows must be 2, 4, 8 or 16");
  __shared__ __align__(16) float lut_s[NL];
  __shared__ double part[2][8][V];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int S = blockDim.x >> 6;
  const int ngroups = (a.N + R - 1) / R;
  TabCopy<F> tab;
  if constexpr (I::kLut) {
    tab.load(a.lut, tid);
    __builtin_amdgcn_sched_barrier(0);  // issued before x and the weights
  }
  const int cbase = wave * 64 * C + lane;
  float xv[B][C][E];
#pragma unroll
  for (int b = 0; b < B; ++b) {
    const float *xb = a.x + (int64_t)min(b, batch - 1) * a.K;
#pragma unroll
    for (int cc = 0; cc < C; ++cc) {
      const int c = min(cbase + cc * 64, a.nchunks - 1);
      load_x<E>(xb + (int64_t)c * E, xv[b][cc]);
    }
  }
  // lanes past the row end (duplicate reads) add exact zeros: x and, for
  // formats with non-finite codes, the weight words are masked
  const bool ragged = __builtin_amdgcn_readfirstlane(wave) * 64 * C + 64 * C > a.nchunks;
  uint32_t keep[C];
#pragma unroll
  for (int cc = 0; cc < C; ++cc) {
    keep[cc] = cbase + cc * 64 < a.nchunks ? ~0u : 0u;
    asm volatile("" : "+v"(keep[cc]));
  }
  // one row group's weight loads (non-temporal: streamed once)
  using Words = uint32_t[R][C][W];
  auto load_group = [&](int g, Words &w) {
    const int r0 = g * R;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t row = min(r0 + r, a.N - 1);
#pragma unroll
      for (int cc = 0; cc < C; ++cc) {
        const int c = min(cbase + cc * 64, a.nchunks - 1);
        load_words_nt<W>(a.body + row * a.row_bytes + (int64_t)c * (W * 4), w[r][cc]);
      }
    }
  };
  // decode + FMA, reductions, epilogue of row group g from its loaded words
  auto group = [&](int g, Words &w, int buf) {
    const int r0 = g * R;
    if constexpr (I::kMayBeNonFinite) {
      if (ragged) {
#pragma unroll
        for (int cc = 0; cc < C; ++cc)
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < W; ++i) w[r][cc][i] &= keep[cc];
      }
    }
    float acc[V];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float sm[B];
#pragma unroll
      for (int b = 0; b < B; ++b) sm[b] = 0.0f;
#pragma unroll
      for (int cc = 0; cc < C; ++cc) {
        float v[E];
        decode_chunk<F>(w[r][cc], v, lut_s, a.scale, a.minv);
#pragma unroll
        for (int e = 0; e < E; ++e)
#pragma unroll
          for (int b = 0; b < B; ++b) sm[b] = fmaf(v[e], xv[b][cc][e], sm[b]);
      }
#pragma unroll
      for (int b = 0; b < B; ++b) acc[r * B + b] = sm[b];
    }
    // lane l: the sum of (row, batch row) l >> (6 - LV) over the wave, in
    // fp32 (64 lane partials: at most 6 roundings of 2^-24 of the sum of
    // magnitudes, far inside the 1e-5 bound); the slices add in f64
    const double v = (double)row_reduce_f32<V>(acc, lane);
    if (S == 1) {
      if ((lane & ((64 >> LV) - 1)) == 0) {
        const int vr = lane >> (6 - LV), row = r0 + vr / B, b = vr % B;
        if (row < a.N && b < batch)
          bias_act_store(v, row, a.bias, a.bias_len, a.act, a.pre, a.post, (int64_t)b * a.N + row);
      }
      return;
    }
    // part is double-buffered: the next group's writes go to the other half,
    // and the barrier of that group orders them after this group's reads
    if ((lane & ((64 >> LV) - 1)) == 0) part[buf][wave][lane >> (6 - LV)] = v;
    __syncthreads();
    if (tid < V) {
      const int row = r0 + tid / B, b = tid % B;
      if (row < a.N && b < batch) {
        double sum = 0;
        for (int q = 0; q < S; ++q) sum += part[buf][q][tid];
        bias_act_store(sum, row, a.bias, a.bias_len, a.act, a.pre, a.post, (int64_t)b * a.N + row);
      }
    }
  };
  // The block walks row groups blockIdx.x, + gridDim.x, ... (the grid never
  // exceeds the group count).  From B = 4 on (at most 3 waves per SIMD) the
  // next group's loads are in flight while it works on the current one, two
  // word buffers alternating; past the last group that prefetch re-reads the
  // last row group (every block the same rows), so the loads stay
  // unconditional.  At B = 2 the extra buffer would cost occupancy instead.
  constexpr bool kPrefetch = B >= 4;
  Words wa, wb;
  int g = blockIdx.x;
  load_group(g, wa);
  if constexpr (I::kLut) {
    tab.store(lut_s, tid);
    lds_barrier();
  }
  if (ragged) {
#pragma unroll
    for (int b = 0; b < B; ++b)
#pragma unroll
      for (int cc = 0; cc < C; ++cc)
#pragma unroll
        for (int e = 0; e < E; ++e) xv[b][cc][e] = __uint_as_float(__float_as_uint(xv[b][cc][e]) & keep[cc]);
  }
  if constexpr (!kPrefetch) {
    for (int buf = 0;; buf ^= 1) {
      group(g, wa, buf);
      g += gridDim.x;
      if (g >= ngroups) break;
      load_group(g, wa);
    }
    return;
  }
  // consecutive groups use opposite halves of part: 0 for wa, 1 for wb
  for (;;) {
    int gn = g + gridDim.x;
    load_group(min(gn, ngroups - 1), wb);
    group(g, wa, 0);
    if (gn >= ngroups) break;
    g = gn;
    gn = g + gridDim.x;
    load_group(min(gn, ngroups - 1), wa);
    group(g, wb, 1);
    if (gn >= ngroups) break;
    g = gn;
  }
}

// Element-wise fallback for shapes whose rows do not start on a chunk
// boundary: a block per output row, f64 accumulation, any batch.
template <int DT>
__global__ void __launch_bounds__(256) gemv_generic_kernel(DevStore w, int batch, const float *x,
                                                           const double *bias, int bias_len, int act,
                                                           float *pre, float *post) {
  __shared__ double red[4];
  const int o = blockIdx.x;
  for (int b = 0; b < batch; ++b) {
    double acc = 0;
    for (int k = threadIdx.x; k < w.cols; k += 256) {
      const int64_t i = (int64_t)o * w.cols + k;
      const uint64_t c = load_code<DT>(w.body, i);
      const double wv = DT == kFloat64 ? u2d(c) : (double)dec_code<DT>(c, w.scale, w.minv);
      acc += wv * (double)x[(int64_t)b * w.cols + k];
    }
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0)
      bias_act_store(red[0] + red[1] + red[2] + red[3], o, bias, bias_len, act, pre, post,
                     (int64_t)b * w.rows + o);
    __syncthreads();
  }
}

// ----------------------------------------------------------------- GEMM
// C[m][n] = sum_k A[m][k] * Wop[k][n] over fp32 MFMA 32x32x2, stream-K.
//   forward: A = x [M][K], Wop[k][n] = W[n][k]        (TRANS = false)
//   dX:      A = dpre [M][K=rows], Wop[k][n] = W[k][n] (TRANS = true)
// The (tile, k-stage) iteration space is cut into equal contiguous shares,
// one per workgroup (two resident per CU), so every CU gets the same work
// whatever the tile count.  Each share stages A and decoded W tiles in
// double-buffered LDS (the next stage's global loads are in flight during
// the current stage's MFMAs) and writes one partial tile per tile it
// touches; sk_reduce_kernel then adds each tile's partials in workgroup
// order in f64.  (Folding that sum into the GEMM, with the last workgroup to
// finish a tile doing it, needs an agent-scope release per partial: the L2
// write-back it costs made the forward GEMM 2.5x slower.)
struct GemmArgs {
  const uint8_t *body;
  const float *lut;
  float scale, minv;
  const float *A;
  int M, K, N;        // product dims
  int64_t row_bytes;  // bytes per stored W row
  int gx, gy, nst;    // tiles along N, along M; k stages
  int per_block, maxspan;
  float *ws;          // [blocks][maxspan][bm][bn] partial tiles
  int bm, bn;         // tile shape
  // the reduction multiplies sums by post (a per-tensor scale the split-x
  // GEMM factors out of the weights)
  float post = 1.0f;
};

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 64, kBN = 64, kBK = 64, kPad = 1;

template <int F, bool TRANS>
struct TileLoader {
  using I = FI<F>;
  static constexpr int E = I::kE, W = I::kW;
  static constexpr int kChunks = TRANS ? kBK * (kBN / E) : kBN * (kBK / E);
  static constexpr int kCPT = (kChunks + 255) / 256;
  static constexpr int kA4 = kBM * kBK / 4 / 256;
  uint32_t w[kCPT][W];
  float av[kA4][4];

  __device__ void load(const GemmArgs &a, int m0, int n0, int k0, int tid) {
#pragma unroll
    for (int i = 0; i < kCPT; ++i) {
      const int q = tid + i * 256;
      bool ok = q < kChunks;
      const uint8_t *p = nullptr;
      if constexpr (!TRANS) {
        const int n = q % kBN, j = q / kBN, k = k0 + j * E, row = n0 + n;
        ok = ok && row < a.N && k < a.K;
        p = a.body + (int64_t)row * a.row_bytes + (int64_t)(k / E) * (W * 4);
      } else {
        const int kl = q % kBK, j = q / kBK, k = k0 + kl, col = n0 + j * E;
        ok = ok && k < a.K && col < a.N;
        p = a.body + (int64_t)k * a.row_bytes + (int64_t)(col / E) * (W * 4);
      }
      if (ok) load_words<W>(p, w[i]);
      else {
#pragma unroll
        for (int j = 0; j < W; ++j) w[i][j] = 0;
      }
    }
    const bool vec = (a.K & 3) == 0;
#pragma unroll
    for (int i = 0; i < kA4; ++i) {
      const int q = tid + i * 256, m = q / (kBK / 4), k = k0 + 4 * (q % (kBK / 4));
      const int mg = m0 + m;
      const float *src = a.A + (int64_t)mg * a.K + k;
      if (mg < a.M && vec && k + 3 < a.K) {
        const float4 v = *(const float4 *)src;
        av[i][0] = v.x; av[i][1] = v.y; av[i][2] = v.z; av[i][3] = v.w;
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) av[i][t] = (mg < a.M && k + t < a.K) ? src[t] : 0.0f;
      }
    }
  }

  __device__ void store(float (*Xs)[kBM + kPad], float (*Ws)[kBN + kPad], const GemmArgs &a,
                        const float *lut, int m0, int n0, int k0, int tid) const {
#pragma unroll
    for (int i = 0; i < kCPT; ++i) {
      const int q = tid + i * 256;
      if (q >= kChunks) break;
      if constexpr (!TRANS) {
        const int n = q % kBN, j = q / kBN;
        const bool ok = n0 + n < a.N && k0 + j * E < a.K;
#pragma unroll
        for (int e = 0; e < E; ++e)
          Ws[j * E + e][n] = ok ? (float)chunk_value<F>(w[i], e, lut, a.scale, a.minv) : 0.0f;
      } else {
        const int kl = q % kBK, j = q / kBK;
        const bool ok = k0 + kl < a.K && n0 + j * E < a.N;
#pragma unroll
        for (int e = 0; e < E; ++e)
          Ws[kl][j * E + e] = ok ? (float)chunk_value<F>(w[i], e, lut, a.scale, a.minv) : 0.0f;
      }
    }
#pragma unroll
    for (int i = 0; i < kA4; ++i) {
      const int q = tid + i * 256, m = q / (kBK / 4), kl = 4 * (q % (kBK / 4));
#pragma unroll
      for (int t = 0; t < 4; ++t) Xs[kl + t][m] = av[i][t];
    }
  }
};

template <int F, bool TRANS>
__global__ void __launch_bounds__(256, 2) gemm_sk_kernel(GemmArgs a) {
  using I = FI<F>;
  __shared__ float Xs[2][kBK][kBM + kPad];
  __shared__ float Ws[2][kBK][kBN + kPad];
  __shared__ float lut_s[I::kTable];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  if constexpr (I::kLut) fill_table<F>(lut_s, a.lut, tid, 256);
  __syncthreads();
  const int T = a.gx * a.gy * a.nst;
  int it = blockIdx.x * a.per_block;
  const int it_end = min(T, it + a.per_block);
  const int first_tile = it / a.nst;
  TileLoader<F, TRANS> L;
  while (it < it_end) {
    const int t = it / a.nst, s0 = it % a.nst;
    const int nseg = min(it_end, (t + 1) * a.nst) - it;
    const int m0 = (t / a.gx) * kBM, n0 = (t % a.gx) * kBN;
    floatx16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
    L.load(a, m0, n0, s0 * kBK, tid);
    L.store(Xs[0], Ws[0], a, lut_s, m0, n0, s0 * kBK, tid);
    __syncthreads();
    for (int s = 0; s < nseg; ++s) {
      const int cur = s & 1;
      const int knext = (s0 + s + 1) * kBK;
      if (s + 1 < nseg) L.load(a, m0, n0, knext, tid);
#pragma unroll
      for (int kk = 0; kk < kBK; kk += 2) {
        const float av = Xs[cur][kk + (lane >> 5)][wm * 32 + (lane & 31)];
        const float bv = Ws[cur][kk + (lane >> 5)][wn * 32 + (lane & 31)];
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc, 0, 0, 0);
      }
      if (s + 1 < nseg) L.store(Xs[cur ^ 1], Ws[cur ^ 1], a, lut_s, m0, n0, knext, tid);
      __syncthreads();
    }
    // D[i][j]: lane = j + 32*((i/4)%2), register = i%4 + 4*(i/8)
    float *dst = a.ws + ((int64_t)blockIdx.x * a.maxspan + (t - first_tile)) * (kBM * kBN);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      dst[m * kBN + wn * 32 + (lane & 31)] = acc[r];
    }
    it += nseg;
  }
}

// Forward GEMM for formats of <= 16 bits with W decoded straight into MFMA
// B-operand registers (no LDS round trip).  Inside a 64-deep k stage the
// MFMA k slot h of step t stands for k = k0 + 32h + t, so lane (j, h) of a
// wave reads 32 consecutive weights of its own row n0 + j (one to four
// 16-byte chunks) and only the x tile goes through LDS, shared by the block's
// four waves.  Wave w computes rows m0..m0+32*MT of output columns
// n0+32w..n0+32w+31 (MT accumulators sharing each decoded B value); the block
// tile is 32*MT x 128.  Stream-K over (tile, stage) like gemm_sk_kernel, with
// the next stage's x and weight words loaded while the current MFMAs run.
constexpr int kRegBN = 128;

template <int F, int MT>
__global__ void __launch_bounds__(256) gemm_reg_kernel(GemmArgs a) {
  using I = FI<F>;
  constexpr int E = I::kE, W = I::kW;
  constexpr int BM = 32 * MT;
  constexpr int NCH = 32 / E;          // chunks per lane per stage
  constexpr int A4 = BM * kBK / 4 / 256;  // float4 of x per thread per stage
  __shared__ float Xs[2][kBK][BM + kPad];
  __shared__ float lut_s[I::kTable];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;
  if constexpr (I::kLut) fill_table<F>(lut_s, a.lut, tid, 256);
  __syncthreads();
  const int T = a.gx * a.gy * a.nst;
  int it = blockIdx.x * a.per_block;
  const int it_end = min(T, it + a.per_block);
  const int first_tile = it / a.nst;
  const bool vec = (a.K & 3) == 0;
  uint32_t wr[NCH][W];
  float xa[A4][4];
  auto load_stage = [&](int m0, int n0, int k0) {
    const int row = n0 + wave * 32 + j;
    const int kk = k0 + 32 * h;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int k = kk + c * E;
      if (row < a.N && k < a.K)
        load_words<W>(a.body + (int64_t)row * a.row_bytes + (int64_t)(k / E) * (W * 4), wr[c]);
      else {
#pragma unroll
        for (int i = 0; i < W; ++i) wr[c][i] = 0;
      }
    }
#pragma unroll
    for (int i = 0; i < A4; ++i) {
      const int q = tid + i * 256, m = q / (kBK / 4), k = k0 + 4 * (q % (kBK / 4)), mg = m0 + m;
      const float *src = a.A + (int64_t)mg * a.K + k;
      if (mg < a.M && vec && k + 3 < a.K) {
        const float4 v = *(const float4 *)src;
        xa[i][0] = v.x; xa[i][1] = v.y; xa[i][2] = v.z; xa[i][3] = v.w;
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) xa[i][t] = (mg < a.M && k + t < a.K) ? src[t] : 0.0f;
      }
    }
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A4; ++i) {
      const int q = tid + i * 256, m = q / (kBK / 4), kl = 4 * (q % (kBK / 4));
#pragma unroll
      for (int t = 0; t < 4; ++t) Xs[buf][kl + t][m] = xa[i][t];
    }
  };
  while (it < it_end) {
    const int t = it / a.nst, s0 = it % a.nst;
    const int nseg = min(it_end, (t + 1) * a.nst) - it;
    const int m0 = (t / a.gx) * BM, n0 = (t % a.gx) * kRegBN;
    floatx16 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mt][i] = 0.0f;
    load_stage(m0, n0, s0 * kBK);
    store_x(0);
    __syncthreads();
    for (int s = 0; s < nseg; ++s) {
      const int cur = s & 1;
      const int k0 = (s0 + s) * kBK;
      float bv[32];
      const bool live = n0 + wave * 32 + j < a.N;
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const bool ok = live && k0 + 32 * h + c * E < a.K;
          bv[c * E + e] = ok ? (float)chunk_value<F>(wr[c], e, lut_s, a.scale, a.minv) : 0.0f;
        }
      if (s + 1 < nseg) load_stage(m0, n0, k0 + kBK);
#pragma unroll
      for (int tt = 0; tt < 32; ++tt) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const float av = Xs[cur][32 * h + tt][mt * 32 + j];
          acc[mt] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv[tt], acc[mt], 0, 0, 0);
        }
      }
      if (s + 1 < nseg) store_x(cur ^ 1);
      __syncthreads();
    }
    float *dst = a.ws + ((int64_t)blockIdx.x * a.maxspan + (t - first_tile)) * (BM * kRegBN);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        dst[m * kRegBN + wave * 32 + j] = acc[mt][r];
      }
    it += nseg;
  }
}

// Small-batch forward GEMM without a k split across workgroups (batch <= 16,
// K <= 2048) on the fp32 MFMA 16x16x4: weights decoded straight into
// B-operand registers and x read from L2 straight into A-operand registers.
// Lane (j, h) of a wave supplies row j of both operands (x row m0 + j, W row
// n0 + j) for k slot h: its KR consecutive k of each stage, so MFMA step t
// covers k = k0 + KR*h + t.  A wave owns a 16 x 16 output tile and walks
// stages g, g + KG, ... (g = its wave group); the KG partial tiles are added
// in f64, in group order, through LDS, and the epilogue (bias + activation,
// pre and post) runs here: no partial tiles in memory, no reduction launch.
// Loads are straight-line from clamped in-range addresses; values past K, N
// or M are zeroed after decode.
template <int F>
struct RegrShape {
  static constexpr int E = FI<F>::kE;
  static constexpr int KR = E >= 8 ? 32 : 4 * E;  // k per lane per stage
  static constexpr int NCH = KR / E;               // chunk loads per lane per stage
  static constexpr int ST = 4 * KR;                // k per stage
};

template <int F, int KG>
__global__ void __launch_bounds__(64 * KG) gemm_regr_kernel(GemmArgs a, const double *bias, int bias_len,
                                                            int act, float *pre, float *post) {
  using I = FI<F>;
  using S = RegrShape<F>;
  constexpr int E = S::E, W = I::kW, KR = S::KR, NCH = S::NCH, ST = S::ST;
  typedef float floatx4 __attribute__((ext_vector_type(4)));
  __shared__ __align__(16) float lut_s[I::kTable];
  __shared__ float ex[KG - 1][4][64];
  const int tid = threadIdx.x, lane = tid & 63, g = tid >> 6;
  const int j = lane & 15, h = lane >> 4;
  const int n0 = blockIdx.x * 16, m0 = blockIdx.y * 16;
  TabCopy<F> tab;
  if constexpr (I::kLut) {
    tab.load(a.lut, tid);
    __builtin_amdgcn_sched_barrier(0);  // issued before the stage loads
  }
  const int mrow = min(m0 + j, a.M - 1), nrow = min(n0 + j, a.N - 1);
  const bool mlive = m0 + j < a.M, nlive = n0 + j < a.N;
  const float *xr = a.A + (int64_t)mrow * a.K;
  const uint8_t *wr = a.body + (int64_t)nrow * a.row_bytes;
  struct Stage {
    uint32_t w[NCH][W];
    float x[KR];
  };
  auto load = [&](Stage &st, int s) {
    const int k0 = s * ST + KR * h;
#pragma unroll
    for (int q = 0; q < KR; q += 4) {
      const float4 v = *(const float4 *)(xr + min(k0 + q, a.K - 4));
      st.x[q] = v.x; st.x[q + 1] = v.y; st.x[q + 2] = v.z; st.x[q + 3] = v.w;
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      load_words<W>(wr + (int64_t)(min(k0 + c * E, a.K - E) / E) * (W * 4), st.w[c]);
  };
  floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&](const Stage &st, int s) {
    const int k0 = s * ST + KR * h;
    float bv[KR];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const bool ok = nlive && k0 + c * E < a.K;
#pragma unroll
      for (int e = 0; e < E; ++e)
        bv[c * E + e] = ok ? (float)chunk_value<F>(st.w[c], e, lut_s, a.scale, a.minv) : 0.0f;
    }
#pragma unroll
    for (int t = 0; t < KR; ++t) {
      const float xv = (mlive && k0 + (t & ~3) < a.K) ? st.x[t] : 0.0f;
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv, bv[t], acc, 0, 0, 0);
    }
  };
  // stage g first, then the next stage of the group is loaded (clamped to
  // the last stage: in range, unused) while the current one computes
  Stage cur, nxt;
  load(cur, min(g, a.nst - 1));
  if constexpr (I::kLut) {
    tab.store(lut_s, tid);
    lds_barrier();
  }
  for (int s = g; s < a.nst; s += KG) {
    load(nxt, min(s + KG, a.nst - 1));
    compute(cur, s);
    cur = nxt;
  }
  // D[4h + r][j] of the tile: groups 1.. hand theirs to group 0
  if (g > 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) ex[g - 1][r][lane] = acc[r];
  }
  lds_barrier();
  if (g != 0) return;
  const int n = n0 + j;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = m0 + 4 * h + r;
    double sum = (double)acc[r];
#pragma unroll
    for (int q = 0; q < KG - 1; ++q) sum += (double)ex[q][r][lane];
    if (a.post != 1.0f) sum *= (double)a.post;
    if (m < a.M && n < a.N) bias_act_store(sum, n, bias, bias_len, act, pre, post, (int64_t)m * a.N + n);
  }
}

// gemm_regr_kernel with x in LDS, for K <= kRegxMaxK: the workgroup's
// threads copy x [M][K] into LDS once, with contiguous 16-byte loads (1 KB per
// wave load instruction), where gemm_regr_kernel's lanes each read 128
// contiguous bytes of one x row per stage (64 cache lines per load
// instruction: at 1024^2, batch 16, the loads took 2.5 of the kernel's 7 us).
// The weights take a chunk-interleaved k order: chunk c of lane group h in
// stage s holds k = s * ST + (4c + h) * E + e, so one chunk load of the wave
// covers 64 contiguous bytes of each of its 16 rows; x is read from LDS in
// the same order.  The first stage's weight loads are issued before the x
// copy waits, so the two latencies overlap.  Rows of the LDS image past M and
// columns past K are zero.  Dynamic LDS: 16 * (kRegxMaxK + 4) floats.
constexpr int kRegxMaxK = 1024;
template <int F, int KG>
__global__ void __launch_bounds__(64 * KG) gemm_regx_kernel(GemmArgs a, const double *bias, int bias_len,
                                                            int act, float *pre, float *post) {
  using I = FI<F>;
  using S = RegrShape<F>;
  constexpr int E = S::E, W = I::kW, KR = S::KR, NCH = S::NCH, ST = S::ST;
  typedef float floatx4 __attribute__((ext_vector_type(4)));
  __shared__ __align__(16) float lut_s[I::kTable];
  __shared__ float ex[KG - 1][4][64];
  extern __shared__ __align__(16) float xs[];
  const int tid = threadIdx.x, lane = tid & 63, g = tid >> 6;
  const int j = lane & 15, h = lane >> 4;
  const int n0 = blockIdx.x * 16;
  constexpr int xp = kRegxMaxK + 4;  // LDS row pitch (floats); the image is kRegxMaxK wide
  TabCopy<F> tab;
  if constexpr (I::kLut) {
    tab.load(a.lut, tid);
    __builtin_amdgcn_sched_barrier(0);  // issued before the x and weight loads
  }
  // x image [16][kRegxMaxK]: wave g copies rows g * RPW .. + RPW - 1, lane l
  // the float4 columns l, l + 64, ...; loads from clamped in-range addresses,
  // zero past M and K at the LDS store (no branches: every slot is written)
  constexpr int RPW = 16 / KG, CPL = kRegxMaxK / 4 / 64;
  float4 xv[RPW][CPL];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int i = 0; i < CPL; ++i)
      xv[r][i] = *(const float4 *)(a.A + (int64_t)min(g * RPW + r, a.M - 1) * a.K + min(4 * (lane + 64 * i), a.K - 4));
  const int nrow = min(n0 + j, a.N - 1);
  const bool nlive = n0 + j < a.N;
  const uint8_t *wr = a.body + (int64_t)nrow * a.row_bytes;
  const int nchunks = a.K / E;  // whole chunks of a row (K % E == 0 on this route)
  struct Stage {
    uint32_t w[NCH][W];
  };
  auto load = [&](Stage &st, int s) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int ch = min(s * (ST / E) + 4 * c + h, nchunks - 1);
      load_words<W>(wr + (int64_t)ch * (W * 4), st.w[c]);
    }
  };
  Stage first;
  load(first, min(g, a.nst - 1));
  __builtin_amdgcn_sched_barrier(0);  // the x copy below waits for the x loads only
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int row = g * RPW + r, c4 = lane + 64 * i;
      const bool ok = row < a.M && 4 * c4 < a.K;
      *(float4 *)(xs + row * xp + 4 * c4) = ok ? xv[r][i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  if constexpr (I::kLut) tab.store(lut_s, tid);
  lds_barrier();
  floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const float *xrow = xs + j * xp;
  auto compute = [&](const Stage &st, int s) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int k0 = s * ST + (4 * c + h) * E;
      const bool ok = nlive && k0 < a.K;
      float xk[E];
      if constexpr (E >= 4) {
#pragma unroll
        for (int q = 0; q < E; q += 4) {
          const float4 v = *(const float4 *)(xrow + k0 + q);
          xk[q] = v.x; xk[q + 1] = v.y; xk[q + 2] = v.z; xk[q + 3] = v.w;
        }
      } else {
#pragma unroll
        for (int q = 0; q < E; ++q) xk[q] = xrow[k0 + q];
      }
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float bv = ok ? (float)chunk_value<F>(st.w[c], e, lut_s, a.scale, a.minv) : 0.0f;
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xk[e], bv, acc, 0, 0, 0);
      }
    }
  };
  // a stage per wave in flight (one or two stages per wave at K <= 1024):
  // the first was requested with x, the rest are loaded and used in turn
  if (g < a.nst) compute(first, g);
  for (int s = g + KG; s < a.nst; s += KG) {
    Stage st;
    load(st, s);
    compute(st, s);
  }
  // D[4h + r][j] of the tile: groups 1.. hand theirs to group 0
  if (g > 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) ex[g - 1][r][lane] = acc[r];
  }
  lds_barrier();
  if (g != 0) return;
  const int n = n0 + j;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * h + r;
    double sum = (double)acc[r];
#pragma unroll
    for (int q = 0; q < KG - 1; ++q) sum += (double)ex[q][r][lane];
    if (a.post != 1.0f) sum *= (double)a.post;
    if (m < a.M && n < a.N) bias_act_store(sum, n, bias, bias_len, act, pre, post, (int64_t)m * a.N + n);
  }
}

// dX of the fp32-MFMA formats at batch <= 16, rows <= 2048, without a k
// split: dX[b][i] = sum_o dpre[b][o] W[o][i] as gemm_regr_kernel's product
// through W^T.  A wave owns 16 output columns i (n0..n0+15) and walks stages
// of ST rows o of W; per stage its lanes load the 16-column piece of each row
// as whole chunks along the row (the stored layout), decode it once into the
// wave's own LDS tile (row pitch 17 floats: the four k slots of a read fall
// on different banks), and MFMA step t reads B = tile[KR*h + t][j]; A is
// dpre row j from L2 as in the forward.  The KG waves take every KG-th stage;
// their tiles are added in f64 in wave order and stored as fl32.
template <int F>
struct RegtShape {
  static constexpr int E = FI<F>::kE;
  static constexpr int KR = E >= 4 ? 16 : 8;         // rows o per lane per stage
  static constexpr int ST = 4 * KR;                   // rows per stage
  static constexpr int CPR = E >= 16 ? 1 : 16 / E;    // chunks per 16-column row piece
  static constexpr int NCH = ST * CPR / 64;           // chunk loads per lane per stage
  static constexpr int DE = E >= 16 ? 16 : E;         // elements decoded per chunk load
  static constexpr int P = 17;                        // tile row pitch (floats)
  static_assert(ST * CPR % 64 == 0, "whole chunk loads per lane");
};

// NEXT: out is the gy of the layer below in a chain, whose piecewise
// activation's derivative is applied here: out = fl32(dX) * act'(next_pre)
// (act_deriv_kernel's expression on the stored dX, so the same bits), so
// that layer's backward needs no derivative launch.  next_pre is loaded with
// the first stage, off the epilogue's critical path.
// XL: dpre [M][K] is copied into (dynamic) LDS once per workgroup with
// contiguous 16-byte loads, as in gemm_regx_kernel, instead of each lane
// loading its KR rows' values per stage; rows past M and past K are zero.
constexpr int kRegtxMaxK = 1024;
template <int F, int KG, bool NEXT, bool XL = false>
__global__ void __launch_bounds__(64 * KG) gemm_regt_kernel(GemmArgs a, float *out, const float *next_pre,
                                                            int next_act) {
  using I = FI<F>;
  using S = RegtShape<F>;
  constexpr int E = S::E, W = I::kW, KR = S::KR, ST = S::ST, CPR = S::CPR, NCH = S::NCH, DE = S::DE,
                P = S::P;
  typedef float floatx4 __attribute__((ext_vector_type(4)));
  __shared__ __align__(16) float lut_s[I::kTable];
  __shared__ float tile[KG][ST * P];
  __shared__ float ex[KG - 1][4][64];
  const int tid = threadIdx.x, lane = tid & 63, g = tid >> 6;
  const int j = lane & 15, h = lane >> 4;
  const int n0 = blockIdx.x * 16, m0 = blockIdx.y * 16;
  TabCopy<F> tab;
  if constexpr (I::kLut) {
    tab.load(a.lut, tid);
    __builtin_amdgcn_sched_barrier(0);  // issued before the stage loads
  }
  const int mrow = min(m0 + j, a.M - 1);
  const bool mlive = m0 + j < a.M;
  const float *xr = a.A + (int64_t)mrow * a.K;
  extern __shared__ __align__(16) float xs[];
  constexpr int xp = kRegtxMaxK + 4;  // XL: LDS row pitch (floats), image kRegtxMaxK wide
  // XL: wave g copies rows g * RPW .. + RPW - 1 of dpre, lane l the float4
  // columns l, l + 64, ... (as gemm_regx_kernel)
  constexpr int RPW = 16 / KG, CPL = XL ? kRegtxMaxK / 4 / 64 : 1;
  float4 xv4[RPW][CPL];
  if constexpr (XL) {
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int i = 0; i < CPL; ++i)
        xv4[r][i] = *(const float4 *)(a.A + (int64_t)min(m0 + g * RPW + r, a.M - 1) * a.K +
                                      min(4 * (lane + 64 * i), a.K - 4));
  }
  // chunk load c of this lane: row r = q / CPR, chunk cc = q % CPR of the
  // piece (q = lane + 64 c); column chunk index along the stored row
  int lr[NCH], lcol[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int q = lane + 64 * c;
    lr[c] = q / CPR;
    lcol[c] = (q % CPR) * DE;  // first column of the piece this load decodes
  }
  const int64_t chunk_bytes = W * 4;
  struct Stage {
    uint32_t w[NCH][W];
    float x[KR];
  };
  auto load = [&](Stage &st, int s) {
    const int k0 = s * ST;
    if constexpr (!XL) {
#pragma unroll
      for (int q = 0; q < KR; q += 4) {
        const float4 v = *(const float4 *)(xr + min(k0 + KR * h + q, a.K - 4));
        st.x[q] = v.x; st.x[q + 1] = v.y; st.x[q + 2] = v.z; st.x[q + 3] = v.w;
      }
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int o = min(k0 + lr[c], a.K - 1);
      const int col = min(n0 + lcol[c], a.N - DE);
      load_words<W>(a.body + (int64_t)o * a.row_bytes + (int64_t)(col / E) * chunk_bytes, st.w[c]);
    }
  };
  // the decoded piece into this wave's tile; elements past K or N are zero.
  // Sub-byte formats (32 per chunk) decode the half that holds n0..n0+15.
  float *tw = tile[g];
  auto put = [&](const Stage &st, int s) {
    const int k0 = s * ST;
    const bool hi = E == 32 && (n0 & 16);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const bool rok = k0 + lr[c] < a.K;
#pragma unroll
      for (int e = 0; e < DE; ++e) {
        const bool ok = rok && n0 + lcol[c] + e < a.N;
        float v;
        if constexpr (E == 32)
          v = hi ? (float)chunk_value<F>(st.w[c], 16 + e, lut_s, a.scale, a.minv)
                 : (float)chunk_value<F>(st.w[c], e, lut_s, a.scale, a.minv);
        else
          v = (float)chunk_value<F>(st.w[c], e, lut_s, a.scale, a.minv);
        tw[lr[c] * P + lcol[c] + e] = ok ? v : 0.0f;
      }
    }
  };
  floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&](const Stage &st, int s) {
    const int k0 = s * ST + KR * h;
    float xl[KR];
    if constexpr (XL) {
#pragma unroll
      for (int q = 0; q < KR; q += 4) {
        const float4 v = *(const float4 *)(xs + j * xp + k0 + q);
        xl[q] = v.x; xl[q + 1] = v.y; xl[q + 2] = v.z; xl[q + 3] = v.w;
      }
    }
#pragma unroll
    for (int t = 0; t < KR; ++t) {
      float xv;
      if constexpr (XL) xv = xl[t];
      else xv = (mlive && k0 + (t & ~3) < a.K) ? st.x[t] : 0.0f;
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv, tw[(KR * h + t) * P + j], acc, 0, 0, 0);
    }
  };
  Stage cur, nxt;
  load(cur, min(g, a.nst - 1));
  if constexpr (XL) {
    __builtin_amdgcn_sched_barrier(0);  // the copy below waits for the dpre loads only
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int row = g * RPW + r, c4 = lane + 64 * i;
        const bool ok = m0 + row < a.M && 4 * c4 < a.K;
        *(float4 *)(xs + row * xp + 4 * c4) = ok ? xv4[r][i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    if constexpr (!I::kLut) lds_barrier();
  }
  float np[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (NEXT) {
    if (g == 0) {  // the storing wave's four outputs, clamped in range
#pragma unroll
      for (int r = 0; r < 4; ++r)
        np[r] = next_pre[(int64_t)min(m0 + 4 * h + r, a.M - 1) * a.N + min(n0 + j, a.N - 1)];
    }
  }
  if constexpr (I::kLut) {
    tab.store(lut_s, tid);
    lds_barrier();
  }
  // LDS operations of one wave complete in order: the previous stage's tile
  // reads are done before the next writes, and the writes before the reads;
  // the clobbers keep the compiler from reordering them
  if constexpr (XL) {
    // dpre in LDS: a stage per wave in flight (the first requested with
    // dpre), the rest loaded and used in turn
    if (g < a.nst) {
      asm volatile("" ::: "memory");
      put(cur, g);
      asm volatile("" ::: "memory");
      compute(cur, g);
      asm volatile("" ::: "memory");
    }
    for (int s = g + KG; s < a.nst; s += KG) {
      load(nxt, s);
      asm volatile("" ::: "memory");
      put(nxt, s);
      asm volatile("" ::: "memory");
      compute(nxt, s);
      asm volatile("" ::: "memory");
    }
  } else {
    for (int s = g; s < a.nst; s += KG) {
      load(nxt, min(s + KG, a.nst - 1));
      asm volatile("" ::: "memory");
      put(cur, s);
      asm volatile("" ::: "memory");
      compute(cur, s);
      asm volatile("" ::: "memory");
      cur = nxt;
    }
  }
  if (g > 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) ex[g - 1][r][lane] = acc[r];
  }
  lds_barrier();
  if (g != 0) return;
  const int n = n0 + j;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = m0 + 4 * h + r;
    double sum = (double)acc[r];
#pragma unroll
    for (int q = 0; q < KG - 1; ++q) sum += (double)ex[q][r][lane];
    if (a.post != 1.0f) sum *= (double)a.post;
    float v = (float)sum;
    if constexpr (NEXT) v = v * act_prime_piecewise(np[r], next_act);
    if (m < a.M && n < a.N) out[(int64_t)m * a.N + n] = v;
  }
}

// ------------------------------------------------------ split-x bf16 GEMM
// For formats whose decoded weights are exact in bf16 once the per-tensor
// scale is factored out (FP8 E4M3 from the decode-ready copy, Int8 codes),
// the fp32 product runs on the bf16 MFMA: each x is split exactly into three
// bf16 parts (8 + 8 + 8 significand bits, by truncation: x = hi + mid + lo
// with no rounding), so every product w * x_part is exact and the MFMA
// accumulates in fp32 — an fp32 GEMM whose products are formed exactly, at
// three bf16 MFMAs per fp32 one (bf16 dense rate is 16x the fp32 rate).
//
// C[m][n] = sum_k x[m][k] W[n][k]: MFMA 32x32x16 bf16 with A = x parts from
// LDS and B = W decoded into registers.  Block = 4 waves x NC column tiles
// of 32 = 128*NC output columns, 32*MT batch rows; 64-deep k stages; lane (i, h)
// of a wave reads 32 consecutive weights k0 + 32h .. + 31 of its row, and
// MFMA step t uses bytes 8t .. 8t + 7 of them (k = k0 + 32h + 8t + j), so x
// parts are read from LDS in the same permuted order.  Stream-K over (tile,
// stage) like gemm_reg_kernel; partial tiles are added by sk_reduce_kernel.
constexpr int kBf3Row = kBK + 8;  // bf16 per LDS row: 144 B keeps 16-lane reads conflict-free

typedef short shortx8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Weight kinds the split-x GEMM takes.  Every decoded weight is exact in
// bf16 once the per-tensor scale (applied by the reduction) is factored out:
// E4M3 and E5M2 from the decode-ready copy, Int8 and FP4 codes as they are,
// and NF4 table values as three exact bf16 parts (hi + mid + lo, like x).
enum Bf3Kind { BK_E4 = 0, BK_I8 = 1, BK_FP4 = 2, BK_NF4 = 3, BK_E5 = 4 };

template <int BK>
struct B3 {
  static constexpr int kBits = (BK <= BK_I8 || BK == BK_E5) ? 8 : 4;
  static constexpr int kWords = kBits;  // words of a lane's 32 weights per stage
  static constexpr int kParts = BK == BK_NF4 ? 3 : 1;
};

typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

inline __device__ bf16x8 bf16x8_of(const uint32_t (&u)[4]) {
  bf16x8 r;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const bf16x2v p = __builtin_bit_cast(bf16x2v, u[q]);
    r[2 * q] = p[0];
    r[2 * q + 1] = p[1];
  }
  return r;
}

// 8 consecutive weights (the words of MFMA step q) as B operands: parts[0..P).
// NF4 reads the split table t3[code] = {hi | mid << 16, lo}.
template <int BK>
__device__ inline void bf3_weights(const uint32_t *w, int q, const uint2 *t3, bf16x8 (&parts)[B3<BK>::kParts]) {
  if constexpr (BK == BK_E4) {
    const uint32_t w0 = w[2 * q], w1 = w[2 * q + 1];
    const uint32_t u[4] = {
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false)),
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true)),
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false)),
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true))};
    parts[0] = bf16x8_of(u);
  } else if constexpr (BK == BK_E5) {
    const uint32_t w0 = w[2 * q], w1 = w[2 * q + 1];
    const uint32_t u[4] = {
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w0, 1.0f, false)),
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w0, 1.0f, true)),
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w1, 1.0f, false)),
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w1, 1.0f, true))};
    parts[0] = bf16x8_of(u);
  } else if constexpr (BK == BK_I8) {
    uint32_t u[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t wd = w[2 * q + (i >> 1)];
      const int sh = (i & 1) * 16;
      const float lo = (float)(int8_t)(uint8_t)(wd >> sh), hi = (float)(int8_t)(uint8_t)(wd >> (sh + 8));
      u[i] = __builtin_amdgcn_perm(f2u(hi), f2u(lo), 0x07060302u);
    }
    parts[0] = bf16x8_of(u);
  } else if constexpr (BK == BK_FP4) {
    const uint32_t wd = w[q];
    const uint32_t u[4] = {
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, 1.0f, 0)),
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, 1.0f, 1)),
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, 1.0f, 2)),
        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, 1.0f, 3))};
    parts[0] = bf16x8_of(u);
  } else {  // NF4
    const uint32_t wd = w[q];
    uint32_t hi[4], mid[4], lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint2 e0 = t3[(wd >> (8 * i)) & 15u], e1 = t3[(wd >> (8 * i + 4)) & 15u];
      hi[i] = __builtin_amdgcn_perm(e1.x, e0.x, 0x05040100u);
      mid[i] = __builtin_amdgcn_perm(e1.x, e0.x, 0x07060302u);
      lo[i] = __builtin_amdgcn_perm(e1.y, e0.y, 0x05040100u);
    }
    parts[0] = bf16x8_of(hi);
    parts[1] = bf16x8_of(mid);
    parts[2] = bf16x8_of(lo);
  }
}

template <int BK, int MT, int D, int NC>
__global__ void __launch_bounds__(256) gemm_bf3_kernel(GemmArgs a) {
  using K3 = B3<BK>;
  constexpr int BM = 32 * MT, BN = 128 * NC, NW = K3::kWords, NP = K3::kParts;
  constexpr int XE = BM * kBK / 256;  // x values per thread per stage (8 or 16)
  constexpr int XT = kBK / XE;        // threads per x row
  __shared__ uint16_t Xs[2][3][BM][kBf3Row];
  __shared__ uint2 t3[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;
  if constexpr (BK == BK_NF4) {
    if (tid < 16) {  // NF4 table values split exactly into three bf16 parts
      const float t = kNf4Tab[tid];
      const uint32_t hi = f2u(t) & 0xffff0000u;
      const float r = t - u2f(hi);
      const uint32_t mid = f2u(r) & 0xffff0000u;
      const uint32_t lo = f2u(r - u2f(mid));
      t3[tid] = make_uint2((hi >> 16) | mid, lo >> 16);
    }
  }
  const int T = a.gx * a.gy * a.nst;
  int it = blockIdx.x * a.per_block;
  const int it_end = min(T, it + a.per_block);
  const int first_tile = it / a.nst;
  // thread's x piece of a stage: row xm, k offset xk .. xk + XE - 1 (K is a
  // multiple of 16, so a piece lies wholly inside or outside the row)
  const int xm = tid / XT, xk = (tid % XT) * XE;
  uint32_t wr[D][NC][NW];  // weights of units u .. u + D - 1 (ring slot = unit offset mod D)
  float xf[D][XE];         // x of the same units
  // unit u of the block's share = (tile u / nst, stage u % nst)
  auto unit_m0 = [&](int u) { return (u / a.nst / a.gx) * BM; };
  auto unit_n0 = [&](int u) { return (u / a.nst % a.gx) * BN; };
  auto load_w = [&](int u, uint32_t (&w)[NC][NW]) {
    const int n0 = unit_n0(u), k0 = (u % a.nst) * kBK;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int row = min(n0 + wave * 32 * NC + c * 32 + j, a.N - 1);
      const uint8_t *src = a.body + (int64_t)row * a.row_bytes + (k0 + 32 * h) * K3::kBits / 8;
#pragma unroll
      for (int i = 0; i < NW; i += 4) {
        const uint4 v = *(const uint4 *)(src + 4 * i);
        w[c][i] = v.x; w[c][i + 1] = v.y; w[c][i + 2] = v.z; w[c][i + 3] = v.w;
      }
    }
  };
  // raw loads: a value is masked where it is stored, so the load's latency
  // is not exposed here
  uint32_t xin[D];         // ~0 when the slot's x piece lies inside x, else 0
  auto load_x = [&](int u, float (&xf)[XE], uint32_t &in_mask) {
    const int m0 = unit_m0(u), k0 = (u % a.nst) * kBK;
    const bool in = m0 + xm < a.M && k0 + xk < a.K;
    in_mask = in ? ~0u : 0u;
    const float *src = a.A + (int64_t)(in ? m0 + xm : 0) * a.K + (in ? k0 + xk : 0);
#pragma unroll
    for (int i = 0; i < XE; i += 4) {
      const float4 v = *(const float4 *)(src + i);
      xf[i] = v.x;
      xf[i + 1] = v.y;
      xf[i + 2] = v.z;
      xf[i + 3] = v.w;
    }
  };
  // x = hi + mid + lo exactly: truncations to the top 8 significand bits,
  // remainders exact in f32; an infinite x keeps its value in hi (the
  // remainders are zero), a NaN carries NaN into the remainders (its hi can
  // read as an infinity when the payload sits in the low 16 bits)
  auto store_x = [&](int buf, const float (&xf)[XE], uint32_t in_mask) {
    uint32_t wp[3][XE / 2];
#pragma unroll
    for (int i = 0; i < XE; i += 2) {
      uint32_t part[3][2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float v = u2f(f2u(xf[i + e]) & in_mask);
        const uint32_t hi = f2u(v) & 0xffff0000u;
        const float r = isinf(v) ? 0.0f : v - u2f(hi);
        const uint32_t mid = f2u(r) & 0xffff0000u;
        part[0][e] = hi;
        part[1][e] = mid;
        part[2][e] = f2u(r - u2f(mid));
      }
#pragma unroll
      for (int p = 0; p < 3; ++p) wp[p][i / 2] = __builtin_amdgcn_perm(part[p][1], part[p][0], 0x07060302u);
    }
#pragma unroll
    for (int p = 0; p < 3; ++p)
#pragma unroll
      for (int q = 0; q < XE / 8; ++q)
        *(uint4 *)&Xs[buf][p][xm][xk + 8 * q] =
            make_uint4(wp[p][4 * q], wp[p][4 * q + 1], wp[p][4 * q + 2], wp[p][4 * q + 3]);
  };
  // One MFMA step: products of x part p with weight part wp for p + wp <= 2
  // (the dropped NF4 terms are below 2^-23 of each product).
  auto mfma_step = [&](floatx16 (&acc)[MT][NC], int buf, int q, const bf16x8 (&bv)[NC][NP]) {
#pragma unroll
    for (int p = 0; p < 3; ++p) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const bf16x8 av = __builtin_bit_cast(bf16x8, *(const shortx8 *)&Xs[buf][p][mt * 32 + j][32 * h + 8 * q]);
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int wp = 0; wp < NP; ++wp)
            if (p + wp <= 2)
              acc[mt][c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv[c][wp], acc[mt][c], 0, 0, 0);
      }
    }
  };
  // The block's units run as one stream across tile boundaries: unit u
  // takes ring slot (u - it) mod D, whose weights and x were loaded D units
  // earlier; the slot is refilled with unit u + D once unit u's weights are
  // decoded (its x went to LDS one unit earlier).  A tile's partial sum is
  // written after its last unit here.  Rows past N read row N - 1 (finite
  // codes) and their columns are never stored.
  floatx16 acc[MT][NC];
  int buf = 0;
  // loads past the share re-read its last unit (valid addresses, unused
  // data): unconditional loads keep the wait counts static
  const int last = max(it, it_end - 1);
#pragma unroll
  for (int d = 0; d < D; ++d) {
    load_w(min(it + d, last), wr[d]);
    load_x(min(it + d, last), xf[d], xin[d]);
  }
  store_x(0, xf[0], xin[0]);
  __syncthreads();
  for (int u0 = it; u0 < it_end; u0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int u = u0 + d;
      if (u >= it_end) break;
      const int t = u / a.nst, st = u - t * a.nst;
      if (u == it || st == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mt][c][i] = 0.0f;
      }
      if constexpr (NP == 1) {
        // decode the unit's weights, refill the slot, then the MFMAs
        bf16x8 bv[4][NC][1];
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            bf16x8 pp[1];
            bf3_weights<BK>(wr[d][c], q, t3, pp);
            bv[q][c][0] = pp[0];
          }
        load_w(min(u + D, last), wr[d]);
        load_x(min(u + D, last), xf[d], xin[d]);
#pragma unroll
        for (int q = 0; q < 4; ++q) mfma_step(acc, buf, q, bv[q]);
      } else {
        // three weight parts: decode step by step, refill the slot afterwards
        load_x(min(u + D, last), xf[d], xin[d]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          bf16x8 bv[NC][NP];
#pragma unroll
          for (int c = 0; c < NC; ++c) bf3_weights<BK>(wr[d][c], q, t3, bv[c]);
          mfma_step(acc, buf, q, bv);
        }
        load_w(min(u + D, last), wr[d]);
      }
      store_x(buf ^ 1, xf[(d + 1) % D], xin[(d + 1) % D]);
      __syncthreads();
      buf ^= 1;
      if (st == a.nst - 1 || u + 1 == it_end) {
        // D[m][n]: lane (j, h) holds column j, rows 8*(r/4) + 4*h + r%4.
        // Groups of 8 rows wholly past M are never read by the reduction:
        // not stored (a wave-uniform test)
        float *dst = a.ws + ((int64_t)blockIdx.x * a.maxspan + (t - first_tile)) * (BM * BN);
        const int mrows = a.M - unit_m0(u);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int m = mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
              if (mt * 32 + 8 * (r >> 2) < mrows) dst[m * BN + wave * 32 * NC + c * 32 + j] = acc[mt][c][r];
            }
      }
    }
  }
}

// gemm_bf3_kernel with two wave groups per workgroup sharing the k range of
// each unit: a unit is (tile, stage pair p), and group g (waves 4g .. 4g + 3,
// the same per-wave tiles as gemm_bf3_kernel) runs stage 2p + g.  At the
// last unit of a tile in the share the groups add their accumulators through
// LDS (the x buffers, idle at that point; group 0's sum + group 1's in fp32)
// and each writes half of the one partial tile.  One workgroup per CU keeps
// two waves per SIMD, like two 4-wave workgroups per CU, while a launch
// writes half the partial tiles.  GemmArgs::nst counts stage pairs here.
template <int BK, int MT, int D, int NC>
__global__ void __launch_bounds__(512) gemm_bf3k_kernel(GemmArgs a) {
  using K3 = B3<BK>;
  constexpr int BM = 32 * MT, BN = 128 * NC, NW = K3::kWords, NP = K3::kParts;
  constexpr int XE = BM * kBK / 256;  // x values per thread per stage (8 or 16)
  constexpr int XT = kBK / XE;        // threads per x row
  constexpr int P = MT * NC;          // 32 x 32 accumulator pieces per wave
  static_assert(P % 2 == 0, "the pieces are shared out between the two groups");
  __shared__ uint16_t Xs[2][2][3][BM][kBf3Row];  // [buffer][group][part][m][k]
  static_assert(sizeof(Xs) >= (size_t)P * 16 * 256 * sizeof(float), "the exchange fits the x buffers");
  __shared__ uint2 t3[16];
  const int tid = threadIdx.x, grp = tid >> 8, gt = tid & 255, lane = tid & 63, wave = gt >> 6;
  const int j = lane & 31, h = lane >> 5;
  if constexpr (BK == BK_NF4) {
    if (tid < 16) {  // NF4 table values split exactly into three bf16 parts
      const float t = kNf4Tab[tid];
      const uint32_t hi = f2u(t) & 0xffff0000u;
      const float r = t - u2f(hi);
      const uint32_t mid = f2u(r) & 0xffff0000u;
      const uint32_t lo = f2u(r - u2f(mid));
      t3[tid] = make_uint2((hi >> 16) | mid, lo >> 16);
    }
  }
  const int T = a.gx * a.gy * a.nst;
  const int it = blockIdx.x * a.per_block;
  const int it_end = min(T, it + a.per_block);
  const int first_tile = it / a.nst;
  const int xm = gt / XT, xk = (gt % XT) * XE;
  uint32_t wr[D][NC][NW];
  float xf[D][XE];
  uint32_t xin[D];
  auto unit_m0 = [&](int u) { return (u / a.nst / a.gx) * BM; };
  auto unit_n0 = [&](int u) { return (u / a.nst % a.gx) * BN; };
  auto unit_k0 = [&](int u) { return (2 * (u % a.nst) + grp) * kBK; };
  auto load_w = [&](int u, uint32_t (&w)[NC][NW]) {
    const int n0 = unit_n0(u), k0 = unit_k0(u);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int row = min(n0 + wave * 32 * NC + c * 32 + j, a.N - 1);
      const uint8_t *src = a.body + (int64_t)row * a.row_bytes + (k0 + 32 * h) * K3::kBits / 8;
#pragma unroll
      for (int i = 0; i < NW; i += 4) {
        const uint4 v = *(const uint4 *)(src + 4 * i);
        w[c][i] = v.x; w[c][i + 1] = v.y; w[c][i + 2] = v.z; w[c][i + 3] = v.w;
      }
    }
  };
  auto load_x = [&](int u, float (&xf)[XE], uint32_t &in_mask) {
    const int m0 = unit_m0(u), k0 = unit_k0(u);
    const bool in = m0 + xm < a.M && k0 + xk < a.K;
    in_mask = in ? ~0u : 0u;
    const float *src = a.A + (int64_t)(in ? m0 + xm : 0) * a.K + (in ? k0 + xk : 0);
#pragma unroll
    for (int i = 0; i < XE; i += 4) {
      const float4 v = *(const float4 *)(src + i);
      xf[i] = v.x;
      xf[i + 1] = v.y;
      xf[i + 2] = v.z;
      xf[i + 3] = v.w;
    }
  };
  auto store_x = [&](int buf, const float (&xf)[XE], uint32_t in_mask) {
    uint32_t wp[3][XE / 2];
#pragma unroll
    for (int i = 0; i < XE; i += 2) {
      uint32_t part[3][2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float v = u2f(f2u(xf[i + e]) & in_mask);
        const uint32_t hi = f2u(v) & 0xffff0000u;
        const float r = isinf(v) ? 0.0f : v - u2f(hi);
        const uint32_t mid = f2u(r) & 0xffff0000u;
        part[0][e] = hi;
        part[1][e] = mid;
        part[2][e] = f2u(r - u2f(mid));
      }
#pragma unroll
      for (int p = 0; p < 3; ++p) wp[p][i / 2] = __builtin_amdgcn_perm(part[p][1], part[p][0], 0x07060302u);
    }
#pragma unroll
    for (int p = 0; p < 3; ++p)
#pragma unroll
      for (int q = 0; q < XE / 8; ++q)
        *(uint4 *)&Xs[buf][grp][p][xm][xk + 8 * q] =
            make_uint4(wp[p][4 * q], wp[p][4 * q + 1], wp[p][4 * q + 2], wp[p][4 * q + 3]);
  };
  auto mfma_step = [&](floatx16 (&acc)[MT][NC], int buf, int q, const bf16x8 (&bv)[NC][NP]) {
#pragma unroll
    for (int p = 0; p < 3; ++p) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const bf16x8 av =
            __builtin_bit_cast(bf16x8, *(const shortx8 *)&Xs[buf][grp][p][mt * 32 + j][32 * h + 8 * q]);
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int wp = 0; wp < NP; ++wp)
            if (p + wp <= 2)
              acc[mt][c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv[c][wp], acc[mt][c], 0, 0, 0);
      }
    }
  };
  floatx16 acc[MT][NC];
  int buf = 0;
  const int last = max(it, it_end - 1);
  // the first unit's loads go out alone: every workgroup asks at once, and
  // the later units' requests would queue in front of them
  load_x(it, xf[0], xin[0]);
  load_w(it, wr[0]);
  store_x(0, xf[0], xin[0]);
  lds_barrier();
#pragma unroll
  for (int d = 1; d < D; ++d) {
    load_x(min(it + d, last), xf[d], xin[d]);
    __builtin_amdgcn_sched_barrier(0);  // x before w, as in the loop (wait counts)
    load_w(min(it + d, last), wr[d]);
  }
  float *xch = reinterpret_cast<float *>(&Xs[0][0][0][0][0]);
  for (int u0 = it; u0 < it_end; u0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int u = u0 + d;
      // leaving the whole loop (not just this unrolled step) keeps the
      // compiler's wait counts for the ring exact: no path runs a step twice
      if (u >= it_end) goto done;
      const int t = u / a.nst, st = u - t * a.nst;
      const bool tile_end = st == a.nst - 1 || u + 1 == it_end;
      // with the ring two units deep, group 1 stages the next unit's x
      // before its MFMAs and group 0 after them, so the two waves of a SIMD
      // overlap one's x split with the other's MFMAs (both after the tile's
      // end, where the exchange takes the x buffers first, and on the first
      // unit, whose successor's x was only just requested)
      const bool early = D >= 2 && grp == 1 && !tile_end && u != it;
      if (early) store_x(buf ^ 1, xf[(d + 1) % D], xin[(d + 1) % D]);
      if (u == it || st == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mt][c][i] = 0.0f;
      }
      if constexpr (NP == 1) {
        bf16x8 bv[4][NC][1];
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            bf16x8 pp[1];
            bf3_weights<BK>(wr[d][c], q, t3, pp);
            bv[q][c][0] = pp[0];
          }
        load_x(min(u + D, last), xf[d], xin[d]);  // first: the early x store waits for it alone
        load_w(min(u + D, last), wr[d]);
#pragma unroll
        for (int q = 0; q < 4; ++q) mfma_step(acc, buf, q, bv[q]);
      } else {
        load_x(min(u + D, last), xf[d], xin[d]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          bf16x8 bv[NC][NP];
#pragma unroll
          for (int c = 0; c < NC; ++c) bf3_weights<BK>(wr[d][c], q, t3, bv[c]);
          mfma_step(acc, buf, q, bv);
        }
        load_w(min(u + D, last), wr[d]);
      }
      if (tile_end) {
        // piece pc = mt * NC + c: group 0 keeps pieces 0 .. P/2 - 1, group 1
        // the rest; each group leaves the other's pieces in region grp of the
        // exchange, lane-major (same wave index and lane = same outputs)
        lds_barrier();  // every wave is done reading x from LDS
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const int pc = mt * NC + c;
            if ((pc < P / 2) != (grp == 0)) {
              float *dst = xch + (size_t)(grp * (P / 2) + pc % (P / 2)) * 16 * 256 + gt;
#pragma unroll
              for (int r = 0; r < 16; ++r) dst[r * 256] = acc[mt][c][r];
            }
          }
        lds_barrier();
        float *dst = a.ws + ((int64_t)blockIdx.x * a.maxspan + (t - first_tile)) * (BM * BN);
        const int mrows = a.M - unit_m0(u);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const int pc = mt * NC + c;
            if ((pc < P / 2) == (grp == 0)) {
              const float *src = xch + (size_t)((1 - grp) * (P / 2) + pc % (P / 2)) * 16 * 256 + gt;
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                const float v = acc[mt][c][r] + src[r * 256];
                const int m = mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (mt * 32 + 8 * (r >> 2) < mrows) dst[m * BN + wave * 32 * NC + c * 32 + j] = v;
              }
            }
          }
        lds_barrier();  // the exchange is read before x goes back into the buffers
      }
      if (!early) store_x(buf ^ 1, xf[(d + 1) % D], xin[(d + 1) % D]);
      // every wave has now stored the next unit's x, early or late; a use
      // on both paths lets the compiler see that, so it does not wait for
      // those loads again where the slot's registers are reused
#pragma unroll
      for (int i = 0; i < XE; ++i) asm volatile("" ::"v"(xf[(d + 1) % D][i]));
      lds_barrier();
      buf ^= 1;
    }
  }
done:;
}

typedef float floatx4 __attribute__((ext_vector_type(4)));

// The split-x GEMM for batch <= 16: one 16-row tile on
// v_mfma_f32_16x16x32_bf16, where the 32-row MFMA would spend three quarters
// of its work on padding rows at batch 8.  Same units, stream-K shares, x
// split and weight decode as gemm_bf3_kernel; per stage a lane (j = lane % 16,
// g = lane / 16) holds for each 16-column group the 16 consecutive weights
// k = 16 g .. 16 g + 15 of column j, and MFMA step q in {0, 1} takes
// k = 16 g + 8 q + i (i < 8) from both operands: a permutation of the stage's
// k order, the same on both sides.  D lane (j, g) holds column j, rows
// 4 g .. 4 g + 3.
template <int BK, int D, int NC>
__global__ void __launch_bounds__(256) gemm_bf3s_kernel(GemmArgs a) {
  using K3 = B3<BK>;
  constexpr int BM = 16, BN = 128 * NC, NW = K3::kWords / 2, NP = K3::kParts;
  constexpr int CG = 2 * NC;          // 16-column groups per wave
  constexpr int XE = BM * kBK / 256;  // 4 x values per thread per stage
  constexpr int XT = kBK / XE;        // 16 threads per x row
  static_assert(XE == 4 && (NW == 2 || NW == 4), "16-row split-x layout");
  __shared__ uint16_t Xs[2][3][BM][kBf3Row];
  __shared__ uint2 t3[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 15, g = lane >> 4;
  if constexpr (BK == BK_NF4) {
    if (tid < 16) {
      const float t = kNf4Tab[tid];
      const uint32_t hi = f2u(t) & 0xffff0000u;
      const float r = t - u2f(hi);
      const uint32_t mid = f2u(r) & 0xffff0000u;
      const uint32_t lo = f2u(r - u2f(mid));
      t3[tid] = make_uint2((hi >> 16) | mid, lo >> 16);
    }
  }
  const int T = a.gx * a.gy * a.nst;
  int it = blockIdx.x * a.per_block;
  const int it_end = min(T, it + a.per_block);
  const int first_tile = it / a.nst;
  const int xm = tid / XT, xk = (tid % XT) * XE;  // xm < 16, xk < 64
  uint32_t wr[D][CG][NW];
  float xf[D][XE];
  uint32_t xin[D];
  auto unit_m0 = [&](int u) { return (u / a.nst / a.gx) * BM; };
  auto unit_n0 = [&](int u) { return (u / a.nst % a.gx) * BN; };
  auto load_w = [&](int u, uint32_t (&w)[CG][NW]) {
    const int n0 = unit_n0(u), k0 = (u % a.nst) * kBK;
#pragma unroll
    for (int c = 0; c < CG; ++c) {
      const int row = min(n0 + wave * 32 * NC + c * 16 + j, a.N - 1);
      const uint8_t *src = a.body + (int64_t)row * a.row_bytes + (k0 + 16 * g) * K3::kBits / 8;
      if constexpr (NW == 4) {
        const uint4 v = *(const uint4 *)src;
        w[c][0] = v.x; w[c][1] = v.y; w[c][2] = v.z; w[c][3] = v.w;
      } else {
        const uint2 v = *(const uint2 *)src;
        w[c][0] = v.x; w[c][1] = v.y;
      }
    }
  };
  auto load_x = [&](int u, float (&xv)[XE], uint32_t &in_mask) {
    const int m0 = unit_m0(u), k0 = (u % a.nst) * kBK;
    const bool in = m0 + xm < a.M && k0 + xk < a.K;
    in_mask = in ? ~0u : 0u;
    const float4 v = *(const float4 *)(a.A + (int64_t)(in ? m0 + xm : 0) * a.K + (in ? k0 + xk : 0));
    xv[0] = v.x; xv[1] = v.y; xv[2] = v.z; xv[3] = v.w;
  };
  auto store_x = [&](int buf, const float (&xv)[XE], uint32_t in_mask) {
    uint32_t wp[3][2];
#pragma unroll
    for (int i = 0; i < XE; i += 2) {
      uint32_t part[3][2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float v = u2f(f2u(xv[i + e]) & in_mask);
        const uint32_t hi = f2u(v) & 0xffff0000u;
        const float r = isinf(v) ? 0.0f : v - u2f(hi);
        const uint32_t mid = f2u(r) & 0xffff0000u;
        part[0][e] = hi;
        part[1][e] = mid;
        part[2][e] = f2u(r - u2f(mid));
      }
#pragma unroll
      for (int p = 0; p < 3; ++p) wp[p][i / 2] = __builtin_amdgcn_perm(part[p][1], part[p][0], 0x07060302u);
    }
#pragma unroll
    for (int p = 0; p < 3; ++p) *(uint2 *)&Xs[buf][p][xm][xk] = make_uint2(wp[p][0], wp[p][1]);
  };
  auto mfma_step = [&](floatx4 (&acc)[CG], int buf, int q, const bf16x8 (&bv)[CG][NP]) {
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      const bf16x8 av = __builtin_bit_cast(bf16x8, *(const shortx8 *)&Xs[buf][p][j][16 * g + 8 * q]);
#pragma unroll
      for (int c = 0; c < CG; ++c)
#pragma unroll
        for (int wp = 0; wp < NP; ++wp)
          if (p + wp <= 2) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv[c][wp], acc[c], 0, 0, 0);
    }
  };
  floatx4 acc[CG];
  int buf = 0;
  const int last = max(it, it_end - 1);
#pragma unroll
  for (int d = 0; d < D; ++d) {
    load_x(min(it + d, last), xf[d], xin[d]);
    __builtin_amdgcn_sched_barrier(0);  // x before w, as in the loop (wait counts)
    load_w(min(it + d, last), wr[d]);
  }
  store_x(0, xf[0], xin[0]);
  lds_barrier();
  for (int u0 = it; u0 < it_end; u0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int u = u0 + d;
      // leaving the whole loop keeps the ring's wait counts exact
      if (u >= it_end) goto done;
      const int t = u / a.nst, st = u - t * a.nst;
      if (u == it || st == 0) {
#pragma unroll
        for (int c = 0; c < CG; ++c)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[c][i] = 0.0f;
      }
      if constexpr (NP == 1) {
        bf16x8 bv[2][CG][1];
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
          for (int c = 0; c < CG; ++c) {
            bf16x8 pp[1];
            bf3_weights<BK>(wr[d][c], q, t3, pp);
            bv[q][c][0] = pp[0];
          }
        load_x(min(u + D, last), xf[d], xin[d]);
        load_w(min(u + D, last), wr[d]);
#pragma unroll
        for (int q = 0; q < 2; ++q) mfma_step(acc, buf, q, bv[q]);
      } else {
        load_x(min(u + D, last), xf[d], xin[d]);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          bf16x8 bv[CG][NP];
#pragma unroll
          for (int c = 0; c < CG; ++c) bf3_weights<BK>(wr[d][c], q, t3, bv[c]);
          mfma_step(acc, buf, q, bv);
        }
        load_w(min(u + D, last), wr[d]);
      }
      store_x(buf ^ 1, xf[(d + 1) % D], xin[(d + 1) % D]);
      lds_barrier();  // the next units' loads stay in flight
      buf ^= 1;
      if (st == a.nst - 1 || u + 1 == it_end) {
        // rows 4 g .. 4 g + 3 of the tile; a group wholly past M is never read
        float *dst = a.ws + ((int64_t)blockIdx.x * a.maxspan + (t - first_tile)) * (BM * BN);
        if (4 * g < a.M - unit_m0(u)) {
#pragma unroll
          for (int c = 0; c < CG; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) dst[(4 * g + r) * BN + wave * 32 * NC + c * 16 + j] = acc[c][r];
        }
      }
    }
  }
done:;
}

// The split-x GEMM for batch <= 16 with no k split across workgroups: a
// workgroup owns 16 * CW output columns (CW waves of 16) over the whole of K,
// and its KG wave groups take every KG-th 64-deep k stage (group g: stages
// g, g + KG, ...), each staging its own stage's x parts in LDS.  At the end
// the groups' fp32 sums meet in LDS, are added in group order in f64 and the
// epilogue (post scale, then bias and activation for the forward, fl32 for
// dX) stores the outputs directly: no partial tiles and no reduction
// launch.  Operand layout, x split and weight decode are gemm_bf3s_kernel's
// (16x16x32 MFMA; a lane holds 16 consecutive weights of one column per
// stage).  Rounds past a group's last stage re-read a valid stage against x
// masked to zero.  NB = 1 (one x buffer per group) only when every group
// has a single round (nst <= KG).
template <int BK, int D, bool FWD, int KG, int CW, int NB>
__global__ void __launch_bounds__(64 * KG * CW) gemm_bf3r_kernel(GemmArgs a, const double *bias,
                                                                 int bias_len, int act, float *out,
                                                                 float *post) {
  using K3 = B3<BK>;
  constexpr int BM = 16, NW = K3::kWords / 2, NP = K3::kParts;
  constexpr int XE = BM * kBK / (64 * CW);  // x values per thread per stage: 8 (CW = 2) or 16
  constexpr int XT = kBK / XE;              // threads per x row
  static_assert((XE == 8 || XE == 16) && (NW == 2 || NW == 4), "16-row split-x layout");
  __shared__ uint16_t Xs[NB][KG][3][BM][kBf3Row];
  __shared__ float ex[KG - 1][CW][4][64];
  __shared__ uint2 t3[16];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int grp = wv / CW, cw = wv % CW, gt = tid & (64 * CW - 1);
  const int j = lane & 15, g = lane >> 4;
  if constexpr (BK == BK_NF4) {
    if (tid < 16) {  // NF4 table values split exactly into three bf16 parts
      const float t = kNf4Tab[tid];
      const uint32_t hi = f2u(t) & 0xffff0000u;
      const float r = t - u2f(hi);
      const uint32_t mid = f2u(r) & 0xffff0000u;
      const uint32_t lo = f2u(r - u2f(mid));
      t3[tid] = make_uint2((hi >> 16) | mid, lo >> 16);
    }
  }
  const int n0 = blockIdx.x * (16 * CW), m0 = blockIdx.y * BM;
  const int rounds = (a.nst + KG - 1) / KG;
  const int xm = gt / XT, xk = (gt % XT) * XE;  // xm < 16, xk < 64
  const int col = n0 + cw * 16 + j;
  const int64_t wrow = (int64_t)min(col, a.N - 1) * a.row_bytes;
  uint32_t wr[D][NW];
  float xf[D][XE];
  uint32_t xin[D];
  auto load_w = [&](int r, uint32_t (&w)[NW]) {
    const int k0 = min(grp + KG * r, a.nst - 1) * kBK;
    const uint8_t *src = a.body + wrow + (k0 + 16 * g) * K3::kBits / 8;
    if constexpr (NW == 4) {
      const uint4 v = *(const uint4 *)src;
      w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else {
      const uint2 v = *(const uint2 *)src;
      w[0] = v.x; w[1] = v.y;
    }
  };
  auto load_x = [&](int r, float (&xv)[XE], uint32_t &in_mask) {
    const int k0 = (grp + KG * r) * kBK;
    const bool in = m0 + xm < a.M && k0 + xk < a.K;
    in_mask = in ? ~0u : 0u;
    const float *src = a.A + (int64_t)(in ? m0 + xm : 0) * a.K + (in ? k0 + xk : 0);
#pragma unroll
    for (int q4 = 0; q4 < XE / 4; ++q4) {
      const float4 v = *(const float4 *)(src + 4 * q4);
      xv[4 * q4] = v.x; xv[4 * q4 + 1] = v.y; xv[4 * q4 + 2] = v.z; xv[4 * q4 + 3] = v.w;
    }
  };
  auto store_x = [&](int buf, const float (&xv)[XE], uint32_t in_mask) {
    uint32_t wp[3][XE / 2];
#pragma unroll
    for (int i = 0; i < XE; i += 2) {
      uint32_t part[3][2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float v = u2f(f2u(xv[i + e]) & in_mask);
        const uint32_t hi = f2u(v) & 0xffff0000u;
        const float r = isinf(v) ? 0.0f : v - u2f(hi);
        const uint32_t mid = f2u(r) & 0xffff0000u;
        part[0][e] = hi;
        part[1][e] = mid;
        part[2][e] = f2u(r - u2f(mid));
      }
#pragma unroll
      for (int p = 0; p < 3; ++p) wp[p][i / 2] = __builtin_amdgcn_perm(part[p][1], part[p][0], 0x07060302u);
    }
#pragma unroll
    for (int p = 0; p < 3; ++p)
#pragma unroll
      for (int h = 0; h < XE / 8; ++h)
        *(uint4 *)&Xs[buf][grp][p][xm][xk + 8 * h] =
            make_uint4(wp[p][4 * h], wp[p][4 * h + 1], wp[p][4 * h + 2], wp[p][4 * h + 3]);
  };
  floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  auto mfma_step = [&](int buf, int q, const bf16x8 (&bv)[NP]) {
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      const bf16x8 av = __builtin_bit_cast(bf16x8, *(const shortx8 *)&Xs[buf][grp][p][j][16 * g + 8 * q]);
#pragma unroll
      for (int wp = 0; wp < NP; ++wp)
        if (p + wp <= 2) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv[wp], acc, 0, 0, 0);
    }
  };
  int buf = 0;
  const int last = rounds - 1;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    load_x(min(d, last), xf[d], xin[d]);
    load_w(min(d, last), wr[d]);
  }
  store_x(0, xf[0], xin[0]);
  lds_barrier();
  for (int r0 = 0; r0 < rounds; r0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int r = r0 + d;
      if (r >= rounds) goto done;
      bf16x8 bv[2][NP];
#pragma unroll
      for (int q = 0; q < 2; ++q) bf3_weights<BK>(wr[d], q, t3, bv[q]);
      load_x(min(r + D, last), xf[d], xin[d]);
      load_w(min(r + D, last), wr[d]);
#pragma unroll
      for (int q = 0; q < 2; ++q) mfma_step(buf, q, bv[q]);
      if constexpr (NB == 2) {  // NB = 1: this was the group's only round
        store_x(buf ^ 1, xf[(d + 1) % D], xin[(d + 1) % D]);
        lds_barrier();
        buf ^= 1;
      }
    }
  }
done:
  // D lane (j, g) holds column j, rows 4 g .. 4 g + 3 of the group's sum
  if (grp > 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) ex[grp - 1][cw][i][lane] = acc[i];
  }
  lds_barrier();
  if (grp == 0 && col < a.N) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + 4 * g + i;
      if (m >= a.M) break;
      double sum = (double)acc[i];
#pragma unroll
      for (int q = 0; q < KG - 1; ++q) sum += (double)ex[q][cw][i][lane];
      if (a.post != 1.0f) sum *= (double)a.post;
      const int64_t idx = (int64_t)m * a.N + col;
      if constexpr (FWD) bias_act_store(sum, col, bias, bias_len, act, out, post, idx);
      else out[idx] = (float)sum;
    }
  }
}

// Sum of a tile's stream-K partials in workgroup order (f64).  Grid: x =
// tile, y = 1024-element slice of the tile; each thread adds four adjacent
// outputs with float4 loads.  The forward applies bias + activation, dX
// stores fl32 of the sum, times act'(next_pre) when next_pre is given (in
// a volume training step the pre of the layer below, act its piecewise
// activation: the derivative act_deriv_kernel would apply, the same
// expression as gemm_regt_kernel's NEXT epilogue).
template <bool FWD>
__global__ void __launch_bounds__(256) sk_reduce_kernel(GemmArgs a, const double *bias, int bias_len,
                                                        int act, float *out, float *post,
                                                        const float *next_pre) {
  const int t = blockIdx.x;
  const int b0 = (int)((int64_t)t * a.nst / a.per_block);
  const int b1 = (int)(((int64_t)(t + 1) * a.nst - 1) / a.per_block);
  const int tile = a.bm * a.bn;
  const int off = (blockIdx.y * 256 + threadIdx.x) * 4;
  if (off >= tile) return;
  const int m = (t / a.gx) * a.bm + off / a.bn, n = (t % a.gx) * a.bn + off % a.bn;
  if (m >= a.M) return;
  double sum[4] = {0, 0, 0, 0};
  // all loads of a group of 8 partials are issued before the first add
  for (int g = b0; g <= b1; g += 8) {
    float4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int b = g + i;
      if (b <= b1) {
        const int slot = t - (int)((int64_t)b * a.per_block / a.nst);
        v[i] = *(const float4 *)(a.ws + ((int64_t)b * a.maxspan + slot) * tile + off);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (g + i <= b1) {
        sum[0] += (double)v[i].x;
        sum[1] += (double)v[i].y;
        sum[2] += (double)v[i].z;
        sum[3] += (double)v[i].w;
      }
    }
  }
  // the epilogue of bias_act_store (or fl32 for dX) on the four sums, stored
  // as one 16-byte write per output array where the row allows it
  float pv[4], qv[4];
  const int nv = min(4, a.N - n);
  const int64_t idx = (int64_t)m * a.N + n;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (a.post != 1.0f) sum[i] *= (double)a.post;
    float p = (float)sum[i];
    if constexpr (FWD) {
      if (bias != nullptr && n + i < bias_len) p = (float)((double)p + bias[n + i]);
      qv[i] = i >= nv ? 0.0f : act == kSwiGated ? act_value(post[idx + i], kSilu) * p : act_value(p, act);
    } else {
      if (next_pre != nullptr && i < nv) p = p * act_prime_piecewise(next_pre[idx + i], act);
    }
    pv[i] = p;
  }
  if (nv == 4 && (a.N & 3) == 0) {
    *(float4 *)(out + idx) = make_float4(pv[0], pv[1], pv[2], pv[3]);
    if constexpr (FWD) *(float4 *)(post + idx) = make_float4(qv[0], qv[1], qv[2], qv[3]);
  } else {
    for (int i = 0; i < nv; ++i) {
      out[idx + i] = pv[i];
      if constexpr (FWD) post[idx + i] = qv[i];
    }
  }
}

__global__ void __launch_bounds__(256) reduce_plain_kernel(const float *ws, int slices, int64_t total,
                                                           float *out) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    double s = 0;
    for (int k = 0; k < slices; ++k) s += (double)ws[(int64_t)k * total + i];
    out[i] = (float)s;
  }
}

// ------------------------------------------------------------- backward
// welvet_dense_act_deriv welvet_dense.metal:107-119
__global__ void __launch_bounds__(256) act_deriv_kernel(const float *gy, const float *pre, int64_t n,
                                                        int act, float *dpre) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    dpre[i] = gy[i] * act_prime(pre[i], act);
}

struct DxArgs {
  const uint8_t *body;
  const float *lut;
  float scale, minv;
  const float *dpre;  // [B][rows]
  int rows, cols, nchunks, seg_rows, nseg;
  int64_t row_bytes;
  float *ws;  // [nseg][B][cols]
};

// dX[b][i] = sum_o W[o][i] dpre[b][o]: lane owns one column chunk, walks the
// rows of its segment.
template <int F, int B>
__global__ void __launch_bounds__(256) dx_small_kernel(DxArgs a) {
  using I = FI<F>;
  using Acc = typename I::Acc;
  constexpr int E = I::kE, W = I::kW;
  __shared__ float lut_s[I::kTable];
  if constexpr (I::kLut) {
    fill_table<F>(lut_s, a.lut, threadIdx.x, 256);
    __syncthreads();
  }
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= a.nchunks) return;
  const int seg = blockIdx.y;
  const int o0 = seg * a.seg_rows, o1 = min(a.rows, o0 + a.seg_rows);
  Acc acc[B][E];
#pragma unroll
  for (int b = 0; b < B; ++b)
#pragma unroll
    for (int e = 0; e < E; ++e) acc[b][e] = 0;
  for (int o = o0; o < o1; ++o) {
    uint32_t w[W];
    load_words<W>(a.body + (int64_t)o * a.row_bytes + (int64_t)c * (W * 4), w);
    Acc dp[B];
#pragma unroll
    for (int b = 0; b < B; ++b) dp[b] = (Acc)a.dpre[(int64_t)b * a.rows + o];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const Acc wv = chunk_value<F>(w, e, lut_s, a.scale, a.minv);
#pragma unroll
      for (int b = 0; b < B; ++b) acc[b][e] = fma(wv, dp[b], acc[b][e]);
    }
  }
#pragma unroll
  for (int b = 0; b < B; ++b)
#pragma unroll
    for (int e = 0; e < E; ++e)
      a.ws[((int64_t)seg * B + b) * a.cols + (int64_t)c * E + e] = (float)acc[b][e];
}

template <int DT>
__global__ void __launch_bounds__(256) dx_generic_kernel(DevStore w, int batch, const float *dpre,
                                                         float *dX) {
  const int64_t total = (int64_t)batch * w.cols;
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += (int64_t)gridDim.x * 256) {
    const int b = (int)(t / w.cols), i = (int)(t % w.cols);
    double acc = 0;
    for (int o = 0; o < w.rows; ++o) {
      const uint64_t c = load_code<DT>(w.body, (int64_t)o * w.cols + i);
      const double wv = DT == kFloat64 ? u2d(c) : (double)dec_code<DT>(c, w.scale, w.minv);
      acc += wv * (double)dpre[(int64_t)b * w.rows + o];
    }
    dX[t] = (float)acc;
  }
}

// dW on the matrix cores with the reference's rounding.  Per output the
// reference accumulates acc = fmaf(dpre[b][o], x[b][i], acc) over b in batch
// order from 0 (welvet_dense.metal:155-178).  v_mfma_f32_32x32x2f32 computes
// each output as fmaf(a1, b1, fmaf(a0, b0, c)): two fused multiply-adds in k
// order, bit-identical to the VALU's fmaf (checked on the device over random
// bit patterns, denormals, infinities, NaNs and signed zeros), so a chain of
// them over k = batch rows reproduces the reference exactly.  An odd batch
// ends with a -0 product, which leaves every accumulator (-0 included) as it
// is.  Block: 128 (o) x 128 (i) outputs, four waves of 64 x 64 (2 x 2 tiles of
// 32 x 32); lane (j, h) supplies batch row b + h of operand column j: the
// A operand dpre[b][o0 + j], the B operand x[b][i0 + j] (coalesced 128-byte
// rows).  Out-of-range rows and columns read a clamped valid element and are
// never stored.
__global__ void __launch_bounds__(256) dw_mfma_kernel(const float *__restrict__ dpre,
                                                      const float *__restrict__ x, int B, int rows,
                                                      int cols, float *__restrict__ dW, int *flag) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 31, h = lane >> 5;
  const int o0 = blockIdx.y * 128 + (wave >> 1) * 64, i0 = blockIdx.x * 128 + (wave & 1) * 64;
  const float *pa[2], *pb[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    pa[t] = dpre + min(o0 + 32 * t + j, rows - 1);
    pb[t] = x + min(i0 + 32 * t + j, cols - 1);
  }
  floatx16 acc[2][2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mt][nt][r] = 0.0f;
  // groups of kU k steps (2 kU batch rows); group g + 1's loads are in flight
  // while group g's MFMAs run (two register sets).  Loads past the batch read
  // row 0; the -0 / 0 padding replaces them where they are used (a select
  // right after a load would make the compiler wait for that load at once).
  constexpr int kU = 6;  // 24 loads per group: two groups fit the 63 loads a wave can have in flight
  const int ng = (B + 2 * kU - 1) / (2 * kU);
  auto load = [&](int g, float (&av)[kU][2], float (&bv)[kU][2]) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int b = g * 2 * kU + 2 * u + h;
      const int64_t bc = b < B ? b : 0;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        av[u][t] = pa[t][bc * rows];
        bv[u][t] = pb[t][bc * cols];
      }
    }
  };
  auto mfmas = [&](int g, const float (&av)[kU][2], const float (&bv)[kU][2]) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int b = g * 2 * kU + 2 * u;
      if (b >= B) break;
      const bool in = b + h < B;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(in ? av[u][mt] : -0.0f, in ? bv[u][nt] : 0.0f,
                                                             acc[mt][nt], 0, 0, 0);
    }
  };
  float a0[kU][2], b0v[kU][2], a1[kU][2], b1v[kU][2];
  load(0, a0, b0v);
  for (int g = 0; g < ng; g += 2) {
    load(g + 1, a1, b1v);
    mfmas(g, a0, b0v);
    if (g + 1 >= ng) break;
    load(g + 2, a0, b0v);
    mfmas(g + 1, a1, b1v);
  }
  // D[m][n]: lane (j, h) holds column j, rows 8 (r / 4) + 4 h + r % 4
  int bad = 0;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int i = i0 + 32 * nt + j;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int o = o0 + 32 * mt + 8 * (r >> 2) + 4 * h + (r & 3);
        if (o < rows && i < cols) {
          dW[(int64_t)o * cols + i] = acc[mt][nt][r];
          bad |= !isfinite(acc[mt][nt][r]);
        }
      }
    }
  if (flag != nullptr && __any(bad) && lane == 0) atomicOr(flag, 1);
}

// out[c][r] = in[r][c] (bytes) through 64 x 64 LDS tiles: coalesced 16-byte
// row reads, 16-byte writes along the output rows.
__global__ void __launch_bounds__(256) transpose_u8_kernel(const uint8_t *__restrict__ in, int rows, int cols,
                                                           uint8_t *__restrict__ out) {
  __shared__ uint8_t t[64][64 + 4];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64, tid = threadIdx.x;
  const int lr = tid >> 2, lc = (tid & 3) * 16;  // 64 rows x 4 pieces of 16 bytes
  const int r = r0 + lr;
  if (r < rows && c0 + lc + 16 <= cols && (cols & 15) == 0) {
    const uint4 v = *(const uint4 *)(in + (int64_t)r * cols + c0 + lc);
    const uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 16; ++j) t[lr][lc + j] = (uint8_t)(q[j >> 2] >> (8 * (j & 3)));
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int c = c0 + lc + j;
      t[lr][lc + j] = (r < rows && c < cols) ? in[(int64_t)r * cols + c] : 0;
    }
  }
  __syncthreads();
  const int oc = c0 + lr;  // output row = input column
  if (oc >= cols) return;
  if (r0 + lc + 16 <= rows && (rows & 15) == 0) {
    uint32_t q[4] = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 16; ++j) q[j >> 2] |= (uint32_t)t[lc + j][lr] << (8 * (j & 3));
    *(uint4 *)(out + (int64_t)oc * rows + r0 + lc) = make_uint4(q[0], q[1], q[2], q[3]);
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int orr = r0 + lc + j;
      if (orr < rows) out[(int64_t)oc * rows + orr] = t[lc + j][lr];
    }
  }
}

// dw_mfma_kernel with its operands staged through LDS (rows and columns
// multiples of 128): per stage of 16 batch rows the block loads the dpre and
// x panels (16 x 128 floats each) with coalesced 16-byte loads into a
// double-buffered LDS ring, the next stage's loads in flight during this
// stage's MFMAs.  Rows are padded to 160 floats so a wave's two k halves
// (batch rows 2s and 2s + 1) read opposite bank halves.  Rows past the batch
// hold the -0 / 0 padding.  Same MFMA chain, so the same bits as
// dw_mfma_kernel.
// The 128 x 128 dW tile at block coordinates (bx, by).
__device__ inline void dw_lds_tile(const float *__restrict__ dpre, const float *__restrict__ x, int B,
                                   int rows, int cols, float *__restrict__ dW, int *flag, int bx, int by) {
  constexpr int kS = 16, kRow = 160;
  __shared__ float As[2][kS][kRow], Bs[2][kS][kRow];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;
  const int ob = by * 128, ib = bx * 128;
  const int wo = (wave >> 1) * 64, wi = (wave & 1) * 64;
  // loader: thread t moves rows t / 32 and t / 32 + 8 of a panel, columns 4 (t % 32) .. + 3
  const int lr = tid >> 5, lc = (tid & 31) * 4;
  floatx16 acc[2][2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mt][nt][r] = 0.0f;
  const int nstage = (B + kS - 1) / kS;
  // stage st's panel rows for this thread (clamped into the batch: the
  // padding replaces them in LDS)
  const float *ga0 = dpre + ob + lc, *gb0 = x + ib + lc;
  float4 ra0, ra1, rb0, rb1;
  {
    const int b0 = min(lr, B - 1), b1 = min(lr + 8, B - 1);
    ra0 = *(const float4 *)(ga0 + (int64_t)b0 * rows);
    ra1 = *(const float4 *)(ga0 + (int64_t)b1 * rows);
    rb0 = *(const float4 *)(gb0 + (int64_t)b0 * cols);
    rb1 = *(const float4 *)(gb0 + (int64_t)b1 * cols);
  }
  // component-wise selects (a select of whole float4 values becomes an
  // indexed private array)
  auto pad = [](bool in, float4 v, float p) {
    return make_float4(in ? v.x : p, in ? v.y : p, in ? v.z : p, in ? v.w : p);
  };
  *(float4 *)&As[0][lr][lc] = pad(lr < B, ra0, -0.0f);
  *(float4 *)&As[0][lr + 8][lc] = pad(lr + 8 < B, ra1, -0.0f);
  *(float4 *)&Bs[0][lr][lc] = pad(lr < B, rb0, 0.0f);
  *(float4 *)&Bs[0][lr + 8][lc] = pad(lr + 8 < B, rb1, 0.0f);
  __syncthreads();
  for (int st = 0; st < nstage; ++st) {
    const int buf = st & 1;
    const int sn = min(st + 1, nstage - 1);
    {
      const int b0 = min(sn * kS + lr, B - 1), b1 = min(sn * kS + lr + 8, B - 1);
      ra0 = *(const float4 *)(ga0 + (int64_t)b0 * rows);
      ra1 = *(const float4 *)(ga0 + (int64_t)b1 * rows);
      rb0 = *(const float4 *)(gb0 + (int64_t)b0 * cols);
      rb1 = *(const float4 *)(gb0 + (int64_t)b1 * cols);
    }
    // steps past the batch multiply the padding (adds -0: no change)
#pragma unroll
    for (int k = 0; k < kS / 2; ++k) {
      const float a0 = As[buf][2 * k + h][wo + j], a1 = As[buf][2 * k + h][wo + 32 + j];
      const float b0 = Bs[buf][2 * k + h][wi + j], b1 = Bs[buf][2 * k + h][wi + 32 + j];
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
    }
    if (st + 1 < nstage) {
      const int r0 = (st + 1) * kS + lr;
      *(float4 *)&As[buf ^ 1][lr][lc] = pad(r0 < B, ra0, -0.0f);
      *(float4 *)&As[buf ^ 1][lr + 8][lc] = pad(r0 + 8 < B, ra1, -0.0f);
      *(float4 *)&Bs[buf ^ 1][lr][lc] = pad(r0 < B, rb0, 0.0f);
      *(float4 *)&Bs[buf ^ 1][lr + 8][lc] = pad(r0 + 8 < B, rb1, 0.0f);
    }
    __syncthreads();
  }
  // D[m][n]: lane (j, h) holds column j, rows 8 (r / 4) + 4 h + r % 4
  int bad = 0;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int i = ib + wi + 32 * nt + j;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int o = ob + wo + 32 * mt + 8 * (r >> 2) + 4 * h + (r & 3);
        dW[(int64_t)o * cols + i] = acc[mt][nt][r];
        bad |= !isfinite(acc[mt][nt][r]);
      }
    }
  if (flag != nullptr && __any(bad) && lane == 0) atomicOr(flag, 1);
}

__global__ void __launch_bounds__(256) dw_mfma_lds_kernel(const float *__restrict__ dpre,
                                                          const float *__restrict__ x, int B, int rows,
                                                          int cols, float *__restrict__ dW, int *flag) {
  dw_lds_tile(dpre, x, B, rows, cols, dW, flag, blockIdx.x, blockIdx.y);
}

// The dW of up to kDwBatch layers in one launch (blockIdx.z = layer; the
// grid covers the largest layer, blocks past a smaller one's tiles exit).
__global__ void __launch_bounds__(256) dw_batch_kernel(DwBatch b) {
  const int l = blockIdx.z;
  if (l >= b.count) return;
  const DwJob &t = b.job[l];
  if ((int)blockIdx.x * 128 >= t.cols || (int)blockIdx.y * 128 >= t.rows) return;
  dw_lds_tile(t.dpre, t.x, b.batch, t.rows, t.cols, t.dW, t.flag, blockIdx.x, blockIdx.y);
}

// ------------------------------------------------------------------ MSE
__global__ void __launch_bounds__(256) mse_partial_kernel(const float *p, const float *t, int64_t n,
                                                          double *part) {
  __shared__ double red[4];
  double s = 0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const double d = (double)p[i] - (double)t[i];
    s += d * d;
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}

__global__ void __launch_bounds__(256) mse_final_kernel(const double *part, int nparts, int64_t n,
                                                        double *loss, int *clear, int64_t nclear) {
  __shared__ double red[4];
  for (int64_t i = threadIdx.x; i < nclear; i += 256) clear[i] = 0;
  double s = 0;
  for (int i = threadIdx.x; i < nparts; i += 256) s += part[i];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) *loss = (red[0] + red[1] + red[2] + red[3]) / (double)n;
}

// welvet_mse_grad welvet_dense.metal:207-215
__global__ void __launch_bounds__(256) mse_grad_kernel(const float *p, const float *t, int64_t n,
                                                       float *g) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    g[i] = (float)((((double)p[i] - (double)t[i]) * 2.0) / (double)n);
}

// --------------------------------------------------- SwiGLU element-wise
// op_swiglu ops_common.metal:27-38.  The forward's h = fl32(silu(gate)) * up
// is the kSwiGated epilogue of the Up projection; the backward (c[1] == 1):
// d_up = fl32(gh * silu(gate));
// d_gate = fl32((gh * up) * silu'(gate)), the product kept wide (exact in f64)
// and rounded once
__global__ void __launch_bounds__(256) swiglu_bwd_kernel(const float *__restrict__ gate,
                                                         const float *__restrict__ up,
                                                         const float *__restrict__ gh, int64_t n,
                                                         float *__restrict__ d_up,
                                                         float *__restrict__ d_gate) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const float g = gate[i], d = gh[i];
    d_up[i] = d * act_value(g, kSilu);
    d_gate[i] = (float)(((double)d * (double)up[i]) * (double)act_prime(g, kSilu));
  }
}

// metal::add: out = fl32(a + b)
__global__ void __launch_bounds__(256) add_kernel(const float *__restrict__ a,
                                                  const float *__restrict__ b, int64_t n,
                                                  float *__restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    out[i] = a[i] + b[i];
}

// --------------------------------------------------------------- dispatch
int g_forward_path = 0;
// Tuning knobs (welvet_hip_set_tuning); defaults are the measured choices.
// Route switches (welvet_hip_set_tuning; kept keys only, the others are
// unknown): read by every launch, written by any thread, hence atomic.
std::atomic<int> g_tune[kNumTune] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 1, 0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 1};
bool tune_key_kept(int key) {
  return key == kTuneBf3 || (key >= kTuneBf3Rows && key <= kTuneRegx);
}
inline int knob(int key) { return g_tune[key].load(std::memory_order_relaxed); }

// Kind of a dtype under the current knobs, -1 when the split-x GEMM does not
// take it.
// Split-x weight kind of a store, -1 when the split-x GEMM does not take it.
// E5M2 only while no stored code is Inf / NaN: x_part * Inf over the three
// parts of x would give NaN where the fp32 product is Inf.
int bf3_kind(const DevStore &w) {
  const int dt = w.dtype;
  if (knob(kTuneBf3) == 0) return -1;
  if (dt == kFP8E4M3) return BK_E4;
  if (dt == kFP8E5M2 && w.finite) return BK_E5;
  if (dt == kInt8) return BK_I8;
  if (dt == kFP4) return BK_FP4;
  if (dt == kNF4) return BK_NF4;
  return -1;
}

inline int blocks_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  return (int)(b < 1 ? 1 : (b > 65536 ? 65536 : b));
}

bool chunk_aligned(const DevStore &w, int64_t len) {
  const int f = fmt_of(w.dtype);
  return f >= 0 && len % fmt_chunk_elems(f) == 0;
}

// Formats whose batch-1 GEMV also has the (1, 4) and (2, 8) shapes of
// (chunks per lane, rows per block) besides the default (C, 8 / C).
constexpr bool gemv_extra_rows(int f) {
  return f == FE4 || f == FE5 || f == FI8 || f == FL4P || f == FF4;
}

// Kernel format of a dtype: FP8 and FP4 through the hardware converters
// (FP8 from the decode-ready copy), Int8 by integer conversion, the other
// 4-bit formats through the byte-pair table, the rest as fmt_of.
int kernel_fmt(int dt) {
  if (dt == kFP8E4M3) return FE4;
  if (dt == kFP8E5M2) return FE5;
  if (dt == kInt8) return FI8;
  if (dt == kFP4) return FF4;
  const int f = fmt_of(dt);
  return f == FL4 ? FL4P : f;
}

// Payload a kernel format reads: the decode-ready copy for the formats
// decoded by the FP8 converters (null when the store has none).
const uint8_t *kernel_body(const DevStore &w, int f) {
  return (f == FE4 || f == FE5) ? w.kbody : w.body;
}

int64_t row_bytes_of(const DevStore &w) {
  return (int64_t)w.cols * dtype_bits(w.dtype) / 8;
}

int num_cus() {
  static int n = [] {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess || v <= 0)
      v = 256;
    return v;
  }();
  return n;
}

struct SkPlan {
  int gx, gy, nst, per_block, blocks, maxspan, bm, bn;
  size_t ws_bytes;
  bool bf3 = false;  // split-x GEMM plan (bn = 128 or 256)
  int kg = 1;        // k stages per unit: 2 = the two-group split-x GEMM
  bool rows = false;  // gemm_bf3r_kernel: whole K per workgroup, no partials
};

// Stream-K split of an M x N x K product over bm x bn tiles into equal
// shares, `occ` workgroups per CU; units of `kg` consecutive k stages (the
// caller makes the stage count a multiple of kg).
SkPlan plan_sk(int M, int K, int N, int bm = kBM, int bn = kBN, int occ = 2, int kg = 1) {
  SkPlan p;
  p.bm = bm;
  p.bn = bn;
  p.kg = kg;
  p.gx = (N + bn - 1) / bn;
  p.gy = (M + bm - 1) / bm;
  p.nst = (K + kBK - 1) / kBK / kg;
  const int64_t T = (int64_t)p.gx * p.gy * p.nst;
  const int64_t G = (int64_t)occ * num_cus();
  p.per_block = (int)((T + G - 1) / G);
  p.blocks = (int)((T + p.per_block - 1) / p.per_block);
  p.maxspan = (p.per_block + p.nst - 1) / p.nst + 1;
  p.ws_bytes = (size_t)p.blocks * p.maxspan * bm * bn * sizeof(float);
  return p;
}

dim3 sk_reduce_grid(const SkPlan &p) {
  return dim3(p.gx * p.gy, (p.bm * p.bn / 4 + 255) / 256);
}

bool reg_gemm_ok(int f) { return f >= 0 && fmt_chunk_elems(f) >= 8; }  // formats of <= 16 bits


// Forward GEMM plan: the split-x bf16 kernel for the formats it takes, the
// register-B kernel for other <= 16-bit formats, else the LDS-staged kernel.
SkPlan plan_fwd_gemm(int f, int bk, int M, int K, int N) {
  if (bk >= 0) {
    const int occ = 2;
    const int bm = M <= 16 ? 16 : M <= 32 ? 32 : 64;
    // tile width: 128 output columns where outputs are few (N <= 8192) for
    // the 16-row tile and for the one-byte kinds' 32-row tile (their
    // stream-K partial tiles then weigh as much as the weights: 4096^2 FP8
    // b16 12.9 against 16.3 us, b32 15.2 against 18.1, NF4 b16 14.3 against
    // 17.2; 11008 -> 4096 FP8 b16 21.4 against 22.9), else 256 (4096 ->
    // 11008 b8 FP8 19.6 against 20.1; the 4-bit kinds' 32-row tile keeps
    // the two-group workgroups, which need 256)
    const bool narrow = N <= 8192 && (bm == 16 || (bm == 32 && bk != BK_NF4 && bk != BK_FP4));
    const int bn = narrow ? 128 : 256;
    const int stages = (K + kBK - 1) / kBK;
    // no k split for K <= 2048 (measured at batch 5-16: 1024^2 6.6 against
    // 10.3 us, 2048 -> 4096 9.4 against 14.3; at K = 4096 about even, at
    // K = 11008 1.6x slower: too few workgroups for the serial K walk)
    const int rk = knob(kTuneBf3Rows);
    if (bm == 16 && K % 8 == 0 && (rk == 2 || (rk == 1 && K <= 2048))) {
      SkPlan p;
      p.bf3 = p.rows = true;
      p.bm = 16;
      p.bn = 32;
      p.gx = (N + 31) / 32;
      p.gy = (M + 15) / 16;
      p.nst = stages;
      p.per_block = stages;
      p.blocks = p.gx * p.gy;
      p.maxspan = 1;
      p.ws_bytes = 0;
      return p;
    }
    // two-group workgroups: every 64-row tile; 32-row tiles only for the
    // 4-bit kinds (FP8 / Int8 measured slower there)
    const bool groups = bn == 256 && stages % 2 == 0 &&
                        (bm == 64 || (bm == 32 && (bk == BK_NF4 || bk == BK_FP4)));
    SkPlan p = groups ? plan_sk(M, K, N, bm, bn, 1, 2)
                      : plan_sk(M, K, N, bm, bn, occ);
    p.bf3 = true;
    return p;
  }
  // batch <= 16 without a k split (gemm_regr_kernel): K <= 2048 as for the
  // split-x 16-row GEMM, and any K (per format, measured at 4096^2, 4096 <->
  // 11008, batch 8 and 16) for at most 8192 outputs outside the half formats
  // (11008 -> 4096 b8: Uint8 29.9 against 44.5 us, Float32 62.4 against
  // 82.9, Int64 72.6 against 114; Float16 57 against 44 at b16), the 16-bit
  // integers there only at K <= 4096 or batch <= 8 (11008 -> 4096 b16 Uint16
  // 57.2 against 46.7), and at more outputs for the formats that gain there
  // too (4096 -> 11008 b8 / b16: Int32 49 / 58 against 83 / 84, the 1- to
  // 3-bit tables 29-30 / 38-40 against 42 / 42, Int64 82 / 86 against 110 /
  // 112, Complex128 167 / 177 against 190 / 183; Uint8, Uint16, FP6, Int5
  // and Complex64 lose at b16)
  const int rk = knob(kTuneBf3Rows);
  const bool half = f == FH16 || f == FB16, int16 = f == FI16 || f == FU16;
  const bool wide_ok = f == FI32 || f == FU32 || f == FI64 || f == FU64 || f == FL1 || f == FL2 ||
                       f == FL3 || f == FC128;
  const bool long_k = !half && (N <= 8192 ? (!int16 || K <= 4096 || M <= 8) : wide_ok);
  if (M <= 16 && K % 4 == 0 && (rk == 2 || (rk == 1 && (K <= 2048 || long_k)))) {
    SkPlan p;
    p.rows = true;
    p.bm = p.bn = 16;
    p.gx = (N + 15) / 16;
    p.gy = (M + 15) / 16;
    const int e = fmt_chunk_elems(f), st = 4 * (e >= 8 ? 32 : 4 * e);  // RegrShape<F>::ST
    p.nst = (K + st - 1) / st;
    p.per_block = p.nst;
    p.blocks = p.gx * p.gy;
    p.maxspan = 1;
    p.ws_bytes = 0;
    return p;
  }
  if (reg_gemm_ok(f)) return plan_sk(M, K, N, M <= 32 ? 32 : 64, kRegBN, 2);
  return plan_sk(M, K, N);
}

constexpr int kDxSegRows = 32;

// Batch 2-8 on gemv_loopb_kernel: B batch rows in registers (the batch
// rounded up to 2, 4 or 8), C chunks per lane (1, 2 or 4), S waves per
// block covering the row (at most 8); false when x of B rows would take more
// than 128 registers per lane or the row more than 8 waves, or for formats
// without that kernel.
struct GemvBatchShape {
  int B, C, S;
};
// formats gemv_loopb_kernel is built for (fp32 partial sums: not Float64)
constexpr bool gemv_batch_fmt(int f) {
  return f == FE4 || f == FE5 || f == FI8 || f == FF4 || f == FL4P || f == FH16 || f == FB16 ||
         f == FF32 || f == FL8 || f == FI16 || f == FU16 || f == FI32 || f == FU32 || f == FI64 ||
         f == FU64 || f == FL1 || f == FL2 || f == FL3 || f == FL5 || f == FL6;
}
bool gemv_batch_shape(int f, int batch, int nchunks, int rows, GemvBatchShape &sh) {
  if (knob(kTuneGemvBatch) == 0 || batch < 2 || batch > 8 || nchunks < 1 || rows < 1) return false;
  if (!gemv_batch_fmt(f)) return false;
  const int E = fmt_chunk_elems(f);
  const int B = batch <= 2 ? 2 : batch <= 4 ? 4 : 8;
  // 8 batch rows of the split-x GEMM's formats only up to 32 M weights (FP8
  // b8: 4096^2 12.3 against 15.8 us on that GEMM, 4096 x 11008 24.6 against
  // 19.9); the others' batch 5-8 GEMM is the fp32 MFMA one, slower still
  const bool split_x = f == FE4 || f == FE5 || f == FI8 || f == FF4 || f == FL4P;
  if (B == 8 && split_x && (int64_t)rows * nchunks * E > ((int64_t)32 << 20)) return false;
  // B * C <= 16: at least one row per group of R = 16 / (B * C)
  for (int C = 1; C <= 4 && B * C <= 16 && B * C * E <= 128; C *= 2) {
    const int S = (nchunks + 64 * C - 1) / (64 * C);
    if (S <= 8) {
      sh = GemvBatchShape{B, C, S};
      return true;
    }
  }
  return false;
}

bool gemv_batch_fits(const DevStore &w, int batch) {
  const int f = kernel_fmt(w.dtype);
  GemvBatchShape sh;
  return f >= 0 && chunk_aligned(w, w.cols) &&
         gemv_batch_shape(f, batch, w.cols / fmt_chunk_elems(f), w.rows, sh);
}

int fwd_route(const DevStore &w, int batch) {
  if (!chunk_aligned(w, w.cols)) return 3;
  if (g_forward_path) return g_forward_path;
  // batch 2-8 where x of the batch fits in registers: gemv_loopb_kernel
  // (4096 x 11008 b4: FP8 14.9 against 19.5 us on the split-x GEMM, NF4 17.1
  // against 22.2; 11008 x 4096 b4: FP8 16.5 against 22.2, NF4 17.1 against
  // 24.9)
  if (batch > 1 && gemv_batch_fits(w, batch)) return 1;
  if (batch <= 2) return 1;
  if (batch > 4) return 2;
  // other batch 3-4: gemv_kernel re-reads x for every chunk, so its time grows with
  // the batch, while the split-x GEMM's does not; measured crossover between
  // 16.8 M weights (4096^2: GEMV 12.5 against 15.3 us at batch 4) and 45 M
  // (4096 x 11008: 22.1 against 19.4 us FP8, 32.3 against 22.0 NF4)
  return (bf3_kind(w) < 0 || (int64_t)w.rows * w.cols <= (int64_t)32 << 20) ? 1 : 2;
}

template <int F, int B>
hipError_t run_gemv(const GemvArgs &a, hipStream_t s) {
  constexpr int R = 4;
  const int groups = (a.N + R - 1) / R;
  gemv_kernel<F, B, R><<<(groups + 3) / 4, 256, 0, s>>>(a);
  return hipGetLastError();
}

template <int F>
hipError_t gemv_dispatch(int batch, const GemvArgs &a, hipStream_t s) {
  switch (batch) {
  case 1: return run_gemv<F, 1>(a, s);
  case 2: return run_gemv<F, 2>(a, s);
  case 3: return run_gemv<F, 3>(a, s);
  case 4: return run_gemv<F, 4>(a, s);
  }
  return hipErrorInvalidValue;
}

#define WH_FMT_SWITCH(f, F)                                                                          \
  switch (f) {                                                                                       \
  case FL1: F(FL1); case FL2: F(FL2); case FL3: F(FL3); case FL5: F(FL5);                            \
  case FL6: F(FL6); case FL8: F(FL8); case FH16: F(FH16); case FB16: F(FB16); case FI16: F(FI16);    \
  case FU16: F(FU16); case FF32: F(FF32); case FI32: F(FI32); case FU32: F(FU32); case FI64: F(FI64); \
  case FU64: F(FU64); case FC64: F(FC64); case FC128: F(FC128); case FF64: F(FF64);                  \
  case FE4: F(FE4); case FE5: F(FE5); case FI8: F(FI8); case FL4P: F(FL4P); case FF4: F(FF4);        \
  default: return hipErrorInvalidValue;                                                              \
  }

#define WH_DT_SWITCH(dt, F)                                                                       \
  switch (dt) {                                                                                   \
  case kFloat64: F(kFloat64); case kFloat32: F(kFloat32); case kFloat16: F(kFloat16);             \
  case kBFloat16: F(kBFloat16); case kFP8E4M3: F(kFP8E4M3); case kFP8E5M2: F(kFP8E5M2);           \
  case kInt64: F(kInt64); case kInt32: F(kInt32); case kInt16: F(kInt16); case kInt8: F(kInt8);   \
  case kUint64: F(kUint64); case kUint32: F(kUint32); case kUint16: F(kUint16);                   \
  case kUint8: F(kUint8); case kInt4: F(kInt4); case kUint4: F(kUint4); case kFP4: F(kFP4);       \
  case kInt2: F(kInt2); case kUint2: F(kUint2); case kTernary: F(kTernary);                       \
  case kBinary: F(kBinary); case kInt: F(kInt); case kUint: F(kUint); case kUintptr: F(kUintptr); \
  case kComplex64: F(kComplex64); case kComplex128: F(kComplex128); case kNF4: F(kNF4);           \
  case kFP6: F(kFP6); case kInt6: F(kInt6); case kUint6: F(kUint6); case kInt5: F(kInt5);         \
  case kUint5: F(kUint5); case kInt3: F(kInt3); case kUint3: F(kUint3);                           \
  default: return hipErrorInvalidValue;                                                           \
  }

}  // namespace

void set_forward_path(int path) { g_forward_path = path; }

int set_tuning(int key, int value) {
  if (key < 0 || key >= kNumTune || !tune_key_kept(key)) return -1;
  return g_tune[key].exchange(value, std::memory_order_relaxed);
}

int tuning(int key) { return key < 0 || key >= kNumTune || !tune_key_kept(key) ? -1 : knob(key); }

size_t forward_workspace_bytes(const DevStore &w, int batch) {
  if (fwd_route(w, batch) != 2) return 0;
  return plan_fwd_gemm(kernel_fmt(w.dtype), bf3_kind(w), batch, w.cols, w.rows).ws_bytes;
}

// gemm_bf3r_kernel for plan p (p.rows): the forward (bias, activation, pre
// and post) or dX (out only, FWD false).
template <bool FWD>
hipError_t launch_bf3r(const SkPlan &p, int bk, const GemmArgs &a, const double *bias, int bias_len,
                       int act, float *out, float *post, hipStream_t s) {
  // Shapes (measured at batch 8-16): K of at most 16 stages on 16 wave groups
  // of one stage each, 16 columns per workgroup (1024^2 b16: FP8 5.78 -> 5.17
  // us, NF4 6.70 -> 5.58, FP4 5.82 -> 4.96; five 1024^2 layers FP8 24.7 ->
  // 21.6); longer K on 8 groups of 16 columns, two rounds of weights in
  // flight (2048 -> 1024 b16 FP8 8.94 -> 7.95, NF4 9.84 -> 8.32; 4096 ->
  // 11008 -> 4096 b8 NF4 68.1 -> 65.7 against 4 groups of 32 columns).  A
  // deeper ring is slower (1024^2 FP8 5.70 us with two rounds, 6.24 with four,
  // 7.5 with eight): the per-stage x split, not the load latency, bounds
  // these.  Rows of x split into 16-value pieces need K % 16 == 0; other K
  // keep 4 groups of 32 columns.
  const dim3 grid32(p.gx, p.gy), grid16((a.N + 15) / 16, p.gy);
  const int shape = a.K % 16 != 0 ? 0 : a.nst <= 16 ? 1 : 2;
#define WH_GR3(BK)                                                                                        \
  if (shape == 1)                                                                                         \
    gemm_bf3r_kernel<BK, 1, FWD, 16, 1, 1><<<grid16, 1024, 0, s>>>(a, bias, bias_len, act, out, post);    \
  else if (shape == 2)                                                                                    \
    gemm_bf3r_kernel<BK, 2, FWD, 8, 1, 2><<<grid16, 512, 0, s>>>(a, bias, bias_len, act, out, post);      \
  else                                                                                                    \
    gemm_bf3r_kernel<BK, 2, FWD, 4, 2, 2><<<grid32, 512, 0, s>>>(a, bias, bias_len, act, out, post);
  switch (bk) {
  case BK_E4: WH_GR3(BK_E4) break;
  case BK_I8: WH_GR3(BK_I8) break;
  case BK_FP4: WH_GR3(BK_FP4) break;
  case BK_NF4: WH_GR3(BK_NF4) break;
  case BK_E5: WH_GR3(BK_E5) break;
  default: return hipErrorInvalidValue;
  }
#undef WH_GR3
  return hipGetLastError();
}

// The split-x GEMM of plan p for weight kind bk (a.body, a.post set).
hipError_t launch_bf3(const SkPlan &p, int bk, GemmArgs &a, hipStream_t s) {
#define WH_GB(BK)                                                                     \
  if (p.bm == 16) {                                                                   \
    if (p.bn == 128) gemm_bf3s_kernel<BK, 1, 1><<<p.blocks, 256, 0, s>>>(a);           \
    else gemm_bf3s_kernel<BK, 1, 2><<<p.blocks, 256, 0, s>>>(a);                       \
  } else if (p.bm == 32) {                                                            \
    if (p.bn == 128) gemm_bf3_kernel<BK, 1, 1, 1><<<p.blocks, 256, 0, s>>>(a);         \
    else gemm_bf3_kernel<BK, 1, 1, 2><<<p.blocks, 256, 0, s>>>(a);                     \
  } else {                                                                            \
    if (p.bn == 128) gemm_bf3_kernel<BK, 2, 1, 1><<<p.blocks, 256, 0, s>>>(a);         \
    else gemm_bf3_kernel<BK, 2, 1, 2><<<p.blocks, 256, 0, s>>>(a);                     \
  }
  if (p.rows) return hipErrorInvalidValue;  // launched with its epilogue by the caller
  if (p.kg == 2) {  // two wave groups, a ring two units deep
#define WH_GK(BK)                                                                             \
  if (p.bm == 32) gemm_bf3k_kernel<BK, 1, 2, 2><<<p.blocks, 512, 0, s>>>(a);                  \
  else gemm_bf3k_kernel<BK, 2, 2, 2><<<p.blocks, 512, 0, s>>>(a);
    switch (bk) {
    case BK_E4: WH_GK(BK_E4) break;
    case BK_I8: WH_GK(BK_I8) break;
    case BK_FP4: WH_GK(BK_FP4) break;
    case BK_NF4: WH_GK(BK_NF4) break;
    case BK_E5: WH_GK(BK_E5) break;
    default: return hipErrorInvalidValue;
    }
#undef WH_GK
    return hipGetLastError();
  }
  switch (bk) {
  case BK_E4: WH_GB(BK_E4) break;
  case BK_I8: WH_GB(BK_I8) break;
  case BK_FP4: WH_GB(BK_FP4) break;
  case BK_NF4: WH_GB(BK_NF4) break;
  case BK_E5: WH_GB(BK_E5) break;
  default: return hipErrorInvalidValue;
  }
#undef WH_GB
  return hipGetLastError();
}

// gemv_loopb_kernel launch: R = 16 / (B * C) rows per group (16 sums per
// group through the butterfly) and a fixed grid walking the row groups.
// Knob 20 at k >= 2: k waves per CU.  Auto: at B = 2 (no prefetch) 16 waves
// per CU for rows of at most 4096 inputs, else 12 (past 4 waves at most half
// the group count); from B = 4 on as many blocks as the CUs hold at once (the
// occupancy query), but at least two row groups per block, so the prefetch
// has a next group (measured on FP8, FP4 and NF4 at 4096^2, 4096 -> 11008
// and 11008 -> 4096: it picks the best of 4, 8, 12 and 16 waves per CU).
// gemm_regx_kernel for plan p: dynamic LDS for the x image, allowed past the
// default per-launch limit once per kernel.
template <int F>
hipError_t launch_regx(const SkPlan &p, const GemmArgs &a, const double *bias, int bias_len, int act,
                       float *pre, float *post, hipStream_t s) {
  constexpr size_t lds = (size_t)16 * (kRegxMaxK + 4) * sizeof(float);
  static const hipError_t attr = hipFuncSetAttribute((const void *)gemm_regx_kernel<F, 8>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  gemm_regx_kernel<F, 8><<<dim3(p.gx, p.gy), 512, lds, s>>>(a, bias, bias_len, act, pre, post);
  return hipGetLastError();
}

// gemm_regt_kernel with dpre in LDS (batch <= 16, rows <= kRegtxMaxK).
template <int F>
hipError_t launch_regtx(const GemmArgs &a, float *dX, const float *next_pre, int next_act, hipStream_t s) {
  constexpr int kMax = (int)(16 * (kRegtxMaxK + 4) * sizeof(float));
  static const hipError_t attr_t = hipFuncSetAttribute((const void *)gemm_regt_kernel<F, 8, true, true>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, kMax);
  static const hipError_t attr_f = hipFuncSetAttribute((const void *)gemm_regt_kernel<F, 8, false, true>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, kMax);
  if (attr_t != hipSuccess) return attr_t;
  if (attr_f != hipSuccess) return attr_f;
  constexpr size_t lds = kMax;
  if (next_pre != nullptr)
    gemm_regt_kernel<F, 8, true, true><<<dim3(a.gx, a.gy), 512, lds, s>>>(a, dX, next_pre, next_act);
  else
    gemm_regt_kernel<F, 8, false, true><<<dim3(a.gx, a.gy), 512, lds, s>>>(a, dX, nullptr, -1);
  return hipGetLastError();
}

template <int F, int C, int R, int B>
hipError_t launch_loopb(const GemvArgs &a, int batch, int S, hipStream_t s) {
  const int ngroups = (a.N + R - 1) / R;
  const int threads = 64 * S;
  const int k = knob(kTuneGemvBatch);
  int blocks;
  if (k >= 2) {
    blocks = k * num_cus() / S;
  } else if (B == 2) {
    // rows of at most 4096 inputs (x of both batch rows in at most 32 KB per
    // block): 16 waves per CU (4096 -> 11008 FP8 10.5 against 11.1 us at 12,
    // 4096^2 Float16 7.4 against 8.4); longer rows 12, and past 4 waves at
    // least two groups per block (x: 88 KB per block at 11008 inputs; NF4
    // 11008 -> 4096 13.0 against 15.6 us, FP4 11.2 against 12.8)
    const bool short_x = a.K <= 4096;
    blocks = (short_x ? 16 : 12) * num_cus() / S;
    if (!short_x && S > 4) blocks = std::min(blocks, (ngroups + 1) / 2);
  } else {
    // resident blocks per CU, per waves-per-block count (the kernel's
    // register count fixes it; queried once per instantiation; concurrent
    // first calls may both query and store the same value)
    static int per_cu[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
    if (per_cu[S] == 0) {
      int nb = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, gemv_loopb_kernel<F, C, R, B>, threads, 0) !=
          hipSuccess) {
        (void)hipGetLastError();  // a failed query must not read as a failed launch
        nb = 1;
      }
      per_cu[S] = std::max(nb, 1);
    }
    blocks = std::min(per_cu[S] * num_cus(), (ngroups + 1) / 2);
  }
  blocks = std::max(1, std::min(ngroups, blocks));
  gemv_loopb_kernel<F, C, R, B><<<blocks, threads, 0, s>>>(a, batch);
  return hipGetLastError();
}

// One instantiation per (B, C) whose x takes at most 128 registers per lane
// (B * C * E <= 128), the shapes gemv_batch_shape can choose.
template <int F>
hipError_t launch_gemv_batch(const GemvArgs &a, int batch, const GemvBatchShape &sh, hipStream_t s) {
  constexpr int E = FI<F>::kE;
  const int key = sh.B * 10 + sh.C;
  if (key == 21) return launch_loopb<F, 1, 8, 2>(a, batch, sh.S, s);
  if constexpr (4 * E <= 128) {
    if (key == 22) return launch_loopb<F, 2, 4, 2>(a, batch, sh.S, s);
    if (key == 41) return launch_loopb<F, 1, 4, 4>(a, batch, sh.S, s);
  }
  if constexpr (8 * E <= 128) {
    if (key == 42) return launch_loopb<F, 2, 2, 4>(a, batch, sh.S, s);
    if (key == 81) return launch_loopb<F, 1, 2, 8>(a, batch, sh.S, s);
  }
  if constexpr (8 * E <= 128) {
    if (key == 24) return launch_loopb<F, 4, 2, 2>(a, batch, sh.S, s);
  }
  if constexpr (16 * E <= 128) {
    if (key == 82) return launch_loopb<F, 2, 1, 8>(a, batch, sh.S, s);
    if (key == 44) return launch_loopb<F, 4, 1, 4>(a, batch, sh.S, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_forward(const DevStore &w, int batch, const float *x, const double *bias,
                          int bias_len, int act, float *pre, float *post, void *ws, size_t ws_bytes,
                          hipStream_t s) {
  const int route = fwd_route(w, batch);
  const int f = kernel_fmt(w.dtype);
  if (kernel_body(w, f) == nullptr) return hipErrorInvalidValue;
  const bool batched = route == 1 && batch > 1 && gemv_batch_fits(w, batch);
  if (route == 3 || (route == 1 && batch > 4 && !batched)) {
#define WH_GEN(D)                                                                        \
  gemv_generic_kernel<D><<<w.rows, 256, 0, s>>>(w, batch, x, bias, bias_len, act, pre, post); \
  return hipGetLastError();
    WH_DT_SWITCH(w.dtype, WH_GEN)
#undef WH_GEN
  }
  if (route == 1) {
    GemvArgs a{kernel_body(w, f), w.lut, w.scale, w.minv, x, w.cols, w.rows, w.cols / fmt_chunk_elems(f),
               row_bytes_of(w), bias, bias_len, act, pre, post};
    if (batch == 1) {
      // (C, R): chunks per lane and rows per block.  The fewest chunks per
      // lane that cover a row with at most 4 waves, and 8 / C rows; for FP8 /
      // Int8 rows of one chunk per lane and for 4-bit rows that two chunks
      // per lane cover, 4 rows (measured best: more blocks in flight for the
      // heavier FP8 decode, one wave per block for 4-bit).  wpc: waves per CU
      // of a fixed grid walking the row groups (0 = one block per group, -1 =
      // the format's default)
      int C = 1, R = 0, wpc = -1;
      while (C < 8 && (a.nchunks + 64 * C - 1) / (64 * C) > 4) C *= 2;
      if ((f == FE4 || f == FE5 || f == FI8) && C == 1) R = 4;
      if (f == FL4P && a.nchunks <= 128) C = 2, R = 4;
      // pair-table rows of at most two waves of one chunk per lane, with
      // more 4-row groups than 16 waves per CU hold: one chunk per lane in
      // the fixed-grid loop (measured at 4096 -> 11008: 8.90-8.96 against
      // 9.22-9.30 us with two chunks per lane, one block per group)
      if (f == FL4P && a.nchunks <= 128 && 16 * num_cus() / ((a.nchunks + 63) / 64) < (a.N + 3) / 4)
        C = 1, R = 4, wpc = 16;
      // rows of 5-8 waves of one chunk per lane (8224-16384 inputs of a
      // 4-bit format): NF4 one chunk per lane, 4 rows per group, the loop
      // at 12 waves per CU (11008 -> 4096: 9.5 against 10.2 us); FP8 rows
      // of 5-8 waves of two chunks per lane: two chunks per lane, 8 rows
      // per block, one block per group (11008 -> 4096: 11.3 against
      // 13.3-13.9 us with four chunks per lane)
      {
        const int s1 = (a.nchunks + 63) / 64, s2 = (a.nchunks + 127) / 128;
        if (f == FL4P && s1 >= 5 && s1 <= 8) C = 1, R = 4, wpc = 12;
        if ((f == FE4 || f == FE5) && s1 > 8 && s2 >= 5 && s2 <= 8) C = 2, R = 8, wpc = 0;
      }
      // 4-bit rows that take three or more waves of two chunks per lane
      // (11008-wide inputs): 8 rows per block (measured at 11008 -> 4096:
      // FP4 8.2 against 9.1 us, NF4 10.2 against 10.6 us with 4)
      if ((f == FL4P || f == FF4) && C == 2 && a.nchunks > 256) R = 8;
      const int S = (a.nchunks + 64 * C - 1) / (64 * C);
      if (S <= 8) {
        if (R == 0 || !gemv_extra_rows(f)) R = 8 / C;
        // grid: one block per row group, or (FP8 and FP4 by default) a fixed
        // number of waves per CU walking the row groups, x loaded once each
        const int ngroups = (a.N + R - 1) / R;
        if (wpc < 0) {
          wpc = (f == FE4 || f == FE5 || f == FF4) ? 16 : 0;
          // FP8 rows whose 16-wave grid would hold every row group: 12
          // waves per CU, so the grid walks them (4096^2 config-2 leg:
          // 5.15 against 5.60 us for one block per group)
          if ((f == FE4 || f == FE5) && 16 * num_cus() / S >= ngroups && 12 * num_cus() / S < ngroups)
            wpc = 12;
        }
        const int blocks = wpc > 0 ? std::max(1, std::min(ngroups, wpc * num_cus() / S)) : ngroups;
#define WH_PF(F)                                                                          \
  if constexpr (F == FE4 || F == FE5 || F == FF4 || F == FL4P) {                          \
    /* the loop's shapes; any other takes one block per row group */                     \
    const bool loop = blocks < ngroups && ((C == 1 && (R == 4 || R == 8)) || (C == 2 && R == 4)); \
    if (loop) {                                                                           \
      if (C == 1 && R == 4) gemv_loop_kernel<F, 1, 4><<<blocks, 64 * S, 0, s>>>(a);       \
      else if (C == 1) gemv_loop_kernel<F, 1, 8><<<blocks, 64 * S, 0, s>>>(a);            \
      else gemv_loop_kernel<F, 2, 4><<<blocks, 64 * S, 0, s>>>(a);                        \
      return hipGetLastError();                                                           \
    }                                                                                     \
  }                                                                                       \
  if constexpr (gemv_extra_rows(F)) {                                                     \
    if (C == 1 && R == 4) {                                                               \
      gemv_pf_kernel<F, 1, 4><<<ngroups, 64 * S, 0, s>>>(a);                              \
      return hipGetLastError();                                                           \
    }                                                                                     \
    if (C == 2 && R == 8) {                                                               \
      gemv_pf_kernel<F, 2, 8><<<ngroups, 64 * S, 0, s>>>(a);                              \
      return hipGetLastError();                                                           \
    }                                                                                     \
  }                                                                                       \
  if (C == 1) gemv_pf_kernel<F, 1, 8><<<ngroups, 64 * S, 0, s>>>(a);                      \
  else if (C == 2) gemv_pf_kernel<F, 2, 4><<<ngroups, 64 * S, 0, s>>>(a);                 \
  else if (C == 4) gemv_pf_kernel<F, 4, 2><<<ngroups, 64 * S, 0, s>>>(a);                 \
  else gemv_pf_kernel<F, 8, 1><<<ngroups, 64 * S, 0, s>>>(a);                             \
  return hipGetLastError();
        WH_FMT_SWITCH(f, WH_PF)
#undef WH_PF
      }
    }
    if (batched) {
      GemvBatchShape sh;
      gemv_batch_shape(f, batch, a.nchunks, a.N, sh);
      switch (f) {
      case FE4: return launch_gemv_batch<FE4>(a, batch, sh, s);
      case FE5: return launch_gemv_batch<FE5>(a, batch, sh, s);
      case FI8: return launch_gemv_batch<FI8>(a, batch, sh, s);
      case FF4: return launch_gemv_batch<FF4>(a, batch, sh, s);
      case FL4P: return launch_gemv_batch<FL4P>(a, batch, sh, s);
      case FH16: return launch_gemv_batch<FH16>(a, batch, sh, s);
      case FB16: return launch_gemv_batch<FB16>(a, batch, sh, s);
      case FF32: return launch_gemv_batch<FF32>(a, batch, sh, s);
      case FL8: return launch_gemv_batch<FL8>(a, batch, sh, s);
      case FI16: return launch_gemv_batch<FI16>(a, batch, sh, s);
      case FU16: return launch_gemv_batch<FU16>(a, batch, sh, s);
      case FI32: return launch_gemv_batch<FI32>(a, batch, sh, s);
      case FU32: return launch_gemv_batch<FU32>(a, batch, sh, s);
      case FI64: return launch_gemv_batch<FI64>(a, batch, sh, s);
      case FU64: return launch_gemv_batch<FU64>(a, batch, sh, s);
      case FL1: return launch_gemv_batch<FL1>(a, batch, sh, s);
      case FL2: return launch_gemv_batch<FL2>(a, batch, sh, s);
      case FL3: return launch_gemv_batch<FL3>(a, batch, sh, s);
      case FL5: return launch_gemv_batch<FL5>(a, batch, sh, s);
      case FL6: return launch_gemv_batch<FL6>(a, batch, sh, s);
      default: return hipErrorInvalidValue;
      }
    }
#define WH_GV(F) return gemv_dispatch<F>(batch, a, s);
    WH_FMT_SWITCH(f, WH_GV)
#undef WH_GV
  }
  const int bk = bf3_kind(w);
  const SkPlan p = plan_fwd_gemm(f, bk, batch, w.cols, w.rows);
  if (ws_bytes < p.ws_bytes) return hipErrorInvalidValue;
  GemmArgs a{kernel_body(w, f), w.lut, w.scale, w.minv, x, batch, w.cols, w.rows, row_bytes_of(w),
             p.gx, p.gy, p.nst, p.per_block, p.maxspan, (float *)ws, p.bm, p.bn};
  if (p.bf3) {
    a.post = (bk == BK_I8 || bk == BK_NF4) ? w.scale : 1.0f;
    if (bk == BK_E4 || bk == BK_E5) a.body = w.kbody;
    if (p.rows) return launch_bf3r<true>(p, bk, a, bias, bias_len, act, pre, post, s);
    const hipError_t e = launch_bf3(p, bk, a, s);
    if (e != hipSuccess) return e;
  } else if (p.rows) {
#define WH_GRR(F)                                                                                     \
  if (batch <= 16 && w.cols <= kRegxMaxK && knob(kTuneRegx) != 0)                                   \
    return launch_regx<F>(p, a, bias, bias_len, act, pre, post, s);                                   \
  gemm_regr_kernel<F, 8><<<dim3(p.gx, p.gy), 512, 0, s>>>(a, bias, bias_len, act, pre, post);          \
  break;
    WH_FMT_SWITCH(f, WH_GRR)
#undef WH_GRR
    return hipGetLastError();
  } else if (p.bn == kRegBN) {
#define WH_GR(F)                                                                      \
  if constexpr (FI<F>::kBits <= 16) {                                                 \
    if (p.bm == 32) gemm_reg_kernel<F, 1><<<p.blocks, 256, 0, s>>>(a);                \
    else gemm_reg_kernel<F, 2><<<p.blocks, 256, 0, s>>>(a);                           \
  }                                                                                   \
  break;
    WH_FMT_SWITCH(f, WH_GR)
#undef WH_GR
  } else {
#define WH_GM(F)                                              \
  gemm_sk_kernel<F, false><<<p.blocks, 256, 0, s>>>(a);      \
  break;
    WH_FMT_SWITCH(f, WH_GM)
#undef WH_GM
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  sk_reduce_kernel<true><<<sk_reduce_grid(p), 256, 0, s>>>(a, bias, bias_len, act, pre, post, nullptr);
  return hipGetLastError();
}

bool forward_pair_fits(const DevStore &g, const DevStore &u, int batch) {
  if (batch != 1 || g.dtype != u.dtype || g.rows != u.rows || g.cols != u.cols) return false;
  const int f = kernel_fmt(g.dtype);
  if (!(f == FE4 || f == FE5 || f == FL4P || f == FF4 || f == FI8) || !chunk_aligned(g, g.cols)) return false;
  const int nchunks = g.cols / fmt_chunk_elems(f);
  return (nchunks + 63) / 64 <= 8;
}

hipError_t launch_forward_pair(const DevStore &g, const DevStore &u, const float *x, float *g_pre,
                               float *u_pre, float *h, hipStream_t s) {
  if (!forward_pair_fits(g, u, 1)) return hipErrorInvalidValue;
  const int f = kernel_fmt(g.dtype);
  if (kernel_body(g, f) == nullptr || kernel_body(u, f) == nullptr) return hipErrorInvalidValue;
  GemvPairArgs pa{GemvArgs{kernel_body(g, f), g.lut, g.scale, g.minv, x, g.cols, g.rows,
                           g.cols / fmt_chunk_elems(f), row_bytes_of(g), nullptr, 0, kLinear, g_pre, h},
                  kernel_body(u, f), u.lut, u.scale, u.minv, u_pre};
  // four rows of each per group, the loop GEMV's 16 waves per CU walking the
  // groups (measured at 4096 -> 11008 against the two launches: see the
  // SwiGLU forward)
  constexpr int R = 4;
  const int S = (pa.a.nchunks + 63) / 64, ngroups = (g.rows + R - 1) / R;
  const int blocks = std::max(1, std::min(ngroups, 16 * num_cus() / S));
  switch (f) {
  case FE4: gemv_pair_kernel<FE4, R><<<blocks, 64 * S, 0, s>>>(pa); break;
  case FE5: gemv_pair_kernel<FE5, R><<<blocks, 64 * S, 0, s>>>(pa); break;
  case FL4P: gemv_pair_kernel<FL4P, R><<<blocks, 64 * S, 0, s>>>(pa); break;
  case FF4: gemv_pair_kernel<FF4, R><<<blocks, 64 * S, 0, s>>>(pa); break;
  case FI8: gemv_pair_kernel<FI8, R><<<blocks, 64 * S, 0, s>>>(pa); break;
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

namespace {
// dX routing: 1 = small-batch column kernel, 2 = transposed MFMA GEMM, 3 = generic.
int dx_route(const DevStore &w, int batch) {
  if (!chunk_aligned(w, w.cols)) return 3;
  return batch <= 2 ? 1 : 2;
}
}  // namespace

// dX of the GEMM route as a forward through W^T on the split-x GEMM: the
// weight kinds of one byte per code whose transposed copy the store keeps
// (-1 when dX takes the fp32 MFMA GEMM).
bool dx_rows(const DevStore &w, int batch);

int dx_bf3_kind(const DevStore &w, int batch) {
  if (dx_route(w, batch) != 2 || w.rows % 16 != 0 || dx_rows(w, batch)) return -1;
  const int bk = bf3_kind(w);
  return (bk == BK_E4 || bk == BK_E5 || bk == BK_I8) ? bk : -1;
}

bool backward_wants_transposed(const DevStore &w, int batch) { return dx_bf3_kind(w, batch) >= 0; }

// dX without a k split (gemm_regt_kernel, every format, no transposed copy):
// batch <= 16 and the same rows bound as the forward's no-split GEMMs
// Up to 4096 rows (at most 8192 columns) for the formats whose dX has no
// transposed split-x copy (a training step of a 4096 -> 4096 -> 4096 stack
// at b8: NF4 256 against 240 us, Float32 283 against 255, Int32 298 against
// 270, Uint8 201 against 186, Float16 272 against 263; FP8 and Int8, whose
// dX runs the split-x GEMM over their transposed codes, equal).
bool dx_rows(const DevStore &w, int batch) {
  const int rk = knob(kTuneBf3Rows);
  if (dx_route(w, batch) != 2 || batch > 16 || w.rows % 4 != 0) return false;
  if (rk == 2) return true;
  if (rk != 1) return false;
  if (w.rows <= 2048) return true;
  const int bk = bf3_kind(w);
  const bool transposed = bk == BK_E4 || bk == BK_E5 || bk == BK_I8;
  return !transposed && w.rows <= 4096 && w.cols <= 8192;
}
int dx_rows_stage(int f) {  // RegtShape<F>::ST
  return 4 * (fmt_chunk_elems(f) >= 4 ? 16 : 8);
}

size_t backward_workspace_bytes(const DevStore &w, int batch) {
  const int route = dx_route(w, batch);
  if (route == 1) {
    const int nseg = (w.rows + kDxSegRows - 1) / kDxSegRows;
    return (size_t)nseg * batch * w.cols * sizeof(float);
  }
  if (route == 2) {
    // either plan (the transposed copy may be refreshed after sizing)
    size_t b = plan_sk(batch, w.rows, w.cols).ws_bytes;
    const int bk = dx_bf3_kind(w, batch);
    if (bk >= 0) b = std::max(b, plan_fwd_gemm(kernel_fmt(w.dtype), bk, batch, w.rows, w.cols).ws_bytes);
    return b;
  }
  return 0;
}

bool dw_batchable(const DevStore &w) {
  return w.rows % 128 == 0 && w.cols % 128 == 0;
}

// Deferring a layer's dW into a batched launch pays where the layer alone
// leaves CUs idle (fewer 128x128 tiles than CUs: config 5's 1024^2 layers,
// 64 tiles, 130-145 us less per step); a layer that fills the GPU runs alone
// (config 4's 2048 x 8192 layers, 1024 tiles each: 50 us per step slower
// batched).
bool dw_defer_pays(const DevStore &w) {
  return dw_batchable(w) && (int64_t)(w.rows / 128) * (w.cols / 128) < num_cus();
}

hipError_t launch_dw_batch(const DwBatch &b, hipStream_t s) {
  if (b.count < 1 || b.count > kDwBatch || b.batch < 1) return hipErrorInvalidValue;
  int gx = 0, gy = 0;
  for (int i = 0; i < b.count; ++i) {
    const DwJob &t = b.job[i];
    if (t.dpre == nullptr || t.x == nullptr || t.dW == nullptr || t.rows % 128 || t.cols % 128 ||
        t.rows < 128 || t.cols < 128)
      return hipErrorInvalidValue;
    gx = std::max(gx, t.cols / 128);
    gy = std::max(gy, t.rows / 128);
  }
  dw_batch_kernel<<<dim3(gx, gy, b.count), 256, 0, s>>>(b);
  return hipGetLastError();
}

// The dX kernels whose epilogue applies the lower layer's derivative: the
// no-split gemm_regt_kernel and the reduction of the stream-K GEMMs
// (sk_reduce_kernel); not the transposed no-split bf3r epilogue.
bool backward_dx_applies_next(const DevStore &w, int batch, int next_act) {
  if (knob(kTuneFoldDeriv) == 0 || !act_piecewise(next_act)) return false;
  if (dx_rows(w, batch)) return true;
  if (dx_route(w, batch) != 2) return false;
  const int bk = dx_bf3_kind(w, batch);
  return bk < 0 || !plan_fwd_gemm(kernel_fmt(w.dtype), bk, batch, w.rows, w.cols).rows;
}

hipError_t launch_backward(const DevStore &w, int batch, const float *x, const float *pre,
                           const float *gy, int act, float *dpre_buf, float *dX, float *dW, int *flag,
                           void *ws, size_t ws_bytes, hipStream_t s, const BackwardChain &chain) {
  const int64_t ny = (int64_t)batch * w.rows;
  // dpre = gy * act'(pre); act' is 1 for Linear (and the ids act_prime
  // treats as Linear), where gy * 1 = gy bit for bit: the kernel is skipped,
  // as it is when the layer above formed dpre in its dX epilogue
  const bool identity = act < kReLU || act > kReLU2;
  const float *dpre = identity || chain.gy_is_dpre ? gy : dpre_buf;
  if (!identity && !chain.gy_is_dpre)
    act_deriv_kernel<<<blocks_for(ny), 256, 0, s>>>(gy, pre, ny, act, dpre_buf);
  if (chain.dx_next_pre != nullptr && (dX == nullptr || !backward_dx_applies_next(w, batch, chain.dx_next_act)))
    return hipErrorInvalidValue;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int route = dx_route(w, batch);
  const int f = kernel_fmt(w.dtype);
  if (kernel_body(w, f) == nullptr) return hipErrorInvalidValue;
  if (ws_bytes < backward_workspace_bytes(w, batch)) return hipErrorInvalidValue;
  if (dX == nullptr) {
    // no input gradient wanted (the first layer of a training step)
  } else if (route == 3) {
#define WH_DXG(D)                                                                         \
  dx_generic_kernel<D><<<blocks_for((int64_t)batch * w.cols), 256, 0, s>>>(w, batch, dpre, dX); \
  break;
    WH_DT_SWITCH(w.dtype, WH_DXG)
#undef WH_DXG
  } else if (route == 1) {
    const int nseg = (w.rows + kDxSegRows - 1) / kDxSegRows;
    DxArgs a{kernel_body(w, f), w.lut, w.scale, w.minv, dpre, w.rows, w.cols, w.cols / fmt_chunk_elems(f),
             kDxSegRows, nseg, row_bytes_of(w), (float *)ws};
    dim3 grid((a.nchunks + 255) / 256, nseg);
#define WH_DXS(F)                                                  \
  if (batch == 1) dx_small_kernel<F, 1><<<grid, 256, 0, s>>>(a);   \
  else dx_small_kernel<F, 2><<<grid, 256, 0, s>>>(a);              \
  break;
    WH_FMT_SWITCH(f, WH_DXS)
#undef WH_DXS
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    reduce_plain_kernel<<<blocks_for((int64_t)batch * w.cols), 256, 0, s>>>(
        (const float *)ws, nseg, (int64_t)batch * w.cols, dX);
  } else if (dx_bf3_kind(w, batch) >= 0 && w.tbody != nullptr) {
    // dX[b][i] = sum_o dpre[b][o] W[o][i]: the forward product through the
    // transposed codes W^T [cols][rows] (rows bytes per row)
    const int bk = dx_bf3_kind(w, batch);
    const SkPlan p = plan_fwd_gemm(f, bk, batch, w.rows, w.cols);
    GemmArgs a{w.tbody, w.lut, w.scale, w.minv, dpre, batch, w.rows, w.cols, (int64_t)w.rows,
               p.gx, p.gy, p.nst, p.per_block, p.maxspan, (float *)ws, p.bm, p.bn};
    a.post = bk == BK_I8 ? w.scale : 1.0f;
    if (p.rows) {
      e = launch_bf3r<false>(p, bk, a, nullptr, 0, -1, dX, nullptr, s);
    } else {
      e = launch_bf3(p, bk, a, s);
      if (e != hipSuccess) return e;
      sk_reduce_kernel<false><<<sk_reduce_grid(p), 256, 0, s>>>(a, nullptr, 0, chain.dx_next_act, dX, nullptr,
                                                                chain.dx_next_pre);
    }
  } else if (dx_rows(w, batch)) {
    const int st = dx_rows_stage(f);
    GemmArgs a{kernel_body(w, f), w.lut, w.scale, w.minv, dpre, batch, w.rows, w.cols, row_bytes_of(w),
               (w.cols + 15) / 16, (batch + 15) / 16, (w.rows + st - 1) / st, 0, 1, nullptr, 16, 16};
#define WH_DXR(F)                                                                                   \
  if (batch <= 16 && w.rows <= kRegtxMaxK && knob(kTuneRegx) != 0) {                              \
    e = launch_regtx<F>(a, dX, chain.dx_next_pre, chain.dx_next_act, s);                            \
    if (e != hipSuccess) return e;                                                                  \
    break;                                                                                          \
  }                                                                                                 \
  if (chain.dx_next_pre != nullptr)                                                                 \
    gemm_regt_kernel<F, 8, true><<<dim3(a.gx, a.gy), 512, 0, s>>>(a, dX, chain.dx_next_pre,          \
                                                                  chain.dx_next_act);               \
  else                                                                                              \
    gemm_regt_kernel<F, 8, false><<<dim3(a.gx, a.gy), 512, 0, s>>>(a, dX, nullptr, -1);              \
  break;
    WH_FMT_SWITCH(f, WH_DXR)
#undef WH_DXR
  } else {
    const SkPlan p = plan_sk(batch, w.rows, w.cols);
    GemmArgs a{kernel_body(w, f), w.lut, w.scale, w.minv, dpre, batch, w.rows, w.cols, row_bytes_of(w),
               p.gx, p.gy, p.nst, p.per_block, p.maxspan, (float *)ws, p.bm, p.bn};
#define WH_DXM(F)                                           \
  gemm_sk_kernel<F, true><<<p.blocks, 256, 0, s>>>(a);     \
  break;
    WH_FMT_SWITCH(f, WH_DXM)
#undef WH_DXM
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    sk_reduce_kernel<false><<<sk_reduce_grid(p), 256, 0, s>>>(a, nullptr, 0, chain.dx_next_act, dX, nullptr,
                                                              chain.dx_next_pre);
  }
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (chain.dpre_out != nullptr) *chain.dpre_out = dpre;
  if (chain.defer_dw) {
    if (!dw_batchable(w)) return hipErrorInvalidValue;
    return hipGetLastError();  // the caller launches this dW with others (launch_dw_batch)
  }
  if (dw_batchable(w)) {
    dim3 g2(w.cols / 128, w.rows / 128);
    dw_mfma_lds_kernel<<<g2, 256, 0, s>>>(dpre, x, batch, w.rows, w.cols, dW, flag);
  } else {
    dim3 g2((w.cols + 127) / 128, (w.rows + 127) / 128);
    dw_mfma_kernel<<<g2, 256, 0, s>>>(dpre, x, batch, w.rows, w.cols, dW, flag);
  }
  return hipGetLastError();
}

// transpose_u8_kernel for rows a multiple of 64 and cols of 256 (every tile
// whole): a 64 x 256-byte tile goes through LDS as 4-byte words; each thread
// reads a 16 x 4 byte block (one word column of 16 input rows), transposes
// its four 4 x 4 blocks in registers and writes four 16-byte pieces of four
// output rows; the 4 threads of one word column write 64 contiguous bytes of
// each of its output rows.
__global__ void __launch_bounds__(256) transpose_u8_tile_kernel(const uint8_t *__restrict__ in, int rows,
                                                                int cols, uint8_t *__restrict__ out) {
  __shared__ uint32_t t[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 256, tid = threadIdx.x;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int lr = k * 16 + (tid >> 4), lw = (tid & 15) * 4;  // 16 pieces of 16 bytes per row
    const uint4 v = *(const uint4 *)(in + (int64_t)(r0 + lr) * cols + c0 + lw * 4);
    t[lr][lw] = v.x;
    t[lr][lw + 1] = v.y;
    t[lr][lw + 2] = v.z;
    t[lr][lw + 3] = v.w;
  }
  __syncthreads();
  const int rb = tid & 3, a = tid >> 2;  // input rows 16rb..16rb+15, input columns 4a..4a+3
  uint32_t w[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) w[k] = t[16 * rb + k][a];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      o[q] = ((w[4 * q] >> (8 * j)) & 0xffu) | (((w[4 * q + 1] >> (8 * j)) & 0xffu) << 8) |
             (((w[4 * q + 2] >> (8 * j)) & 0xffu) << 16) | (((w[4 * q + 3] >> (8 * j)) & 0xffu) << 24);
    *(uint4 *)(out + (int64_t)(c0 + 4 * a + j) * rows + r0 + 16 * rb) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

hipError_t launch_transpose_u8(const uint8_t *in, int rows, int cols, uint8_t *out, hipStream_t s) {
  if (rows % 64 == 0 && cols % 256 == 0)
    transpose_u8_tile_kernel<<<dim3(cols / 256, rows / 64), 256, 0, s>>>(in, rows, cols, out);
  else
    transpose_u8_kernel<<<dim3((cols + 63) / 64, (rows + 63) / 64), 256, 0, s>>>(in, rows, cols, out);
  return hipGetLastError();
}

size_t mse_workspace_bytes(int64_t n) {
  (void)n;
  return 1024 * sizeof(double);
}

hipError_t launch_swiglu_bwd(const float *gate, const float *up, const float *gh, int64_t n,
                             float *d_up, float *d_gate, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  swiglu_bwd_kernel<<<blocks_for(n), 256, 0, s>>>(gate, up, gh, n, d_up, d_gate);
  return hipGetLastError();
}

hipError_t launch_add(const float *a, const float *b, int64_t n, float *out, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  add_kernel<<<blocks_for(n), 256, 0, s>>>(a, b, n, out);
  return hipGetLastError();
}

namespace {
// Streaming-read probe: each thread loads four 16-byte words 4 KB apart
// (non-temporal, all four in flight before any use) and folds them into one
// value; a store that only the value 0x9e3779b9 reaches keeps the loads live
// without writing anything in practice.  The bytes are read once in one
// launch: the floor for a kernel that streams the same bytes once.
__global__ void __launch_bounds__(256) read_probe_kernel(const uint4 *__restrict__ p, int64_t n16,
                                                         uint32_t *sink) {
  const int64_t i = (int64_t)blockIdx.x * 1024 + threadIdx.x;
  typedef uint32_t u4v __attribute__((ext_vector_type(4)));
  u4v v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t k = min(i + 256 * j, n16 - 1);
    v[j] = __builtin_nontemporal_load((const u4v *)(p + k));
  }
  uint32_t acc = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) acc ^= v[j][0] ^ v[j][1] ^ v[j][2] ^ v[j][3];
  if (acc == 0x9e3779b9u) sink[blockIdx.x & 1023] = acc;
}
}  // namespace

hipError_t launch_read_probe(const void *p, int64_t bytes, uint32_t *sink, hipStream_t s) {
  const int64_t n16 = bytes / 16;
  if (n16 <= 0) return hipErrorInvalidValue;
  const int64_t blocks = (n16 + 1023) / 1024;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  read_probe_kernel<<<(unsigned)blocks, 256, 0, s>>>((const uint4 *)p, n16, sink);
  return hipGetLastError();
}

hipError_t launch_mse(const float *pred, const float *target, int64_t n, double *loss, float *grad,
                      void *ws, size_t ws_bytes, hipStream_t s, int *clear, int64_t nclear) {
  if (ws_bytes < mse_workspace_bytes(n)) return hipErrorInvalidValue;
  if (nclear > 0 && (clear == nullptr || loss == nullptr)) return hipErrorInvalidValue;
  if (loss != nullptr) {
    int parts = blocks_for(n);
    if (parts > 1024) parts = 1024;
    mse_partial_kernel<<<parts, 256, 0, s>>>(pred, target, n, (double *)ws);
    mse_final_kernel<<<1, 256, 0, s>>>((const double *)ws, parts, n, loss, clear, nclear > 0 ? nclear : 0);
  }
  if (grad != nullptr) mse_grad_kernel<<<blocks_for(n), 256, 0, s>>>(pred, target, n, grad);
  return hipGetLastError();
}

}  // namespace wh
