// codec.hip — device encode (pack with fresh per-tensor statistics), decode
// (export_f32), decode tables, and the SGD update with fixed-scale re-encode.
//
// These replace the reference's host pack_native / weight_at loops
// (native_codec.cpp:189-813) and its single-thread op_native_sgd
// (ops_storage.metal:924-958) with one-thread-per-unit HBM-streaming kernels.
// A unit is the smallest group of elements that owns whole bytes, so no two
// threads ever write the same byte.
#include <algorithm>

#include "codec.hpp"
#include "kernels.hpp"

namespace wh {
namespace {

constexpr int kThreads = 256;

inline int grid_for(int64_t units) {
  int64_t g = (units + kThreads - 1) / kThreads;
  if (g > 65536) g = 65536;
  return (int)(g < 1 ? 1 : g);
}

// Order-preserving map of a non-NaN float to uint32 with -0 folded onto +0,
// so that equal values compare equal and the element index breaks ties.
__device__ inline uint32_t sortable(float v) {
  const uint32_t u = f2u(v == 0.0f ? 0.0f : v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// abs_max (native_codec.cpp:22-30) and min_max (:32-40) in one pass.  The
// sequential min/max keep the first element that attains the extreme value;
// the (value, index) keys reproduce that, including the sign of a zero.
__global__ void __launch_bounds__(kThreads) stats_kernel(const float *__restrict__ w, int64_t n,
                                                         Stats *acc) {
  float am = 0.0f;
  uint64_t kmin = ~0ull, kmax = 0ull;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    const float v = w[i];
    const float a = fabsf(v);
    if (a > am) am = a;
    if (v == v) {
      const uint64_t key = (uint64_t)sortable(v) << 32;
      const uint64_t lo = key | (uint32_t)i, hi = key | (0xffffffffu - (uint32_t)i);
      kmin = lo < kmin ? lo : kmin;
      kmax = hi > kmax ? hi : kmax;
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
    const float o = __shfl_xor(am, off);
    am = o > am ? o : am;
    const uint64_t a = __shfl_xor(kmin, off), b = __shfl_xor(kmax, off);
    kmin = a < kmin ? a : kmin;
    kmax = b > kmax ? b : kmax;
  }
  __shared__ float s_am[kThreads / 64];
  __shared__ uint64_t s_min[kThreads / 64], s_max[kThreads / 64];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_am[wave] = am;
    s_min[wave] = kmin;
    s_max[wave] = kmax;
  }
  __syncthreads();
  if (threadIdx.x == 0) {  // one atomic triple per block
    for (int i = 1; i < kThreads / 64; ++i) {
      am = s_am[i] > am ? s_am[i] : am;
      kmin = s_min[i] < kmin ? s_min[i] : kmin;
      kmax = s_max[i] > kmax ? s_max[i] : kmax;
    }
    atomicMax(&acc->absmax_bits, f2u(am));  // non-negative: bit order == value order
    atomicMin(&acc->minkey, (unsigned long long)kmin);
    atomicMax(&acc->maxkey, (unsigned long long)kmax);
  }
}

__global__ void stats_init_kernel(Stats *acc) {
  acc->absmax_bits = 0;
  acc->minkey = ~0ull;
  acc->maxkey = 0ull;
}

// Per-dtype scale rules of pack_native (native_codec.cpp:148-560).
template <int DT>
__global__ void finalize_kernel(const float *__restrict__ w, const Stats *acc, Meta *meta) {
  const float absmax = u2f(acc->absmax_bits);
  float mn, mx;
  if (w[0] != w[0]) {
    mn = mx = w[0];  // the sequential scan never leaves a NaN first element
  } else {
    mn = w[(uint32_t)acc->minkey];
    mx = w[0xffffffffu - (uint32_t)acc->maxkey];
  }
  Meta m{1.0f, 1.0f, 0.0f, 0.0f};
  if constexpr (DT == kInt64 || DT == kInt || DT == kInt32 || DT == kInt16) {
    float s = absmax;
    if (s == 0) s = 1;
    m.s = s;
    m.scale = s / (DT == kInt32 ? 2147483647.0f : (DT == kInt16 ? 32767.0f : 1e6f));
  } else if constexpr (DT == kInt8 || DT == kInt4 || DT == kInt6 || DT == kFP6 || DT == kInt5 ||
                       DT == kInt3) {
    constexpr int bits = dtype_bits(DT);
    float s = absmax / (float)((1 << (bits - 1)) - 1);
    if (s == 0) s = 1;
    m.s = m.scale = s;
  } else if constexpr (DT == kInt2 || DT == kTernary || DT == kBinary || DT == kNF4) {
    float s = absmax;
    if (s == 0) s = 1;
    m.s = m.scale = s;
  } else if constexpr (dtype_has_min(DT)) {
    float span = mx - mn;
    if (span == 0) span = 1;
    float k;
    if constexpr (DT == kUint8) k = 255.0f;
    else if constexpr (DT == kUint16) k = 65535.0f;
    else if constexpr (DT == kUint32) k = 4294967296.0f;  // float(4294967295u)
    else if constexpr (DT == kUint2) k = 3.0f;
    else if constexpr (DT == kUint64 || DT == kUint || DT == kUintptr) k = 1e15f;
    else k = (float)((1 << dtype_bits(DT)) - 1);
    m.s = span;
    m.minv = mn;
    m.scale = span / k;
  }
  *meta = m;
}

// The statistics of op_native_repack ops_storage.metal:983-1024: Metal's
// max / min return the other operand of a NaN, so NaN elements (element 0
// included) never become the min or max; with no number at all min = max =
// NaN.  Scale rules as pack's (the same divisors; Int8 / Int4 / n-bit use the
// absmax, 0 -> 1).
template <int DT>
__global__ void repack_finalize_kernel(const float *__restrict__ w, const Stats *acc, Meta *meta) {
  const float absmax = u2f(acc->absmax_bits);
  float mn = __builtin_nanf(""), mx = mn;
  if (acc->minkey != ~0ull) {
    mn = w[(uint32_t)acc->minkey];
    mx = w[0xffffffffu - (uint32_t)acc->maxkey];
  }
  Meta m{1.0f, 1.0f, 0.0f, 0.0f};
  if constexpr (DT == kInt64 || DT == kInt || DT == kInt32 || DT == kInt16) {
    float s = absmax;
    if (s == 0) s = 1;
    m.s = s;
    m.scale = s / (DT == kInt32 ? 2147483647.0f : (DT == kInt16 ? 32767.0f : 1e6f));
  } else if constexpr (DT == kInt8 || DT == kInt4 || DT == kInt6 || DT == kFP6 || DT == kInt5 ||
                       DT == kInt3) {
    constexpr int bits = dtype_bits(DT);
    float s = absmax / (float)((1 << (bits - 1)) - 1);
    if (s == 0) s = 1;
    m.s = m.scale = s;
  } else if constexpr (DT == kInt2 || DT == kTernary || DT == kBinary || DT == kNF4) {
    float s = absmax;
    if (s == 0) s = 1;
    m.s = m.scale = s;
  } else if constexpr (dtype_has_min(DT)) {
    float span = mx - mn;
    if (span == 0) span = 1;
    float k;
    if constexpr (DT == kUint8) k = 255.0f;
    else if constexpr (DT == kUint16) k = 65535.0f;
    else if constexpr (DT == kUint32) k = 4294967296.0f;  // float(4294967295)
    else if constexpr (DT == kUint2) k = 3.0f;
    else if constexpr (DT == kUint64 || DT == kUint || DT == kUintptr) k = 1e15f;
    else k = (float)((1 << dtype_bits(DT)) - 1);
    m.s = span;
    m.minv = mn;
    m.scale = span / k;
  }
  *meta = m;
}

template <int DT, bool REPACK = false>
__global__ void __launch_bounds__(kThreads) pack_kernel(const float *__restrict__ w, int64_t n,
                                                        uint8_t *__restrict__ body,
                                                        uint8_t *__restrict__ kbody,
                                                        const Meta *__restrict__ meta) {
  constexpr int bits = dtype_bits(DT);
  constexpr int U = unit_elems<DT>();
  const Meta m = *meta;
  const int64_t units = (n + U - 1) / U;
  for (int64_t u = (int64_t)blockIdx.x * kThreads + threadIdx.x; u < units;
       u += (int64_t)gridDim.x * kThreads) {
    if constexpr (bits >= 8) {
      const uint64_t c = REPACK ? repack_code<DT>(w[u], m) : pack_code<DT>(w[u], m);
      if constexpr (has_kcopy<DT>()) kbody[u] = kcode<DT>((uint32_t)c);
      if constexpr (bits == 8) body[u] = (uint8_t)c;
      else if constexpr (bits == 16) ((uint16_t *)body)[u] = (uint16_t)c;
      else if constexpr (bits == 32) ((uint32_t *)body)[u] = (uint32_t)c;
      else if constexpr (bits == 64) {
        ((uint32_t *)body)[2 * u] = (uint32_t)c;
        ((uint32_t *)body)[2 * u + 1] = (uint32_t)(c >> 32);
      } else {
        uint32_t *p = (uint32_t *)body + 4 * u;
        p[0] = (uint32_t)c;
        p[1] = (uint32_t)(c >> 32);
        p[2] = 0;
        p[3] = 0;
      }
    } else {
      uint64_t acc = 0;
#pragma unroll
      for (int j = 0; j < U; ++j) {
        const int64_t i = u * U + j;
        if (i < n) acc |= (REPACK ? repack_code<DT>(w[i], m) : pack_code<DT>(w[i], m)) << (j * bits);
      }
      constexpr int ubytes = U * bits / 8;
#pragma unroll
      for (int b = 0; b < ubytes; ++b) body[u * ubytes + b] = (uint8_t)(acc >> (8 * b));
    }
  }
}

template <int DT>
__global__ void __launch_bounds__(kThreads) decode_kernel(const uint8_t *__restrict__ body, int64_t n,
                                                          float scale, float minv,
                                                          float *__restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads)
    out[i] = dec_code<DT>(load_code<DT>(body, i), scale, minv);
}

template <int DT>
__global__ void lut_kernel(float scale, float minv, float *lut) {
  const int c = threadIdx.x;
  if (c < (1 << dtype_bits(DT))) lut[c] = dec_code<DT>((uint64_t)c, scale, minv);
  if constexpr (dtype_bits(DT) == 4) {  // byte c = codes (c & 15, c >> 4)
    lut[kPairLut + 2 * c] = dec_code<DT>((uint64_t)(c & 15), scale, minv);
    lut[kPairLut + 2 * c + 1] = dec_code<DT>((uint64_t)(c >> 4), scale, minv);
  }
}

// op_native_sgd ops_storage.metal:924-958 with the f64 contract: each element
// becomes fl32(old - lr*g) re-encoded with the stored scale/min; element 0 is
// first decoded and re-encoded once (the reference's probe, :941-945).
template <int DT>
__device__ inline float sgd_value(uint64_t code, int64_t i, float g, double lr, float scale, float minv) {
  float old = dec_code<DT>(code, scale, minv);
  if (i == 0) old = dec_code<DT>(fix_code<DT>(old, scale, minv), scale, minv);
  return (float)((double)old - lr * (double)g);
}

// True when an SGD launch must leave the weights alone: an earlier cell's
// step stopped (*stop != 0), or this cell's gradient holds a non-finite value
// (*bad != 0, found by the kernel that produced it), which then sets the
// stop code for this and every later cell.
__device__ inline bool sgd_stopped(int *stop, const int *bad, int bad_value) {
  if (bad != nullptr && *bad != 0) {
    if (stop != nullptr && blockIdx.x == 0 && threadIdx.x == 0) atomicCAS(stop, 0, bad_value);
    return true;
  }
  return stop != nullptr && *stop != 0;
}

// The SGD of unit u (unit_elems elements, so no two threads touch a byte).
template <int DT>
__device__ inline void sgd_unit(uint8_t *__restrict__ body, uint8_t *__restrict__ kbody, int64_t n,
                                const float *__restrict__ g, double lr, float scale, float minv, int64_t u) {
  constexpr int bits = dtype_bits(DT);
  constexpr int U = unit_elems<DT>();
  if constexpr (bits >= 8) {
    const uint64_t c = fix_code<DT>(sgd_value<DT>(load_code<DT>(body, u), u, g[u], lr, scale, minv),
                                    scale, minv);
    constexpr int fb = fix_bytes<DT>();
    if constexpr (has_kcopy<DT>()) kbody[u] = kcode<DT>((uint32_t)c);
    if constexpr (fb == 1) body[u] = (uint8_t)c;
    else if constexpr (fb == 2) ((uint16_t *)body)[u] = (uint16_t)c;
    else if constexpr (fb == 4) ((uint32_t *)(body + u * (bits / 8)))[0] = (uint32_t)c;
    else {
      uint32_t *p = (uint32_t *)(body + u * (bits / 8));
      p[0] = (uint32_t)c;
      p[1] = (uint32_t)(c >> 32);
    }
  } else {
    constexpr int ubytes = U * bits / 8;
    uint64_t acc = 0;
#pragma unroll
    for (int b = 0; b < ubytes; ++b) acc |= (uint64_t)body[u * ubytes + b] << (8 * b);
    constexpr uint64_t mask = (1ull << bits) - 1;
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int64_t i = u * U + j;
      if (i < n) {
        const uint64_t c = (acc >> (j * bits)) & mask;
        const uint64_t nc = fix_code<DT>(sgd_value<DT>(c, i, g[i], lr, scale, minv), scale, minv);
        acc = (acc & ~(mask << (j * bits))) | ((nc & mask) << (j * bits));
      }
    }
#pragma unroll
    for (int b = 0; b < ubytes; ++b) body[u * ubytes + b] = (uint8_t)(acc >> (8 * b));
  }
}

// The SGD element loops below take their block index and block count as
// arguments: one launch per store (the block grid) or one launch for several
// stores (sgd_batch_kernel: blockIdx.y picks the store).
template <int DT>
__device__ inline void sgd_units(uint8_t *__restrict__ body, uint8_t *__restrict__ kbody, int64_t n,
                                 const float *__restrict__ g, double lr, float scale, float minv,
                                 int64_t blk, int64_t nblk) {
  constexpr int U = unit_elems<DT>();
  const int64_t units = (n + U - 1) / U;
  for (int64_t u = blk * kThreads + threadIdx.x; u < units; u += nblk * kThreads)
    sgd_unit<DT>(body, kbody, n, g, lr, scale, minv, u);
}

// Elements per thread of sgdw_units: a whole number of 32-bit code words —
// 16 (`bits` / 2 words) for the 2-, 4- and 6-bit formats, 32 (`bits` words)
// for the 1-, 3- and 5-bit ones, 8 for the 16-bit ones, 4 for Int32 /
// Uint32; 0 where it does not apply.
template <int DT>
__host__ __device__ constexpr int sgdw_group() {
  constexpr int b = dtype_bits(DT);
  if (DT == kFloat32 || has_kcopy<DT>()) return 0;
  if (b < 8) return b % 2 == 0 ? 16 : 32;
  if (b == 16 && fix_bytes<DT>() == 2) return 8;
  if (b == 32 && fix_bytes<DT>() == 4) return 4;
  return 0;
}

// sgd_units over groups of sgdw_group<DT>() elements per thread: the codes
// of a group are whole words (loaded and stored as such, every bit of them
// rewritten), the gradient is read as float4; the elements past the last
// whole group go unit by unit through block 0.  The per-element arithmetic
// is sgd_units'.  FP4 / NF4 decode through a copy of their 16 values in LDS
// (a lookup in the constant table takes 16 registers per element in
// flight); every thread of the block must call this.
template <int DT>
__device__ __forceinline__ void sgdw_units(uint8_t *__restrict__ body, int64_t n, const float *__restrict__ g,
                                           double lr, float scale, float minv, int64_t blk, int64_t nblk) {
  constexpr int bits = dtype_bits(DT), G = sgdw_group<DT>(), NW = G * bits / 32;
  static_assert(G > 0 && G % 4 == 0 && G * bits % 32 == 0 && G % unit_elems<DT>() == 0,
                "whole words and units per group");
  constexpr uint32_t mask = bits >= 32 ? ~0u : (1u << bits) - 1;
  constexpr bool kTab = DT == kFP4 || DT == kNF4;
  // FP4 / NF4: the decoded values and the windowed search in LDS
  __shared__ float tab[kTab ? 16 : 1];
  __shared__ __align__(16) TabSearch search_s[1];
  if constexpr (kTab) {
    const uint32_t *from = (const uint32_t *)(DT == kNF4 ? &kNf4Search : &kFp4Search);
    if (threadIdx.x < 16) tab[threadIdx.x] = dec_code<DT>(threadIdx.x, scale, minv);
    for (int i = threadIdx.x; i < (int)(sizeof(TabSearch) / 4); i += kThreads) ((uint32_t *)search_s)[i] = from[i];
    __syncthreads();
  }
  auto value = [&](uint32_t c, int64_t i, float gj) {
    if constexpr (kTab) {
      float old = tab[c];
      if (i == 0) old = dec_code<DT>(fix_code<DT>(old, scale, minv), scale, minv);
      return (float)((double)old - lr * (double)gj);
    } else {
      return sgd_value<DT>(c, i, gj, lr, scale, minv);
    }
  };
  // fix_code<DT> (the NF4 / FP4 search through the window)
  auto code_of = [&](float v) -> uint32_t {
    if constexpr (DT == kNF4) return nearest_window<true>(search_s[0], v / (scale == 0.0f ? 1.0f : scale));
    else if constexpr (DT == kFP4) return nearest_window<false>(search_s[0], v);
    else return (uint32_t)fix_code<DT>(v, scale, minv);
  };
  const int64_t groups = n / G;
  for (int64_t q = blk * kThreads + threadIdx.x; q < groups; q += nblk * kThreads) {
    uint32_t *words = (uint32_t *)(body + q * (NW * 4));
    uint32_t cw[NW + 1];
    if constexpr (NW == 4) {
      const uint4 v = *(const uint4 *)words;
      cw[0] = v.x; cw[1] = v.y; cw[2] = v.z; cw[3] = v.w;
    } else {
#pragma unroll
      for (int k = 0; k < NW; ++k) cw[k] = words[k];
    }
    cw[NW] = 0;
    float gv[G];
#pragma unroll
    for (int v = 0; v < G / 4; ++v) {
      const float4 t = *(const float4 *)(g + q * G + 4 * v);
      gv[4 * v] = t.x; gv[4 * v + 1] = t.y; gv[4 * v + 2] = t.z; gv[4 * v + 3] = t.w;
    }
    uint32_t ow[NW + 1];
#pragma unroll
    for (int k = 0; k <= NW; ++k) ow[k] = 0;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const int off = j * bits, k = off >> 5, sh = off & 31;
      uint32_t c;
      if constexpr (bits == 32) c = cw[k];
      else c = (uint32_t)((((uint64_t)cw[k + 1] << 32) | cw[k]) >> sh) & mask;
      const uint32_t nc = code_of(value(c, q * G + j, gv[j])) & mask;
      ow[k] |= nc << sh;
      if (sh + bits > 32) ow[k + 1] |= nc >> (32 - sh);
    }
    if constexpr (NW == 4) {
      *(uint4 *)words = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    } else {
#pragma unroll
      for (int k = 0; k < NW; ++k) words[k] = ow[k];
    }
  }
  if (blk == 0) {
    constexpr int U = unit_elems<DT>();
    const int64_t u = groups * (G / U) + threadIdx.x, units = (n + U - 1) / U;
    if (u < units) sgd_unit<DT>(body, nullptr, n, g, lr, scale, minv, u);
  }
}

// Threads the SGD of an n-element store of a packed format takes.
template <int DT, bool WIDE = true>
int64_t sgd_threads(int64_t n) {
  if constexpr (WIDE && sgdw_group<DT>() > 0) return n / sgdw_group<DT>() + 1;
  else return (n + unit_elems<DT>() - 1) / unit_elems<DT>();
}

// WIDE: the grouped path where the format has one (the gradient then must
// be 16-byte aligned); else one unit per thread.
template <int DT, bool WIDE>
__global__ void __launch_bounds__(kThreads) sgd_kernel(uint8_t *__restrict__ body,
                                                       uint8_t *__restrict__ kbody, int64_t n,
                                                       const float *__restrict__ g, double lr,
                                                       float scale, float minv, int *stop,
                                                       const int *bad, int bad_value) {
  if (sgd_stopped(stop, bad, bad_value)) return;
  if constexpr (WIDE && sgdw_group<DT>() > 0) sgdw_units<DT>(body, n, g, lr, scale, minv, blockIdx.x, gridDim.x);
  else sgd_units<DT>(body, kbody, n, g, lr, scale, minv, blockIdx.x, gridDim.x);
}

// sgd_kernel for the one-byte formats, 16 elements per thread: one 16-byte
// code load, four float4 gradient loads and 16-byte stores (of the
// decode-ready copy too, for FP8); the first block's threads take the
// n mod 16 tail.  The per-element arithmetic is sgd_kernel's.
// E5M2 (nf non-null): *nf |= 1 when a new decode-ready code has the all-ones
// exponent (Inf or NaN), so the store's finiteness is known after the step.
template <int DT, int G>
__device__ inline void sgd8_units(uint8_t *__restrict__ body, uint8_t *__restrict__ kbody, int64_t n,
                                  const float *__restrict__ g, double lr, float scale, float minv,
                                  int64_t blk, int64_t nblk, int *nf = nullptr) {
  static_assert(dtype_bits(DT) == 8 && fix_bytes<DT>() == 1, "one-byte codes");
  static_assert(G == 4 || G == 16, "elements per thread");
  constexpr int NWD = G / 4;  // code words per thread
  constexpr bool kTrack = DT == kFP8E5M2;
  // a byte of w is an E5M2 Inf / NaN code: (b & 0x7c) == 0x7c, i.e. a zero
  // byte in (w & 0x7c7c7c7c) ^ 0x7c7c7c7c (whose bytes are below 0x80)
  auto nonfinite4 = [](uint32_t w) {
    const uint32_t v = (w & 0x7c7c7c7cu) ^ 0x7c7c7c7cu;
    return ((v - 0x01010101u) & ~v & 0x80808080u) != 0;
  };
  bool bad = false;
  const int64_t groups = n / G;
  for (int64_t q = blk * kThreads + threadIdx.x; q < groups; q += nblk * kThreads) {
    const int64_t i0 = q * G;
    uint32_t cw[NWD];
    if constexpr (G == 16) {
      const uint4 cv = *(const uint4 *)(body + i0);
      cw[0] = cv.x; cw[1] = cv.y; cw[2] = cv.z; cw[3] = cv.w;
    } else {
      cw[0] = *(const uint32_t *)(body + i0);
    }
    float gv[G];
#pragma unroll
    for (int v = 0; v < NWD; ++v) {
      const float4 t = *(const float4 *)(g + i0 + 4 * v);
      gv[4 * v] = t.x; gv[4 * v + 1] = t.y; gv[4 * v + 2] = t.z; gv[4 * v + 3] = t.w;
    }
    uint32_t ow[NWD], kw[NWD];
#pragma unroll
    for (int v = 0; v < NWD; ++v) ow[v] = kw[v] = 0;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const uint32_t c = (cw[j >> 2] >> (8 * (j & 3))) & 0xffu;
      const uint32_t nc = (uint32_t)fix_code<DT>(sgd_value<DT>(c, i0 + j, gv[j], lr, scale, minv), scale, minv) & 0xffu;
      ow[j >> 2] |= nc << (8 * (j & 3));
      if constexpr (has_kcopy<DT>()) kw[j >> 2] |= (uint32_t)kcode<DT>(nc) << (8 * (j & 3));
    }
    if constexpr (G == 16) {
      *(uint4 *)(body + i0) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
      if constexpr (has_kcopy<DT>()) *(uint4 *)(kbody + i0) = make_uint4(kw[0], kw[1], kw[2], kw[3]);
    } else {
      *(uint32_t *)(body + i0) = ow[0];
      if constexpr (has_kcopy<DT>()) *(uint32_t *)(kbody + i0) = kw[0];
    }
    if constexpr (kTrack) {
#pragma unroll
      for (int v = 0; v < NWD; ++v) bad |= nonfinite4(kw[v]);
    }
  }
  const int64_t i = groups * G + threadIdx.x;
  if (blk == 0 && i < n) {
    const uint32_t nc = (uint32_t)fix_code<DT>(sgd_value<DT>(body[i], i, g[i], lr, scale, minv), scale, minv) & 0xffu;
    if constexpr (has_kcopy<DT>()) {
      const uint8_t k = kcode<DT>(nc);
      kbody[i] = k;
      if constexpr (kTrack) bad |= (k & 0x7cu) == 0x7cu;
    }
    body[i] = (uint8_t)nc;
  }
  if constexpr (kTrack) {
    if (nf != nullptr && __any(bad) && (threadIdx.x & 63) == 0) atomicOr(nf, 1);
  }
}

template <int DT, int G>
__global__ void __launch_bounds__(kThreads) sgd8_kernel(uint8_t *__restrict__ body, uint8_t *__restrict__ kbody,
                                                        int64_t n, const float *__restrict__ g, double lr,
                                                        float scale, float minv, int *stop, const int *bad,
                                                        int bad_value, int *nf) {
  if (sgd_stopped(stop, bad, bad_value)) return;
  sgd8_units<DT, G>(body, kbody, n, g, lr, scale, minv, blockIdx.x, gridDim.x, nf);
}

// Float64 storage keeps full f64: w = w - lr*g (native_codec.cpp:933-939
// pinned to the f64 value its soft-double approximates).
__device__ inline void sgd_f64_units(double *__restrict__ w, int64_t n, const float *__restrict__ g,
                                     double lr, int64_t blk, int64_t nblk) {
  for (int64_t i = blk * kThreads + threadIdx.x; i < n; i += nblk * kThreads) w[i] = w[i] - lr * (double)g[i];
}
__global__ void __launch_bounds__(kThreads) sgd_f64_kernel(double *__restrict__ w, int64_t n,
                                                           const float *__restrict__ g, double lr,
                                                           int *stop, const int *bad, int bad_value) {
  if (sgd_stopped(stop, bad, bad_value)) return;
  sgd_f64_units(w, n, g, lr, blockIdx.x, gridDim.x);
}

// welvet_sgd_f32_f64_grad welvet_dense.metal:263-281: the step is rounded to
// f32 first, then subtracted in f32.
// WIDE: four weights per thread (float4 loads and stores; w and g 16-byte
// aligned), block 0 taking the n mod 4 tail; else one per thread.
template <bool WIDE = true>
__device__ inline void sgd_f32_units(float *__restrict__ w, int64_t n, const float *__restrict__ g, double lr,
                                     int64_t blk, int64_t nblk) {
  auto step = [lr](float wi, float gi) { return wi - (float)(lr * (double)gi); };
  if constexpr (!WIDE) {
    for (int64_t i = blk * kThreads + threadIdx.x; i < n; i += nblk * kThreads) w[i] = step(w[i], g[i]);
    return;
  }
  const int64_t quads = n / 4;
  for (int64_t q = blk * kThreads + threadIdx.x; q < quads; q += nblk * kThreads) {
    float4 wv = *(const float4 *)(w + 4 * q);
    const float4 gv = *(const float4 *)(g + 4 * q);
    wv.x = step(wv.x, gv.x);
    wv.y = step(wv.y, gv.y);
    wv.z = step(wv.z, gv.z);
    wv.w = step(wv.w, gv.w);
    *(float4 *)(w + 4 * q) = wv;
  }
  const int64_t i = quads * 4 + threadIdx.x;
  if (blk == 0 && i < n) w[i] = step(w[i], g[i]);
}
template <bool WIDE>
__global__ void __launch_bounds__(kThreads) sgd_f32_kernel(float *__restrict__ w, int64_t n,
                                                           const float *__restrict__ g, double lr,
                                                           int *stop, const int *bad, int bad_value) {
  if (sgd_stopped(stop, bad, bad_value)) return;
  sgd_f32_units<WIDE>(w, n, g, lr, blockIdx.x, gridDim.x);
}

// The SGD of up to kSgdBatch stores of one dtype in one launch (blockIdx.y =
// store, blockIdx.x = block within it).  Every gradient was checked before
// the launch (bad[k] != 0: store k's gradient holds a non-finite value), so
// store c of the batch (index first + c in the sequence) is skipped when any
// store k <= first + c is bad, exactly as a launch per store in sequence
// order skips it; the first bad store records its code in *stop.  The skip
// rule reads only bad[], which no block of this launch writes: *stop is
// written here but never read, since a block of a later bad store may set it
// while blocks of earlier, good stores of the same launch are still to run.
// G: codes per thread of the one-byte formats.
template <int DT, int G>
__global__ void __launch_bounds__(kThreads) sgd_batch_kernel(SgdBatch b, double lr, int *stop,
                                                             const int *bad, int first) {
  const int c = blockIdx.y;
  if (c >= b.count) return;
  const SgdStore &t = b.store[c];
  // the first bad store up to this one: each lane reads one flag, a ballot
  // finds the lowest set (one memory round trip per 64 stores)
  const int upto = first + c, lane = threadIdx.x & 63;
  int fb = -1;
  for (int k0 = 0; k0 <= upto && fb < 0; k0 += 64) {
    const int k = k0 + lane;
    const uint64_t m = __ballot(k <= upto && bad[min(k, upto)] != 0);
    if (m != 0) fb = k0 + __ffsll((unsigned long long)m) - 1;
  }
  if (fb >= 0) {
    if (fb == upto && blockIdx.x == 0 && threadIdx.x == 0) atomicCAS(stop, 0, t.code);
    return;
  }
  if constexpr (DT == kFloat32) sgd_f32_units((float *)t.body, t.n, t.g, lr, blockIdx.x, gridDim.x);
  else if constexpr (DT == kFloat64) sgd_f64_units((double *)t.body, t.n, t.g, lr, blockIdx.x, gridDim.x);
  else if constexpr (dtype_bits(DT) == 8 && fix_bytes<DT>() == 1)
    sgd8_units<DT, G>(t.body, t.kbody, t.n, t.g, lr, t.scale, t.minv, blockIdx.x, gridDim.x, t.nonfinite);
  else if constexpr (sgdw_group<DT>() > 0)
    sgdw_units<DT>(t.body, t.n, t.g, lr, t.scale, t.minv, blockIdx.x, gridDim.x);
  else
    sgd_units<DT>(t.body, t.kbody, t.n, t.g, lr, t.scale, t.minv, blockIdx.x, gridDim.x);
}

// flag := value when g holds a non-finite element and flag is still 0 (the
// first failing check of a sequence keeps its value).
__global__ void __launch_bounds__(kThreads) nonfinite_kernel(const float *__restrict__ g, int64_t n,
                                                             int *flag, int value) {
  int bad = 0;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads)
    bad |= !isfinite(g[i]);
  if (__any(bad) && (threadIdx.x & 63) == 0) atomicCAS(flag, 0, value);
}

__global__ void __launch_bounds__(kThreads) e5m2_nonfinite_kernel(const uint8_t *__restrict__ c, int64_t n,
                                                                  int *flag) {
  int bad = 0;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    bad |= (c[i] & 0x7cu) == 0x7cu;
  if (__any(bad) && (threadIdx.x & 63) == 0) atomicOr(flag, 1);
}

}  // namespace

#define WH_DTYPE_SWITCH(dt, F)                                                                    \
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

hipError_t launch_encode(int dt, const float *w, int64_t n, uint8_t *body, uint8_t *kbody, Meta *meta,
                         Stats *stats, hipStream_t s, bool repack) {
  if (n <= 0) return hipErrorInvalidValue;
  if ((dt == kFP8E4M3 || dt == kFP8E5M2) && kbody == nullptr) return hipErrorInvalidValue;
  stats_init_kernel<<<1, 1, 0, s>>>(stats);
  int sblocks = grid_for(n / 4 + 1);
  if (sblocks > 1024) sblocks = 1024;
  stats_kernel<<<sblocks, kThreads, 0, s>>>(w, n, stats);
#define WH_ENC(D)                                                                                  \
  if (repack) {                                                                                    \
    repack_finalize_kernel<D><<<1, 1, 0, s>>>(w, stats, meta);                                     \
    pack_kernel<D, true><<<grid_for((n + unit_elems<D>() - 1) / unit_elems<D>()), kThreads, 0, s>>>( \
        w, n, body, kbody, meta);                                                                  \
  } else {                                                                                         \
    finalize_kernel<D><<<1, 1, 0, s>>>(w, stats, meta);                                            \
    pack_kernel<D><<<grid_for((n + unit_elems<D>() - 1) / unit_elems<D>()), kThreads, 0, s>>>(     \
        w, n, body, kbody, meta);                                                                  \
  }                                                                                                \
  return hipGetLastError();
  WH_DTYPE_SWITCH(dt, WH_ENC)
#undef WH_ENC
}

hipError_t launch_decode(int dt, const uint8_t *body, int64_t n, float scale, float minv, float *out,
                         hipStream_t s) {
#define WH_DEC(D)                                                                    \
  decode_kernel<D><<<grid_for(n), kThreads, 0, s>>>(body, n, scale, minv, out);      \
  return hipGetLastError();
  WH_DTYPE_SWITCH(dt, WH_DEC)
#undef WH_DEC
}

hipError_t launch_lut(int dt, float scale, float minv, float *lut, hipStream_t s) {
  if (!dtype_lut(dt) || dt == kFloat32) return hipSuccess;
#define WH_LUT(D)                                             \
  if constexpr (dtype_bits(D) <= 8) {                          \
    lut_kernel<D><<<1, 256, 0, s>>>(scale, minv, lut);         \
    return hipGetLastError();                                 \
  } else {                                                    \
    return hipSuccess;                                        \
  }
  WH_DTYPE_SWITCH(dt, WH_LUT)
#undef WH_LUT
}

hipError_t launch_sgd(int dt, uint8_t *body, uint8_t *kbody, int64_t n, const float *g, double lr,
                      float scale, float minv, int *stop, const int *bad, int bad_value, hipStream_t s,
                      int *nonfinite) {
  if ((dt == kFP8E4M3 || dt == kFP8E5M2) && kbody == nullptr) return hipErrorInvalidValue;
  // the grouped kernels read the gradient as float4; a gradient at another
  // alignment (a slice of a concatenated buffer) takes one element or unit
  // per thread
  const bool wide = ((uintptr_t)g & 15) == 0;
  if (dt == kFloat32) {
    if (wide)
      sgd_f32_kernel<true><<<grid_for(n / 4 + 1), kThreads, 0, s>>>((float *)body, n, g, lr, stop, bad, bad_value);
    else
      sgd_f32_kernel<false><<<grid_for(n), kThreads, 0, s>>>((float *)body, n, g, lr, stop, bad, bad_value);
    return hipGetLastError();
  }
  if (dt == kFloat64) {
    sgd_f64_kernel<<<grid_for(n), kThreads, 0, s>>>((double *)body, n, g, lr, stop, bad, bad_value);
    return hipGetLastError();
  }
#define WH_SGD(D)                                                                           \
  if constexpr (dtype_bits(D) == 8 && fix_bytes<D>() == 1) {                               \
    if (!wide) {                                                                            \
      sgd_kernel<D, false><<<grid_for(n), kThreads, 0, s>>>(body, kbody, n, g, lr, scale, minv, stop, \
                                                            bad, bad_value);                \
      if (D == kFP8E5M2 && nonfinite != nullptr) /* every code was rewritten */             \
        e5m2_nonfinite_kernel<<<grid_for(n / 16 + 1), kThreads, 0, s>>>(kbody, n, nonfinite); \
    } else if (n >= ((int64_t)4 << 20))                                                     \
      sgd8_kernel<D, 16><<<grid_for(n / 16 + 1), kThreads, 0, s>>>(body, kbody, n, g, lr, scale, minv, \
                                                                  stop, bad, bad_value, nonfinite); \
    else /* small stores: four codes per thread, four times the threads */                \
      sgd8_kernel<D, 4><<<grid_for(n / 4 + 1), kThreads, 0, s>>>(body, kbody, n, g, lr, scale, minv, \
                                                                stop, bad, bad_value, nonfinite); \
    return hipGetLastError();                                                               \
  } else if constexpr (D != kFloat32 && D != kFloat64) {                                    \
    if (wide)                                                                               \
      sgd_kernel<D, true><<<grid_for(sgd_threads<D>(n)), kThreads, 0, s>>>(                 \
          body, kbody, n, g, lr, scale, minv, stop, bad, bad_value);                        \
    else                                                                                    \
      sgd_kernel<D, false><<<grid_for(sgd_threads<D, false>(n)), kThreads, 0, s>>>(         \
          body, kbody, n, g, lr, scale, minv, stop, bad, bad_value);                        \
    return hipGetLastError();                                                               \
  } else {                                                                                  \
    return hipErrorInvalidValue;                                                            \
  }
  WH_DTYPE_SWITCH(dt, WH_SGD)
#undef WH_SGD
}

hipError_t launch_e5m2_nonfinite(const uint8_t *codes, int64_t n, int *flag, hipStream_t s) {
  e5m2_nonfinite_kernel<<<grid_for(n / 16 + 1), kThreads, 0, s>>>(codes, n, flag);
  return hipGetLastError();
}

hipError_t launch_sgd_batch(int dt, const SgdBatch &b, double lr, int *stop, const int *bad, int first,
                            hipStream_t s) {
  if (b.count < 1 || b.count > kSgdBatch || stop == nullptr || bad == nullptr) return hipErrorInvalidValue;
  int64_t maxn = 0;
  for (int i = 0; i < b.count; ++i) {
    if (b.store[i].body == nullptr || b.store[i].g == nullptr || b.store[i].n < 0) return hipErrorInvalidValue;
    if (((uintptr_t)b.store[i].g & 15) != 0) return hipErrorInvalidValue;  // read as float4
    if ((dt == kFP8E4M3 || dt == kFP8E5M2) && b.store[i].kbody == nullptr) return hipErrorInvalidValue;
    maxn = std::max(maxn, b.store[i].n);
  }
#define WH_SGDB(D)                                                                                  \
  if constexpr (dtype_bits(D) == 8 && fix_bytes<D>() == 1) {                                       \
    if (maxn >= ((int64_t)4 << 20))                                                                 \
      sgd_batch_kernel<D, 16><<<dim3(grid_for(maxn / 16 + 1), b.count), kThreads, 0, s>>>(b, lr, stop, bad, first); \
    else                                                                                            \
      sgd_batch_kernel<D, 4><<<dim3(grid_for(maxn / 4 + 1), b.count), kThreads, 0, s>>>(b, lr, stop, bad, first);   \
  } else {                                                                                          \
    const int64_t units = D == kFloat32 ? maxn / 4 + 1 : D == kFloat64 ? maxn : sgd_threads<D>(maxn); \
    sgd_batch_kernel<D, 4><<<dim3(grid_for(units), b.count), kThreads, 0, s>>>(b, lr, stop, bad, first); \
  }                                                                                                 \
  return hipGetLastError();
  WH_DTYPE_SWITCH(dt, WH_SGDB)
#undef WH_SGDB
}

hipError_t launch_nonfinite(const float *g, int64_t n, int *flag, int value, hipStream_t s) {
  nonfinite_kernel<<<grid_for(n / 4 + 1), kThreads, 0, s>>>(g, n, flag, value);
  return hipGetLastError();
}

}  // namespace wh
