// dense.hip — Dense forward / backward over packed native weights.
//
// Replaces the reference's float2 soft-double mirror kernels
// (welvet_dense.metal:54-178): weights stay packed in HBM and are decoded in
// registers (through LDS tables for formats of <= 8 bits) inside the product.
//
//   forward, batch <= 4   gemv_kernel: a 64-lane wave owns R rows, lanes
//                         stream 16-byte chunks of each row (coalesced), x
//                         chunks are reused across the R rows, DPP/shuffle
//                         reduction, bias + activation fused in the store.
//   forward, batch > 4    gemm_kernel: decoded W tiles and x tiles staged in
//                         LDS, fp32 MFMA 32x32x2, split-K with an ordered f64
//                         reduction that applies bias + activation.
//   dX, batch <= 2        dx_small_kernel: lanes own column chunks and walk a
//                         segment of rows (coalesced), ordered f64 reduction
//                         over segments.
//   dX, batch > 2         gemm_kernel with the transposed W tile loader.
//   dW                    dw_kernel: VALU sequential fmaf over the batch in
//                         batch order, bit-identical to the reference's
//                         outer-product accumulation (welvet_dense.metal:155-178).
//
// Accumulation is fp32 inside a lane/tile and f64 across split-K / segment
// partials; outputs are fl32 of that, within the stated tolerance of the f64
// contract.  Float64 storage accumulates in f64 on the GEMV path.
#include <type_traits>

#include "codec.hpp"
#include "kernels.hpp"

namespace wh {
namespace {

// Kernel formats: dtypes sharing a body layout and decode share a kernel.
enum Fmt {
  FL1, FL2, FL3, FL4, FL5, FL6, FL8, FH16, FB16, FI16, FU16, FF32, FI32, FU32, FI64, FU64, FC64,
  FC128, FF64, kNumFmt
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
  static constexpr int kBits = F == FL1 ? 1 : F == FL2 ? 2 : F == FL3 ? 3 : F == FL4 ? 4 : F == FL5 ? 5
                             : F == FL6 ? 6 : F == FL8 ? 8 : (F == FH16 || F == FB16 || F == FI16 || F == FU16) ? 16
                             : (F == FF32 || F == FI32 || F == FU32) ? 32 : F == FC128 ? 128 : 64;
  static constexpr bool kLut = kBits <= 8;
  static constexpr int kE = kBits <= 6 ? 32 : 128 / kBits;
  static constexpr int kW = kBits <= 6 ? kBits : 4;
  using Acc = std::conditional_t<F == FF64, double, float>;
};

int fmt_chunk_elems(int f) {
  switch (f) {
  case FL1: case FL2: case FL3: case FL4: case FL5: case FL6: return 32;
  case FL8: return 16;
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
  if constexpr (I::kLut) return lut[chunk_code<I::kBits, I::kW>(w, e)];
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

// ----------------------------------------------------------------- GEMV
template <int F, int B, int R>
__global__ void __launch_bounds__(256) gemv_kernel(GemvArgs a) {
  using I = FI<F>;
  using Acc = typename I::Acc;
  constexpr int E = I::kE, W = I::kW;
  __shared__ float lut_s[I::kLut ? (1 << I::kBits) : 1];
  if constexpr (I::kLut) {
    for (int i = threadIdx.x; i < (1 << I::kBits); i += 256) lut_s[i] = a.lut[i];
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
// C[m][n] = sum_k A[m][k] * Wop[k][n] over fp32 MFMA 32x32x2.
//   forward: A = x [M][K], Wop[k][n] = W[n][k]   (TRANS = false)
//   dX:      A = dpre [M][K=rows], Wop[k][n] = W[k][n] (TRANS = true)
struct GemmArgs {
  const uint8_t *body;
  const float *lut;
  float scale, minv;
  const float *A;
  int M, K, N;       // product dims
  int64_t row_bytes;  // bytes per stored W row
  int stages_per_slice, nstages;
  float *ws;          // split-K partials [slices][M][N] (unused when direct)
  int direct;
  const double *bias;
  int bias_len, act;
  float *pre, *post;  // direct forward outputs; dX writes `pre`
};

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 64, kBN = 64, kBK = 32, kPad = 1;

template <int F, bool TRANS>
__global__ void __launch_bounds__(256) gemm_kernel(GemmArgs a) {
  using I = FI<F>;
  constexpr int E = I::kE, W = I::kW;
  __shared__ float Xs[kBK][kBM + kPad];
  __shared__ float Ws[kBK][kBN + kPad];
  __shared__ float lut_s[I::kLut ? (1 << I::kBits) : 1];
  if constexpr (I::kLut) {
    for (int i = threadIdx.x; i < (1 << I::kBits); i += 256) lut_s[i] = a.lut[i];
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int n0 = blockIdx.x * kBN, m0 = blockIdx.y * kBM, slice = blockIdx.z;
  const int st0 = slice * a.stages_per_slice;
  const int st1 = min(a.nstages, st0 + a.stages_per_slice);
  floatx16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;

  for (int st = st0; st < st1; ++st) {
    const int k0 = st * kBK;
    __syncthreads();
    // W tile -> Ws[k][n] (decoded f32)
    if constexpr (!TRANS) {
      constexpr int CPR = (kBK + E - 1) / E;  // chunks per row in a stage
      for (int q = tid; q < kBN * CPR; q += 256) {
        const int n = q % kBN, j = q / kBN, k = k0 + j * E, row = n0 + n;
        uint32_t w[W];
        const bool ok = row < a.N && k < a.K;
        if (ok) load_words<W>(a.body + (int64_t)row * a.row_bytes + (int64_t)(k / E) * (W * 4), w);
#pragma unroll
        for (int e = 0; e < E; ++e)
          if (j * E + e < kBK) Ws[j * E + e][n] = ok ? (float)chunk_value<F>(w, e, lut_s, a.scale, a.minv) : 0.0f;
      }
    } else {
      constexpr int CPR = kBN / E;  // chunks across the tile's columns
      for (int q = tid; q < kBK * CPR; q += 256) {
        const int kl = q % kBK, j = q / kBK, k = k0 + kl, col = n0 + j * E;
        uint32_t w[W];
        const bool ok = k < a.K && col < a.N;
        if (ok) load_words<W>(a.body + (int64_t)k * a.row_bytes + (int64_t)(col / E) * (W * 4), w);
#pragma unroll
        for (int e = 0; e < E; ++e)
          Ws[kl][j * E + e] = (ok && col + e < a.N) ? (float)chunk_value<F>(w, e, lut_s, a.scale, a.minv) : 0.0f;
      }
    }
    // A tile -> Xs[k][m]
    for (int q = tid; q < kBM * kBK; q += 256) {
      const int kl = q % kBK, m = q / kBK, k = k0 + kl;  // lanes walk k: coalesced rows of A
      Xs[kl][m] = (m0 + m < a.M && k < a.K) ? a.A[(int64_t)(m0 + m) * a.K + k] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 2) {
      const float av = Xs[kk + (lane >> 5)][wm * 32 + (lane & 31)];
      const float bv = Ws[kk + (lane >> 5)][wn * 32 + (lane & 31)];
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc, 0, 0, 0);
    }
  }
  // D[i][j]: lane = j + 32*((i/4)%2), register = i%4 + 4*(i/8)
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = m0 + wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    const int n = n0 + wn * 32 + (lane & 31);
    if (m < a.M && n < a.N) {
      const int64_t idx = (int64_t)m * a.N + n;
      if (a.direct) {
        if constexpr (TRANS) a.pre[idx] = acc[r];
        else bias_act_store((double)acc[r], n, a.bias, a.bias_len, a.act, a.pre, a.post, idx);
      } else {
        a.ws[(int64_t)slice * a.M * a.N + idx] = acc[r];
      }
    }
  }
}

// Ordered f64 sum of split-K / segment partials.
__global__ void __launch_bounds__(256) reduce_fwd_kernel(const float *ws, int slices, int M, int N,
                                                         const double *bias, int bias_len, int act,
                                                         float *pre, float *post) {
  const int64_t total = (int64_t)M * N;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    double s = 0;
    for (int k = 0; k < slices; ++k) s += (double)ws[(int64_t)k * total + i];
    bias_act_store(s, (int)(i % N), bias, bias_len, act, pre, post, i);
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
  __shared__ float lut_s[I::kLut ? (1 << I::kBits) : 1];
  if constexpr (I::kLut) {
    for (int i = threadIdx.x; i < (1 << I::kBits); i += 256) lut_s[i] = a.lut[i];
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

// dW[o][i] = sequential fmaf over b (welvet_dense.metal:155-178).
__global__ void __launch_bounds__(256) dw_kernel(const float *__restrict__ dpre,
                                                 const float *__restrict__ x, int B, int rows, int cols,
                                                 float *__restrict__ dW, int *flag) {
  __shared__ float Ds[32][64];
  __shared__ float Xs[32][64];
  const int tid = threadIdx.x, to = tid >> 4, ti = tid & 15;
  const int o0 = blockIdx.y * 64, i0 = blockIdx.x * 64;
  float acc[4][4] = {};
  for (int b0 = 0; b0 < B; b0 += 32) {
    __syncthreads();
    for (int q = tid; q < 32 * 64; q += 256) {
      const int bb = q >> 6, j = q & 63, b = b0 + bb;
      Ds[bb][j] = (b < B && o0 + j < rows) ? dpre[(int64_t)b * rows + o0 + j] : 0.0f;
      Xs[bb][j] = (b < B && i0 + j < cols) ? x[(int64_t)b * cols + i0 + j] : 0.0f;
    }
    __syncthreads();
    const int nb = min(32, B - b0);
    for (int bb = 0; bb < nb; ++bb) {
      float d[4], xv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) d[r] = Ds[bb][to * 4 + r];
#pragma unroll
      for (int c = 0; c < 4; ++c) xv[c] = Xs[bb][ti * 4 + c];
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[r][c] = fmaf(d[r], xv[c], acc[r][c]);
    }
  }
  int bad = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int o = o0 + to * 4 + r;
    if (o >= rows) continue;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int i = i0 + ti * 4 + c;
      if (i < cols) {
        dW[(int64_t)o * cols + i] = acc[r][c];
        bad |= !isfinite(acc[r][c]);
      }
    }
  }
  if (flag != nullptr && __any(bad) && (tid & 63) == 0) atomicOr(flag, 1);
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
                                                        double *loss) {
  __shared__ double red[4];
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

// --------------------------------------------------------------- dispatch
int g_forward_path = 0;

inline int blocks_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  return (int)(b < 1 ? 1 : (b > 65536 ? 65536 : b));
}

bool chunk_aligned(const DevStore &w, int64_t len) {
  const int f = fmt_of(w.dtype);
  return f >= 0 && len % fmt_chunk_elems(f) == 0;
}

int64_t row_bytes_of(const DevStore &w) {
  return (int64_t)w.cols * dtype_bits(w.dtype) / 8;
}

struct GemmPlan {
  int slices, stages_per_slice, nstages, gx, gy;
};

GemmPlan plan_gemm(int M, int K, int N) {
  GemmPlan p;
  p.nstages = (K + kBK - 1) / kBK;
  p.gx = (N + kBN - 1) / kBN;
  p.gy = (M + kBM - 1) / kBM;
  const int tiles = p.gx * p.gy;
  int s = (1024 + tiles - 1) / tiles;
  if (s > p.nstages) s = p.nstages;
  if (s > 64) s = 64;
  if (s < 1) s = 1;
  p.stages_per_slice = (p.nstages + s - 1) / s;
  p.slices = (p.nstages + p.stages_per_slice - 1) / p.stages_per_slice;
  return p;
}

constexpr int kDxSegRows = 32;

int fwd_route(const DevStore &w, int batch) {
  if (!chunk_aligned(w, w.cols)) return 3;
  if (g_forward_path) return g_forward_path;
  return batch <= 4 ? 1 : 2;
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
  case FL1: F(FL1); case FL2: F(FL2); case FL3: F(FL3); case FL4: F(FL4); case FL5: F(FL5);          \
  case FL6: F(FL6); case FL8: F(FL8); case FH16: F(FH16); case FB16: F(FB16); case FI16: F(FI16);    \
  case FU16: F(FU16); case FF32: F(FF32); case FI32: F(FI32); case FU32: F(FU32); case FI64: F(FI64); \
  case FU64: F(FU64); case FC64: F(FC64); case FC128: F(FC128); case FF64: F(FF64);                  \
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

size_t forward_workspace_bytes(const DevStore &w, int batch) {
  if (fwd_route(w, batch) != 2) return 0;
  const GemmPlan p = plan_gemm(batch, w.cols, w.rows);
  return p.slices > 1 ? (size_t)p.slices * batch * w.rows * sizeof(float) : 0;
}

hipError_t launch_forward(const DevStore &w, int batch, const float *x, const double *bias,
                          int bias_len, int act, float *pre, float *post, void *ws, size_t ws_bytes,
                          hipStream_t s) {
  const int route = fwd_route(w, batch);
  const int f = fmt_of(w.dtype);
  if (route == 3 || (route == 1 && batch > 4)) {
#define WH_GEN(D)                                                                        \
  gemv_generic_kernel<D><<<w.rows, 256, 0, s>>>(w, batch, x, bias, bias_len, act, pre, post); \
  return hipGetLastError();
    WH_DT_SWITCH(w.dtype, WH_GEN)
#undef WH_GEN
  }
  if (route == 1) {
    GemvArgs a{w.body, w.lut, w.scale, w.minv, x, w.cols, w.rows, w.cols / fmt_chunk_elems(f),
               row_bytes_of(w), bias, bias_len, act, pre, post};
#define WH_GV(F) return gemv_dispatch<F>(batch, a, s);
    WH_FMT_SWITCH(f, WH_GV)
#undef WH_GV
  }
  const GemmPlan p = plan_gemm(batch, w.cols, w.rows);
  if (p.slices > 1 && ws_bytes < (size_t)p.slices * batch * w.rows * sizeof(float))
    return hipErrorInvalidValue;
  GemmArgs a{w.body, w.lut, w.scale, w.minv, x, batch, w.cols, w.rows, row_bytes_of(w),
             p.stages_per_slice, p.nstages, (float *)ws, p.slices == 1, bias, bias_len, act, pre, post};
  dim3 grid(p.gx, p.gy, p.slices);
#define WH_GM(F)                                      \
  gemm_kernel<F, false><<<grid, 256, 0, s>>>(a);      \
  break;
  WH_FMT_SWITCH(f, WH_GM)
#undef WH_GM
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.slices == 1) return e;
  reduce_fwd_kernel<<<blocks_for((int64_t)batch * w.rows), 256, 0, s>>>(
      (const float *)ws, p.slices, batch, w.rows, bias, bias_len, act, pre, post);
  return hipGetLastError();
}

namespace {
// dX routing: 1 = small-batch column kernel, 2 = transposed MFMA GEMM, 3 = generic.
int dx_route(const DevStore &w, int batch) {
  if (!chunk_aligned(w, w.cols)) return 3;
  return batch <= 2 ? 1 : 2;
}
}  // namespace

size_t backward_workspace_bytes(const DevStore &w, int batch) {
  const int route = dx_route(w, batch);
  if (route == 1) {
    const int nseg = (w.rows + kDxSegRows - 1) / kDxSegRows;
    return (size_t)nseg * batch * w.cols * sizeof(float);
  }
  if (route == 2) {
    const GemmPlan p = plan_gemm(batch, w.rows, w.cols);
    return p.slices > 1 ? (size_t)p.slices * batch * w.cols * sizeof(float) : 0;
  }
  return 0;
}

hipError_t launch_backward(const DevStore &w, int batch, const float *x, const float *pre,
                           const float *gy, int act, float *dpre, float *dX, float *dW, int *flag,
                           void *ws, size_t ws_bytes, hipStream_t s) {
  const int64_t ny = (int64_t)batch * w.rows;
  act_deriv_kernel<<<blocks_for(ny), 256, 0, s>>>(gy, pre, ny, act, dpre);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int route = dx_route(w, batch);
  const int f = fmt_of(w.dtype);
  if (ws_bytes < backward_workspace_bytes(w, batch)) return hipErrorInvalidValue;
  if (route == 3) {
#define WH_DXG(D)                                                                         \
  dx_generic_kernel<D><<<blocks_for((int64_t)batch * w.cols), 256, 0, s>>>(w, batch, dpre, dX); \
  break;
    WH_DT_SWITCH(w.dtype, WH_DXG)
#undef WH_DXG
  } else if (route == 1) {
    const int nseg = (w.rows + kDxSegRows - 1) / kDxSegRows;
    DxArgs a{w.body, w.lut, w.scale, w.minv, dpre, w.rows, w.cols, w.cols / fmt_chunk_elems(f),
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
  } else {
    const GemmPlan p = plan_gemm(batch, w.rows, w.cols);
    GemmArgs a{w.body, w.lut, w.scale, w.minv, dpre, batch, w.rows, w.cols, row_bytes_of(w),
               p.stages_per_slice, p.nstages, (float *)ws, p.slices == 1, nullptr, 0, -1, dX, nullptr};
    dim3 grid(p.gx, p.gy, p.slices);
#define WH_DXM(F)                                   \
  gemm_kernel<F, true><<<grid, 256, 0, s>>>(a);     \
  break;
    WH_FMT_SWITCH(f, WH_DXM)
#undef WH_DXM
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (p.slices > 1)
      reduce_plain_kernel<<<blocks_for((int64_t)batch * w.cols), 256, 0, s>>>(
          (const float *)ws, p.slices, (int64_t)batch * w.cols, dX);
  }
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  dim3 g2((w.cols + 63) / 64, (w.rows + 63) / 64);
  dw_kernel<<<g2, 256, 0, s>>>(dpre, x, batch, w.rows, w.cols, dW, flag);
  return hipGetLastError();
}

size_t mse_workspace_bytes(int64_t n) {
  (void)n;
  return 1024 * sizeof(double);
}

hipError_t launch_mse(const float *pred, const float *target, int64_t n, double *loss, float *grad,
                      void *ws, size_t ws_bytes, hipStream_t s) {
  if (ws_bytes < mse_workspace_bytes(n)) return hipErrorInvalidValue;
  if (loss != nullptr) {
    int parts = blocks_for(n);
    if (parts > 1024) parts = 1024;
    mse_partial_kernel<<<parts, 256, 0, s>>>(pred, target, n, (double *)ws);
    mse_final_kernel<<<1, 256, 0, s>>>((const double *)ws, parts, n, loss);
  }
  if (grad != nullptr) mse_grad_kernel<<<blocks_for(n), 256, 0, s>>>(pred, target, n, grad);
  return hipGetLastError();
}

}  // namespace wh
