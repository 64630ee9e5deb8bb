// kernels.hpp — host-side launch interface of the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wh {

struct Meta;

// Device scratch of the statistics pass (absmax, first min, first max).
struct Stats {
  unsigned int absmax_bits;
  unsigned int pad;
  unsigned long long minkey;
  unsigned long long maxkey;
};

// The store's decode table (Store::lut, kLutFloats floats): the 2^bits
// decoded values from float 0, and for 4-bit formats the 256 byte-pair
// entries {value of the low nibble, value of the high nibble} from float
// kPairLut on, so a block copies its pair table instead of building it.
constexpr int kPairLut = 256;
constexpr int kLutFloats = kPairLut + 512;

// Resident weight matrix: rows = out, cols = in (native_codec.cpp:112-136
// bitstream order, header split off into minv).
struct DevStore {
  int dtype;
  int rows;
  int cols;
  float scale;
  float minv;
  const uint8_t *body;
  const uint8_t *kbody;  // FP8 formats: decode-ready copy of body (codec.hpp kcode)
  const float *lut;  // decoded values for formats of <= 8 bits (layout: kPairLut)
  bool finite;       // no stored code decodes to Inf or NaN (known on the host)
  // codes of one byte (the decode-ready copy for FP8) transposed, [cols][rows],
  // for dX on the split-x GEMM; null when absent or stale
  const uint8_t *tbody;
};

// ---- codec.hip
// FP8 formats also write the decode-ready copy kbody (required for them).
// repack: the statistics and codes of op_native_repack instead of pack_native.
hipError_t launch_encode(int dt, const float *w, int64_t n, uint8_t *body, uint8_t *kbody, Meta *meta,
                         Stats *stats, hipStream_t s, bool repack = false);
hipError_t launch_decode(int dt, const uint8_t *body, int64_t n, float scale, float minv, float *out,
                         hipStream_t s);
hipError_t launch_lut(int dt, float scale, float minv, float *lut, hipStream_t s);
// SGD with fixed-scale re-encode; a no-op when `stop` is non-null and
// *stop != 0, or when `bad` is non-null and *bad != 0 (a non-finite gradient
// found upstream; then *stop = bad_value if it was 0).  FP8 formats also
// refresh the decode-ready copy kbody (required for them).  E5M2 with
// `nonfinite` non-null: *nonfinite |= 1 when a new code decodes to Inf or NaN
// (the caller zeroes it first).
hipError_t launch_sgd(int dt, uint8_t *body, uint8_t *kbody, int64_t n, const float *g, double lr,
                      float scale, float minv, int *stop, const int *bad, int bad_value,
                      hipStream_t s, int *nonfinite = nullptr);
// The SGD of up to kSgdBatch stores of one dtype in one launch, as
// launch_sgd on each in sequence: store c is skipped when bad[k] != 0 for any
// k <= first + c (its own gradient or an earlier store's is non-finite), and
// the first such store sets *stop = its code if *stop was 0.  The skip rule
// reads bad[] only (never *stop), so a stop with another cause must end the
// sequence before a batch is launched.  The stores' parameters travel in
// the kernel arguments.
constexpr int kSgdBatch = 16;
struct SgdStore {
  uint8_t *body;
  uint8_t *kbody;  // FP8 formats: the decode-ready copy (required), else null
  const float *g;
  int64_t n;
  float scale, minv;
  int code;  // the stop code when this store's gradient is the first non-finite one
  int *nonfinite;  // E5M2: |= 1 when a new code decodes to Inf or NaN (nullable)
};
struct SgdBatch {
  SgdStore store[kSgdBatch];
  int count;
};
hipError_t launch_sgd_batch(int dt, const SgdBatch &b, double lr, int *stop, const int *bad, int first,
                            hipStream_t s);
// *flag = value if g holds a non-finite element and *flag is still 0.
hipError_t launch_nonfinite(const float *g, int64_t n, int *flag, int value, hipStream_t s);
// *flag |= 1 if one of the n FP8 E5M2 codes is Inf or NaN (exponent field all ones).
hipError_t launch_e5m2_nonfinite(const uint8_t *codes, int64_t n, int *flag, hipStream_t s);

// ---- dense.hip
// Bytes of workspace the forward / backward launches below need.
size_t forward_workspace_bytes(const DevStore &w, int batch);
size_t backward_workspace_bytes(const DevStore &w, int batch);

// pre/post [batch][rows] = act(x[batch][cols] . W^T (+ bias)).
hipError_t launch_forward(const DevStore &w, int batch, const float *x, const double *bias,
                          int bias_len, int act, float *pre, float *post, void *ws, size_t ws_bytes,
                          hipStream_t s);
// SwiGLU's Gate and Up projections at batch 1 in one launch (two stores of
// one format and shape): g_pre = Gate x, u_pre = Up x, h = fl32(silu(g)) * u.
// forward_pair_fits: whether the pair kernel takes the stores (FP8, NF4 /
// Int4 / Uint4, FP4, Int8; rows of at most 8 waves of chunks).
bool forward_pair_fits(const DevStore &g, const DevStore &u, int batch);
hipError_t launch_forward_pair(const DevStore &g, const DevStore &u, const float *x, float *g_pre,
                               float *u_pre, float *h, hipStream_t s);
// out[c][r] = in[r][c] for a rows x cols byte matrix.
hipError_t launch_transpose_u8(const uint8_t *in, int rows, int cols, uint8_t *out, hipStream_t s);
// True when launch_backward's dX would use the store's transposed codes
// (DevStore::tbody); the caller refreshes them before the launch.
bool backward_wants_transposed(const DevStore &w, int batch);
// dpre = gy * act'(pre); dX = dpre . W (skipped when dX is null); dW =
// sum_b dpre^T x (sequential FMA); flag |= 1 when dW holds a non-finite value.
// A backward inside a chain of layers (the volume runtime's reverse walk):
// gy_is_dpre: gy already holds dpre (the layer above applied this layer's
// derivative in its dX epilogue), so no derivative launch; dx_next_pre /
// dx_next_act: dX becomes the layer below's dpre, fl32(dX) * act'(pre of the
// layer below), allowed only where backward_dx_applies_next holds (else the
// launch fails with hipErrorInvalidValue).
// defer_dw: no dW launch (the caller batches it with launch_dw_batch, from
// the dpre written to *dpre_out, which must stay intact until then); allowed
// only where dw_batchable holds.
struct BackwardChain {
  bool gy_is_dpre = false;
  const float *dx_next_pre = nullptr;
  int dx_next_act = -1;
  bool defer_dw = false;
  const float **dpre_out = nullptr;
};
bool backward_dx_applies_next(const DevStore &w, int batch, int next_act);
// dW of up to kDwBatch layers in one launch, each as launch_backward computes
// it (LDS-staged fp32 MFMA, sequential FMA over the batch; rows and columns
// multiples of 128: dw_batchable), flag |= 1 per layer on a non-finite value.
constexpr int kDwBatch = 16;
struct DwJob {
  const float *dpre;  // [batch][rows]
  const float *x;     // [batch][cols]
  int rows, cols;
  float *dW;
  int *flag;
};
struct DwBatch {
  DwJob job[kDwBatch];
  int count;
  int batch;
};
bool dw_batchable(const DevStore &w);
bool dw_defer_pays(const DevStore &w);  // batchable, and the layer alone leaves CUs idle
hipError_t launch_dw_batch(const DwBatch &b, hipStream_t s);
hipError_t launch_backward(const DevStore &w, int batch, const float *x, const float *pre,
                           const float *gy, int act, float *dpre, float *dX, float *dW, int *flag,
                           void *ws, size_t ws_bytes, hipStream_t s, const BackwardChain &chain = {});
// SwiGLU's backward element-wise step (op_swiglu): d_up = fl32(gh *
// silu(gate)), d_gate = fl32(gh * up * silu'(gate)).  The forward product is
// the kSwiGated epilogue of the Up projection (common.hpp).
hipError_t launch_swiglu_bwd(const float *gate, const float *up, const float *gh, int64_t n,
                             float *d_up, float *d_gate, hipStream_t s);
// out = fl32(a + b)
hipError_t launch_add(const float *a, const float *b, int64_t n, float *out, hipStream_t s);
// loss = sum (p - t)^2 / n (f64);  grad = fl32(2 (p - t) / n).  With
// nclear > 0 the loss launch also zeroes the nclear ints at clear (a step's
// flags, cleared before the launches that follow on the stream; needs loss).
hipError_t launch_mse(const float *pred, const float *target, int64_t n, double *loss, float *grad,
                      void *ws, size_t ws_bytes, hipStream_t s, int *clear = nullptr, int64_t nclear = 0);
size_t mse_workspace_bytes(int64_t n);

// Reads `bytes` (a multiple of 16) at p once, 16 bytes per load; sink: 1024
// words the kernel practically never writes.
hipError_t launch_read_probe(const void *p, int64_t bytes, uint32_t *sink, hipStream_t s);

// Kernel-selection knobs, exposed for sweeps: forward path for a batch
// (0 = auto, 1 = GEMV, 2 = MFMA GEMM, 3 = generic element-wise).
void set_forward_path(int path);

// Route switches (the C-ABI's welvet_hip_set_tuning documents each value):
// 10 the split-x GEMM, 16 no-split batch <= 16 forward / dX, 17 the folded
// activation derivative, 18 the batched SGD, 19 the batched dW, 20 the batch
// 2-8 GEMV (k >= 2: k waves per CU), 21 the LDS-staged no-split kernels.
// Atomic; the other key numbers are unknown (set_tuning and tuning return -1).
enum TuneKey {
  kTuneBf3 = 10, kTuneBf3Rows = 16, kTuneFoldDeriv = 17, kTuneSgdBatch = 18, kTuneDwBatch = 19,
  kTuneGemvBatch = 20, kTuneRegx = 21, kNumTune = 22
};
int set_tuning(int key, int value);  // the previous value (-1 for an unknown key)
int tuning(int key);  // the current value (-1 for an unknown key)

}  // namespace wh
