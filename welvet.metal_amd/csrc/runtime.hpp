// runtime.hpp — host-side pieces shared by the Dense session runtime and
// the volume runtime: status helpers, device bring-up and the resident
// packed weight store.  Internal to the library (not installed).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/welvet_c.h"
#include "codec.hpp"
#include "kernels.hpp"

namespace wh {
namespace rt {

welvet_status make_status(int code, const char *fmt, ...);
inline welvet_status ok() { return welvet_status{}; }

#define WH_HIP(expr)                                                                   \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess)                                                              \
      return make_status(kInternal, "hip: %s at %s:%d", hipGetErrorString(e_), __FILE__, __LINE__); \
  } while (0)

// Brings up device 0 once (gfx950 only); code 2 when unusable.
welvet_status require_device();
void device_init();
bool device_ready();
const char *device_identity();

// ------------------------------------------------------- resident store
struct Store {
  int dtype = kFloat32, rows = 0, cols = 0;
  float scale = 1.0f, minv = 0.0f;
  uint8_t *body = nullptr;  // payload without the unsigned header
  uint8_t *kbody = nullptr; // FP8: decode-ready copy of body (same size), else null
  size_t body_bytes = 0;    // payload bytes in the reference layout minus header
  float *lut = nullptr;
  double *bias = nullptr;
  int bias_len = 0;

  // no code decodes to Inf / NaN: found at encode (FP8 E5M2 can hold them),
  // cleared by an SGD step of a format that can produce them
  bool finite = true;
  // transposed codes for dX on the split-x GEMM (tbody_ok: current with body)
  uint8_t *tbody = nullptr;
  bool tbody_ok = false;

  DevStore dev() const {
    return DevStore{dtype, rows, cols, scale, minv, body, kbody, lut, finite, tbody_ok ? tbody : nullptr};
  }
  int64_t n() const { return (int64_t)rows * cols; }
};

void free_store(Store *w);
// Refreshes the transposed codes when a backward at this batch reads them.
welvet_status store_prepare_backward(Store *w, int batch, hipStream_t s);
// WeightStore::make on the device from f32 values already in HBM.
welvet_status store_make(Store *w, int dtype, int rows, int cols, const float *d_w, hipStream_t s);
// Re-encodes a made store from f32 values in HBM (pack_native, or the fresh
// statistics and codes of op_native_repack when repack is set).
welvet_status store_encode(Store *w, const float *d_w, bool repack, hipStream_t s);
// WeightStore::set_from_f32_gpu (native_codec.cpp:872-907): the store
// replaced by the op_native_repack encode of host values [rows*cols].
welvet_status store_repack_host(Store *w, const float *values, hipStream_t s);
welvet_status store_set_bias(Store *w, const double *bias, size_t bias_len, hipStream_t s);
// A store from the fields of a WeightStore snapshot (model_session.cpp:128-151
// read_store): Float32 takes the f32 payload, the other dtypes the native
// bytes in the reference layout (4-byte min header for the unsigned types).
welvet_status store_from_native(Store *w, int dtype, int rows, int cols, float scale,
                                const float *f32, size_t nf32, const uint8_t *raw, size_t nraw,
                                hipStream_t s);
welvet_status store_from_host(Store *w, int dtype, int rows, int cols, const float *W_init,
                              hipStream_t s);
// WeightStore::apply_sgd with a device gradient; synchronises to check it.
welvet_status store_sgd(Store *w, const float *d_dW, double lr, int *d_flag, hipStream_t s);
welvet_status store_native(const Store &w, uint8_t *out, size_t cap, size_t *len, hipStream_t s);
welvet_status store_export(const Store &w, float *d_out, hipStream_t s);
bool dims_ok(int32_t rows, int32_t cols);

// Volume hooks for the model sessions (volume.cpp): bind a ready store (taken
// over), read a bound cell's store, change the batch, and
// cameral_train::train_volume_mse of the BP family (forward, MSE loss, then
// backward and SGD unless `frozen` or lr == 0).
welvet_status grid_bind_store(welvet_hip_grid *g, int z, int y, int x, int l, int in, int out,
                              int act, Store *W);
const Store *grid_store(welvet_hip_grid *g, int z, int y, int x, int l);
int grid_batch(const welvet_hip_grid *g);
welvet_status grid_set_batch(welvet_hip_grid *g, int batch);
welvet_status grid_train_volume_mse(welvet_hip_grid *g, const float *x, int in, const float *target,
                                    int out, double lr, bool frozen, double *loss);

}  // namespace rt
}  // namespace wh
