// runtime.cpp — host side of the Dense path and its C ABI (include/welvet_c.h).
//
// Mirrors the reference's flow and error behaviour:
//   welvet_dense_mount / execute / release   c_abi.cpp:102-128, session.cpp:37-97
//   welvet_dense_forward_f32                 c_abi.cpp:130-140
//   welvet_dense_normalbp_f32                c_abi.cpp:142-207 with the checks of
//                                            WeightStore::apply_sgd native_codec.cpp:909-945
//                                            and the Float32 launcher training.mm:71-128
// but keeps the native payload packed in HBM (encoded and decoded on the
// device) instead of a host WeightStore plus a float2 mirror.  One stream per
// session; calls on one session are serialised by its mutex.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/welvet_c.h"
#include "codec.hpp"
#include "runtime.hpp"

using namespace wh;
using namespace wh::rt;

namespace wh {
namespace rt {

welvet_status make_status(int code, const char *fmt, ...) {
  welvet_status st{};
  st.code = code;
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(st.message, sizeof(st.message), fmt, ap);
  va_end(ap);
  return st;
}



// ------------------------------------------------------------ device state
struct Device {
  std::once_flag once;
  int status = kUnsupported;
  std::string message = "no HIP device";
  std::string identity = "hip:unavailable";
  int id = -1;
};
Device g_dev;

void device_init() {
  std::call_once(g_dev.once, [] {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
      g_dev.message = "no HIP device";
      return;
    }
    hipDeviceProp_t p{};
    if (hipGetDeviceProperties(&p, 0) != hipSuccess) {
      g_dev.message = "hipGetDeviceProperties failed";
      return;
    }
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0) {
      g_dev.message = std::string("kernels are built for gfx950; device is ") + p.gcnArchName;
      return;
    }
    g_dev.id = 0;
    char buf[512];
    std::snprintf(buf, sizeof(buf), "hip:%s:%s:cu=%d:hbm=%.0fGiB:welvet-hip-dense", p.gcnArchName,
                  p.name, p.multiProcessorCount, (double)p.totalGlobalMem / (1024.0 * 1024 * 1024));
    g_dev.identity = buf;
    g_dev.status = kOk;
    g_dev.message.clear();
  });
}

welvet_status require_device() {
  device_init();
  if (g_dev.status != kOk) return make_status(g_dev.status, "%s", g_dev.message.c_str());
  if (hipSetDevice(g_dev.id) != hipSuccess) return make_status(kInternal, "hipSetDevice failed");
  return ok();
}

bool device_ready() {
  device_init();
  return g_dev.status == kOk;
}

const char *device_identity() {
  device_init();
  return g_dev.identity.c_str();
}

// ------------------------------------------------------- resident store
void free_store(Store *w) {
  if (w->body) (void)hipFree(w->body);
  if (w->kbody) (void)hipFree(w->kbody);
  if (w->tbody) (void)hipFree(w->tbody);
  w->tbody = nullptr;
  w->tbody_ok = false;
  if (w->lut) (void)hipFree(w->lut);
  if (w->bias) (void)hipFree(w->bias);
  w->body = nullptr;
  w->kbody = nullptr;
  w->lut = nullptr;
  w->bias = nullptr;
}

welvet_status store_prepare_backward(Store *w, int batch, hipStream_t s) {
  if (w->tbody_ok || !backward_wants_transposed(w->dev(), batch)) return ok();
  const size_t bytes = (size_t)w->rows * w->cols;
  if (w->tbody == nullptr) {
    // padding: the GEMM's last 64-column stage may read past the last row
    const size_t alloc = ((bytes + 64 + 255) / 256) * 256;
    WH_HIP(hipMalloc(&w->tbody, alloc));
    WH_HIP(hipMemsetAsync(w->tbody, 0, alloc, s));
  }
  const uint8_t *src = (w->dtype == kFP8E4M3 || w->dtype == kFP8E5M2) ? w->kbody : w->body;
  WH_HIP(launch_transpose_u8(src, w->rows, w->cols, w->tbody, s));
  w->tbody_ok = true;
  return ok();
}

// Device scratch reused by encode: Meta + Stats.
struct EncodeScratch {
  Meta meta;
  Stats stats;
  int nonfinite;
};

// WeightStore::make + encode_format_none (store.cpp:7-22, native_codec.cpp:819-833)
// on the device.  `d_w` holds the f32 init values.
welvet_status store_make(Store *w, int dtype, int rows, int cols, const float *d_w, hipStream_t s) {
  w->dtype = dtype;
  w->rows = rows;
  w->cols = cols;
  const int64_t n = w->n();
  const int bits = dtype_bits(dtype);
  w->body_bytes = (size_t)((n * bits + 7) / 8);
  // padding: a full 16-byte chunk past the last element stays in the allocation
  const size_t alloc = ((w->body_bytes + 64 + 255) / 256) * 256;
  WH_HIP(hipMalloc(&w->body, alloc));
  WH_HIP(hipMemsetAsync(w->body, 0, alloc, s));
  if (dtype == kFP8E4M3 || dtype == kFP8E5M2) {
    WH_HIP(hipMalloc(&w->kbody, alloc));
    WH_HIP(hipMemsetAsync(w->kbody, 0, alloc, s));
  }
  return store_encode(w, d_w, false, s);
}

// Encodes f32 values already in HBM into the store's existing allocation:
// pack_native's statistics and codes, or op_native_repack's (repack); then
// the scale, min, decode tables and non-finite flag follow the new codes and
// the transposed copy is stale.
welvet_status store_encode(Store *w, const float *d_w, bool repack, hipStream_t s) {
  const int dtype = w->dtype;
  const int64_t n = w->n();
  w->tbody_ok = false;
  if (dtype == kFloat32) {
    WH_HIP(hipMemcpyAsync(w->body, d_w, (size_t)n * 4, hipMemcpyDeviceToDevice, s));
    w->scale = 1.0f;
    w->minv = 0.0f;
    return ok();
  }
  EncodeScratch *scratch = nullptr;
  WH_HIP(hipMalloc(&scratch, sizeof(EncodeScratch)));
  hipError_t e = launch_encode(dtype, d_w, n, w->body, w->kbody, &scratch->meta, &scratch->stats, s, repack);
  Meta m{};
  int nonfinite = 0;
  if (dtype == kFP8E5M2) {
    if (e == hipSuccess) e = hipMemsetAsync(&scratch->nonfinite, 0, sizeof(int), s);
    if (e == hipSuccess) e = launch_e5m2_nonfinite(w->kbody, n, &scratch->nonfinite, s);
    if (e == hipSuccess) e = hipMemcpyAsync(&nonfinite, &scratch->nonfinite, sizeof(int), hipMemcpyDeviceToHost, s);
  }
  if (e == hipSuccess) e = hipMemcpyAsync(&m, &scratch->meta, sizeof(Meta), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  (void)hipFree(scratch);
  WH_HIP(e);
  w->scale = m.scale;
  w->minv = m.minv;
  w->finite = nonfinite == 0;
  if (dtype_lut(dtype)) {
    if (w->lut == nullptr) WH_HIP(hipMalloc(&w->lut, kLutFloats * sizeof(float)));
    WH_HIP(launch_lut(dtype, w->scale, w->minv, w->lut, s));
    WH_HIP(hipStreamSynchronize(s));
  }
  return ok();
}

welvet_status store_from_native(Store *w, int dtype, int rows, int cols, float scale,
                                const float *f32, size_t nf32, const uint8_t *raw, size_t nraw,
                                hipStream_t s) {
  if (dtype < 0 || dtype >= kNumDTypes || !dims_ok(rows, cols) || !std::isfinite(scale))
    return make_status(kInvalid, "native store metadata mismatch");
  const int64_t n = (int64_t)rows * cols;
  const bool is_f32 = dtype == kFloat32;
  if (is_f32 ? (nf32 != (size_t)n || nraw != 0) : (nf32 != 0 || nraw != (size_t)native_bytes(dtype, n)))
    return make_status(kInvalid, "native store payload length mismatch");
  w->dtype = dtype;
  w->rows = rows;
  w->cols = cols;
  w->body_bytes = (size_t)((n * dtype_bits(dtype) + 7) / 8);
  const size_t alloc = ((w->body_bytes + 64 + 255) / 256) * 256;
  WH_HIP(hipMalloc(&w->body, alloc));
  WH_HIP(hipMemsetAsync(w->body, 0, alloc, s));
  if (is_f32) {  // WeightStore::f32; the scale of a Float32 store is 1 (encode_format_none)
    WH_HIP(hipMemcpyAsync(w->body, f32, (size_t)n * 4, hipMemcpyHostToDevice, s));
    w->scale = 1.0f;
    w->minv = 0.0f;
    WH_HIP(hipStreamSynchronize(s));
    return ok();
  }
  const size_t hdr = dtype_has_min(dtype) ? 4 : 0;
  w->scale = scale;
  w->minv = 0.0f;
  if (hdr) std::memcpy(&w->minv, raw, 4);
  WH_HIP(hipMemcpyAsync(w->body, raw + hdr, w->body_bytes, hipMemcpyHostToDevice, s));
  std::vector<uint8_t> k;
  if (dtype == kFP8E4M3 || dtype == kFP8E5M2) {  // the decode-ready copy, made on the host
    k.resize(w->body_bytes);
    bool finite = true;
    for (size_t i = 0; i < k.size(); ++i) {
      const uint32_t c = raw[hdr + i];
      if (dtype == kFP8E4M3) {
        k[i] = kcode<kFP8E4M3>(c);
      } else {
        k[i] = kcode<kFP8E5M2>(c);
        finite = finite && (c & 0x7cu) != 0x7cu;
      }
    }
    w->finite = finite;
    WH_HIP(hipMalloc(&w->kbody, alloc));
    WH_HIP(hipMemsetAsync(w->kbody, 0, alloc, s));
    WH_HIP(hipMemcpyAsync(w->kbody, k.data(), k.size(), hipMemcpyHostToDevice, s));
  }
  if (dtype_lut(dtype)) {
    WH_HIP(hipMalloc(&w->lut, kLutFloats * sizeof(float)));
    WH_HIP(launch_lut(dtype, w->scale, w->minv, w->lut, s));
  }
  WH_HIP(hipStreamSynchronize(s));  // k and the caller's buffers outlive the copies
  return ok();
}

welvet_status store_repack_host(Store *w, const float *values, hipStream_t s) {
  float *d = nullptr;
  const size_t bytes = (size_t)w->n() * sizeof(float);
  WH_HIP(hipMalloc(&d, bytes));
  hipError_t e = hipMemcpyAsync(d, values, bytes, hipMemcpyHostToDevice, s);
  welvet_status st = e == hipSuccess ? store_encode(w, d, true, s)
                                     : make_status(kInternal, "hip: %s", hipGetErrorString(e));
  e = hipStreamSynchronize(s);
  (void)hipFree(d);
  if (st.code) return st;
  WH_HIP(e);
  return ok();
}

welvet_status store_set_bias(Store *w, const double *bias, size_t bias_len, hipStream_t s) {
  if (bias == nullptr || bias_len == 0) return ok();
  if (bias_len > (size_t)INT32_MAX) return make_status(kInvalid, "bias too long");
  WH_HIP(hipMalloc(&w->bias, bias_len * sizeof(double)));
  WH_HIP(hipMemcpyAsync(w->bias, bias, bias_len * sizeof(double), hipMemcpyHostToDevice, s));
  w->bias_len = (int)bias_len;
  return ok();
}

// Upload f32 weights and build the store.
welvet_status store_from_host(Store *w, int dtype, int rows, int cols, const float *W_init,
                              hipStream_t s) {
  float *d_w = nullptr;
  const size_t bytes = (size_t)rows * cols * sizeof(float);
  WH_HIP(hipMalloc(&d_w, bytes));
  hipError_t e = hipMemcpyAsync(d_w, W_init, bytes, hipMemcpyHostToDevice, s);
  welvet_status st = e == hipSuccess ? store_make(w, dtype, rows, cols, d_w, s)
                                     : make_status(kInternal, "hip: %s", hipGetErrorString(e));
  (void)hipStreamSynchronize(s);
  (void)hipFree(d_w);
  return st;
}

// WeightStore::apply_sgd (native_codec.cpp:909-945) on a device gradient,
// with the Float32 launcher's checks (training.mm:71-128).
welvet_status store_sgd(Store *w, const float *d_dW, double lr, int *d_flag, hipStream_t s) {
  if (!std::isfinite(lr)) return make_status(kInvalid, "weights: bad SGD arguments");
  const int64_t n = w->n();
  if (n > INT32_MAX) return make_status(kInvalid, "SGD: tensor too large");
  int flag = 0;
  WH_HIP(hipMemsetAsync(d_flag, 0, sizeof(int), s));
  WH_HIP(launch_nonfinite(d_dW, n, d_flag, 1, s));
  WH_HIP(hipMemcpyAsync(&flag, d_flag, sizeof(int), hipMemcpyDeviceToHost, s));
  WH_HIP(hipStreamSynchronize(s));
  if (w->dtype == kFloat32) {
    if (flag) return make_status(kUnsupported, "SGD: gradient is not a finite f32");
    if (std::fabs(lr) > FLT_MAX || (lr != 0.0 && std::fabs(lr) < FLT_MIN))
      return make_status(kUnsupported, "SGD: learning rate outside the f32 range");
  } else if (flag) {
    return make_status(kInvalid, "weights: nonfinite gradient");
  }
  // *d_flag is 0 here (the gradient check passed); an E5M2 update sets it
  // when a new code is Inf or NaN, which decides the store's decode route
  const bool e5 = w->dtype == kFP8E5M2;
  WH_HIP(launch_sgd(w->dtype, w->body, w->kbody, n, d_dW, lr, w->scale, w->minv, nullptr, nullptr, 0, s,
                    e5 ? d_flag : nullptr));
  w->tbody_ok = false;
  if (e5) {
    WH_HIP(hipMemcpyAsync(&flag, d_flag, sizeof(int), hipMemcpyDeviceToHost, s));
    WH_HIP(hipStreamSynchronize(s));
    w->finite = flag == 0;
  }
  return ok();
}

// Native bytes in the reference layout (header + payload).
welvet_status store_native(const Store &w, uint8_t *out, size_t cap, size_t *len, hipStream_t s) {
  const size_t hdr = dtype_has_min(w.dtype) ? 4 : 0;
  const size_t need = hdr + w.body_bytes;
  if (len) *len = need;
  if (out == nullptr || cap < need) return make_status(kInvalid, "native: buffer too small (%zu)", need);
  if (hdr) std::memcpy(out, &w.minv, 4);
  WH_HIP(hipMemcpyAsync(out + hdr, w.body, w.body_bytes, hipMemcpyDeviceToHost, s));
  WH_HIP(hipStreamSynchronize(s));
  return ok();
}

welvet_status store_export(const Store &w, float *d_out, hipStream_t s) {
  WH_HIP(launch_decode(w.dtype, w.body, w.n(), w.scale, w.minv, d_out, s));
  return ok();
}

bool dims_ok(int32_t rows, int32_t cols) {
  return rows > 0 && cols > 0 && (int64_t)rows * cols <= INT32_MAX;
}

}  // namespace rt
}  // namespace wh

// ------------------------------------------------------------- session
struct welvet_dense_session {
  std::mutex mu;
  Store W;
  int batch = 0, act = kLinear;
  hipStream_t stream = nullptr;
  float *d_x = nullptr, *d_pre = nullptr, *d_post = nullptr;
  void *ws = nullptr;
  size_t ws_bytes = 0;
  int *d_flag = nullptr;
};

namespace {

void session_free(welvet_dense_session *s) {
  if (!s) return;
  if (s->stream) (void)hipStreamSynchronize(s->stream);
  free_store(&s->W);
  if (s->d_x) (void)hipFree(s->d_x);
  if (s->d_pre) (void)hipFree(s->d_pre);
  if (s->d_post) (void)hipFree(s->d_post);
  if (s->ws) (void)hipFree(s->ws);
  if (s->d_flag) (void)hipFree(s->d_flag);
  if (s->stream) (void)hipStreamDestroy(s->stream);
  delete s;
}

welvet_status session_alloc_io(welvet_dense_session *s) {
  const size_t xb = (size_t)s->batch * s->W.cols * sizeof(float);
  const size_t yb = (size_t)s->batch * s->W.rows * sizeof(float);
  WH_HIP(hipMalloc(&s->d_x, xb));
  WH_HIP(hipMalloc(&s->d_pre, yb));
  WH_HIP(hipMalloc(&s->d_post, yb));
  WH_HIP(hipMalloc(&s->d_flag, 256));
  s->ws_bytes = forward_workspace_bytes(s->W.dev(), s->batch);
  const size_t mb = mse_workspace_bytes(0);
  if (s->ws_bytes < mb) s->ws_bytes = mb;
  WH_HIP(hipMalloc(&s->ws, s->ws_bytes));
  return ok();
}

welvet_status ensure_ws(welvet_dense_session *s, size_t bytes) {
  if (bytes <= s->ws_bytes) return ok();
  // the old workspace may be in use on a caller's stream: drain the device
  WH_HIP(hipDeviceSynchronize());
  if (s->ws) WH_HIP(hipFree(s->ws));
  s->ws = nullptr;
  WH_HIP(hipMalloc(&s->ws, bytes));
  s->ws_bytes = bytes;
  return ok();
}

welvet_status forward_device(welvet_dense_session *s, const float *x, float *pre, float *post,
                             hipStream_t st) {
  // the kernel plan (and so the workspace) can change with the tuning knobs
  welvet_status ws = ensure_ws(s, forward_workspace_bytes(s->W.dev(), s->batch));
  if (ws.code) return ws;
  WH_HIP(launch_forward(s->W.dev(), s->batch, x, s->W.bias, s->W.bias_len, s->act, pre, post, s->ws,
                        s->ws_bytes, st));
  return ok();
}

// ------------------------------------------------- no-allocation forward
// The stream-K partial tiles of welvet_hip_dense_forward_noalloc live in this
// file-scope device array instead of a session workspace, so that call
// allocates nothing.  Every GPU the library runs on holds its own copy for the
// life of the process; host code reaches it only through the address
// hipGetSymbolAddress returns for the current device (the array's name on the
// host is a stand-in, not a device address).  Every slot a reduce reads is
// written by the same launch's GEMM first, so nothing needs clearing.
constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
struct ScratchAddr {
  std::once_flag once;
  void *ptr = nullptr;
  hipError_t err = hipErrorNotInitialized;
};
ScratchAddr g_scratch[kMaxDevices];

// The current device's copy of `scratch`, looked up once per device (with
// that device current); null when the lookup failed.
void *scratch_ptr(hipError_t *err) {
  int dev = -1;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  ScratchAddr &a = g_scratch[dev];
  std::call_once(a.once, [&a] { a.err = hipGetSymbolAddress(&a.ptr, HIP_SYMBOL(scratch)); });
  *err = a.err;
  return a.err == hipSuccess ? a.ptr : nullptr;
}

// Where a mount's weights come from: f32 values on the host or the device
// (encoded on the device), or a store snapshot in the reference's native
// byte layout (taken byte for byte).
struct WeightSource {
  enum Kind { kHostF32, kDeviceF32, kNative } kind = kHostF32;
  const float *f32 = nullptr;
  const uint8_t *raw = nullptr;
  size_t raw_len = 0;
  float scale = 1.0f;
};

// session_mount session.cpp:37-84 (dtype -> 2, dims/batch -> 1)
welvet_status mount(int32_t batch, int32_t in, int32_t out, int32_t act, int32_t dtype,
                    const WeightSource &src, const double *bias, size_t bias_len,
                    welvet_dense_session **sess) {
  if (!sess || (src.kind == WeightSource::kNative ? !src.raw : !src.f32))
    return make_status(kInvalid, "invalid argument");
  if (dtype < 0 || dtype >= kNumDTypes)
    return make_status(kUnsupported, "dense HIP unsupported dtype %d", dtype);
  welvet_status st = require_device();
  if (st.code) return st;
  if (!dims_ok(out, in)) return make_status(kInvalid, "weights: bad shape");
  if (batch <= 0) return make_status(kInvalid, "bad resident dims");
  auto *s = new welvet_dense_session();
  s->batch = batch;
  s->act = act;
  if (hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking) != hipSuccess) {
    delete s;
    return make_status(kInternal, "hipStreamCreate failed");
  }
  if (src.kind == WeightSource::kDeviceF32) {
    st = store_make(&s->W, dtype, out, in, src.f32, s->stream);
  } else if (src.kind == WeightSource::kHostF32) {
    st = store_from_host(&s->W, dtype, out, in, src.f32, s->stream);
  } else if (dtype == kFloat32) {
    st = src.raw_len % 4 ? make_status(kInvalid, "native store payload length mismatch")
                         : store_from_native(&s->W, dtype, out, in, 1.0f, (const float *)src.raw,
                                             src.raw_len / 4, nullptr, 0, s->stream);
  } else {
    st = store_from_native(&s->W, dtype, out, in, src.scale, nullptr, 0, src.raw, src.raw_len, s->stream);
  }
  if (!st.code) st = store_set_bias(&s->W, bias, bias_len, s->stream);
  if (!st.code) st = session_alloc_io(s);
  if (!st.code && hipStreamSynchronize(s->stream) != hipSuccess)
    st = make_status(kInternal, "mount: stream failed");
  if (st.code) {
    session_free(s);
    return st;
  }
  *sess = s;
  return ok();
}

welvet_status execute(welvet_dense_session *s, const float *x, float *pre, float *post) {
  if (!s || !x || !pre || !post) return make_status(kInvalid, "null execute args");
  std::lock_guard<std::mutex> lock(s->mu);
  const size_t xb = (size_t)s->batch * s->W.cols * sizeof(float);
  const size_t yb = (size_t)s->batch * s->W.rows * sizeof(float);
  WH_HIP(hipSetDevice(g_dev.id));
  WH_HIP(hipMemcpyAsync(s->d_x, x, xb, hipMemcpyHostToDevice, s->stream));
  welvet_status st = forward_device(s, s->d_x, s->d_pre, s->d_post, s->stream);
  if (st.code) return st;
  WH_HIP(hipMemcpyAsync(pre, s->d_pre, yb, hipMemcpyDeviceToHost, s->stream));
  WH_HIP(hipMemcpyAsync(post, s->d_post, yb, hipMemcpyDeviceToHost, s->stream));
  WH_HIP(hipStreamSynchronize(s->stream));
  return ok();
}

// Device buffers of one NormalBP / backward call.
struct Bwd {
  float *gy = nullptr, *dpre = nullptr, *dX = nullptr, *dW = nullptr, *pre = nullptr;
  double *loss = nullptr;
  ~Bwd() {
    for (void *p : {(void *)gy, (void *)dpre, (void *)dX, (void *)dW, (void *)pre, (void *)loss})
      if (p) (void)hipFree(p);
  }
};

welvet_status backward_device(welvet_dense_session *s, const float *d_x, const float *d_pre,
                              const float *d_gy, Bwd *b) {
  const int64_t ny = (int64_t)s->batch * s->W.rows, nx = (int64_t)s->batch * s->W.cols;
  WH_HIP(hipMalloc(&b->dpre, ny * sizeof(float)));
  WH_HIP(hipMalloc(&b->dX, nx * sizeof(float)));
  WH_HIP(hipMalloc(&b->dW, s->W.n() * sizeof(float)));
  welvet_status st = ensure_ws(s, backward_workspace_bytes(s->W.dev(), s->batch));
  if (st.code == 0) st = store_prepare_backward(&s->W, s->batch, s->stream);
  if (st.code) return st;
  WH_HIP(hipMemsetAsync(s->d_flag, 0, sizeof(int), s->stream));
  WH_HIP(launch_backward(s->W.dev(), s->batch, d_x, d_pre, d_gy, s->act, b->dpre, b->dX, b->dW,
                         s->d_flag, s->ws, s->ws_bytes, s->stream));
  return ok();
}

}  // namespace

extern "C" {

const char *welvet_version(void) { return "0.71"; }

const char *welvet_runtime_identity(void) {
  device_init();
  static thread_local std::string id;
  id = g_dev.identity;
  return id.c_str();
}

welvet_status welvet_metal_init(void) {
  welvet_status st = require_device();
  if (st.code) return st;
  // probe: encode and decode two values through the device codec
  const float w[2] = {0.5f, -0.25f};
  welvet_dense_session *s = nullptr;
  WeightSource src;
  src.f32 = w;
  st = mount(1, 2, 1, kLinear, kFP8E4M3, src, nullptr, 0, &s);
  if (st.code) return st;
  float back[2] = {0, 0};
  st = welvet_hip_dense_export_f32(s, back);
  session_free(s);
  if (st.code) return st;
  if (back[0] != 0.5f || back[1] != -0.25f) return make_status(kInternal, "device codec probe failed");
  return ok();
}

int32_t welvet_metal_available(void) {
  device_init();
  return g_dev.status == kOk ? 1 : 0;
}

welvet_status welvet_dense_mount(int32_t batch, int32_t in, int32_t out, int32_t act, int32_t dtype,
                                 const float *W_init, const double *bias, size_t bias_len,
                                 welvet_dense_session **sess) {
  WeightSource src;
  src.f32 = W_init;
  return mount(batch, in, out, act, dtype, src, bias, bias_len, sess);
}

welvet_status welvet_hip_dense_mount_device(int32_t batch, int32_t in, int32_t out, int32_t act,
                                            int32_t dtype, const float *d_W_init,
                                            const double *bias, size_t bias_len,
                                            welvet_dense_session **sess) {
  if ((uintptr_t)d_W_init & 15) return make_status(kInvalid, "device pointers must be 16-byte aligned");
  WeightSource src;
  src.kind = WeightSource::kDeviceF32;
  src.f32 = d_W_init;
  return mount(batch, in, out, act, dtype, src, bias, bias_len, sess);
}

welvet_status welvet_hip_dense_mount_native(int32_t batch, int32_t in, int32_t out, int32_t act,
                                            int32_t dtype, const uint8_t *native, size_t native_len,
                                            float scale, const double *bias, size_t bias_len,
                                            welvet_dense_session **sess) {
  WeightSource src;
  src.kind = WeightSource::kNative;
  src.raw = native;
  src.raw_len = native_len;
  src.scale = scale;
  return mount(batch, in, out, act, dtype, src, bias, bias_len, sess);
}

welvet_status welvet_dense_execute(welvet_dense_session *s, const float *x, float *pre, float *post) {
  return execute(s, x, pre, post);
}

void welvet_dense_release(welvet_dense_session *s) { session_free(s); }

welvet_status welvet_dense_forward_f32(int32_t batch, int32_t in, int32_t out, int32_t act,
                                       int32_t dtype, int32_t /*backend*/, const float *W_init,
                                       const double *bias, size_t bias_len, const float *x,
                                       float *pre, float *post) {
  welvet_dense_session *s = nullptr;
  WeightSource src;
  src.f32 = W_init;
  welvet_status st = mount(batch, in, out, act, dtype, src, bias, bias_len, &s);
  if (st.code) return st;
  st = execute(s, x, pre, post);
  session_free(s);
  return st;
}

welvet_status welvet_dense_normalbp_f32(int32_t batch, int32_t in, int32_t out, int32_t act,
                                        int32_t dtype, int32_t /*backend*/, const float *W_init,
                                        const double *bias, size_t bias_len, const float *x,
                                        const float *grad_or_target, int32_t use_target, double lr,
                                        float *pre, float *post, float *dX, float *dW,
                                        float *W_after, double *loss) {
  if (batch <= 0 || in <= 0 || out <= 0 || !W_init || !x || !grad_or_target || !pre || !post ||
      !dX || !dW || !W_after || !loss)
    return make_status(kInvalid, "invalid argument");
  if (dtype < 0 || dtype >= kNumDTypes) return make_status(kInvalid, "bad dtype %d", dtype);
  welvet_dense_session *s = nullptr;
  WeightSource src;
  src.f32 = W_init;
  welvet_status st = mount(batch, in, out, act, dtype, src, bias, bias_len, &s);
  if (st.code) return st;
  const int64_t ny = (int64_t)batch * out, nx = (int64_t)batch * in, nw = (int64_t)out * in;
  hipStream_t strm = s->stream;
  Bwd b;
  auto run = [&]() -> welvet_status {
    WH_HIP(hipMemcpyAsync(s->d_x, x, nx * sizeof(float), hipMemcpyHostToDevice, strm));
    st = forward_device(s, s->d_x, s->d_pre, s->d_post, strm);
    if (st.code) return st;
    WH_HIP(hipMalloc(&b.gy, ny * sizeof(float)));
    WH_HIP(hipMalloc(&b.loss, sizeof(double)));
    double h_loss = 0.0;
    if (use_target) {
      float *d_t = nullptr;
      WH_HIP(hipMalloc(&d_t, ny * sizeof(float)));
      hipError_t e = hipMemcpyAsync(d_t, grad_or_target, ny * sizeof(float), hipMemcpyHostToDevice, strm);
      if (e == hipSuccess)
        e = launch_mse(s->d_post, d_t, ny, b.loss, b.gy, s->ws, s->ws_bytes, strm);
      if (e == hipSuccess) e = hipMemcpyAsync(&h_loss, b.loss, sizeof(double), hipMemcpyDeviceToHost, strm);
      if (e == hipSuccess) e = hipStreamSynchronize(strm);
      (void)hipFree(d_t);
      WH_HIP(e);
    } else {
      WH_HIP(hipMemcpyAsync(b.gy, grad_or_target, ny * sizeof(float), hipMemcpyHostToDevice, strm));
    }
    st = backward_device(s, s->d_x, s->d_pre, b.gy, &b);
    if (st.code) return st;
    if (lr != 0.0) {
      st = store_sgd(&s->W, b.dW, lr, s->d_flag, strm);
      if (st.code) return st;
    }
    float *d_after = nullptr;
    WH_HIP(hipMalloc(&d_after, nw * sizeof(float)));
    st = store_export(s->W, d_after, strm);
    hipError_t e = st.code ? hipSuccess
                           : hipMemcpyAsync(W_after, d_after, nw * sizeof(float), hipMemcpyDeviceToHost, strm);
    if (e == hipSuccess) e = hipStreamSynchronize(strm);
    (void)hipFree(d_after);
    if (st.code) return st;
    WH_HIP(e);
    WH_HIP(hipMemcpyAsync(pre, s->d_pre, ny * sizeof(float), hipMemcpyDeviceToHost, strm));
    WH_HIP(hipMemcpyAsync(post, s->d_post, ny * sizeof(float), hipMemcpyDeviceToHost, strm));
    WH_HIP(hipMemcpyAsync(dX, b.dX, nx * sizeof(float), hipMemcpyDeviceToHost, strm));
    WH_HIP(hipMemcpyAsync(dW, b.dW, nw * sizeof(float), hipMemcpyDeviceToHost, strm));
    WH_HIP(hipStreamSynchronize(strm));
    *loss = h_loss;
    return ok();
  };
  st = run();
  (void)hipStreamSynchronize(strm);
  session_free(s);
  return st;
}

welvet_status welvet_hip_dense_forward_device(welvet_dense_session *s, const float *d_x,
                                              float *d_pre, float *d_post, void *stream) {
  if (!s || !d_x || !d_pre || !d_post) return make_status(kInvalid, "null execute args");
  if (((uintptr_t)d_x | (uintptr_t)d_pre | (uintptr_t)d_post) & 15)
    return make_status(kInvalid, "device pointers must be 16-byte aligned");
  std::lock_guard<std::mutex> lock(s->mu);
  return forward_device(s, d_x, d_pre, d_post, (hipStream_t)stream);
}

welvet_status welvet_hip_dense_forward_noalloc(welvet_dense_session *s, int32_t batch,
                                               const float *d_x, float *d_pre, float *d_post,
                                               void *stream) {
  if (!s || !d_x || !d_pre || !d_post) return make_status(kInvalid, "null execute args");
  if (((uintptr_t)d_x | (uintptr_t)d_pre | (uintptr_t)d_post) & 15)
    return make_status(kInvalid, "device pointers must be 16-byte aligned");
  if (batch <= 0) return make_status(kInvalid, "bad batch %d", batch);
  const size_t need = forward_workspace_bytes(s->W.dev(), batch);
  if (need > kScratchBytes)
    return make_status(kInvalid, "no-allocation forward: batch %d needs %zu bytes of scratch (limit %zu)",
                       batch, need, kScratchBytes);
  WH_HIP(hipSetDevice(g_dev.id));
  hipError_t e = hipSuccess;
  void *ws = scratch_ptr(&e);
  if (ws == nullptr)
    return make_status(kInternal, "no-allocation forward: scratch address: %s", hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(s->mu);
  WH_HIP(launch_forward(s->W.dev(), batch, d_x, s->W.bias, s->W.bias_len, s->act, d_pre, d_post, ws,
                        kScratchBytes, (hipStream_t)stream));
  return ok();
}

welvet_status welvet_hip_dense_native(welvet_dense_session *s, uint8_t *out, size_t cap,
                                      size_t *len, float *scale) {
  if (!s) return make_status(kInvalid, "null session");
  std::lock_guard<std::mutex> lock(s->mu);
  if (scale) *scale = s->W.scale;
  if (s->W.dtype == kFloat32) {  // WeightStore::f32
    if (scale) *scale = 1.0f;
  }
  return store_native(s->W, out, cap, len, s->stream);
}

welvet_status welvet_hip_dense_repack(welvet_dense_session *s, const float *values, size_t len) {
  if (!s) return make_status(kInvalid, "null session");
  if (!values || len == 0 || len != (size_t)s->W.n())
    return make_status(kInvalid, "blend: invalid native store replacement");
  std::lock_guard<std::mutex> lock(s->mu);
  WH_HIP(hipSetDevice(g_dev.id));
  return store_repack_host(&s->W, values, s->stream);
}

welvet_status welvet_hip_dense_export_f32(welvet_dense_session *s, float *W_out) {
  if (!s || !W_out) return make_status(kInvalid, "weights: nil dst");
  std::lock_guard<std::mutex> lock(s->mu);
  const size_t bytes = (size_t)s->W.n() * sizeof(float);
  float *d = nullptr;
  WH_HIP(hipMalloc(&d, bytes));
  welvet_status st = store_export(s->W, d, s->stream);
  hipError_t e = st.code ? hipSuccess : hipMemcpyAsync(W_out, d, bytes, hipMemcpyDeviceToHost, s->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
  (void)hipFree(d);
  if (st.code) return st;
  WH_HIP(e);
  return ok();
}

welvet_status welvet_hip_dense_backward(welvet_dense_session *s, const float *x, const float *pre,
                                        const float *gy, float *dX, float *dW) {
  if (!s || !x || !pre || !gy || !dX || !dW) return make_status(kInvalid, "null resident backward");
  std::lock_guard<std::mutex> lock(s->mu);
  const int64_t ny = (int64_t)s->batch * s->W.rows, nx = (int64_t)s->batch * s->W.cols;
  Bwd b;
  WH_HIP(hipMalloc(&b.gy, ny * sizeof(float)));
  WH_HIP(hipMalloc(&b.pre, ny * sizeof(float)));
  WH_HIP(hipMemcpyAsync(s->d_x, x, nx * sizeof(float), hipMemcpyHostToDevice, s->stream));
  WH_HIP(hipMemcpyAsync(b.pre, pre, ny * sizeof(float), hipMemcpyHostToDevice, s->stream));
  WH_HIP(hipMemcpyAsync(b.gy, gy, ny * sizeof(float), hipMemcpyHostToDevice, s->stream));
  welvet_status st = backward_device(s, s->d_x, b.pre, b.gy, &b);
  if (st.code) return st;
  WH_HIP(hipMemcpyAsync(dX, b.dX, nx * sizeof(float), hipMemcpyDeviceToHost, s->stream));
  WH_HIP(hipMemcpyAsync(dW, b.dW, s->W.n() * sizeof(float), hipMemcpyDeviceToHost, s->stream));
  WH_HIP(hipStreamSynchronize(s->stream));
  return ok();
}

welvet_status welvet_hip_dense_sgd(welvet_dense_session *s, const float *dW, double lr) {
  if (!s || !dW) return make_status(kInvalid, "weights: bad SGD arguments");
  std::lock_guard<std::mutex> lock(s->mu);
  float *d = nullptr;
  const size_t bytes = (size_t)s->W.n() * sizeof(float);
  WH_HIP(hipMalloc(&d, bytes));
  hipError_t e = hipMemcpyAsync(d, dW, bytes, hipMemcpyHostToDevice, s->stream);
  welvet_status st = e == hipSuccess ? store_sgd(&s->W, d, lr, s->d_flag, s->stream)
                                     : make_status(kInternal, "hip: %s", hipGetErrorString(e));
  (void)hipStreamSynchronize(s->stream);
  (void)hipFree(d);
  return st;
}

welvet_status welvet_hip_mse_f32(const float *pred, const float *target, size_t n, double *loss,
                                 float *grad) {
  if (!pred || !target || n == 0 || (!loss && !grad))
    return make_status(kInvalid, "MSE: invalid arguments");
  welvet_status st = require_device();
  if (st.code) return st;
  float *dp = nullptr, *dt = nullptr, *dg = nullptr;
  double *dl = nullptr;
  void *ws = nullptr;
  auto run = [&]() -> welvet_status {
    WH_HIP(hipMalloc(&dp, n * 4));
    WH_HIP(hipMalloc(&dt, n * 4));
    WH_HIP(hipMalloc(&dg, n * 4));
    WH_HIP(hipMalloc(&dl, 8));
    WH_HIP(hipMalloc(&ws, mse_workspace_bytes((int64_t)n)));
    WH_HIP(hipMemcpy(dp, pred, n * 4, hipMemcpyHostToDevice));
    WH_HIP(hipMemcpy(dt, target, n * 4, hipMemcpyHostToDevice));
    WH_HIP(launch_mse(dp, dt, (int64_t)n, loss ? dl : nullptr, grad ? dg : nullptr, ws,
                      mse_workspace_bytes((int64_t)n), nullptr));
    WH_HIP(hipDeviceSynchronize());
    if (loss) WH_HIP(hipMemcpy(loss, dl, 8, hipMemcpyDeviceToHost));
    if (grad) WH_HIP(hipMemcpy(grad, dg, n * 4, hipMemcpyDeviceToHost));
    return ok();
  };
  st = run();
  for (void *p : {(void *)dp, (void *)dt, (void *)dg, (void *)dl, ws})
    if (p) (void)hipFree(p);
  return st;
}

void welvet_hip_set_forward_path(int32_t path) { set_forward_path(path); }

int32_t welvet_hip_set_tuning(int32_t key, int32_t value) { return set_tuning(key, value); }

welvet_status welvet_hip_probe_read(const void *d_bytes, uint64_t bytes, void *d_sink, void *stream) {
  if (!d_bytes || !d_sink) return make_status(kInvalid, "null probe args");
  if ((((uintptr_t)d_bytes | (uintptr_t)d_sink) & 15) || bytes == 0 || bytes % 16)
    return make_status(kInvalid, "probe: 16-byte aligned pointers and a non-zero multiple of 16 bytes");
  WH_HIP(launch_read_probe(d_bytes, (int64_t)bytes, (uint32_t *)d_sink, (hipStream_t)stream));
  return ok();
}

}  // extern "C"
