// swiglu.cpp — SwiGLU over three resident Dense stores, behind the
// reference's C ABI entries
//   welvet_swiglu_forward_f32                  c_abi.cpp:326-361
//   welvet_swiglu_normalbp_f32                 c_abi.cpp:363-432
// with the layer semantics of src/layers/swiglu/swiglu.cpp:
//   Gate, Up  = Dense(in -> inter, Linear), Down = Dense(inter -> in, Linear),
//   forward   h = silu(Gate x) * (Up x), post = Down h, pre = h   (:93-141)
//   backward  Down's dX and dW on h, op_swiglu's split of grad_h into the
//             Gate and Up output gradients, grad_in = dX_gate + dX_up,
//             dW = concat(dW_gate, dW_up, dW_down)                  (:164-252)
//   SGD       Gate, Up, Down in that order, the first failure stops (:254-275)
// The three stores stay packed in HBM and every step is a kernel of this
// library (the Dense GEMV/GEMM, dX and dW kernels; op_swiglu's forward in
// the epilogue of the Up projection, its backward as one element-wise
// kernel); nothing round-trips through the host between the layers.  The backward reuses the forward's gate, up, h and Down pre
// values: the reference recomputes them with the same deterministic kernels.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <vector>

#include "../../include/welvet_c.h"
#include "runtime.hpp"

using namespace wh;
using namespace wh::rt;

namespace {

struct Swiglu {
  Store gate, up, down;
  int bs = 0, in = 0, inter = 0;
  hipStream_t stream = nullptr;
  void *ws = nullptr;
  size_t ws_bytes = 0;
  std::vector<void *> bufs;
  float *x = nullptr, *g_pre = nullptr, *u_pre = nullptr;
  float *h = nullptr, *d_pre = nullptr, *d_post = nullptr;
  int *flag = nullptr;

  ~Swiglu() {
    if (stream) (void)hipStreamSynchronize(stream);
    for (void *p : bufs) (void)hipFree(p);
    if (ws) (void)hipFree(ws);
    free_store(&gate);
    free_store(&up);
    free_store(&down);
    if (stream) (void)hipStreamDestroy(stream);
  }
  template <class T>
  welvet_status alloc(T **p, int64_t elems) {
    WH_HIP(hipMalloc((void **)p, (size_t)std::max<int64_t>(elems, 1) * sizeof(T)));
    bufs.push_back(*p);
    return ok();
  }
  welvet_status grow_ws(size_t bytes) {
    if (bytes <= ws_bytes) return ok();
    WH_HIP(hipStreamSynchronize(stream));
    if (ws) WH_HIP(hipFree(ws));
    ws = nullptr;
    ws_bytes = 0;
    WH_HIP(hipMalloc(&ws, bytes));
    ws_bytes = bytes;
    return ok();
  }
};

welvet_status prefixed(const char *part, welvet_status st) {
  if (st.code == 0) return st;
  char msg[sizeof st.message];
  std::snprintf(msg, sizeof msg, "swiglu %s: %s", part, st.message);
  std::memcpy(st.message, msg, sizeof msg);
  return st;
}

// swiglu::new_configured swiglu.cpp:70-91 (dense::new_layer per part) and the
// device buffers of one forward at bs = batch * seq rows.
welvet_status make(Swiglu *L, int bs, int in, int inter, int dtype, const float *Gate,
                   const float *Up, const float *Down) {
  welvet_status st = require_device();
  if (st.code) return st;
  if (dtype < 0 || dtype >= kNumDTypes)
    return make_status(kUnsupported, "swiglu Gate: dense HIP unsupported dtype %d", dtype);
  if (!dims_ok(inter, in) || (int64_t)bs * inter > INT32_MAX || (int64_t)bs * in > INT32_MAX)
    return make_status(kInvalid, "swiglu Gate: weights: bad shape");
  L->bs = bs, L->in = in, L->inter = inter;
  WH_HIP(hipStreamCreateWithFlags(&L->stream, hipStreamNonBlocking));
  st = prefixed("Gate", store_from_host(&L->gate, dtype, inter, in, Gate, L->stream));
  if (st.code == 0) st = prefixed("Up", store_from_host(&L->up, dtype, inter, in, Up, L->stream));
  if (st.code == 0) st = prefixed("Down", store_from_host(&L->down, dtype, in, inter, Down, L->stream));
  if (st.code) return st;
  const int64_t nh = (int64_t)bs * inter, nx = (int64_t)bs * in;
  for (float **p : {&L->g_pre, &L->u_pre, &L->h})
    if ((st = L->alloc(p, nh)).code) return st;
  for (float **p : {&L->x, &L->d_pre, &L->d_post})
    if ((st = L->alloc(p, nx)).code) return st;
  if ((st = L->alloc(&L->flag, 4)).code) return st;
  size_t need = 0;
  for (const Store *w : {&L->gate, &L->up, &L->down})
    need = std::max({need, forward_workspace_bytes(w->dev(), bs), backward_workspace_bytes(w->dev(), bs),
                     mse_workspace_bytes(nx)});
  return L->grow_ws(need);
}

// swiglu::forward swiglu.cpp:93-141: x [bs][in] -> h [bs][inter] (the
// layer's pre), post [bs][in], enqueued on s
// Gate writes g to pre and to h; Up's epilogue (kSwiGated) turns each h
// element into fl32(silu(g)) * u, op_swiglu's product, and keeps u in u_pre
// (Linear: post = pre); then Down on h.
// At batch 1 both projections run as one launch (x read once per block, the
// product in its epilogue).
welvet_status forward(Swiglu *L, const float *x, float *h, float *post, hipStream_t s) {
  if (forward_pair_fits(L->gate.dev(), L->up.dev(), L->bs)) {
    WH_HIP(launch_forward_pair(L->gate.dev(), L->up.dev(), x, L->g_pre, L->u_pre, h, s));
  } else {
    WH_HIP(launch_forward(L->gate.dev(), L->bs, x, nullptr, 0, kLinear, L->g_pre, h, L->ws, L->ws_bytes, s));
    WH_HIP(launch_forward(L->up.dev(), L->bs, x, nullptr, 0, kSwiGated, L->u_pre, h, L->ws, L->ws_bytes, s));
  }
  WH_HIP(launch_forward(L->down.dev(), L->bs, h, nullptr, 0, kLinear, L->d_pre, post, L->ws,
                        L->ws_bytes, s));
  return ok();
}
welvet_status forward(Swiglu *L) { return forward(L, L->x, L->h, L->d_post, L->stream); }

bool bad_dims(int32_t batch, int32_t seq, int32_t in, int32_t inter) {
  return batch <= 0 || seq <= 0 || in <= 0 || inter <= 0 || (int64_t)batch * seq > INT32_MAX;
}

}  // namespace

extern "C" {

welvet_status welvet_swiglu_forward_f32(int32_t batch, int32_t seq, int32_t input_dim,
                                        int32_t intermediate_dim, int32_t dtype, int32_t /*backend*/,
                                        const float *Gate, const float *Up, const float *Down,
                                        const float *x, float *pre, float *post) {
  if (bad_dims(batch, seq, input_dim, intermediate_dim) || !Gate || !Up || !Down || !x || !pre ||
      !post)
    return make_status(kInvalid, "swiglu: invalid argument");
  Swiglu L;
  const int bs = batch * seq;
  welvet_status st = make(&L, bs, input_dim, intermediate_dim, dtype, Gate, Up, Down);
  if (st.code) return st;
  const int64_t nh = (int64_t)bs * intermediate_dim, nx = (int64_t)bs * input_dim;
  WH_HIP(hipMemcpyAsync(L.x, x, nx * sizeof(float), hipMemcpyHostToDevice, L.stream));
  if ((st = forward(&L)).code) return st;
  WH_HIP(hipMemcpyAsync(pre, L.h, nh * sizeof(float), hipMemcpyDeviceToHost, L.stream));
  WH_HIP(hipMemcpyAsync(post, L.d_post, nx * sizeof(float), hipMemcpyDeviceToHost, L.stream));
  WH_HIP(hipStreamSynchronize(L.stream));
  return ok();
}

welvet_status welvet_swiglu_normalbp_f32(int32_t batch, int32_t seq, int32_t input_dim,
                                         int32_t intermediate_dim, int32_t dtype, int32_t /*backend*/,
                                         const float *Gate, const float *Up, const float *Down,
                                         const float *x, const float *grad_or_target,
                                         int32_t use_target, double lr, float *pre, float *post,
                                         float *dX, float *dW, float *W_after, double *loss) {
  if (bad_dims(batch, seq, input_dim, intermediate_dim) || !Gate || !Up || !Down || !x ||
      !grad_or_target || !pre || !post || !dX || !dW || !W_after || !loss)
    return make_status(kInvalid, "swiglu nbp: invalid argument");
  if (dtype < 0 || dtype >= kNumDTypes) return make_status(kInvalid, "swiglu nbp: bad dtype %d", dtype);
  Swiglu L;
  const int bs = batch * seq, in = input_dim, inter = intermediate_dim;
  welvet_status st = make(&L, bs, in, inter, dtype, Gate, Up, Down);
  if (st.code) return st;
  const hipStream_t s = L.stream;
  const int64_t nh = (int64_t)bs * inter, nx = (int64_t)bs * in, nw = (int64_t)inter * in;
  WH_HIP(hipMemcpyAsync(L.x, x, nx * sizeof(float), hipMemcpyHostToDevice, s));
  if ((st = forward(&L)).code) return st;

  // output gradient: the caller's, or the MSE gradient against the target
  float *gy = nullptr, *grad_h = nullptr, *d_up = nullptr, *d_gate = nullptr, *dpre = nullptr;
  float *gx_g = nullptr, *gx_u = nullptr, *gx = nullptr, *dw = nullptr, *w_after = nullptr;
  double *d_loss = nullptr;
  for (auto pe : {std::make_pair(&gy, nx), std::make_pair(&gx_g, nx), std::make_pair(&gx_u, nx),
                  std::make_pair(&gx, nx), std::make_pair(&grad_h, nh), std::make_pair(&d_up, nh),
                  std::make_pair(&d_gate, nh), std::make_pair(&dpre, std::max(nh, nx)),
                  std::make_pair(&dw, 3 * nw), std::make_pair(&w_after, 3 * nw)})
    if ((st = L.alloc(pe.first, pe.second)).code) return st;
  if ((st = L.alloc(&d_loss, 1)).code) return st;
  double h_loss = 0.0;
  if (use_target) {
    float *d_t = nullptr;
    if ((st = L.alloc(&d_t, nx)).code) return st;
    WH_HIP(hipMemcpyAsync(d_t, grad_or_target, nx * sizeof(float), hipMemcpyHostToDevice, s));
    WH_HIP(launch_mse(L.d_post, d_t, nx, d_loss, gy, L.ws, L.ws_bytes, s));
    WH_HIP(hipMemcpyAsync(&h_loss, d_loss, sizeof(double), hipMemcpyDeviceToHost, s));
  } else {
    WH_HIP(hipMemcpyAsync(gy, grad_or_target, nx * sizeof(float), hipMemcpyHostToDevice, s));
  }

  // swiglu::backward_f32: Down on h, op_swiglu, Gate and Up on x
  float *dw_g = dw, *dw_u = dw + nw, *dw_d = dw + 2 * nw;
  if ((st = store_prepare_backward(&L.down, bs, s)).code) return st;
  WH_HIP(launch_backward(L.down.dev(), bs, L.h, L.d_pre, gy, kLinear, dpre, grad_h, dw_d, L.flag,
                         L.ws, L.ws_bytes, s));
  WH_HIP(launch_swiglu_bwd(L.g_pre, L.u_pre, grad_h, nh, d_up, d_gate, s));
  if ((st = store_prepare_backward(&L.gate, bs, s)).code) return st;
  WH_HIP(launch_backward(L.gate.dev(), bs, L.x, L.g_pre, d_gate, kLinear, dpre, gx_g, dw_g, L.flag,
                         L.ws, L.ws_bytes, s));
  if ((st = store_prepare_backward(&L.up, bs, s)).code) return st;
  WH_HIP(launch_backward(L.up.dev(), bs, L.x, L.u_pre, d_up, kLinear, dpre, gx_u, dw_u, L.flag,
                         L.ws, L.ws_bytes, s));
  WH_HIP(launch_add(gx_g, gx_u, nx, gx, s));

  if (lr != 0.0) {  // swiglu::apply_grad_sgd: Gate, Up, Down; the first error stops
    if ((st = store_sgd(&L.gate, dw_g, lr, L.flag, s)).code) return st;
    if ((st = store_sgd(&L.up, dw_u, lr, L.flag, s)).code) return st;
    if ((st = store_sgd(&L.down, dw_d, lr, L.flag, s)).code) return st;
  }
  // swiglu::export_weights_f32: concat(Gate, Up, Down)
  if ((st = store_export(L.gate, w_after, s)).code) return st;
  if ((st = store_export(L.up, w_after + nw, s)).code) return st;
  if ((st = store_export(L.down, w_after + 2 * nw, s)).code) return st;
  WH_HIP(hipMemcpyAsync(W_after, w_after, 3 * nw * sizeof(float), hipMemcpyDeviceToHost, s));
  WH_HIP(hipMemcpyAsync(pre, L.h, nh * sizeof(float), hipMemcpyDeviceToHost, s));
  WH_HIP(hipMemcpyAsync(post, L.d_post, nx * sizeof(float), hipMemcpyDeviceToHost, s));
  WH_HIP(hipMemcpyAsync(dX, gx, nx * sizeof(float), hipMemcpyDeviceToHost, s));
  WH_HIP(hipMemcpyAsync(dW, dw, 3 * nw * sizeof(float), hipMemcpyDeviceToHost, s));
  WH_HIP(hipStreamSynchronize(s));
  *loss = h_loss;
  return ok();
}

// ---- resident SwiGLU (extension): the three stores stay mounted ----------

welvet_status welvet_hip_swiglu_mount(int32_t rows, int32_t input_dim, int32_t intermediate_dim,
                                      int32_t dtype, const float *Gate, const float *Up,
                                      const float *Down, welvet_hip_swiglu **out) {
  if (!out) return make_status(kInvalid, "swiglu: invalid argument");
  *out = nullptr;
  if (bad_dims(rows, 1, input_dim, intermediate_dim) || !Gate || !Up || !Down)
    return make_status(kInvalid, "swiglu: invalid argument");
  auto *L = new Swiglu();
  welvet_status st = make(L, rows, input_dim, intermediate_dim, dtype, Gate, Up, Down);
  if (st.code == 0 && hipStreamSynchronize(L->stream) != hipSuccess)
    st = make_status(kInternal, "swiglu: mount failed");
  if (st.code) {
    delete L;
    return st;
  }
  *out = reinterpret_cast<welvet_hip_swiglu *>(L);
  return ok();
}

welvet_status welvet_hip_swiglu_forward_device(welvet_hip_swiglu *s, const float *d_x, float *d_pre,
                                               float *d_post, void *stream) {
  if (!s || !d_x || !d_pre || !d_post) return make_status(kInvalid, "swiglu: invalid argument");
  if (((uintptr_t)d_x | (uintptr_t)d_pre | (uintptr_t)d_post) & 15)
    return make_status(kInvalid, "device pointers must be 16-byte aligned");
  auto *L = reinterpret_cast<Swiglu *>(s);
  return forward(L, d_x, d_pre, d_post, (hipStream_t)stream);
}

void welvet_hip_swiglu_release(welvet_hip_swiglu *s) { delete reinterpret_cast<Swiglu *>(s); }

}  // extern "C"
