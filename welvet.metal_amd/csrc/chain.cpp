// chain.cpp — Sequential and Residual chains of Dense children, behind the
// reference's C ABI entries
//   welvet_sequential_forward_f32 / _normalbp_f32   c_abi.cpp:918-1011
//   welvet_residual_forward_f32 / _normalbp_f32     c_abi.cpp:1013-1090
// with the layer semantics of src/layers/sequential/sequential.cpp and
// src/layers/residual/residual.cpp: `depth` Dense children of dim x dim, all
// with child_act and no bias, packed [depth][dim][dim]; rows = batch * seq.
//   Sequential  post = the last child's post, pre = the last child's pre;
//               backward through the children in reverse, grad_in = the
//               first child's dX                     (sequential.cpp:117-207)
//   Residual    post = fl32(F(x) + x) with F the chain; grad_in =
//               fl32(dX_F + grad_out)                 (residual.cpp:117-240)
//   SGD         children in order, the first failure stops; dW and W_after
//               are the children's, concatenated     (:209-245)
// Every child's packed weights, inputs, pre and post stay in HBM for the
// whole call; the backward reuses the forward's values (the reference
// recomputes them with the same deterministic kernels).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/welvet_c.h"
#include "runtime.hpp"

using namespace wh;
using namespace wh::rt;

namespace {

struct Chain {
  bool residual = false;
  std::vector<Store> child;
  int rows = 0, dim = 0, act = kLinear;
  hipStream_t stream = nullptr;
  void *ws = nullptr;
  size_t ws_bytes = 0;
  std::vector<void *> bufs;
  float *x = nullptr, *y = nullptr;          // input, the layer's post
  std::vector<float *> pre, post;            // per child [rows][dim]
  int *flag = nullptr;

  ~Chain() {
    if (stream) (void)hipStreamSynchronize(stream);
    for (void *p : bufs) (void)hipFree(p);
    if (ws) (void)hipFree(ws);
    for (Store &w : child) free_store(&w);
    if (stream) (void)hipStreamDestroy(stream);
  }
  template <class T>
  welvet_status alloc(T **p, int64_t elems) {
    WH_HIP(hipMalloc((void **)p, (size_t)std::max<int64_t>(elems, 1) * sizeof(T)));
    bufs.push_back(*p);
    return ok();
  }
  const char *name() const { return residual ? "residual F child" : "sequential child"; }
  // the layer's input of child i
  const float *in_of(int i) const { return i == 0 ? x : post[i - 1]; }
};

// sequential/residual::new_configured (dense::new_layer per child) and the
// device buffers of one forward
welvet_status make(Chain *L, bool residual, int rows, int dim, int depth, int act, int dtype,
                   const float *packed) {
  L->residual = residual;
  welvet_status st = require_device();
  if (st.code) return st;
  if (dtype < 0 || dtype >= kNumDTypes)
    return make_status(kUnsupported, "%s 0: dense HIP unsupported dtype %d", L->name(), dtype);
  if (!dims_ok(dim, dim) || (int64_t)rows * dim > INT32_MAX)
    return make_status(kInvalid, "%s 0: weights: bad shape", L->name());
  L->rows = rows, L->dim = dim, L->act = act;
  WH_HIP(hipStreamCreateWithFlags(&L->stream, hipStreamNonBlocking));
  L->child.resize((size_t)depth);
  const int64_t cn = (int64_t)dim * dim, n = (int64_t)rows * dim;
  for (int i = 0; i < depth; ++i) {
    st = store_from_host(&L->child[i], dtype, dim, dim, packed + i * cn, L->stream);
    if (st.code) {
      char msg[sizeof st.message];
      std::snprintf(msg, sizeof msg, "%s %d: %s", L->name(), i, st.message);
      std::memcpy(st.message, msg, sizeof msg);
      return st;
    }
  }
  L->pre.assign((size_t)depth, nullptr);
  L->post.assign((size_t)depth, nullptr);
  for (int i = 0; i < depth; ++i) {
    if ((st = L->alloc(&L->pre[i], n)).code) return st;
    if ((st = L->alloc(&L->post[i], n)).code) return st;
  }
  if ((st = L->alloc(&L->x, n)).code || (st = L->alloc(&L->y, n)).code ||
      (st = L->alloc(&L->flag, 4)).code)
    return st;
  size_t need = mse_workspace_bytes(n);
  for (const Store &w : L->child)
    need = std::max({need, forward_workspace_bytes(w.dev(), rows), backward_workspace_bytes(w.dev(), rows)});
  WH_HIP(hipMalloc(&L->ws, need));
  L->ws_bytes = need;
  return ok();
}

welvet_status forward(Chain *L) {
  const hipStream_t s = L->stream;
  const int depth = (int)L->child.size();
  for (int i = 0; i < depth; ++i)
    WH_HIP(launch_forward(L->child[i].dev(), L->rows, L->in_of(i), nullptr, 0, L->act, L->pre[i],
                          L->post[i], L->ws, L->ws_bytes, s));
  const int64_t n = (int64_t)L->rows * L->dim;
  if (L->residual)
    WH_HIP(launch_add(L->post[depth - 1], L->x, n, L->y, s));
  else
    WH_HIP(hipMemcpyAsync(L->y, L->post[depth - 1], n * sizeof(float), hipMemcpyDeviceToDevice, s));
  return ok();
}

welvet_status run_forward(bool residual, int32_t batch, int32_t seq, int32_t dim, int32_t depth,
                          int32_t act, int32_t dtype, const float *packed, const float *x,
                          float *pre, float *post) {
  Chain L;
  const int rows = batch * seq;
  welvet_status st = make(&L, residual, rows, dim, depth, act, dtype, packed);
  if (st.code) return st;
  const int64_t n = (int64_t)rows * dim;
  WH_HIP(hipMemcpyAsync(L.x, x, n * sizeof(float), hipMemcpyHostToDevice, L.stream));
  if ((st = forward(&L)).code) return st;
  WH_HIP(hipMemcpyAsync(pre, L.pre[depth - 1], n * sizeof(float), hipMemcpyDeviceToHost, L.stream));
  WH_HIP(hipMemcpyAsync(post, L.y, n * sizeof(float), hipMemcpyDeviceToHost, L.stream));
  WH_HIP(hipStreamSynchronize(L.stream));
  return ok();
}

welvet_status run_normalbp(bool residual, int32_t batch, int32_t seq, int32_t dim, int32_t depth,
                           int32_t act, int32_t dtype, const float *packed, const float *x,
                           const float *grad_or_target, int32_t use_target, double lr, float *pre,
                           float *post, float *dX, float *dW, float *W_after, double *loss) {
  Chain L;
  const int rows = batch * seq;
  welvet_status st = make(&L, residual, rows, dim, depth, act, dtype, packed);
  if (st.code) return st;
  const hipStream_t s = L.stream;
  const int64_t n = (int64_t)rows * dim, cn = (int64_t)dim * dim;
  WH_HIP(hipMemcpyAsync(L.x, x, n * sizeof(float), hipMemcpyHostToDevice, s));
  if ((st = forward(&L)).code) return st;
  float *gy = nullptr, *g[2] = {nullptr, nullptr}, *gin = nullptr, *dpre = nullptr, *dw = nullptr;
  float *w_after = nullptr;
  double *d_loss = nullptr;
  for (float **p : {&gy, &g[0], &g[1], &gin, &dpre})
    if ((st = L.alloc(p, n)).code) return st;
  if ((st = L.alloc(&dw, depth * cn)).code || (st = L.alloc(&w_after, depth * cn)).code ||
      (st = L.alloc(&d_loss, 1)).code)
    return st;
  double h_loss = 0.0;
  if (use_target) {
    float *d_t = nullptr;
    if ((st = L.alloc(&d_t, n)).code) return st;
    WH_HIP(hipMemcpyAsync(d_t, grad_or_target, n * sizeof(float), hipMemcpyHostToDevice, s));
    WH_HIP(launch_mse(L.y, d_t, n, d_loss, gy, L.ws, L.ws_bytes, s));
    WH_HIP(hipMemcpyAsync(&h_loss, d_loss, sizeof(double), hipMemcpyDeviceToHost, s));
  } else {
    WH_HIP(hipMemcpyAsync(gy, grad_or_target, n * sizeof(float), hipMemcpyHostToDevice, s));
  }
  // the children in reverse; each one's dX is the gradient of the one before
  const float *gcur = gy;
  for (int i = depth - 1; i >= 0; --i) {
    float *gx = g[i & 1];
    if ((st = store_prepare_backward(&L.child[i], rows, s)).code) return st;
    WH_HIP(launch_backward(L.child[i].dev(), rows, L.in_of(i), L.pre[i], gcur, act, dpre, gx,
                           dw + i * cn, L.flag, L.ws, L.ws_bytes, s));
    gcur = gx;
  }
  if (residual)
    WH_HIP(launch_add(gcur, gy, n, gin, s));
  else
    WH_HIP(hipMemcpyAsync(gin, gcur, n * sizeof(float), hipMemcpyDeviceToDevice, s));
  if (lr != 0.0)
    for (int i = 0; i < depth; ++i)
      if ((st = store_sgd(&L.child[i], dw + i * cn, lr, L.flag, s)).code) return st;
  for (int i = 0; i < depth; ++i)
    if ((st = store_export(L.child[i], w_after + i * cn, s)).code) return st;
  WH_HIP(hipMemcpyAsync(W_after, w_after, depth * cn * sizeof(float), hipMemcpyDeviceToHost, s));
  WH_HIP(hipMemcpyAsync(pre, L.pre[depth - 1], n * sizeof(float), hipMemcpyDeviceToHost, s));
  WH_HIP(hipMemcpyAsync(post, L.y, n * sizeof(float), hipMemcpyDeviceToHost, s));
  WH_HIP(hipMemcpyAsync(dX, gin, n * sizeof(float), hipMemcpyDeviceToHost, s));
  WH_HIP(hipMemcpyAsync(dW, dw, depth * cn * sizeof(float), hipMemcpyDeviceToHost, s));
  WH_HIP(hipStreamSynchronize(s));
  *loss = h_loss;
  return ok();
}

bool bad_dims(int32_t batch, int32_t seq, int32_t dim, int32_t depth) {
  return batch <= 0 || seq <= 0 || dim <= 0 || depth <= 0 || (int64_t)batch * seq > INT32_MAX ||
         (int64_t)dim * dim > INT32_MAX || (int64_t)depth * dim * dim > INT32_MAX;
}

}  // namespace

extern "C" {

welvet_status welvet_sequential_forward_f32(int32_t batch, int32_t seq, int32_t dim, int32_t depth,
                                            int32_t child_act, int32_t dtype, int32_t /*backend*/,
                                            const float *packed, const float *x, float *pre,
                                            float *post) {
  if (bad_dims(batch, seq, dim, depth) || !packed || !x || !pre || !post)
    return make_status(kInvalid, "sequential: invalid argument");
  return run_forward(false, batch, seq, dim, depth, child_act, dtype, packed, x, pre, post);
}

welvet_status welvet_sequential_normalbp_f32(int32_t batch, int32_t seq, int32_t dim, int32_t depth,
                                             int32_t child_act, int32_t dtype, int32_t /*backend*/,
                                             const float *packed, const float *x,
                                             const float *grad_or_target, int32_t use_target,
                                             double lr, float *pre, float *post, float *dX,
                                             float *dW, float *W_after, double *loss) {
  if (bad_dims(batch, seq, dim, depth) || !packed || !x || !grad_or_target || !pre || !post || !dX ||
      !dW || !W_after || !loss)
    return make_status(kInvalid, "sequential nbp: invalid argument");
  return run_normalbp(false, batch, seq, dim, depth, child_act, dtype, packed, x, grad_or_target,
                      use_target, lr, pre, post, dX, dW, W_after, loss);
}

welvet_status welvet_residual_forward_f32(int32_t batch, int32_t seq, int32_t dim, int32_t depth,
                                          int32_t child_act, int32_t dtype, int32_t /*backend*/,
                                          const float *packed, const float *x, float *pre,
                                          float *post) {
  if (bad_dims(batch, seq, dim, depth) || !packed || !x || !pre || !post)
    return make_status(kInvalid, "residual: invalid argument");
  return run_forward(true, batch, seq, dim, depth, child_act, dtype, packed, x, pre, post);
}

welvet_status welvet_residual_normalbp_f32(int32_t batch, int32_t seq, int32_t dim, int32_t depth,
                                           int32_t child_act, int32_t dtype, int32_t /*backend*/,
                                           const float *packed, const float *x,
                                           const float *grad_or_target, int32_t use_target,
                                           double lr, float *pre, float *post, float *dX, float *dW,
                                           float *W_after, double *loss) {
  if (bad_dims(batch, seq, dim, depth) || !packed || !x || !grad_or_target || !pre || !post || !dX ||
      !dW || !W_after || !loss)
    return make_status(kInvalid, "residual nbp: invalid argument");
  return run_normalbp(true, batch, seq, dim, depth, child_act, dtype, packed, x, grad_or_target,
                      use_target, lr, pre, post, dX, dW, W_after, loss);
}

}  // extern "C"
