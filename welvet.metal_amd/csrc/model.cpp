// model.cpp — the versioned model-session ABI (welvet_model_*) for models
// whose operations are all Dense, over this library's resident stores:
//   descriptor WMN1, mount             src/interop/model_session.cpp:319-404
//   forward / forward_pair / backward / apply_sgd / train_mse
//                                      :405-520
//   snapshot NWS1 (export_weights)     :521-550
//   child grammar and Cameral controls include/welvet/interop/child_wire.hpp:21-60,
//                                      include/welvet/interop/model_wire.hpp:195-263
// Roots: Stack (0) of Dense children, and Grid (2) of Dense cells with the
// enabled / remote-link metadata.  A mount takes every store byte for byte
// from the descriptor's store snapshots (dtype, scale, f32 or native bytes,
// bias), exactly as the reference's read_store does, so an NWS1 export of an
// untouched session returns the snapshot it was given.
// Training follows cameral_train::train_stack_mse / train_volume_mse for the
// back-propagation family: Inherit resolves to NormalBP; Freeze and Shadow
// compute the loss only; a Grid skips the update at lr == 0 while a Stack
// still applies it (the reference's order of checks).  What needs the other
// layer families or systems (a Parallel root, non-Dense children, Line/Mesh/
// Tween credit, mixed per-child modes, CamSync, Dense proxies) answers
// code 2 (unsupported) with a message naming it.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <vector>

#include "../../include/welvet_c.h"
#include "runtime.hpp"

using namespace wh;
using namespace wh::rt;

namespace {

enum { kKindNone = 0, kKindDense = 1 };
enum { kRootStack = 0, kRootParallel = 1, kRootGrid = 2 };
enum {
  kModeInherit = 0, kModeNormalBP = 1, kModeTweenChain = 4, kModeFreeze = 30, kModeShadow = 31,
  kModeAdversarial = 32, kModeMemory = 33
};

#define WH_HIP_THROW(expr)                                                             \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess) throw Coded(make_status(kInternal, "hip: %s", hipGetErrorString(e_))); \
  } while (0)

struct Invalid : std::runtime_error {  // code 1 (std::invalid_argument in the reference)
  using std::runtime_error::runtime_error;
};
struct Coded : std::runtime_error {  // a library status
  welvet_status st;
  explicit Coded(const welvet_status &s) : std::runtime_error(s.message), st(s) {}
};
void require(bool ok, const char *why) {
  if (!ok) throw Invalid(why);
}
void good(const welvet_status &st) {
  if (st.code) throw Coded(st);
}
welvet_status unsupported(const char *what) {
  return make_status(kUnsupported, "model: %s is not part of this build (Dense only)", what);
}
template <class F>
welvet_status guarded(F fn) {
  try {
    fn();
    return ok();
  } catch (const Coded &e) {
    return e.st;
  } catch (const Invalid &e) {
    return make_status(kInvalid, "%s", e.what());
  } catch (const std::bad_alloc &) {
    return make_status(kInternal, "out of host memory");
  } catch (const std::exception &e) {
    return make_status(kInternal, "%s", e.what());
  }
}

// Bounded little-endian reader with the reference's limits.
struct Reader {
  const uint8_t *p;
  size_t left;
  bool allow_count(size_t n) const { return n <= left / 4; }
  template <class T>
  bool read(T *out, size_t n) {
    if (n > left / sizeof(T)) return false;
    if (n) std::memcpy(out, p, n * sizeof(T));
    p += n * sizeof(T);
    left -= n * sizeof(T);
    return true;
  }
  template <class T>
  T one() {
    T v{};
    if (!read(&v, 1)) throw Invalid("truncated descriptor");
    return v;
  }
  template <class T>
  std::vector<T> vec() {
    const int32_t n = one<int32_t>();
    if (n < 0 || (size_t)n > left / sizeof(T)) throw Invalid("invalid vector length");
    std::vector<T> v((size_t)n);
    if (!read(v.data(), v.size())) throw Invalid("short vector");
    return v;
  }
  void end() const {
    if (left) throw Invalid("trailing descriptor bytes");
  }
};

struct Writer {
  std::vector<uint8_t> data;
  template <class T>
  void one(T v) {
    const auto *b = reinterpret_cast<const uint8_t *>(&v);
    data.insert(data.end(), b, b + sizeof(T));
  }
  template <class T>
  void vec(const T *v, size_t n) {
    one((int32_t)n);
    const auto *b = reinterpret_cast<const uint8_t *>(v);
    if (n) data.insert(data.end(), b, b + n * sizeof(T));
  }
};

// model_session.cpp:99-113: rank 1..5, positive dims, <= 2^26 values, raw f32
struct Tensor {
  std::vector<int32_t> shape;
  std::vector<float> data;
};
Tensor read_tensor(Reader &r) {
  Tensor t;
  const int32_t rank = r.one<int32_t>();
  require(rank > 0 && rank <= 5, "tensor rank must be 1..5");
  size_t n = 1;
  for (int i = 0; i < rank; ++i) {
    const int32_t d = r.one<int32_t>();
    require(d > 0 && n <= (size_t(1) << 26) / (size_t)d, "invalid tensor shape");
    n *= (size_t)d;
    t.shape.push_back(d);
  }
  require(n <= r.left / 4, "short tensor data");
  t.data.resize(n);
  require(r.read(t.data.data(), n), "short tensor");
  return t;
}
void write_tensor(Writer &w, const std::vector<int32_t> &shape, const float *v, size_t n) {
  w.one((int32_t)shape.size());
  for (int32_t d : shape) w.one(d);
  w.vec(v, n);
}
void to_blob(const Writer &w, welvet_metal_blob *out) {
  require(out != nullptr, "null output");
  out->data = nullptr;
  out->size = 0;
  void *p = std::malloc(std::max<size_t>(w.data.size(), 1));
  if (!p) throw std::bad_alloc();
  if (!w.data.empty()) std::memcpy(p, w.data.data(), w.data.size());
  out->data = static_cast<uint8_t *>(p);
  out->size = w.data.size();
}

// interop::wire::checked_count (child_wire.hpp:15-20)
size_t checked_count(Reader &r, int64_t n, bool empty) {
  if (n < 0 || (!empty && n == 0) || n > (1 << 26) || !r.allow_count((size_t)n))
    throw Invalid("invalid model payload size");
  return (size_t)n;
}

// cameral::Controls (model_wire.hpp:195-253); only what the Dense-only build
// acts on is kept: whether any mode is set and whether CamSync is enabled
struct Controls {
  bool mixed = false, sync = false;
};
bool read_controls(Reader &r, Controls *c) {
  int32_t n = 0;
  if (!r.read(&n, 1) || n < 0 || n > 4096) return false;
  for (int i = 0; i < n; ++i) {
    int32_t m;
    if (!r.read(&m, 1) || m < 0 || m > 33) return false;
    c->mixed = c->mixed || m != kModeInherit;
  }
  std::vector<double> d;
  if (!r.read(&n, 1) || n < 0 || n > 4096) return false;
  d.resize((size_t)n);
  if (!r.read(d.data(), d.size())) return false;
  double three[3];
  if (!r.read(three, 3)) return false;
  int32_t present;
  if (!r.read(&present, 1)) return false;
  if (!present) return true;
  int32_t enabled, when;
  double alpha;
  if (!r.read(&enabled, 1) || !r.read(&alpha, 1) || !r.read(&when, 1) || when < 0 || when > 3)
    return false;
  c->sync = enabled != 0;
  if (!r.read(&n, 1) || n < 0 || n > 4096) return false;
  d.resize((size_t)n);
  if (!r.read(d.data(), d.size())) return false;
  if (!r.read(&n, 1) || n < 0 || n > 4096) return false;
  for (int g = 0; g < n; ++g) {
    int32_t count;
    if (!r.read(&count, 1) || count < 0 || count > 4096) return false;
    std::vector<int32_t> grp((size_t)count);
    if (!r.read(grp.data(), grp.size())) return false;
  }
  if (!r.read(&n, 1) || n < 0 || n > 4096) return false;
  std::vector<int32_t> cross((size_t)n * 6);
  return r.read(cross.data(), cross.size());
}

struct Snapshot {  // a WeightStore as the descriptor carries it
  int32_t dtype = 0, rows = 0, cols = 0;
  float scale = 1.0f;
  std::vector<float> f32;
  std::vector<uint8_t> raw;
  std::vector<double> bias;
};

struct Child {
  int kind = kKindNone;
  int in = 0, out = 0, act = kLinear;
  bool enabled = true;  // Grid cells: the descriptor's enabled flag
  int remote = 0, tz = 0, ty = 0, tx = 0, tl = 0;
  Controls controls;
  Snapshot snap;
  Store W;  // the snapshot's store, resident (moved into the grid for a Grid root)
};

// child_wire.hpp:21-55 for the kinds this build holds
bool read_child(Reader &r, Child *c) {
  int32_t kind = 0;
  if (!r.read(&kind, 1)) return false;
  c->kind = kind;
  if (kind == kKindNone) return true;
  if (kind != kKindDense) throw Coded(unsupported("a non-Dense child"));
  int32_t in = 0, out = 0, act = 0, dtype = 1;
  if (!r.read(&in, 1) || !r.read(&out, 1) || !r.read(&act, 1) || !r.read(&dtype, 1)) return false;
  // the initial weights are replaced by the store snapshot that follows
  const size_t nw = checked_count(r, (int64_t)out * in, false);
  if (nw > r.left / 4) return false;
  r.p += nw * 4;
  r.left -= nw * 4;
  uint32_t bias_len = 0;
  if (!r.read(&bias_len, 1)) return false;
  const size_t nb = checked_count(r, bias_len, true);
  if (nb > r.left / 8) return false;
  r.p += nb * 8;
  r.left -= nb * 8;
  if (in <= 0 || out <= 0 || dtype < 0 || dtype >= kNumDTypes) return false;  // dense::new_layer
  c->in = in, c->out = out, c->act = act;
  return true;
}

}  // namespace

struct welvet_model_session {
  std::mutex mu;
  int root = kRootStack;
  Controls controls;
  std::vector<Child> children;  // Stack: in order; Grid: in hop order (stores moved into the grid)
  welvet_hip_grid *grid = nullptr;
  int dims[4] = {1, 1, 1, 1};
  hipStream_t stream = nullptr;

  ~welvet_model_session() {
    if (stream) (void)hipStreamSynchronize(stream);
    for (Child &c : children) free_store(&c.W);
    if (grid) welvet_hip_grid_release(grid);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

namespace {

using Session = welvet_model_session;

// Device buffers of one Stack pass at `batch` rows: the input, and per child
// pre and post.
struct StackPass {
  int batch = 0;
  std::vector<void *> bufs;
  float *x = nullptr;
  std::vector<float *> pre, post;
  void *ws = nullptr;
  size_t ws_bytes = 0;
  int *flag = nullptr;
  ~StackPass() {
    for (void *p : bufs) (void)hipFree(p);
  }
  float *alloc(size_t elems) {
    void *p = nullptr;
    if (hipMalloc(&p, std::max<size_t>(elems, 1) * sizeof(float)) != hipSuccess)
      throw Coded(make_status(kInternal, "hip: out of device memory"));
    bufs.push_back(p);
    return static_cast<float *>(p);
  }
};

std::vector<Child *> stack_ops(Session &s) {
  std::vector<Child *> ops;
  for (Child &c : s.children)
    if (c.kind == kKindDense) ops.push_back(&c);
  return ops;
}

// stack::forward stack.cpp:446-470 (children in order, each a dense::forward_f32
// on [batch, in]); leaves every child's pre and post on the device
void stack_forward(Session &s, const Tensor &x, StackPass *P) {
  auto ops = stack_ops(s);
  require(!ops.empty(), "stack: no operations");
  if (x.shape.size() != 2)
    throw Invalid("stack fwd: dense: input shape need [batch,in]");
  const int batch = x.shape[0];
  P->batch = batch;
  int width = x.shape[1];
  size_t need = 0;
  for (Child *c : ops) {
    if (width != c->in) throw Invalid("stack fwd: dense: input width mismatch");
    need = std::max({need, forward_workspace_bytes(c->W.dev(), batch),
                     backward_workspace_bytes(c->W.dev(), batch)});
    width = c->out;
  }
  need = std::max(need, mse_workspace_bytes((int64_t)batch * width));
  P->ws = P->alloc(need / sizeof(float) + 1);
  P->ws_bytes = need;
  P->flag = reinterpret_cast<int *>(P->alloc(4));
  P->x = P->alloc(x.data.size());
  WH_HIP_THROW(hipMemcpyAsync(P->x, x.data.data(), x.data.size() * 4, hipMemcpyHostToDevice, s.stream));
  const float *cur = P->x;
  for (Child *c : ops) {
    float *pre = P->alloc((size_t)batch * c->out), *post = P->alloc((size_t)batch * c->out);
    WH_HIP_THROW(launch_forward(c->W.dev(), batch, cur, c->W.bias, c->W.bias_len, c->act, pre, post,
                                P->ws, P->ws_bytes, s.stream));
    P->pre.push_back(pre);
    P->post.push_back(post);
    cur = post;
  }
}

// stack::backward_f32 stack.cpp:480-535 after stack_forward: gx [batch, in0]
// and dW (children's, concatenated) on the device
void stack_backward(Session &s, StackPass *P, const float *d_gy, float **gx_out, float **dw_out,
                    size_t *nw_out) {
  auto ops = stack_ops(s);
  const int n = (int)ops.size(), batch = P->batch;
  size_t nw = 0, maxw = 0;
  for (Child *c : ops) {
    nw += (size_t)c->out * c->in;
    maxw = std::max<size_t>(maxw, std::max(c->in, c->out));
  }
  float *dw = P->alloc(nw), *dpre = P->alloc((size_t)batch * maxw);
  float *g[2] = {P->alloc((size_t)batch * maxw), P->alloc((size_t)batch * maxw)};
  size_t off = nw;
  const float *gcur = d_gy;
  for (int i = n - 1; i >= 0; --i) {
    Child *c = ops[i];
    off -= (size_t)c->out * c->in;
    good(store_prepare_backward(&c->W, batch, s.stream));
    const float *in = i == 0 ? P->x : P->post[i - 1];
    WH_HIP_THROW(launch_backward(c->W.dev(), batch, in, P->pre[i], gcur, c->act, dpre, g[i & 1],
                                 dw + off, P->flag, P->ws, P->ws_bytes, s.stream));
    gcur = g[i & 1];
  }
  *gx_out = const_cast<float *>(gcur);
  *dw_out = dw;
  *nw_out = nw;
}

// stack::apply_grad_sgd stack.cpp:537-556: children in order, the first error stops
void stack_sgd(Session &s, const float *d_dw, size_t nw, double lr, int *d_flag) {
  size_t off = 0;
  for (Child *c : stack_ops(s)) {
    const size_t cn = (size_t)c->out * c->in;
    require(off + cn <= nw, "stack: dW short");
    good(store_sgd(&c->W, d_dw + off, lr, d_flag, s.stream));
    off += cn;
  }
}

template <class T>
std::vector<T> to_host(Session &s, const T *d, size_t n) {
  std::vector<T> h(n);
  WH_HIP_THROW(hipMemcpyAsync(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost, s.stream));
  WH_HIP_THROW(hipStreamSynchronize(s.stream));
  return h;
}

// The grid at this batch (the batch of a volume is fixed per pass).
void grid_batch_for(Session &s, int batch) { good(grid_set_batch(s.grid, batch)); }

void write_store(Writer &w, Session &s, const Store &st) {
  // model_session.cpp:152-160: dtype, rows, cols, scale, f32, native, bias
  w.one((int32_t)st.dtype);
  w.one((int32_t)st.rows);
  w.one((int32_t)st.cols);
  w.one(st.dtype == kFloat32 ? 1.0f : st.scale);
  const size_t n = (size_t)st.rows * st.cols;
  if (st.dtype == kFloat32) {
    auto f = to_host(s, reinterpret_cast<const float *>(st.body), n);
    w.vec(f.data(), n);
    w.vec((const uint8_t *)nullptr, 0);
  } else {
    size_t len = 0;
    (void)store_native(st, nullptr, 0, &len, s.stream);
    std::vector<uint8_t> raw(len);
    good(store_native(st, raw.data(), raw.size(), &len, s.stream));
    w.vec((const float *)nullptr, 0);
    w.vec(raw.data(), raw.size());
  }
  std::vector<double> b;
  if (st.bias_len > 0) b = to_host(s, st.bias, (size_t)st.bias_len);
  w.vec(b.data(), b.size());
}

}  // namespace

extern "C" {

int32_t welvet_model_abi_version(void) { return 1; }

welvet_status welvet_model_mount(const uint8_t *descriptor, size_t size, welvet_model_session **out) {
  if (out) *out = nullptr;
  return guarded([&] {
    require(out && descriptor && size >= 28 && size <= (1u << 28), "invalid mount arguments");
    Reader r{descriptor, size};
    require(r.one<uint32_t>() == 0x314e4d57u, "unsupported model descriptor version");
    auto s = std::make_unique<Session>();
    s->root = r.one<int32_t>();
    const int count = r.one<int32_t>();
    require(s->root >= 0 && s->root <= 2 && count > 0 && count <= 4096, "invalid model root/count");
    for (int &d : s->dims) d = r.one<int32_t>();
    if (s->root == kRootParallel) throw Coded(unsupported("a Parallel root"));
    // the whole descriptor is parsed before any device work
    s->children.resize((size_t)count);
    for (Child &c : s->children) require(read_child(r, &c), "invalid model child");
    require(read_controls(r, &s->controls), "invalid root controls");
    for (Child &c : s->children) require(read_controls(r, &c.controls), "invalid child controls");
    int stores = 0;
    for (const Child &c : s->children) stores += c.kind == kKindDense ? 1 : 0;
    require(r.one<int32_t>() == stores, "store count mismatch");
    for (Child &c : s->children) {
      if (c.kind != kKindDense) continue;
      // model_session.cpp:128-151 read_store
      Snapshot &sn = c.snap;
      sn.dtype = r.one<int32_t>(), sn.rows = r.one<int32_t>(), sn.cols = r.one<int32_t>();
      sn.scale = r.one<float>();
      require(sn.dtype >= 0 && sn.dtype <= 33 && sn.rows == c.out && sn.cols == c.in &&
                  std::isfinite(sn.scale),
              "native store metadata mismatch");
      sn.f32 = r.vec<float>();
      sn.raw = r.vec<uint8_t>();
      sn.bias = r.vec<double>();
      const size_t n = (size_t)sn.rows * sn.cols;
      const bool f = sn.dtype == kFloat32;
      require(f ? (sn.f32.size() == n && sn.raw.empty())
                : (sn.f32.empty() && sn.raw.size() == (size_t)native_bytes(sn.dtype, (int64_t)n)),
              "native store payload length mismatch");
    }
    if (s->root == kRootGrid) {
      int64_t n = 1;
      for (int d : s->dims) {
        require(d > 0 && d <= 4096 && n <= 4096 / d, "invalid grid dimensions");
        n *= d;
      }
      require(n == count, "grid cell count mismatch");
      for (Child &c : s->children) {
        c.enabled = r.one<int32_t>() != 0;
        require(!c.enabled || c.kind != kKindNone, "enabled grid cell has no operation");
        c.remote = r.one<int32_t>();
        c.tz = r.one<int32_t>(), c.ty = r.one<int32_t>(), c.tx = r.one<int32_t>(), c.tl = r.one<int32_t>();
        if (c.remote != 0)
          require(c.tz >= 0 && c.tz < s->dims[0] && c.ty >= 0 && c.ty < s->dims[1] && c.tx >= 0 &&
                      c.tx < s->dims[2] && c.tl >= 0 && c.tl < s->dims[3],
                  "invalid remote link");
      }
    }
    r.end();
    if (s->controls.sync) throw Coded(unsupported("CamSync"));
    for (const Child &c : s->children)
      if (c.controls.sync) throw Coded(unsupported("CamSync"));
    good(require_device());
    WH_HIP_THROW(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking));
    for (Child &c : s->children) {
      if (c.kind != kKindDense) continue;
      Snapshot &sn = c.snap;
      good(store_from_native(&c.W, sn.dtype, sn.rows, sn.cols, sn.scale, sn.f32.data(),
                             sn.f32.size(), sn.raw.data(), sn.raw.size(), s->stream));
      good(store_set_bias(&c.W, sn.bias.data(), sn.bias.size(), s->stream));
      c.snap = Snapshot();  // the bytes now live in HBM
    }
    WH_HIP_THROW(hipStreamSynchronize(s->stream));
    if (s->root == kRootGrid) {
      good(welvet_hip_grid_new(s->dims[0], s->dims[1], s->dims[2], s->dims[3], 1, &s->grid));
      int i = 0;
      for (int z = 0; z < s->dims[0]; ++z)
        for (int y = 0; y < s->dims[1]; ++y)
          for (int x = 0; x < s->dims[2]; ++x)
            for (int l = 0; l < s->dims[3]; ++l, ++i) {
              Child &c = s->children[(size_t)i];
              if (c.kind == kKindDense)
                good(grid_bind_store(s->grid, z, y, x, l, c.in, c.out, c.act, &c.W));
              good(welvet_hip_grid_set_disabled(s->grid, z, y, x, l, !c.enabled));
              if (c.remote != 0)
                good(welvet_hip_grid_set_remote_link(s->grid, z, y, x, l, c.tz, c.ty, c.tx, c.tl));
            }
    }
    *out = s.release();
  });
}

welvet_status welvet_model_forward(welvet_model_session *s, const uint8_t *input, size_t size,
                                   welvet_metal_blob *out) {
  return guarded([&] {
    require(s && input && out, "invalid forward arguments");
    std::lock_guard<std::mutex> lock(s->mu);
    Reader r{input, size};
    Tensor x = read_tensor(r);
    r.end();
    Writer w;
    if (s->root == kRootStack) {
      StackPass P;
      stack_forward(*s, x, &P);
      const int width = stack_ops(*s).back()->out;
      auto y = to_host(*s, P.post.back(), (size_t)P.batch * width);
      write_tensor(w, {P.batch, width}, y.data(), y.size());
    } else {
      // runtime::forward::volume_dense on [batch, in]
      if (x.shape.size() != 2) throw Invalid("dense: input shape need [batch,in]");
      grid_batch_for(*s, x.shape[0]);
      int width = 0;  // the output is the last enabled cell's post
      for (auto it = s->children.rbegin(); it != s->children.rend() && !width; ++it)
        if (it->kind == kKindDense && it->enabled) width = it->out;
      std::vector<float> y((size_t)x.shape[0] * width);
      good(welvet_hip_volume_forward(s->grid, x.data.data(), x.shape[1], y.data(), width));
      write_tensor(w, {x.shape[0], width}, y.data(), y.size());
    }
    to_blob(w, out);
  });
}

welvet_status welvet_model_forward_pair(welvet_model_session *s, const uint8_t *data, size_t size,
                                        welvet_metal_blob *out) {
  return guarded([&] {
    require(s && data && out, "invalid segment forward arguments");
    std::lock_guard<std::mutex> lock(s->mu);
    require(s->root != kRootGrid, "segment forward expects Stack or Parallel");
    Reader r{data, size};
    Tensor x = read_tensor(r);
    r.end();
    StackPass P;
    stack_forward(*s, x, &P);
    const int width = stack_ops(*s).back()->out;
    auto pre = to_host(*s, P.pre.back(), (size_t)P.batch * width);
    auto post = to_host(*s, P.post.back(), (size_t)P.batch * width);
    Writer w;
    write_tensor(w, {P.batch, width}, pre.data(), pre.size());
    write_tensor(w, {P.batch, width}, post.data(), post.size());
    to_blob(w, out);
  });
}

welvet_status welvet_model_backward(welvet_model_session *s, const uint8_t *data, size_t size,
                                    welvet_metal_blob *out) {
  return guarded([&] {
    require(s && data && out, "invalid segment backward arguments");
    std::lock_guard<std::mutex> lock(s->mu);
    require(s->root != kRootGrid, "segment backward expects Stack or Parallel");
    Reader r{data, size};
    Tensor x = read_tensor(r), gy = read_tensor(r);
    r.end();
    StackPass P;
    stack_forward(*s, x, &P);
    const int width = stack_ops(*s).back()->out;
    require(gy.shape == std::vector<int32_t>{P.batch, width} && gy.data.size() == (size_t)P.batch * width,
            "segment output gradient shape mismatch");
    float *d_gy = P.alloc(gy.data.size());
    WH_HIP_THROW(hipMemcpyAsync(d_gy, gy.data.data(), gy.data.size() * 4, hipMemcpyHostToDevice,
                                s->stream));
    float *gx = nullptr, *dw = nullptr;
    size_t nw = 0;
    stack_backward(*s, &P, d_gy, &gx, &dw, &nw);
    auto hgx = to_host(*s, gx, x.data.size());
    auto hdw = to_host(*s, dw, nw);
    Writer w;
    write_tensor(w, x.shape, hgx.data(), hgx.size());
    write_tensor(w, {1, (int32_t)nw}, hdw.data(), hdw.size());
    to_blob(w, out);
  });
}

welvet_status welvet_model_apply_sgd(welvet_model_session *s, double lr, const uint8_t *data,
                                     size_t size) {
  return guarded([&] {
    require(s && data && std::isfinite(lr), "invalid segment SGD arguments");
    std::lock_guard<std::mutex> lock(s->mu);
    require(s->root != kRootGrid, "segment SGD expects Stack or Parallel");
    Reader r{data, size};
    Tensor dw = read_tensor(r);
    r.end();
    size_t n = 0;
    for (Child *c : stack_ops(*s)) n += (size_t)c->out * c->in;
    require(dw.data.size() == n, "segment weight gradient size mismatch");
    StackPass P;
    float *d = P.alloc(n);
    P.flag = reinterpret_cast<int *>(P.alloc(4));
    WH_HIP_THROW(hipMemcpyAsync(d, dw.data.data(), n * 4, hipMemcpyHostToDevice, s->stream));
    stack_sgd(*s, d, n, lr, P.flag);
    WH_HIP_THROW(hipStreamSynchronize(s->stream));
  });
}

welvet_status welvet_model_train_mse(welvet_model_session *s, int32_t mode, double lr, int32_t ticks,
                                     const uint8_t *data, size_t size, double *loss) {
  return guarded([&] {
    require(s && data && loss && mode >= 0 && mode <= 33 && std::isfinite(lr) && ticks > 0 &&
                ticks <= 4096,
            "invalid train arguments");
    std::lock_guard<std::mutex> lock(s->mu);
    Reader r{data, size};
    Tensor x = read_tensor(r), t = read_tensor(r);
    r.end();
    const int m = mode == kModeInherit ? kModeNormalBP : mode;
    const bool frozen = m == kModeFreeze || m == kModeShadow;
    if (s->root == kRootGrid) {
      // model_session.cpp:236-299: the BP family goes to train_volume_mse
      // (TweenChain as NormalBP); Tween, Mesh and split credit do not
      if (!(m == kModeNormalBP || m == kModeTweenChain || frozen || m == kModeAdversarial ||
            m == kModeMemory))
        throw Coded(unsupported("this TrainMode on a Grid (Tween / Mesh / split credit)"));
      if (x.shape.size() != 2) throw Invalid("dense: input shape need [batch,in]");
      grid_batch_for(*s, x.shape[0]);
      const int width = (int)(t.data.size() / (size_t)x.shape[0]);
      good(grid_train_volume_mse(s->grid, x.data.data(), x.shape[1], t.data.data(), width, lr,
                                 frozen, loss));
      return;
    }
    // cameral_train::train_stack_mse cameral_train.cpp:348-403, BP family
    const bool bp = !(m == 2 || m == 3 || (m >= 5 && m <= 29));
    if (!bp) throw Coded(unsupported("this TrainMode on a Stack (Line / Tween / split credit)"));
    bool mixed = s->controls.mixed;
    for (const Child &c : s->children) mixed = mixed || c.controls.mixed;
    StackPass P;
    stack_forward(*s, x, &P);
    const int width = stack_ops(*s).back()->out;
    const size_t ny = (size_t)P.batch * width;
    require(t.data.size() == ny, "training: MSE shape");
    float *d_t = P.alloc(ny), *d_gy = P.alloc(ny);
    double *d_loss = reinterpret_cast<double *>(P.alloc(2));
    WH_HIP_THROW(hipMemcpyAsync(d_t, t.data.data(), ny * 4, hipMemcpyHostToDevice, s->stream));
    WH_HIP_THROW(launch_mse(P.post.back(), d_t, (int64_t)ny, d_loss, frozen ? nullptr : d_gy, P.ws,
                            P.ws_bytes, s->stream));
    *loss = to_host(*s, d_loss, 1)[0];
    if (frozen) return;
    if (mixed) throw Coded(unsupported("mixed per-child train modes"));
    float *gx = nullptr, *dw = nullptr;
    size_t nw = 0;
    stack_backward(*s, &P, d_gy, &gx, &dw, &nw);
    stack_sgd(*s, dw, nw, lr, P.flag);
    WH_HIP_THROW(hipStreamSynchronize(s->stream));
  });
}

welvet_status welvet_model_train_credit(welvet_model_session *s, int32_t, double,
                                        const uint8_t *, size_t) {
  if (!s) return make_status(kInvalid, "invalid credit arguments");
  return unsupported("Cameral credit training");
}

welvet_status welvet_model_dense_proxy(welvet_model_session *s, int32_t, const uint8_t *, size_t,
                                       welvet_metal_blob *out) {
  if (out) *out = welvet_metal_blob{nullptr, 0};
  if (!s) return make_status(kInvalid, "invalid Dense proxy arguments");
  return unsupported("the Dense proxy");
}

welvet_status welvet_model_export_weights(welvet_model_session *s, welvet_metal_blob *out) {
  return guarded([&] {
    require(s && out, "invalid export arguments");
    std::lock_guard<std::mutex> lock(s->mu);
    // NWS1: store count, each store (collect_stores order: children in order,
    // one store per Dense), then the count of Mamba/GDN records (none here)
    Writer w;
    w.one((uint32_t)0x3153574eu);
    std::vector<const Store *> stores;
    if (s->root == kRootStack) {
      for (Child *c : stack_ops(*s)) stores.push_back(&c->W);
    } else {
      int i = 0;
      for (int z = 0; z < s->dims[0]; ++z)
        for (int y = 0; y < s->dims[1]; ++y)
          for (int x = 0; x < s->dims[2]; ++x)
            for (int l = 0; l < s->dims[3]; ++l, ++i)
              if (s->children[(size_t)i].kind == kKindDense) stores.push_back(grid_store(s->grid, z, y, x, l));
    }
    w.one((int32_t)stores.size());
    for (const Store *st : stores) write_store(w, *s, *st);
    w.one((int32_t)0);
    to_blob(w, out);
  });
}

welvet_status welvet_model_sync(welvet_model_session *s, int32_t event) {
  return guarded([&] {
    require(s && event >= 0 && event <= 3, "invalid sync arguments");
    std::lock_guard<std::mutex> lock(s->mu);
    if (s->root == kRootGrid) throw Invalid("grid synchronization is configured per cell at mount");
    // no CamSync configuration is mounted (mount refuses an enabled one), so
    // no event has stores to blend
  });
}

void welvet_model_release(welvet_model_session *s) { delete s; }

void welvet_metal_blob_free(welvet_metal_blob *b) {
  if (b) {
    std::free(b->data);
    b->data = nullptr;
    b->size = 0;
  }
}

}  // extern "C"
