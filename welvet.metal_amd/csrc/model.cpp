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
#include <cstdio>
#include <initializer_list>
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

// Values of one payload (a tensor, a weight matrix, a bias) the wire admits.
constexpr uint64_t kMaxValues = uint64_t(1) << 26;

// ---------------------------------------------------------------- outcome
// The status a model call returns.  The first failure recorded wins: later
// checks may record theirs, but the caller sees the one that happened first
// (a malformed child's own message rather than the generic one its parser
// adds on the way out).  Every recorder returns whether the call is still
// good, so a check reads `if (!v.need(cond, "...")) return ...`.
class Verdict {
 public:
  bool ok() const { return st_.code == 0; }
  const welvet_status &status() const { return st_; }
  bool fail(int code, const char *message) {
    if (ok()) {
      st_.code = code;
      std::snprintf(st_.message, sizeof(st_.message), "%s", message);
    }
    return false;
  }
  bool need(bool cond, const char *message) { return cond || fail(kInvalid, message); }
  bool adopt(const welvet_status &s) {
    if (s.code != 0 && ok()) st_ = s;
    return ok();
  }
  bool hip(hipError_t e) {
    if (e != hipSuccess && ok()) st_ = make_status(kInternal, "hip: %s", hipGetErrorString(e));
    return ok();
  }

 private:
  welvet_status st_{};
};

welvet_status unsupported(const char *what) {
  return make_status(kUnsupported, "model: %s is not part of this build (Dense only)", what);
}

// --------------------------------------------------------------- wire in
// A message consumed front to back: little-endian scalars, arrays as an i32
// count and their elements.  get<T>() reports a message that ends early as
// "truncated descriptor" (once, in the verdict) and from then on yields
// zeros, so a parser can read a fixed layout straight through and look at
// the verdict where a value decides something.  pull() is the quiet form for
// sub-grammars that name their own failure.
class WireIn {
 public:
  WireIn(const uint8_t *data, size_t size, Verdict &v) : cur_(data), end_(data + size), v_(v) {}
  size_t remaining() const { return (size_t)(end_ - cur_); }
  bool pull(void *dst, size_t bytes) {
    if (bytes > remaining()) return false;
    if (bytes) std::memcpy(dst, cur_, bytes);
    cur_ += bytes;
    return true;
  }
  template <class T>
  bool pull(T *dst) {
    return pull(dst, sizeof(T));
  }
  bool skip(size_t bytes) {
    if (bytes > remaining()) return false;
    cur_ += bytes;
    return true;
  }
  template <class T>
  T get() {
    T out{};
    if (v_.ok() && !pull(&out)) {
      v_.fail(kInvalid, "truncated descriptor");
      cur_ = end_;
    }
    return out;
  }
  // i32 count, then that many elements
  template <class T>
  std::vector<T> get_array() {
    std::vector<T> out;
    const int32_t n = get<int32_t>();
    if (!v_.ok()) return out;
    if (n < 0 || (size_t)n > remaining() / sizeof(T)) {
      v_.fail(kInvalid, "invalid vector length");
      return out;
    }
    out.resize((size_t)n);
    pull(out.data(), out.size() * sizeof(T));
    return out;
  }
  bool finish() { return v_.need(remaining() == 0, "trailing descriptor bytes"); }

 private:
  const uint8_t *cur_, *end_;
  Verdict &v_;
};

// -------------------------------------------------------------- wire out
class WireOut {
 public:
  template <class T>
  void put(T v) {
    append(&v, sizeof(T));
  }
  template <class T>
  void put_array(const T *v, size_t n) {
    put((int32_t)n);
    append(v, n * sizeof(T));
  }
  // rank, dims, then the values as a counted array
  void put_tensor(std::initializer_list<int32_t> shape, const std::vector<float> &v) {
    put_tensor(std::vector<int32_t>(shape), v);
  }
  void put_tensor(const std::vector<int32_t> &shape, const std::vector<float> &v) {
    put((int32_t)shape.size());
    for (int32_t d : shape) put(d);
    put_array(v.data(), v.size());
  }
  // The bytes in a malloc'd blob the caller frees with welvet_metal_blob_free.
  bool emit(welvet_metal_blob *out, Verdict &v) const {
    if (!v.need(out != nullptr, "null output")) return false;
    out->data = nullptr;
    out->size = 0;
    auto *p = static_cast<uint8_t *>(std::malloc(std::max<size_t>(bytes_.size(), 1)));
    if (p == nullptr) return v.fail(kInternal, "out of host memory");
    std::copy(bytes_.begin(), bytes_.end(), p);
    out->data = p;
    out->size = bytes_.size();
    return true;
  }

 private:
  void append(const void *src, size_t n) {
    const auto *b = static_cast<const uint8_t *>(src);
    bytes_.insert(bytes_.end(), b, b + n);
  }
  std::vector<uint8_t> bytes_;
};

// ---------------------------------------------------------------- tensors
// A tensor argument (model_session.cpp:99-113): rank 1..5, every dimension
// positive, at most 2^26 values, then the f32 values without a count.
struct Tensor {
  std::vector<int32_t> shape;
  std::vector<float> data;
};
bool get_tensor(WireIn &in, Verdict &v, Tensor *t) {
  const int32_t rank = in.get<int32_t>();
  if (!v.ok() || !v.need(rank >= 1 && rank <= 5, "tensor rank must be 1..5")) return false;
  uint64_t count = 1;
  t->shape.assign((size_t)rank, 0);
  for (int32_t &d : t->shape) {
    d = in.get<int32_t>();
    if (!v.ok() || !v.need(d > 0 && count * (uint64_t)d <= kMaxValues, "invalid tensor shape"))
      return false;
    count *= (uint64_t)d;
  }
  if (!v.need(count <= in.remaining() / sizeof(float), "short tensor data")) return false;
  t->data.resize((size_t)count);
  return v.need(in.pull(t->data.data(), t->data.size() * sizeof(float)), "short tensor");
}

// The element count of a child payload (interop::wire::checked_count,
// child_wire.hpp:15-20): 1..2^26 (0 allowed where `may_be_empty`), and no
// more four-byte values than the message still holds.
bool payload_count(WireIn &in, Verdict &v, int64_t n, bool may_be_empty, size_t *out) {
  const bool fits = n >= (may_be_empty ? 0 : 1) && (uint64_t)n <= kMaxValues &&
                    (uint64_t)n <= in.remaining() / 4;
  *out = fits ? (size_t)n : 0;
  return v.need(fits, "invalid model payload size");
}

// cameral::Controls (model_wire.hpp:195-253); only what the Dense-only build
// acts on is kept: whether any mode is set and whether CamSync is enabled
struct Controls {
  bool mixed = false, sync = false;
};
// A counted list of `elem`-byte records, at most 4096 of them; false when
// short or over the limit.
bool skip_counted(WireIn &in, size_t elem, int32_t *count = nullptr) {
  int32_t n = 0;
  if (!in.pull(&n) || n < 0 || n > 4096) return false;
  if (count) *count = n;
  return in.skip((size_t)n * elem);
}
bool read_controls(WireIn &in, Controls *c) {
  int32_t n = 0;
  if (!in.pull(&n) || n < 0 || n > 4096) return false;
  for (int i = 0; i < n; ++i) {
    int32_t m = 0;
    if (!in.pull(&m) || m < 0 || m > 33) return false;
    c->mixed = c->mixed || m != kModeInherit;
  }
  if (!skip_counted(in, sizeof(double)) || !in.skip(3 * sizeof(double))) return false;
  int32_t present = 0;
  if (!in.pull(&present)) return false;
  if (!present) return true;
  int32_t enabled = 0, when = 0;
  double alpha = 0;
  if (!in.pull(&enabled) || !in.pull(&alpha) || !in.pull(&when) || when < 0 || when > 3) return false;
  c->sync = enabled != 0;
  if (!skip_counted(in, sizeof(double))) return false;
  int32_t groups = 0;
  if (!in.pull(&groups) || groups < 0 || groups > 4096) return false;
  for (int g = 0; g < groups; ++g)
    if (!skip_counted(in, sizeof(int32_t))) return false;
  return skip_counted(in, 6 * sizeof(int32_t));
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

// child_wire.hpp:21-55 for the kinds this build holds.  False when the record
// is malformed (the caller names it) or is a kind this build does not hold
// (recorded here as code 2).  A Dense child's initial weights and bias are
// passed over: the store snapshot that follows the children replaces them.
bool read_child(WireIn &in, Verdict &v, Child *c) {
  int32_t kind = 0;
  if (!in.pull(&kind)) return false;
  c->kind = kind;
  if (kind == kKindNone) return true;
  if (kind != kKindDense) return v.adopt(unsupported("a non-Dense child"));
  int32_t dims[4] = {0, 0, 0, 1};  // in, out, act, dtype
  for (int32_t &d : dims)
    if (!in.pull(&d)) return false;
  const int32_t in_w = dims[0], out_w = dims[1], act = dims[2], dtype = dims[3];
  size_t nw = 0, nb = 0;
  if (!payload_count(in, v, (int64_t)out_w * in_w, false, &nw) || !in.skip(nw * sizeof(float)))
    return false;
  uint32_t bias_len = 0;
  if (!in.pull(&bias_len)) return false;
  if (!payload_count(in, v, bias_len, true, &nb) || !in.skip(nb * sizeof(double))) return false;
  if (in_w <= 0 || out_w <= 0 || dtype < 0 || dtype >= kNumDTypes) return false;  // dense::new_layer
  c->in = in_w, c->out = out_w, c->act = act;
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
// pre and post.  alloc() records an out-of-memory failure and returns null.
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
  float *alloc(Verdict &v, size_t elems) {
    void *p = nullptr;
    if (!v.ok()) return nullptr;
    if (!v.hip(hipMalloc(&p, std::max<size_t>(elems, 1) * sizeof(float)))) return nullptr;
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
bool stack_forward(Session &s, Verdict &v, const Tensor &x, StackPass *P) {
  auto ops = stack_ops(s);
  if (!v.need(!ops.empty(), "stack: no operations") ||
      !v.need(x.shape.size() == 2, "stack fwd: dense: input shape need [batch,in]"))
    return false;
  const int batch = x.shape[0];
  P->batch = batch;
  int width = x.shape[1];
  size_t need = 0;
  for (Child *c : ops) {
    if (!v.need(width == c->in, "stack fwd: dense: input width mismatch")) return false;
    need = std::max({need, forward_workspace_bytes(c->W.dev(), batch),
                     backward_workspace_bytes(c->W.dev(), batch)});
    width = c->out;
  }
  need = std::max(need, mse_workspace_bytes((int64_t)batch * width));
  P->ws = P->alloc(v, need / sizeof(float) + 1);
  P->ws_bytes = need;
  P->flag = reinterpret_cast<int *>(P->alloc(v, 4));
  P->x = P->alloc(v, x.data.size());
  if (!v.ok() ||
      !v.hip(hipMemcpyAsync(P->x, x.data.data(), x.data.size() * 4, hipMemcpyHostToDevice, s.stream)))
    return false;
  const float *cur = P->x;
  for (Child *c : ops) {
    float *pre = P->alloc(v, (size_t)batch * c->out), *post = P->alloc(v, (size_t)batch * c->out);
    if (!v.ok() || !v.hip(launch_forward(c->W.dev(), batch, cur, c->W.bias, c->W.bias_len, c->act,
                                         pre, post, P->ws, P->ws_bytes, s.stream)))
      return false;
    P->pre.push_back(pre);
    P->post.push_back(post);
    cur = post;
  }
  return true;
}

// stack::backward_f32 stack.cpp:480-535 after stack_forward: gx [batch, in0]
// and dW (children's, concatenated) on the device
bool stack_backward(Session &s, Verdict &v, StackPass *P, const float *d_gy, const float **gx_out,
                    float **dw_out, size_t *nw_out) {
  auto ops = stack_ops(s);
  const int n = (int)ops.size(), batch = P->batch;
  size_t nw = 0, maxw = 0;
  for (Child *c : ops) {
    nw += (size_t)c->out * c->in;
    maxw = std::max<size_t>(maxw, std::max(c->in, c->out));
  }
  float *dw = P->alloc(v, nw), *dpre = P->alloc(v, (size_t)batch * maxw);
  float *g[2] = {P->alloc(v, (size_t)batch * maxw), P->alloc(v, (size_t)batch * maxw)};
  if (!v.ok()) return false;
  size_t off = nw;
  const float *gcur = d_gy;
  for (int i = n - 1; i >= 0; --i) {
    Child *c = ops[i];
    off -= (size_t)c->out * c->in;
    const float *in = i == 0 ? P->x : P->post[i - 1];
    if (!v.adopt(store_prepare_backward(&c->W, batch, s.stream)) ||
        !v.hip(launch_backward(c->W.dev(), batch, in, P->pre[i], gcur, c->act, dpre, g[i & 1],
                               dw + off, P->flag, P->ws, P->ws_bytes, s.stream)))
      return false;
    gcur = g[i & 1];
  }
  *gx_out = gcur;
  *dw_out = dw;
  *nw_out = nw;
  return true;
}

// stack::apply_grad_sgd stack.cpp:537-556: children in order, the first error stops
bool stack_sgd(Session &s, Verdict &v, const float *d_dw, size_t nw, double lr, int *d_flag) {
  size_t off = 0;
  for (Child *c : stack_ops(s)) {
    const size_t cn = (size_t)c->out * c->in;
    if (!v.need(off + cn <= nw, "stack: dW short") ||
        !v.adopt(store_sgd(&c->W, d_dw + off, lr, d_flag, s.stream)))
      return false;
    off += cn;
  }
  return true;
}

// n values from the device (synchronises the session's stream); empty on failure
template <class T>
std::vector<T> to_host(Session &s, Verdict &v, const T *d, size_t n) {
  std::vector<T> h(n);
  if (!v.ok() || !v.hip(hipMemcpyAsync(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost, s.stream)) ||
      !v.hip(hipStreamSynchronize(s.stream)))
    h.clear();
  return h;
}

// One store as the NWS1 snapshot carries it (model_session.cpp:152-160):
// dtype, rows, cols, scale, counted f32, counted native bytes, counted bias.
bool put_store(WireOut &w, Session &s, Verdict &v, const Store &st) {
  w.put((int32_t)st.dtype);
  w.put((int32_t)st.rows);
  w.put((int32_t)st.cols);
  w.put(st.dtype == kFloat32 ? 1.0f : st.scale);
  const size_t n = (size_t)st.rows * st.cols;
  if (st.dtype == kFloat32) {
    auto f = to_host(s, v, reinterpret_cast<const float *>(st.body), n);
    w.put_array(f.data(), f.size());
    w.put_array((const uint8_t *)nullptr, 0);
  } else {
    size_t len = 0;
    (void)store_native(st, nullptr, 0, &len, s.stream);
    std::vector<uint8_t> raw(len);
    if (!v.adopt(store_native(st, raw.data(), raw.size(), &len, s.stream))) return false;
    w.put_array((const float *)nullptr, 0);
    w.put_array(raw.data(), raw.size());
  }
  std::vector<double> b;
  if (st.bias_len > 0) b = to_host(s, v, st.bias, (size_t)st.bias_len);
  w.put_array(b.data(), b.size());
  return v.ok();
}

// The WMN1 descriptor (model_session.cpp:319-404) parsed into a session with
// no device work; false with the verdict's message otherwise.
bool parse_descriptor(WireIn &in, Verdict &v, Session *s) {
  if (!v.need(in.get<uint32_t>() == 0x314e4d57u, "unsupported model descriptor version")) return false;
  s->root = in.get<int32_t>();
  const int count = in.get<int32_t>();
  if (!v.ok() ||
      !v.need(s->root >= 0 && s->root <= 2 && count > 0 && count <= 4096, "invalid model root/count"))
    return false;
  for (int &d : s->dims) d = in.get<int32_t>();
  if (s->root == kRootParallel) return v.adopt(unsupported("a Parallel root"));
  s->children.resize((size_t)count);
  for (Child &c : s->children)
    if (!read_child(in, v, &c)) return v.fail(kInvalid, "invalid model child");
  if (!v.need(read_controls(in, &s->controls), "invalid root controls")) return false;
  for (Child &c : s->children)
    if (!v.need(read_controls(in, &c.controls), "invalid child controls")) return false;
  int stores = 0;
  for (const Child &c : s->children) stores += c.kind == kKindDense ? 1 : 0;
  if (!v.need(in.get<int32_t>() == stores && v.ok(), "store count mismatch")) return false;
  for (Child &c : s->children) {
    if (c.kind != kKindDense) continue;
    // model_session.cpp:128-151 read_store
    Snapshot &sn = c.snap;
    sn.dtype = in.get<int32_t>();
    sn.rows = in.get<int32_t>();
    sn.cols = in.get<int32_t>();
    sn.scale = in.get<float>();
    if (!v.ok() || !v.need(sn.dtype >= 0 && sn.dtype <= 33 && sn.rows == c.out && sn.cols == c.in &&
                               std::isfinite(sn.scale),
                           "native store metadata mismatch"))
      return false;
    sn.f32 = in.get_array<float>();
    sn.raw = in.get_array<uint8_t>();
    sn.bias = in.get_array<double>();
    const size_t n = (size_t)sn.rows * sn.cols;
    const bool f = sn.dtype == kFloat32;
    if (!v.ok() || !v.need(f ? (sn.f32.size() == n && sn.raw.empty())
                             : (sn.f32.empty() && sn.raw.size() == (size_t)native_bytes(sn.dtype, (int64_t)n)),
                           "native store payload length mismatch"))
      return false;
  }
  if (s->root == kRootGrid) {
    int64_t cells = 1;
    for (int d : s->dims) {
      if (!v.need(d > 0 && d <= 4096 && cells <= 4096 / d, "invalid grid dimensions")) return false;
      cells *= d;
    }
    if (!v.need(cells == count, "grid cell count mismatch")) return false;
    for (Child &c : s->children) {
      c.enabled = in.get<int32_t>() != 0;
      c.remote = in.get<int32_t>();
      c.tz = in.get<int32_t>(), c.ty = in.get<int32_t>(), c.tx = in.get<int32_t>(), c.tl = in.get<int32_t>();
      if (!v.ok() || !v.need(!c.enabled || c.kind != kKindNone, "enabled grid cell has no operation"))
        return false;
      const bool inside = c.tz >= 0 && c.tz < s->dims[0] && c.ty >= 0 && c.ty < s->dims[1] &&
                          c.tx >= 0 && c.tx < s->dims[2] && c.tl >= 0 && c.tl < s->dims[3];
      if (!v.need(c.remote == 0 || inside, "invalid remote link")) return false;
    }
  }
  if (!in.finish()) return false;
  bool sync = s->controls.sync;
  for (const Child &c : s->children) sync = sync || c.controls.sync;
  return !sync || v.adopt(unsupported("CamSync"));
}

// The parsed session's stores into HBM (byte for byte) and, for a Grid root,
// its grid of cells.
bool place_on_device(Session *s, Verdict &v) {
  if (!v.adopt(require_device()) || !v.hip(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking)))
    return false;
  for (Child &c : s->children) {
    if (c.kind != kKindDense) continue;
    Snapshot &sn = c.snap;
    if (!v.adopt(store_from_native(&c.W, sn.dtype, sn.rows, sn.cols, sn.scale, sn.f32.data(),
                                   sn.f32.size(), sn.raw.data(), sn.raw.size(), s->stream)) ||
        !v.adopt(store_set_bias(&c.W, sn.bias.data(), sn.bias.size(), s->stream)))
      return false;
    c.snap = Snapshot();  // the bytes now live in HBM
  }
  if (!v.hip(hipStreamSynchronize(s->stream))) return false;
  if (s->root != kRootGrid) return true;
  if (!v.adopt(welvet_hip_grid_new(s->dims[0], s->dims[1], s->dims[2], s->dims[3], 1, &s->grid)))
    return false;
  int i = 0;
  for (int z = 0; z < s->dims[0]; ++z)
    for (int y = 0; y < s->dims[1]; ++y)
      for (int x = 0; x < s->dims[2]; ++x)
        for (int l = 0; l < s->dims[3]; ++l, ++i) {
          Child &c = s->children[(size_t)i];
          if (c.kind == kKindDense && !v.adopt(grid_bind_store(s->grid, z, y, x, l, c.in, c.out, c.act, &c.W)))
            return false;
          if (!v.adopt(welvet_hip_grid_set_disabled(s->grid, z, y, x, l, !c.enabled))) return false;
          if (c.remote != 0 &&
              !v.adopt(welvet_hip_grid_set_remote_link(s->grid, z, y, x, l, c.tz, c.ty, c.tx, c.tl)))
            return false;
        }
  return true;
}

// The stores of the session in NWS1 order (collect_stores: children in
// order, one store per Dense).
std::vector<const Store *> session_stores(Session &s) {
  std::vector<const Store *> stores;
  if (s.root == kRootStack) {
    for (Child *c : stack_ops(s)) stores.push_back(&c->W);
    return stores;
  }
  int i = 0;
  for (int z = 0; z < s.dims[0]; ++z)
    for (int y = 0; y < s.dims[1]; ++y)
      for (int x = 0; x < s.dims[2]; ++x)
        for (int l = 0; l < s.dims[3]; ++l, ++i)
          if (s.children[(size_t)i].kind == kKindDense) stores.push_back(grid_store(s.grid, z, y, x, l));
  return stores;
}

// runtime::forward::volume_dense of a Grid root on [batch, in]: the output is
// the last enabled cell's post
bool grid_forward(Session &s, Verdict &v, const Tensor &x, WireOut &w) {
  if (!v.need(x.shape.size() == 2, "dense: input shape need [batch,in]") ||
      !v.adopt(grid_set_batch(s.grid, x.shape[0])))
    return false;
  int width = 0;
  for (auto it = s.children.rbegin(); it != s.children.rend() && !width; ++it)
    if (it->kind == kKindDense && it->enabled) width = it->out;
  std::vector<float> y((size_t)x.shape[0] * width);
  if (!v.adopt(welvet_hip_volume_forward(s.grid, x.data.data(), x.shape[1], y.data(), width))) return false;
  w.put_tensor({x.shape[0], width}, y);
  return true;
}

}  // namespace

extern "C" {

int32_t welvet_model_abi_version(void) { return 1; }

welvet_status welvet_model_mount(const uint8_t *descriptor, size_t size, welvet_model_session **out) {
  if (out) *out = nullptr;
  Verdict v;
  if (!v.need(out && descriptor && size >= 28 && size <= (1u << 28), "invalid mount arguments"))
    return v.status();
  auto s = std::make_unique<Session>();
  WireIn in(descriptor, size, v);
  // the whole descriptor is checked before any device work
  if (parse_descriptor(in, v, s.get()) && place_on_device(s.get(), v)) *out = s.release();
  return v.status();
}

welvet_status welvet_model_forward(welvet_model_session *s, const uint8_t *input, size_t size,
                                   welvet_metal_blob *out) {
  Verdict v;
  if (!v.need(s && input && out, "invalid forward arguments")) return v.status();
  std::lock_guard<std::mutex> lock(s->mu);
  WireIn in(input, size, v);
  Tensor x;
  if (!get_tensor(in, v, &x) || !in.finish()) return v.status();
  WireOut w;
  if (s->root == kRootStack) {
    StackPass P;
    if (!stack_forward(*s, v, x, &P)) return v.status();
    const int width = stack_ops(*s).back()->out;
    w.put_tensor({P.batch, width}, to_host(*s, v, P.post.back(), (size_t)P.batch * width));
  } else if (!grid_forward(*s, v, x, w)) {
    return v.status();
  }
  if (v.ok()) w.emit(out, v);
  return v.status();
}

welvet_status welvet_model_forward_pair(welvet_model_session *s, const uint8_t *data, size_t size,
                                        welvet_metal_blob *out) {
  Verdict v;
  if (!v.need(s && data && out, "invalid segment forward arguments")) return v.status();
  std::lock_guard<std::mutex> lock(s->mu);
  if (!v.need(s->root != kRootGrid, "segment forward expects Stack or Parallel")) return v.status();
  WireIn in(data, size, v);
  Tensor x;
  StackPass P;
  if (!get_tensor(in, v, &x) || !in.finish() || !stack_forward(*s, v, x, &P)) return v.status();
  const int width = stack_ops(*s).back()->out;
  const size_t ny = (size_t)P.batch * width;
  WireOut w;
  w.put_tensor({P.batch, width}, to_host(*s, v, P.pre.back(), ny));
  w.put_tensor({P.batch, width}, to_host(*s, v, P.post.back(), ny));
  if (v.ok()) w.emit(out, v);
  return v.status();
}

welvet_status welvet_model_backward(welvet_model_session *s, const uint8_t *data, size_t size,
                                    welvet_metal_blob *out) {
  Verdict v;
  if (!v.need(s && data && out, "invalid segment backward arguments")) return v.status();
  std::lock_guard<std::mutex> lock(s->mu);
  if (!v.need(s->root != kRootGrid, "segment backward expects Stack or Parallel")) return v.status();
  WireIn in(data, size, v);
  Tensor x, gy;
  StackPass P;
  if (!get_tensor(in, v, &x) || !get_tensor(in, v, &gy) || !in.finish() || !stack_forward(*s, v, x, &P))
    return v.status();
  const int width = stack_ops(*s).back()->out;
  if (!v.need(gy.shape == std::vector<int32_t>{P.batch, width} && gy.data.size() == (size_t)P.batch * width,
              "segment output gradient shape mismatch"))
    return v.status();
  float *d_gy = P.alloc(v, gy.data.size());
  const float *gx = nullptr;
  float *dw = nullptr;
  size_t nw = 0;
  if (!v.ok() ||
      !v.hip(hipMemcpyAsync(d_gy, gy.data.data(), gy.data.size() * 4, hipMemcpyHostToDevice, s->stream)) ||
      !stack_backward(*s, v, &P, d_gy, &gx, &dw, &nw))
    return v.status();
  WireOut w;
  w.put_tensor(x.shape, to_host(*s, v, gx, x.data.size()));
  w.put_tensor({1, (int32_t)nw}, to_host(*s, v, (const float *)dw, nw));
  if (v.ok()) w.emit(out, v);
  return v.status();
}

welvet_status welvet_model_apply_sgd(welvet_model_session *s, double lr, const uint8_t *data,
                                     size_t size) {
  Verdict v;
  if (!v.need(s && data && std::isfinite(lr), "invalid segment SGD arguments")) return v.status();
  std::lock_guard<std::mutex> lock(s->mu);
  if (!v.need(s->root != kRootGrid, "segment SGD expects Stack or Parallel")) return v.status();
  WireIn in(data, size, v);
  Tensor dw;
  if (!get_tensor(in, v, &dw) || !in.finish()) return v.status();
  size_t n = 0;
  for (Child *c : stack_ops(*s)) n += (size_t)c->out * c->in;
  if (!v.need(dw.data.size() == n, "segment weight gradient size mismatch")) return v.status();
  StackPass P;
  float *d = P.alloc(v, n);
  P.flag = reinterpret_cast<int *>(P.alloc(v, 4));
  if (v.ok() && v.hip(hipMemcpyAsync(d, dw.data.data(), n * 4, hipMemcpyHostToDevice, s->stream)) &&
      stack_sgd(*s, v, d, n, lr, P.flag))
    v.hip(hipStreamSynchronize(s->stream));
  return v.status();
}

welvet_status welvet_model_train_mse(welvet_model_session *s, int32_t mode, double lr, int32_t ticks,
                                     const uint8_t *data, size_t size, double *loss) {
  Verdict v;
  if (!v.need(s && data && loss && mode >= 0 && mode <= 33 && std::isfinite(lr) && ticks > 0 &&
                  ticks <= 4096,
              "invalid train arguments"))
    return v.status();
  std::lock_guard<std::mutex> lock(s->mu);
  WireIn in(data, size, v);
  Tensor x, t;
  if (!get_tensor(in, v, &x) || !get_tensor(in, v, &t) || !in.finish()) return v.status();
  const int m = mode == kModeInherit ? kModeNormalBP : mode;
  const bool frozen = m == kModeFreeze || m == kModeShadow;
  if (s->root == kRootGrid) {
    // model_session.cpp:236-299: the BP family goes to train_volume_mse
    // (TweenChain as NormalBP); Tween, Mesh and split credit do not
    if (!(m == kModeNormalBP || m == kModeTweenChain || frozen || m == kModeAdversarial ||
          m == kModeMemory)) {
      v.adopt(unsupported("this TrainMode on a Grid (Tween / Mesh / split credit)"));
      return v.status();
    }
    if (v.need(x.shape.size() == 2, "dense: input shape need [batch,in]") &&
        v.adopt(grid_set_batch(s->grid, x.shape[0]))) {
      const int width = (int)(t.data.size() / (size_t)x.shape[0]);
      v.adopt(grid_train_volume_mse(s->grid, x.data.data(), x.shape[1], t.data.data(), width, lr,
                                    frozen, loss));
    }
    return v.status();
  }
  // cameral_train::train_stack_mse cameral_train.cpp:348-403, BP family
  const bool bp = !(m == 2 || m == 3 || (m >= 5 && m <= 29));
  if (!bp) {
    v.adopt(unsupported("this TrainMode on a Stack (Line / Tween / split credit)"));
    return v.status();
  }
  bool mixed = s->controls.mixed;
  for (const Child &c : s->children) mixed = mixed || c.controls.mixed;
  StackPass P;
  if (!stack_forward(*s, v, x, &P)) return v.status();
  const int width = stack_ops(*s).back()->out;
  const size_t ny = (size_t)P.batch * width;
  if (!v.need(t.data.size() == ny, "training: MSE shape")) return v.status();
  float *d_t = P.alloc(v, ny), *d_gy = P.alloc(v, ny);
  double *d_loss = reinterpret_cast<double *>(P.alloc(v, 2));
  if (!v.ok() || !v.hip(hipMemcpyAsync(d_t, t.data.data(), ny * 4, hipMemcpyHostToDevice, s->stream)) ||
      !v.hip(launch_mse(P.post.back(), d_t, (int64_t)ny, d_loss, frozen ? nullptr : d_gy, P.ws,
                        P.ws_bytes, s->stream)))
    return v.status();
  const auto l = to_host(*s, v, (const double *)d_loss, 1);
  if (!v.ok()) return v.status();
  *loss = l[0];
  if (frozen) return v.status();
  if (mixed) {
    v.adopt(unsupported("mixed per-child train modes"));
    return v.status();
  }
  const float *gx = nullptr;
  float *dw = nullptr;
  size_t nw = 0;
  if (stack_backward(*s, v, &P, d_gy, &gx, &dw, &nw) && stack_sgd(*s, v, dw, nw, lr, P.flag))
    v.hip(hipStreamSynchronize(s->stream));
  return v.status();
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
  Verdict v;
  if (!v.need(s && out, "invalid export arguments")) return v.status();
  std::lock_guard<std::mutex> lock(s->mu);
  // NWS1: store count, each store, then the count of Mamba/GDN records (none here)
  WireOut w;
  w.put((uint32_t)0x3153574eu);
  const auto stores = session_stores(*s);
  w.put((int32_t)stores.size());
  for (const Store *st : stores)
    if (!put_store(w, *s, v, *st)) return v.status();
  w.put((int32_t)0);
  w.emit(out, v);
  return v.status();
}

welvet_status welvet_model_sync(welvet_model_session *s, int32_t event) {
  Verdict v;
  if (!v.need(s && event >= 0 && event <= 3, "invalid sync arguments")) return v.status();
  std::lock_guard<std::mutex> lock(s->mu);
  // no CamSync configuration is mounted (mount refuses an enabled one), so
  // no event has stores to blend
  v.need(s->root != kRootGrid, "grid synchronization is configured per cell at mount");
  return v.status();
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
