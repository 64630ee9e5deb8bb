// volume.cpp — the volume runtime over Dense cells, device-resident.
//
// Mirrors the reference's grid and volume sequencing:
//   architecture::new_grid / bind_dense / set_remote_link / hop_order
//                                              grid.cpp:31-117
//   runtime::forward::volume_dense             forward.cpp:74-132
//   runtime::backward::volume_dense            backward.cpp:88-127
//   runtime::training::{mse, mse_grad, sgd_dense, step_dense}
//                                              training.cpp:43-184
// with the same hop order (z, y, x, l), skip rules, remote-link inputs,
// tape, reverse backward (the gradient of each step feeds the step before it
// in tape order), SGD in forward order, and error messages.  Unlike the
// reference, nothing leaves the GPU between cells: each cell keeps its
// packed weights, pre and post in HBM, all launches go to one stream, and a
// training step synchronises once at its end.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <mutex>
#include <initializer_list>
#include <vector>

#include "runtime.hpp"

using namespace wh;
using namespace wh::rt;

struct welvet_hip_grid {
  struct Cell {
    bool bound = false, disabled = false, remote = false;
    int tz = 0, ty = 0, tx = 0, tl = 0;
    int in = 0, out = 0, act = kLinear;
    Store W;
    float *pre = nullptr, *post = nullptr, *dW = nullptr;
    // training: this cell's output gradient, then its dpre in place ([batch][out]),
    // kept until the step's batched dW has read it
    float *grad = nullptr;
  };
  std::mutex mu;
  int depth = 1, rows = 1, cols = 1, layers = 1, batch = 1;
  std::vector<Cell> cells;
  hipStream_t stream = nullptr;
  void *ws = nullptr;
  size_t ws_bytes = 0;
  float *gx[2] = {nullptr, nullptr};
  int64_t gx_elems = 0;
  float *dpre = nullptr;
  int64_t dpre_elems = 0;
  float *d_x = nullptr, *d_t = nullptr, *d_gy = nullptr;
  int64_t x_elems = 0, t_elems = 0, gy_elems = 0;
  // A training step's status block, one device allocation: the loss (f64)
  // at byte 0, then the flags from byte 8 — [1] SGD stop code, [2 + i] an
  // Inf / NaN code after tape entry i's E5M2 update, [2 + n + i] (n cells)
  // non-finite dW of tape entry i.  The step clears the flags in its loss
  // kernel and ends with one copy of the block's head into the pinned
  // mirror h_status.
  void *d_status = nullptr;
  void *h_status = nullptr;
  double *d_loss = nullptr;
  int *d_flag = nullptr;
  // tape of the last forward: cell index and the input it read
  std::vector<int> tape;
  std::vector<const float *> tape_in;
};

namespace {

using Grid = welvet_hip_grid;

int cell_index(const Grid &g, int z, int y, int x, int l) {
  return ((z * g.rows + y) * g.cols + x) * g.layers + l;
}

bool in_grid(const Grid &g, int z, int y, int x, int l) {
  return z >= 0 && z < g.depth && y >= 0 && y < g.rows && x >= 0 && x < g.cols && l >= 0 &&
         l < g.layers;
}

// grid.cpp:8-13
welvet_status bad_coord(const char *which, int z, int y, int x, int l) {
  return make_status(kInvalid, "architecture: bad %s coord z=%d y=%d x=%d l=%d", which, z, y, x, l);
}

void free_cell(Grid::Cell *c) {
  free_store(&c->W);
  for (float *p : {c->pre, c->post, c->dW, c->grad})
    if (p) (void)hipFree(p);
  c->pre = c->post = c->dW = c->grad = nullptr;
  c->bound = false;
}

void grid_free(Grid *g) {
  if (!g) return;
  if (g->stream) (void)hipStreamSynchronize(g->stream);
  for (auto &c : g->cells) free_cell(&c);
  for (void *p : {(void *)g->ws, (void *)g->gx[0], (void *)g->gx[1], (void *)g->dpre,
                  (void *)g->d_x, (void *)g->d_t, (void *)g->d_gy, g->d_status})
    if (p) (void)hipFree(p);
  if (g->h_status) (void)hipHostFree(g->h_status);
  if (g->stream) (void)hipStreamDestroy(g->stream);
  delete g;
}

// Grows a device buffer of `elems` floats (contents are not kept).
welvet_status grow(float **p, int64_t *have, int64_t elems) {
  if (elems <= *have) return ok();
  // the old buffer may still be read on a caller's stream: drain the device
  if (*p) WH_HIP(hipDeviceSynchronize());
  if (*p) WH_HIP(hipFree(*p));
  *p = nullptr;
  *have = 0;
  WH_HIP(hipMalloc(p, (size_t)elems * sizeof(float)));
  *have = elems;
  return ok();
}

welvet_status grow_ws(Grid *g, size_t bytes) {
  if (bytes <= g->ws_bytes) return ok();
  WH_HIP(hipDeviceSynchronize());
  if (g->ws) WH_HIP(hipFree(g->ws));
  g->ws = nullptr;
  g->ws_bytes = 0;
  WH_HIP(hipMalloc(&g->ws, bytes));
  g->ws_bytes = bytes;
  return ok();
}

// The forward tape in hop order with the reference's checks, before any
// launch: disabled cells are skipped, an enabled cell without an op, a remote
// link to a cell that has not run, or a width mismatch is an error.
welvet_status plan_forward(Grid *g, const float *d_x, int in_width, int *out_width) {
  g->tape.clear();
  g->tape_in.clear();
  std::vector<char> ran(g->cells.size(), 0);
  const float *cur = d_x;
  int cur_w = in_width;
  for (int z = 0; z < g->depth; ++z)
    for (int y = 0; y < g->rows; ++y)
      for (int x = 0; x < g->cols; ++x)
        for (int l = 0; l < g->layers; ++l) {
          const int idx = cell_index(*g, z, y, x, l);
          Grid::Cell &c = g->cells[idx];
          if (c.disabled) continue;
          if (!c.bound)
            return make_status(kInvalid, "runtime.forward: no op at z=%d y=%d x=%d l=%d", z, y, x, l);
          const float *in = cur;
          int in_w = cur_w;
          if (c.remote) {
            const int t = cell_index(*g, c.tz, c.ty, c.tx, c.tl);
            if (!ran[t])
              return make_status(kInvalid,
                                 "runtime.forward: remote hop has no recorded activation -> "
                                 "z=%d y=%d x=%d l=%d",
                                 c.tz, c.ty, c.tx, c.tl);
            in = g->cells[t].post;
            in_w = g->cells[t].out;
          }
          if (in_w != c.in) return make_status(kInvalid, "dense: input width mismatch");
          g->tape.push_back(idx);
          g->tape_in.push_back(in);
          ran[idx] = 1;
          cur = c.post;
          cur_w = c.out;
        }
  if (g->tape.empty())
    return make_status(kInvalid, "runtime.forward: grid has no enabled cells with ops");
  *out_width = cur_w;
  return ok();
}

// Enqueues the planned forward on `s`.
// final_post (nullable): where the last tape entry writes its activation
// instead of its cell's post buffer (then tape_output does not hold it).
welvet_status run_forward(Grid *g, hipStream_t s, float *final_post = nullptr) {
  for (int idx : g->tape) {  // the kernel plans (and workspace) follow the tuning knobs
    welvet_status st = grow_ws(g, forward_workspace_bytes(g->cells[idx].W.dev(), g->batch));
    if (st.code) return st;
  }
  for (size_t i = 0; i < g->tape.size(); ++i) {
    Grid::Cell &c = g->cells[g->tape[i]];
    float *post = final_post != nullptr && i + 1 == g->tape.size() ? final_post : c.post;
    WH_HIP(launch_forward(c.W.dev(), g->batch, g->tape_in[i], c.W.bias, c.W.bias_len, c.act, c.pre,
                          post, g->ws, g->ws_bytes, s));
  }
  return ok();
}

const float *tape_output(const Grid *g) { return g->cells[g->tape.back()].post; }

// training::step_dense after a forward: MSE loss and gradient, backward
// through the tape in reverse, then SGD per cell in forward order.  Errors a
// kernel finds (non-finite dW) stop every later cell's SGD on the device; the
// host reads the first code once, at the end.  grad_in (host, nullable)
// receives backward::Result::grad_in, the first entry's input gradient.
welvet_status run_step(Grid *g, const float *d_target, int out_width, double lr, double *loss,
                       float *grad_in, hipStream_t s, bool loss_only = false) {
  const int64_t ny = (int64_t)g->batch * out_width;
  const size_t ncells = g->cells.size();
  // the loss, and the flags the step clears in the loss kernel (before any
  // backward launch)
  WH_HIP(launch_mse(tape_output(g), d_target, ny, g->d_loss, g->d_gy, g->ws, g->ws_bytes, s, g->d_flag,
                    (int64_t)(2 + 2 * ncells)));
  // one copy of the status block's head (the loss and `flags` flags) to the
  // pinned mirror, then the step's only synchronisation
  auto read_status = [&](size_t flags) -> hipError_t {
    hipError_t e = hipMemcpyAsync(g->h_status, g->d_status, sizeof(double) + flags * sizeof(int),
                                  hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    return e;
  };
  const double *h_loss = (const double *)g->h_status;
  const int *h_flag = (const int *)((const char *)g->h_status + sizeof(double));
  if (loss_only) {
    WH_HIP(read_status(0));
    if (loss) *loss = *h_loss;
    return ok();
  }
  // the gradient a step passes back must fit the step before it in the tape
  // (a remote hop can break the chain: dense::backward_f32 dense.cpp:171-178)
  for (size_t i = g->tape.size() - 1; i > 0; --i) {
    if (g->cells[g->tape[i]].in != g->cells[g->tape[i - 1]].out) {
      WH_HIP(read_status(0));
      if (loss) *loss = *h_loss;
      return make_status(kInvalid, "dense: bwd shape mismatch");
    }
  }
  // The first entry's input gradient is computed only when the caller asks
  // for it (training::step_dense does not return it).  Each dW launch flags
  // its own non-finite values, which the SGD of that cell reads.
  // Where the dX kernel allows it, a layer's dX epilogue also applies the
  // piecewise activation derivative of the layer below it in the tape, whose
  // backward then takes gy as dpre (one launch less per layer, same bits).
  //
  // With batched dW (knob on), each layer's dX goes to the cell below's grad
  // buffer, the derivative is applied there in place, and the dW launches of
  // layers too small to fill the GPU wait until the walk is done and run a
  // batch at a time: the walk is then only the chain of dX launches.
  const bool batch_dw = tuning(kTuneDwBatch) != 0;
  int *const dw_flag = g->d_flag + 2 + ncells, *const e5_flag = g->d_flag + 2;
  DwBatch dwb{};
  dwb.batch = g->batch;
  const float *gy = g->d_gy;
  bool gy_is_dpre = false;
  for (int i = (int)g->tape.size() - 1; i >= 0; --i) {
    Grid::Cell &c = g->cells[g->tape[i]];
    float *gx = nullptr;
    if (i > 0) gx = batch_dw ? g->cells[g->tape[i - 1]].grad : g->gx[i & 1];
    else if (grad_in) gx = g->gx[0];
    if (gx != nullptr) {
      welvet_status st = store_prepare_backward(&c.W, g->batch, s);
      if (st.code) return st;
    }
    BackwardChain chain;
    chain.gy_is_dpre = gy_is_dpre;
    if (i > 0) {
      const Grid::Cell &below = g->cells[g->tape[i - 1]];
      if (backward_dx_applies_next(c.W.dev(), g->batch, below.act)) {
        chain.dx_next_pre = below.pre;
        chain.dx_next_act = below.act;
      }
    }
    const float *dpre = nullptr;
    chain.defer_dw = batch_dw && dw_defer_pays(c.W.dev());
    chain.dpre_out = &dpre;
    WH_HIP(launch_backward(c.W.dev(), g->batch, g->tape_in[i], c.pre, gy, c.act, batch_dw ? c.grad : g->dpre,
                           gx, c.dW, dw_flag + i, g->ws, g->ws_bytes, s, chain));
    if (chain.defer_dw) {
      dwb.job[dwb.count++] = DwJob{dpre, g->tape_in[i], c.W.rows, c.W.cols, c.dW, dw_flag + i};
      if (dwb.count == kDwBatch) {
        WH_HIP(launch_dw_batch(dwb, s));
        dwb.count = 0;
      }
    }
    gy = gx;
    gy_is_dpre = chain.dx_next_pre != nullptr;
  }
  if (dwb.count > 0) WH_HIP(launch_dw_batch(dwb, s));
  if (grad_in)
    WH_HIP(hipMemcpyAsync(grad_in, g->gx[0],
                          (size_t)g->batch * g->cells[g->tape[0]].in * sizeof(float),
                          hipMemcpyDeviceToHost, s));
  welvet_status late = ok();  // a host-side SGD error found part-way (codes after kernel codes)
  size_t e5_sent = 0;         // tape entries whose SGD was launched
  if (lr == 0.0) {
    late = make_status(kInvalid, "training: LR is 0");
  } else if (!std::isfinite(lr)) {
    late = make_status(kInvalid, "weights: bad SGD arguments");
  } else {
    // Consecutive cells of one dtype share a launch (every dW and its flag
    // exist by now, so a batch skips exactly the cells a launch per cell in
    // this order would); a pending batch goes out before anything that
    // stops the sequence.
    const bool batched = tuning(kTuneSgdBatch) != 0;
    SgdBatch batch{};
    int batch_dt = -1, batch_first = 0;
    auto flush = [&]() -> hipError_t {
      if (batch.count == 0) return hipSuccess;
      const hipError_t e = launch_sgd_batch(batch_dt, batch, lr, g->d_flag + 1, dw_flag, batch_first, s);
      batch.count = 0;
      return e;
    };
    for (size_t j = 0; j < g->tape.size(); ++j) {
      Grid::Cell &c = g->cells[g->tape[j]];
      const int64_t n = c.W.n();
      const int code = c.W.dtype == kFloat32 ? kUnsupported : kInvalid;
      // the gradient check comes first, then the Float32 rate check (store_sgd order)
      if (c.W.dtype == kFloat32 && (std::fabs(lr) > FLT_MAX || std::fabs(lr) < FLT_MIN)) {
        WH_HIP(flush());
        WH_HIP(launch_nonfinite(c.dW, n, g->d_flag + 1, code, s));
        late = make_status(kUnsupported, "SGD: learning rate outside the f32 range");
        break;
      }
      if (batched) {
        if (batch.count == kSgdBatch || (batch.count > 0 && batch_dt != c.W.dtype)) WH_HIP(flush());
        if (batch.count == 0) {
          batch_dt = c.W.dtype;
          batch_first = (int)j;
        }
        batch.store[batch.count++] =
            SgdStore{c.W.body, c.W.kbody, c.dW, n, c.W.scale, c.W.minv, code, e5_flag + j};
      } else {
        WH_HIP(launch_sgd(c.W.dtype, c.W.body, c.W.kbody, n, c.dW, lr, c.W.scale, c.W.minv,
                          g->d_flag + 1, dw_flag + j, code, s, e5_flag + j));
      }
      e5_sent = j + 1;
      c.W.tbody_ok = false;
    }
    WH_HIP(flush());
  }
  WH_HIP(read_status(2 + e5_sent));
  const int stop = h_flag[1];
  const int *e5 = h_flag + 2;
  if (loss) *loss = *h_loss;
  // E5M2 stores whose SGD was launched: finite unless a new code is Inf /
  // NaN; after a stop, a launched store may have been skipped (its codes
  // unchanged, its flag 0), so each is marked non-finite, which is always
  // safe (it only selects the decode that handles Inf / NaN)
  for (size_t j = 0; j < e5_sent; ++j) {
    Grid::Cell &c = g->cells[g->tape[j]];
    if (c.W.dtype == kFP8E5M2) c.W.finite = stop == 0 && e5[j] == 0;
  }
  if (lr == 0.0 || !std::isfinite(lr)) return late;  // no cell was updated
  if (stop == kUnsupported) return make_status(kUnsupported, "SGD: gradient is not a finite f32");
  if (stop == kInvalid) return make_status(kInvalid, "weights: nonfinite gradient");
  return late;
}

// Buffers a training step needs beyond the forward's (allocated once, kept).
welvet_status prepare_step(Grid *g, int out_width) {
  int64_t max_in = 0, max_out = 0;
  for (int idx : g->tape) {
    Grid::Cell &c = g->cells[idx];
    max_in = std::max<int64_t>(max_in, c.in);
    max_out = std::max<int64_t>(max_out, c.out);
    if (!c.dW) WH_HIP(hipMalloc(&c.dW, (size_t)c.W.n() * sizeof(float)));
    if (!c.grad) WH_HIP(hipMalloc(&c.grad, (size_t)g->batch * c.out * sizeof(float)));
    welvet_status st = grow_ws(g, backward_workspace_bytes(c.W.dev(), g->batch));
    if (st.code) return st;
  }
  const int64_t ng = g->batch * max_in;
  if (ng > g->gx_elems) {
    WH_HIP(hipDeviceSynchronize());
    for (float *&p : g->gx) {
      if (p) WH_HIP(hipFree(p));
      p = nullptr;
    }
    g->gx_elems = 0;
    for (float *&p : g->gx) WH_HIP(hipMalloc(&p, (size_t)ng * sizeof(float)));
    g->gx_elems = ng;
  }
  welvet_status st = grow(&g->d_gy, &g->gy_elems, (int64_t)g->batch * out_width);
  if (st.code) return st;
  return grow(&g->dpre, &g->dpre_elems, g->batch * max_out);
}

// bind_dense's work after its checks: the cell's store is *W (taken over)
// when W is given, else W_init encoded into dtype with the bias; then the
// cell's pre/post buffers and the forward workspace.
welvet_status bind_cell(Grid *g, int z, int y, int x, int l, int in, int out, int act, Store *W,
                        int dtype, const float *W_init, const double *bias, size_t bias_len) {
  Grid::Cell &c = g->cells[cell_index(*g, z, y, x, l)];
  WH_HIP(hipStreamSynchronize(g->stream));
  const bool remote = c.remote, disabled = c.disabled;
  const int tz = c.tz, ty = c.ty, tx = c.tx, tl = c.tl;
  free_cell(&c);
  c = Grid::Cell();
  c.remote = remote;
  c.disabled = disabled;
  c.tz = tz, c.ty = ty, c.tx = tx, c.tl = tl;
  c.in = in;
  c.out = out;
  c.act = act;
  welvet_status st = ok();
  if (W != nullptr) {  // take the store over
    c.W = *W;
    *W = Store();
  } else {
    st = store_from_host(&c.W, dtype, out, in, W_init, g->stream);
    if (st.code == 0) st = store_set_bias(&c.W, bias, bias_len, g->stream);
  }
  if (st.code == 0) {
    const size_t yb = (size_t)g->batch * out * sizeof(float);
    hipError_t e = hipMalloc(&c.pre, yb);
    if (e == hipSuccess) e = hipMalloc(&c.post, yb);
    if (e == hipSuccess) e = hipStreamSynchronize(g->stream);
    if (e != hipSuccess) st = make_status(kInternal, "hip: %s", hipGetErrorString(e));
  }
  if (st.code == 0) st = grow_ws(g, forward_workspace_bytes(c.W.dev(), g->batch));
  if (st.code) {
    free_cell(&c);
    return st;
  }
  c.bound = true;
  g->tape.clear();
  return ok();
}

welvet_status cell_at(Grid *g, int z, int y, int x, int l, Grid::Cell **c) {
  if (!in_grid(*g, z, y, x, l)) return bad_coord("cell", z, y, x, l);
  *c = &g->cells[cell_index(*g, z, y, x, l)];
  if (!(*c)->bound) return make_status(kInvalid, "no Dense op at z=%d y=%d x=%d l=%d", z, y, x, l);
  return ok();
}

}  // namespace

extern "C" {

welvet_status welvet_hip_grid_new(int32_t depth, int32_t rows, int32_t cols, int32_t layers_per_cell,
                                  int32_t batch, welvet_hip_grid **out) {
  if (!out) return make_status(kInvalid, "invalid argument");
  *out = nullptr;
  if (batch <= 0) return make_status(kInvalid, "bad resident dims");
  welvet_status st = require_device();
  if (st.code) return st;
  auto *g = new welvet_hip_grid();
  g->depth = depth < 1 ? 1 : depth;  // grid.cpp:32-35
  g->rows = rows < 1 ? 1 : rows;
  g->cols = cols < 1 ? 1 : cols;
  g->layers = layers_per_cell < 1 ? 1 : layers_per_cell;
  g->batch = batch;
  int64_t n = 1;  // at most 2^20 cells, checked factor by factor (no overflow)
  for (const int d : {g->depth, g->rows, g->cols, g->layers}) {
    if (n > (int64_t(1) << 20) / d) {
      delete g;
      return make_status(kInvalid, "architecture: grid too large");
    }
    n *= d;
  }
  g->cells.resize((size_t)n);
  if (hipStreamCreateWithFlags(&g->stream, hipStreamNonBlocking) != hipSuccess) {
    delete g;
    return make_status(kInternal, "hipStreamCreate failed");
  }
  auto fail = [&](hipError_t e) {
    grid_free(g);
    return make_status(kInternal, "hip: %s", hipGetErrorString(e));
  };
  const size_t status_bytes = sizeof(double) + (2 + 2 * (size_t)n) * sizeof(int);
  hipError_t e = hipMalloc(&g->d_status, status_bytes);
  if (e == hipSuccess) e = hipMemset(g->d_status, 0, status_bytes);
  if (e == hipSuccess) e = hipHostMalloc(&g->h_status, status_bytes, hipHostMallocDefault);
  if (e != hipSuccess) return fail(e);
  g->d_loss = (double *)g->d_status;
  g->d_flag = (int *)((char *)g->d_status + sizeof(double));
  st = grow_ws(g, mse_workspace_bytes(0));
  if (st.code) {
    grid_free(g);
    return st;
  }
  *out = g;
  return ok();
}

void welvet_hip_grid_release(welvet_hip_grid *g) { grid_free(g); }

welvet_status welvet_hip_grid_bind_dense(welvet_hip_grid *g, int32_t z, int32_t y, int32_t x,
                                         int32_t l, int32_t in, int32_t out, int32_t act,
                                         int32_t dtype, const float *W_init, const double *bias,
                                         size_t bias_len) {
  if (!g || !W_init) return make_status(kInvalid, "invalid argument");
  std::lock_guard<std::mutex> lk(g->mu);
  if (!in_grid(*g, z, y, x, l)) return bad_coord("bind", z, y, x, l);
  if (dtype < 0 || dtype >= kNumDTypes)
    return make_status(kUnsupported, "dense HIP unsupported dtype %d", dtype);
  if (!dims_ok(out, in)) return make_status(kInvalid, "weights: bad shape");
  return bind_cell(g, z, y, x, l, in, out, act, nullptr, dtype, W_init, bias, bias_len);
}

}  // extern "C"

namespace wh {
namespace rt {

welvet_status grid_bind_store(welvet_hip_grid *g, int z, int y, int x, int l, int in, int out,
                              int act, Store *W) {
  std::lock_guard<std::mutex> lk(g->mu);
  if (!in_grid(*g, z, y, x, l)) return bad_coord("bind", z, y, x, l);
  return bind_cell(g, z, y, x, l, in, out, act, W, 0, nullptr, nullptr, 0);
}

const Store *grid_store(welvet_hip_grid *g, int z, int y, int x, int l) {
  if (!g || !in_grid(*g, z, y, x, l)) return nullptr;
  const Grid::Cell &c = g->cells[cell_index(*g, z, y, x, l)];
  return c.bound ? &c.W : nullptr;
}

welvet_status grid_train_volume_mse(welvet_hip_grid *g, const float *x, int in, const float *target,
                                    int out, double lr, bool frozen, double *loss) {
  if (!g || !loss) return make_status(kInvalid, "cameral volume arguments");
  if (!x || in <= 0) return make_status(kInvalid, "runtime.forward: empty input");
  std::lock_guard<std::mutex> lk(g->mu);
  welvet_status st = grow(&g->d_x, &g->x_elems, (int64_t)g->batch * in);
  if (st.code) return st;
  int out_w = 0;
  st = plan_forward(g, g->d_x, in, &out_w);
  if (st.code) return st;
  if (!target || out != out_w) return make_status(kInvalid, "training: MSE shape");
  st = grow(&g->d_t, &g->t_elems, (int64_t)g->batch * out);
  if (st.code == 0) st = prepare_step(g, out);
  if (st.code) return st;
  WH_HIP(hipMemcpyAsync(g->d_x, x, (size_t)g->batch * in * sizeof(float), hipMemcpyHostToDevice,
                        g->stream));
  WH_HIP(hipMemcpyAsync(g->d_t, target, (size_t)g->batch * out * sizeof(float),
                        hipMemcpyHostToDevice, g->stream));
  st = run_forward(g, g->stream);
  if (st.code) return st;
  return run_step(g, g->d_t, out, lr, loss, nullptr, g->stream, frozen || lr == 0.0);
}

int grid_batch(const welvet_hip_grid *g) { return g->batch; }

welvet_status grid_set_batch(welvet_hip_grid *g, int batch) {
  if (batch <= 0) return make_status(kInvalid, "bad resident dims");
  std::lock_guard<std::mutex> lk(g->mu);
  if (batch == g->batch) return ok();
  WH_HIP(hipStreamSynchronize(g->stream));
  for (Grid::Cell &c : g->cells) {
    if (!c.bound) continue;
    for (float **p : {&c.pre, &c.post}) {
      if (*p) WH_HIP(hipFree(*p));
      *p = nullptr;
      WH_HIP(hipMalloc(p, (size_t)batch * c.out * sizeof(float)));
    }
    // the training gradient is [batch][out] too: the next step allocates it
    // at the new batch (prepare_step)
    if (c.grad) WH_HIP(hipFree(c.grad));
    c.grad = nullptr;
  }
  g->batch = batch;  // the step buffers regrow on demand
  g->tape.clear();
  return ok();
}

}  // namespace rt
}  // namespace wh

extern "C" {

welvet_status welvet_hip_grid_set_remote_link(welvet_hip_grid *g, int32_t z, int32_t y, int32_t x,
                                              int32_t l, int32_t tz, int32_t ty, int32_t tx,
                                              int32_t tl) {
  if (!g) return make_status(kInvalid, "invalid argument");
  std::lock_guard<std::mutex> lk(g->mu);
  if (!in_grid(*g, z, y, x, l)) return bad_coord("source", z, y, x, l);
  if (!in_grid(*g, tz, ty, tx, tl)) return bad_coord("target", tz, ty, tx, tl);
  Grid::Cell &c = g->cells[cell_index(*g, z, y, x, l)];
  c.remote = true;
  c.tz = tz, c.ty = ty, c.tx = tx, c.tl = tl;
  return ok();
}

welvet_status welvet_hip_grid_set_disabled(welvet_hip_grid *g, int32_t z, int32_t y, int32_t x,
                                           int32_t l, int32_t disabled) {
  if (!g) return make_status(kInvalid, "invalid argument");
  std::lock_guard<std::mutex> lk(g->mu);
  if (!in_grid(*g, z, y, x, l)) return bad_coord("cell", z, y, x, l);
  g->cells[cell_index(*g, z, y, x, l)].disabled = disabled != 0;
  return ok();
}

welvet_status welvet_hip_volume_forward(welvet_hip_grid *g, const float *x, int32_t in, float *y,
                                        int32_t out) {
  if (!g || !y) return make_status(kInvalid, "runtime.forward: nil result");
  if (!x || in <= 0) return make_status(kInvalid, "runtime.forward: empty input");
  std::lock_guard<std::mutex> lk(g->mu);
  welvet_status st = grow(&g->d_x, &g->x_elems, (int64_t)g->batch * in);
  if (st.code) return st;
  int out_w = 0;
  st = plan_forward(g, g->d_x, in, &out_w);
  if (st.code) return st;
  if (out != out_w)
    return make_status(kInvalid, "runtime.forward: output width %d, volume gives %d", out, out_w);
  WH_HIP(hipMemcpyAsync(g->d_x, x, (size_t)g->batch * in * sizeof(float), hipMemcpyHostToDevice,
                        g->stream));
  st = run_forward(g, g->stream);
  if (st.code) return st;
  WH_HIP(hipMemcpyAsync(y, tape_output(g), (size_t)g->batch * out * sizeof(float),
                        hipMemcpyDeviceToHost, g->stream));
  WH_HIP(hipStreamSynchronize(g->stream));
  return ok();
}

welvet_status welvet_hip_volume_forward_device(welvet_hip_grid *g, const float *d_x, int32_t in,
                                               float *d_y, int32_t out, void *stream) {
  if (!g || !d_y) return make_status(kInvalid, "runtime.forward: nil result");
  if (!d_x || in <= 0) return make_status(kInvalid, "runtime.forward: empty input");
  std::lock_guard<std::mutex> lk(g->mu);
  int out_w = 0;
  welvet_status st = plan_forward(g, d_x, in, &out_w);
  if (st.code) return st;
  if (out != out_w)
    return make_status(kInvalid, "runtime.forward: output width %d, volume gives %d", out, out_w);
  const hipStream_t s = (hipStream_t)stream;
  // the last layer writes d_y itself (one copy command less per call) unless
  // d_y overlaps that layer's input, which it still reads while writing, or
  // is not 16-byte aligned (the reduction epilogues store float4)
  const Grid::Cell &last = g->cells[g->tape.back()];
  const uintptr_t y0 = (uintptr_t)d_y, y1 = y0 + (size_t)g->batch * out * sizeof(float);
  const uintptr_t i0 = (uintptr_t)g->tape_in.back(), i1 = i0 + (size_t)g->batch * last.in * sizeof(float);
  const bool direct = (y0 % 16 == 0) && (y1 <= i0 || i1 <= y0);
  st = run_forward(g, s, direct ? d_y : nullptr);
  if (st.code) return st;
  if (!direct)
    WH_HIP(hipMemcpyAsync(d_y, tape_output(g), (size_t)g->batch * out * sizeof(float),
                          hipMemcpyDeviceToDevice, s));
  return ok();
}

welvet_status welvet_hip_volume_train_step(welvet_hip_grid *g, const float *x, int32_t in,
                                           const float *target, int32_t out, double lr,
                                           double *loss, float *y) {
  return welvet_hip_volume_train_step_grad(g, x, in, target, out, lr, loss, y, nullptr);
}

welvet_status welvet_hip_volume_train_step_grad(welvet_hip_grid *g, const float *x, int32_t in,
                                                const float *target, int32_t out, double lr,
                                                double *loss, float *y, float *grad_in) {
  if (!g || !loss) return make_status(kInvalid, "training: nil loss");
  if (!x || in <= 0) return make_status(kInvalid, "runtime.forward: empty input");
  std::lock_guard<std::mutex> lk(g->mu);
  welvet_status st = grow(&g->d_x, &g->x_elems, (int64_t)g->batch * in);
  if (st.code) return st;
  int out_w = 0;
  st = plan_forward(g, g->d_x, in, &out_w);
  if (st.code) return st;
  if (!target || out != out_w) return make_status(kInvalid, "training: MSE shape");
  st = grow(&g->d_t, &g->t_elems, (int64_t)g->batch * out);
  if (st.code == 0) st = prepare_step(g, out);
  if (st.code) return st;
  WH_HIP(hipMemcpyAsync(g->d_x, x, (size_t)g->batch * in * sizeof(float), hipMemcpyHostToDevice,
                        g->stream));
  WH_HIP(hipMemcpyAsync(g->d_t, target, (size_t)g->batch * out * sizeof(float),
                        hipMemcpyHostToDevice, g->stream));
  st = run_forward(g, g->stream);
  if (st.code) return st;
  if (y)
    WH_HIP(hipMemcpyAsync(y, tape_output(g), (size_t)g->batch * out * sizeof(float),
                          hipMemcpyDeviceToHost, g->stream));
  return run_step(g, g->d_t, out, lr, loss, grad_in, g->stream);
}

welvet_status welvet_hip_volume_train_step_device(welvet_hip_grid *g, const float *d_x, int32_t in,
                                                  const float *d_target, int32_t out, double lr,
                                                  double *loss, void *stream) {
  if (!g || !loss) return make_status(kInvalid, "training: nil loss");
  if (!d_x || in <= 0) return make_status(kInvalid, "runtime.forward: empty input");
  std::lock_guard<std::mutex> lk(g->mu);
  int out_w = 0;
  welvet_status st = plan_forward(g, d_x, in, &out_w);
  if (st.code) return st;
  if (!d_target || out != out_w) return make_status(kInvalid, "training: MSE shape");
  st = prepare_step(g, out);
  if (st.code) return st;
  const hipStream_t s = (hipStream_t)stream;
  st = run_forward(g, s);
  if (st.code) return st;
  return run_step(g, d_target, out, lr, loss, nullptr, s);
}

welvet_status welvet_hip_grid_export_f32(welvet_hip_grid *g, int32_t z, int32_t y, int32_t x,
                                         int32_t l, float *W_out) {
  if (!W_out) return make_status(kInvalid, "invalid argument");
  if (!g) return make_status(kInvalid, "invalid argument");
  std::lock_guard<std::mutex> lk(g->mu);
  Grid::Cell *c = nullptr;
  welvet_status st = cell_at(g, z, y, x, l, &c);
  if (st.code) return st;
  float *d = nullptr;
  WH_HIP(hipMalloc(&d, (size_t)c->W.n() * sizeof(float)));
  st = store_export(c->W, d, g->stream);
  hipError_t e = hipSuccess;
  if (st.code == 0) e = hipMemcpyAsync(W_out, d, (size_t)c->W.n() * sizeof(float),
                                       hipMemcpyDeviceToHost, g->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(g->stream);
  (void)hipFree(d);
  if (st.code) return st;
  WH_HIP(e);
  return ok();
}

welvet_status welvet_hip_grid_repack(welvet_hip_grid *g, int32_t z, int32_t y, int32_t x, int32_t l,
                                     const float *values, size_t len) {
  if (!g) return make_status(kInvalid, "invalid argument");
  std::lock_guard<std::mutex> lk(g->mu);
  Grid::Cell *c = nullptr;
  welvet_status st = cell_at(g, z, y, x, l, &c);
  if (st.code) return st;
  if (!values || len == 0 || len != (size_t)c->W.n())
    return make_status(kInvalid, "blend: invalid native store replacement");
  return store_repack_host(&c->W, values, g->stream);
}

welvet_status welvet_hip_grid_native(welvet_hip_grid *g, int32_t z, int32_t y, int32_t x, int32_t l,
                                     uint8_t *out, size_t cap, size_t *len, float *scale) {
  if (!g) return make_status(kInvalid, "invalid argument");
  std::lock_guard<std::mutex> lk(g->mu);
  Grid::Cell *c = nullptr;
  welvet_status st = cell_at(g, z, y, x, l, &c);
  if (st.code) return st;
  if (scale) *scale = c->W.scale;
  return store_native(c->W, out, cap, len, g->stream);
}

}  // extern "C"
