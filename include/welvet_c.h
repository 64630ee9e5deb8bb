#ifndef WELVET_C_H
#define WELVET_C_H
/*
 * welvet_c.h — C ABI of the MI355X-native (HIP, gfx950) quantized-storage
 * Dense path.  A drop-in for the Dense subset of the reference's
 * include/welvet_c.h: same symbols, argument order, meaning, ownership and
 * status codes.  Every input is copied during the call, no caller pointer is
 * retained, and the caller allocates every output.
 *
 * Entry points prefixed welvet_hip_ are extensions with no counterpart in the
 * reference: device-resident execution and inspection of the packed store,
 * for callers that keep activations in HBM (benchmarks, device training loops).
 */
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WELVET_API __attribute__((visibility("default")))

/* reference include/welvet_c.h:22-25; codes 0 ok, 1 invalid, 2 unsupported,
 * 3 gap, 4 internal (include/welvet/status.hpp:8-14) */
typedef struct welvet_status {
  int32_t code;
  char message[256];
} welvet_status;

/* reference include/welvet_c.h:28 — version string of the Dense ABI ("0.71") */
WELVET_API const char *welvet_version(void);
/* reference include/welvet_c.h:29 — here "hip:<gcnArch>:<device>:cu=<n>:..." */
WELVET_API const char *welvet_runtime_identity(void);
/* reference include/welvet_c.h:31 — device init + kernel probe; the name keeps
 * the reference's "metal" spelling so existing bindings resolve */
WELVET_API welvet_status welvet_metal_init(void);
/* reference include/welvet_c.h:32 — 1 when a gfx950 device is usable */
WELVET_API int32_t welvet_metal_available(void);

/* reference include/welvet_c.h:35-56 — versioned model sessions (ABI 1):
 * descriptor WMN1 in, snapshot NWS1 out (reference docs/GO_INTEGRATION.md:
 * 139-157).  This build mounts Stack and Grid roots whose operations are all
 * Dense, with every store taken byte for byte from the descriptor's
 * snapshots; other roots, layer kinds, credit families and CamSync answer
 * code 2.  Inputs are copied during the call; blobs are freed with
 * welvet_metal_blob_free. */
typedef struct welvet_model_session welvet_model_session;
typedef struct welvet_metal_blob {
  uint8_t *data;
  size_t size;
} welvet_metal_blob;
WELVET_API int32_t welvet_model_abi_version(void);
WELVET_API welvet_status welvet_model_mount(const uint8_t *descriptor, size_t size,
                                            welvet_model_session **out);
WELVET_API welvet_status welvet_model_forward(welvet_model_session *s, const uint8_t *input,
                                              size_t size, welvet_metal_blob *out);
WELVET_API welvet_status welvet_model_train_credit(welvet_model_session *s, int32_t mode,
                                                   double lr, const uint8_t *data, size_t size);
WELVET_API welvet_status welvet_model_dense_proxy(welvet_model_session *s, int32_t kind,
                                                  const uint8_t *data, size_t size,
                                                  welvet_metal_blob *out);
WELVET_API welvet_status welvet_model_forward_pair(welvet_model_session *s, const uint8_t *data,
                                                   size_t size, welvet_metal_blob *out);
WELVET_API welvet_status welvet_model_backward(welvet_model_session *s, const uint8_t *data,
                                               size_t size, welvet_metal_blob *out);
WELVET_API welvet_status welvet_model_apply_sgd(welvet_model_session *s, double lr,
                                                const uint8_t *data, size_t size);
WELVET_API welvet_status welvet_model_train_mse(welvet_model_session *s, int32_t mode, double lr,
                                                int32_t ticks, const uint8_t *data, size_t size,
                                                double *loss);
WELVET_API welvet_status welvet_model_export_weights(welvet_model_session *s,
                                                     welvet_metal_blob *out);
WELVET_API welvet_status welvet_model_sync(welvet_model_session *s, int32_t event);
WELVET_API void welvet_model_release(welvet_model_session *s);
WELVET_API void welvet_metal_blob_free(welvet_metal_blob *b);

/* reference include/welvet_c.h:59-62 — one-shot mount + execute + release.
 * W_init [out*in] row-major f32, encoded into `dtype` (0..33); bias [bias_len]
 * f64 (nullable) added for o < bias_len; x [batch*in]; pre/post [batch*out].
 * `backend` is ignored, as in the reference (c_abi.cpp:131). */
WELVET_API welvet_status welvet_dense_forward_f32(int32_t batch, int32_t in, int32_t out,
                                                  int32_t act, int32_t dtype, int32_t backend,
                                                  const float *W_init, const double *bias,
                                                  size_t bias_len, const float *x, float *pre,
                                                  float *post);

/* reference include/welvet_c.h:64-73 — NormalBP leaf: forward, then the MSE
 * gradient against grad_or_target (use_target = 1) or grad_or_target as the
 * output gradient (use_target = 0), backward, SGD in the native dtype when
 * lr != 0, and W_after = decode of the stored weights.  Outputs: pre/post
 * [batch*out], dX [batch*in], dW [out*in], W_after [out*in], *loss (0 when
 * use_target = 0).  All pointers except bias must be non-null. */
WELVET_API welvet_status welvet_dense_normalbp_f32(
    int32_t batch, int32_t in, int32_t out, int32_t act, int32_t dtype, int32_t backend,
    const float *W_init, const double *bias, size_t bias_len, const float *x,
    const float *grad_or_target, int32_t use_target, double lr, float *pre, float *post,
    float *dX, float *dW, float *W_after, double *loss);

/* reference include/welvet_c.h:105-109 — SwiGLU forward (the WVS1 wire):
 * Gate and Up [inter*in], Down [in*inter] row-major f32, each encoded into
 * `dtype` as a Linear Dense layer without bias; x [batch*seq*in] ->
 * pre = h = silu(Gate x) * (Up x) [batch*seq*inter], post = Down h
 * [batch*seq*in] (src/layers/swiglu/swiglu.cpp:93-141). */
WELVET_API welvet_status welvet_swiglu_forward_f32(int32_t batch, int32_t seq, int32_t input_dim,
                                                   int32_t intermediate_dim, int32_t dtype,
                                                   int32_t backend, const float *Gate,
                                                   const float *Up, const float *Down,
                                                   const float *x, float *pre, float *post);
/* reference include/welvet_c.h:111-119 — SwiGLU NormalBP leaf: forward, the
 * MSE gradient (use_target = 1) or grad_or_target as the output gradient,
 * backward, SGD of Gate, Up, Down when lr != 0.  Outputs pre [batch*seq*inter],
 * post and dX [batch*seq*in], dW and W_after = concat(Gate, Up, Down). */
WELVET_API welvet_status welvet_swiglu_normalbp_f32(
    int32_t batch, int32_t seq, int32_t input_dim, int32_t intermediate_dim, int32_t dtype,
    int32_t backend, const float *Gate, const float *Up, const float *Down, const float *x,
    const float *grad_or_target, int32_t use_target, double lr, float *pre, float *post, float *dX,
    float *dW, float *W_after, double *loss);

/* reference include/welvet_c.h:184-189 — Sequential Dense chain (the WSQ1
 * wire): packed [depth][dim][dim] f32, each child a Dense dim -> dim layer
 * with child_act and no bias, encoded into `dtype`; x [batch*seq*dim] ->
 * pre = the last child's pre, post = the last child's post. */
WELVET_API welvet_status welvet_sequential_forward_f32(int32_t batch, int32_t seq, int32_t dim,
                                                       int32_t depth, int32_t child_act,
                                                       int32_t dtype, int32_t backend,
                                                       const float *packed, const float *x,
                                                       float *pre, float *post);
/* reference include/welvet_c.h:191-197 — Sequential NormalBP leaf;
 * dW and W_after [depth][dim][dim]; lr == 0 skips the SGD. */
WELVET_API welvet_status welvet_sequential_normalbp_f32(
    int32_t batch, int32_t seq, int32_t dim, int32_t depth, int32_t child_act, int32_t dtype,
    int32_t backend, const float *packed, const float *x, const float *grad_or_target,
    int32_t use_target, double lr, float *pre, float *post, float *dX, float *dW, float *W_after,
    double *loss);
/* reference include/welvet_c.h:199-203 — Residual y = F(x) + x (the WRE1
 * wire), F the Dense chain as in welvet_sequential_forward_f32; pre = the
 * last F child's pre, post = fl32(F(x) + x). */
WELVET_API welvet_status welvet_residual_forward_f32(int32_t batch, int32_t seq, int32_t dim,
                                                     int32_t depth, int32_t child_act,
                                                     int32_t dtype, int32_t backend,
                                                     const float *packed, const float *x,
                                                     float *pre, float *post);
/* reference include/welvet_c.h:205-211 — Residual NormalBP leaf; dX includes
 * the skip path; dW and W_after are the F children's. */
WELVET_API welvet_status welvet_residual_normalbp_f32(
    int32_t batch, int32_t seq, int32_t dim, int32_t depth, int32_t child_act, int32_t dtype,
    int32_t backend, const float *packed, const float *x, const float *grad_or_target,
    int32_t use_target, double lr, float *pre, float *post, float *dX, float *dW, float *W_after,
    double *loss);

/* reference include/welvet_c.h:75-85 — resident session: the packed weights
 * and the [batch] activation buffers stay in HBM; batch is fixed at mount. */
typedef struct welvet_dense_session welvet_dense_session;
WELVET_API welvet_status welvet_dense_mount(int32_t batch, int32_t in, int32_t out, int32_t act,
                                            int32_t dtype, const float *W_init,
                                            const double *bias, size_t bias_len,
                                            welvet_dense_session **sess);
WELVET_API welvet_status welvet_dense_execute(welvet_dense_session *s, const float *x, float *pre,
                                              float *post);
WELVET_API void welvet_dense_release(welvet_dense_session *s);

/* ---- extensions (no reference counterpart) ------------------------------ */

/* welvet_dense_mount with W_init already in device memory (16-byte aligned). */
WELVET_API welvet_status welvet_hip_dense_mount_device(int32_t batch, int32_t in, int32_t out,
                                                       int32_t act, int32_t dtype,
                                                       const float *d_W_init, const double *bias,
                                                       size_t bias_len,
                                                       welvet_dense_session **sess);

/* welvet_dense_mount from a store snapshot instead of f32 values: the native
 * bytes in the reference's WeightStore::native layout (4-byte f32 min header
 * for the unsigned types; the f32 bytes for Float32) and the store's scale,
 * taken byte for byte as the model-session import does
 * (reference src/interop/model_session.cpp:128-151 read_store).  Code 1 when
 * native_len is not the layout's size for [out*in] or the scale is not finite. */
WELVET_API welvet_status welvet_hip_dense_mount_native(int32_t batch, int32_t in, int32_t out,
                                                       int32_t act, int32_t dtype,
                                                       const uint8_t *native, size_t native_len,
                                                       float scale, const double *bias,
                                                       size_t bias_len,
                                                       welvet_dense_session **sess);

/* Forward on device pointers (16-byte aligned) enqueued on `stream`
 * (a hipStream_t; NULL = the HIP null stream); returns once enqueued.
 * The launch uses the session's own workspace (stream-K partial tiles), so
 * calls on one session must not overlap: forwards on one stream are ordered
 * by that stream; before a call on the same session from another stream,
 * or a host-buffer call (execute, backward, sgd, export, native: these run
 * on the session's internal stream and return when done), synchronise
 * `stream`.  Sessions are independent of each other. */
WELVET_API welvet_status welvet_hip_dense_forward_device(welvet_dense_session *s, const float *d_x,
                                                         float *d_pre, float *d_post,
                                                         void *stream);
/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): welvet_hip_dense_forward_device for `batch` rows
 * (any batch >= 1, independent of the mount's) that allocates nothing.  Its
 * stream-K partial tiles live in one library-wide 64 MiB device array per
 * GPU, held until the process ends, instead of the session's workspace; code
 * 1 when the batch's plan needs more than 64 MiB (4096 x 11008 weights:
 * batch 64 needs 60 MB).  Every call on one GPU shares that array, whatever
 * the session or stream: calls that overlap on one GPU race, so order them
 * on one stream or synchronise between them.  Enqueued on `stream`; returns
 * once enqueued. */
WELVET_API welvet_status welvet_hip_dense_forward_noalloc(welvet_dense_session *s, int32_t batch,
                                                          const float *d_x, float *d_pre,
                                                          float *d_post, void *stream);
/* The store in the reference's byte layout (WeightStore::native, with the
 * 4-byte min header of the unsigned types; f32 bytes for Float32).  *len gets
 * the payload size; fails with code 1 when cap is too small. */
WELVET_API welvet_status welvet_hip_dense_native(welvet_dense_session *s, uint8_t *out,
                                                 size_t cap, size_t *len, float *scale);
/* WeightStore::set_from_f32_gpu (reference src/weights/native_codec.cpp:
 * 872-907, kernel shaders/ops_storage.metal:971-1144 op_native_repack): the
 * resident store replaced by `values` [out*in] re-encoded in its dtype with
 * fresh statistics (a new scale, and min for the unsigned types); Float32
 * takes the values as they are.  Code 1 "blend: invalid native store
 * replacement" when len != out*in (or 0).  The reference calls it for
 * CamSync's blended weights (src/systems/cam_sync.cpp:148). */
WELVET_API welvet_status welvet_hip_dense_repack(welvet_dense_session *s, const float *values,
                                                 size_t len);
/* WeightStore::export_f32 of the resident store into W_out [out*in]. */
WELVET_API welvet_status welvet_hip_dense_export_f32(welvet_dense_session *s, float *W_out);
/* Backward against the resident weights (host pointers): x [batch*in], pre and
 * gy [batch*out] -> dX [batch*in], dW [out*in] (resident_backward semantics). */
WELVET_API welvet_status welvet_hip_dense_backward(welvet_dense_session *s, const float *x,
                                                   const float *pre, const float *gy, float *dX,
                                                   float *dW);
/* WeightStore::apply_sgd with a host gradient dW [out*in] (f32, widened). */
WELVET_API welvet_status welvet_hip_dense_sgd(welvet_dense_session *s, const float *dW,
                                              double lr);
/* MSE loss and/or gradient of n values (host pointers; either output may be NULL). */
WELVET_API welvet_status welvet_hip_mse_f32(const float *pred, const float *target, size_t n,
                                            double *loss, float *grad);
/* ---- volume runtime over Dense cells (extensions) ------------------------
 * The reference runs volumes through its C++ API (architecture::Grid,
 * runtime::forward/backward::volume_dense, runtime::training::step_dense);
 * these entry points expose the same sequencing with its argument meaning
 * and error messages.  Every cell's packed weights and activations stay in
 * HBM; batch is fixed for the whole grid at creation. */
typedef struct welvet_hip_grid welvet_hip_grid;
/* architecture::new_grid grid.cpp:31-60 (a dimension < 1 becomes 1). */
WELVET_API welvet_status welvet_hip_grid_new(int32_t depth, int32_t rows, int32_t cols,
                                             int32_t layers_per_cell, int32_t batch,
                                             welvet_hip_grid **g);
WELVET_API void welvet_hip_grid_release(welvet_hip_grid *g);
/* architecture::bind_dense grid.cpp:109-117 of dense::new_layer dense.cpp:101-119:
 * W_init [out*in] row-major f32 encoded into dtype; bias as in mount. */
WELVET_API welvet_status welvet_hip_grid_bind_dense(welvet_hip_grid *g, int32_t z, int32_t y,
                                                    int32_t x, int32_t l, int32_t in, int32_t out,
                                                    int32_t act, int32_t dtype, const float *W_init,
                                                    const double *bias, size_t bias_len);
/* architecture::set_remote_link grid.cpp:97-107: the cell reads the recorded
 * post of (tz,ty,tx,tl) instead of the previous hop's output. */
WELVET_API welvet_status welvet_hip_grid_set_remote_link(welvet_hip_grid *g, int32_t z, int32_t y,
                                                         int32_t x, int32_t l, int32_t tz,
                                                         int32_t ty, int32_t tx, int32_t tl);
/* CellMeta::is_disabled: the hop skips the cell (forward.cpp:90). */
WELVET_API welvet_status welvet_hip_grid_set_disabled(welvet_hip_grid *g, int32_t z, int32_t y,
                                                      int32_t x, int32_t l, int32_t disabled);
/* runtime::forward::volume_dense forward.cpp:74-132 in hop order z,y,x,l
 * (grid.cpp:82-95): x [batch*in] -> y [batch*out], out = the last hop's width. */
WELVET_API welvet_status welvet_hip_volume_forward(welvet_hip_grid *g, const float *x, int32_t in,
                                                   float *y, int32_t out);
/* The same on device pointers, enqueued on `stream` (NULL = null stream);
 * returns once enqueued.  The cells' activation buffers and workspace belong
 * to the grid: calls on one grid must not overlap (synchronise `stream`
 * before a call on the same grid from another stream or a host-buffer
 * call). */
WELVET_API welvet_status welvet_hip_volume_forward_device(welvet_hip_grid *g, const float *d_x,
                                                          int32_t in, float *d_y, int32_t out,
                                                          void *stream);
/* A volume forward followed by runtime::training::step_dense training.cpp:161-184:
 * *loss = MSE(y, target) (target [batch*out]), backward through the tape in
 * reverse (backward.cpp:88-127), SGD of every cell in forward order with
 * re-encode (training.cpp:61-159).  y [batch*out] receives the forward
 * output when non-NULL. */
WELVET_API welvet_status welvet_hip_volume_train_step(welvet_hip_grid *g, const float *x,
                                                      int32_t in, const float *target, int32_t out,
                                                      double lr, double *loss, float *y);
/* welvet_hip_volume_train_step that also returns runtime::backward::Result::
 * grad_in (backward.cpp:125): grad_in [batch*in] (nullable) receives the input
 * gradient of the first hop, which the WVN1 wire's WVNO reply carries
 * (tools/dense_fwd/volume_fwd.cpp:1897-1902). */
WELVET_API welvet_status welvet_hip_volume_train_step_grad(welvet_hip_grid *g, const float *x,
                                                           int32_t in, const float *target,
                                                           int32_t out, double lr, double *loss,
                                                           float *y, float *grad_in);
/* The same on device pointers on `stream`; returns after the step completed. */
WELVET_API welvet_status welvet_hip_volume_train_step_device(welvet_hip_grid *g, const float *d_x,
                                                             int32_t in, const float *d_target,
                                                             int32_t out, double lr, double *loss,
                                                             void *stream);
/* WeightStore::export_f32 / native bytes of one bound cell. */
WELVET_API welvet_status welvet_hip_grid_export_f32(welvet_hip_grid *g, int32_t z, int32_t y,
                                                    int32_t x, int32_t l, float *W_out);
/* welvet_hip_dense_repack of one bound cell's store. */
WELVET_API welvet_status welvet_hip_grid_repack(welvet_hip_grid *g, int32_t z, int32_t y,
                                                int32_t x, int32_t l, const float *values,
                                                size_t len);
WELVET_API welvet_status welvet_hip_grid_native(welvet_hip_grid *g, int32_t z, int32_t y,
                                                int32_t x, int32_t l, uint8_t *out, size_t cap,
                                                size_t *len, float *scale);

/* Resident SwiGLU: welvet_swiglu_forward_f32's layer kept mounted (the
 * three stores packed in HBM, `rows` = batch * seq fixed at mount), its
 * forward on device pointers (16-byte aligned) enqueued on `stream`:
 * x [rows*in] -> pre = h [rows*inter], post [rows*in].  Calls on one handle
 * must not overlap (they share its intermediate buffers). */
typedef struct welvet_hip_swiglu welvet_hip_swiglu;
WELVET_API welvet_status welvet_hip_swiglu_mount(int32_t rows, int32_t input_dim,
                                                 int32_t intermediate_dim, int32_t dtype,
                                                 const float *Gate, const float *Up,
                                                 const float *Down, welvet_hip_swiglu **s);
WELVET_API welvet_status welvet_hip_swiglu_forward_device(welvet_hip_swiglu *s, const float *d_x,
                                                          float *d_pre, float *d_post,
                                                          void *stream);
WELVET_API void welvet_hip_swiglu_release(welvet_hip_swiglu *s);

/* Kernel route of the forward: 0 auto, 1 GEMV, 2 MFMA GEMM, 3 element-wise. */
WELVET_API void welvet_hip_set_forward_path(int32_t path);
/* Route switch `key` := value, returns the previous value (-1 = unknown key,
 * the value unchanged).  Process-wide and atomic: a call on one thread is seen
 * by launches on any other, and a launch reads each switch once.  Every
 * setting computes the same result within the same tolerance (dW and the
 * SGD bit for bit); the switches exist so that tests can compare routes and
 * sweeps can time them.  Keys (default in brackets; the other key numbers
 * are unknown):
 *   10 split-x bf16 MFMA GEMM (x split exactly into three bf16 parts) for
 *      FP8 E4M3 / E5M2, Int8, FP4 and NF4 weights at batch > 4, 0 = the
 *      fp32 MFMA GEMMs [1]
 *   16 batch <= 16 forward and dX without a k split across workgroups
 *      (epilogue in the kernel, no reduction launch; the split-x GEMM for
 *      its formats, the fp32 MFMA for the others): 0 off, 1 for a
 *      reduction length <= 2048 (and, for the fp32-MFMA forward outside
 *      Float16 / BFloat16, any length at <= 8192 outputs, for 16-bit
 *      integers at lengths <= 4096 or batch <= 8, and at any width for
 *      32- and 64-bit integer, 1- to 3-bit table and Complex128 weights;
 *      the dX up to 4096 rows and 8192 columns outside FP8 and Int8),
 *      2 always [1]
 *   17 volume training steps: a piecewise activation's derivative (ReLU,
 *      ReLU2, LeakyReLU) applied in the epilogue of the layer above's
 *      no-split dX instead of a launch of its own [1]
 *   18 volume training steps: the SGD of consecutive cells of one dtype in
 *      one launch (up to 16 cells), 0 = one launch per cell [1]
 *   19 volume training steps: every layer's dW after the backward's dX
 *      chain, up to 16 layers per launch (layers whose sizes are multiples
 *      of 128), 0 = each with its layer's backward [1]
 *   20 batch 2-8 forward as a GEMV that keeps x of every batch row in
 *      registers (every format but Float64 and the complex ones; rows of at
 *      most 8 waves, x of at most 128 registers per lane; the split-x
 *      formats' batch 5-8 up to 32 M weights):
 *      0 off, 1 on with an automatic grid, k >= 2 on with k waves per CU
 *      walking the row groups [1]
 *   21 the fp32-MFMA no-split forward and the no-split dX of key 16 with x /
 *      dpre copied into LDS once per workgroup when the reduction length is
 *      at most 1024, 0 = each lane loads its own [1] */
WELVET_API int32_t welvet_hip_set_tuning(int32_t key, int32_t value);

/* No counterpart in the reference: a measurement aid.  Streams `bytes`
 * (a non-zero multiple of 16) of device memory at d_bytes once, in one
 * launch on `stream`, with the loads the batch-1 GEMVs use (16 bytes per
 * lane, non-temporal, four in flight per thread); the single-launch floor
 * for a kernel that reads the same bytes once.  d_sink: 4 KB of device
 * memory the probe may write (practically never does).  Code 1 on null or
 * misaligned arguments. */
WELVET_API welvet_status welvet_hip_probe_read(const void *d_bytes, uint64_t bytes, void *d_sink,
                                               void *stream);

#ifdef __cplusplus
}
#endif
#endif
