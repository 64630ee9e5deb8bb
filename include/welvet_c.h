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

/* Forward on device pointers (16-byte aligned) enqueued on `stream`
 * (a hipStream_t; NULL = the HIP null stream); returns once enqueued. */
WELVET_API welvet_status welvet_hip_dense_forward_device(welvet_dense_session *s, const float *d_x,
                                                         float *d_pre, float *d_post,
                                                         void *stream);
/* The store in the reference's byte layout (WeightStore::native, with the
 * 4-byte min header of the unsigned types; f32 bytes for Float32).  *len gets
 * the payload size; fails with code 1 when cap is too small. */
WELVET_API welvet_status welvet_hip_dense_native(welvet_dense_session *s, uint8_t *out,
                                                 size_t cap, size_t *len, float *scale);
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
/* Kernel route of the forward: 0 auto, 1 GEMV, 2 MFMA GEMM, 3 element-wise. */
WELVET_API void welvet_hip_set_forward_path(int32_t path);
/* Kernel tuning knob `key` := value, returns the previous value (-1 = unknown
 * key).  Process-wide; results stay within the same tolerance whatever the
 * setting.  Keys (default in brackets):
 *   0 batch-1 GEMV kernel: 0 row-group, 1 all-loads-in-flight [1],
 *     2 column-stationary
 *   1 column-stationary rows per block [0 = 16]
 *   2 column-stationary in-lane f64 accumulation [0]
 *   3 all-loads-in-flight chunks per lane: 0 auto, 1 two, 2 four, 3 one,
 *     4 eight [0]
 *   4 register-B MFMA GEMM for formats of <= 16 bits [1]
 *   5 its workgroups per CU [0 = 2]
 *   6 hardware FP8 conversions and integer Int8 decode instead of tables [1]
 *   7 byte-pair decode table for 4-bit formats [1] */
WELVET_API int32_t welvet_hip_set_tuning(int32_t key, int32_t value);

#ifdef __cplusplus
}
#endif
#endif
