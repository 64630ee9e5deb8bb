/*
 * oracle.h — CPU restatement of welvet.metal's quantized-storage Dense path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the HIP path is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links it and never
 * falls back to it.
 *
 * Every function restates one piece of the reference and cites the file:line
 * it follows (paths relative to the reference checkout).  Where the reference
 * is the Apple-GPU soft-double arithmetic, the restatement pins the Go f64
 * contract that arithmetic approximates (welvet_dense.metal:1-3).
 *
 * Platform-dependent casts are pinned to the reference platform (arm64):
 * float->integer conversions saturate and NaN converts to 0.
 *
 * Parity pinning (what checks each function):
 *   codecs (or_f32_to_*, or_*_to_f32)  golden vectors + exhaustive compare
 *                                      against oracle/_ref (compiled reference)
 *   or_pack / or_decode / or_decode_f64 golden vectors + oracle/_ref compare
 *   or_set (fixed-scale re-encode)     round-trip invariants + closed forms;
 *                                      the float formats share the scalar
 *                                      codecs pinned above
 *   or_native_sgd / or_sgd_f32         closed forms (lr=0 identity apart from
 *                                      the element-0 probe, exact dyadic steps)
 *                                      + the release_smoke KAT
 *   or_dense_forward / or_dense_backward brute force on dyadic inputs (every
 *                                      summation order exact) + the KAT
 *   or_act / or_act_prime              closed forms and finite differences
 *   or_mse / or_mse_grad               KAT (loss 0.15625) + closed forms
 *   or_swiglu_h / or_swiglu_split      closed forms through the composed
 *                                      SwiGLU layer (identity weights, swapped
 *                                      roles distinguishable) and finite
 *                                      differences of its forward (oracle.py)
 */
#ifndef WELVET_ORACLE_H
#define WELVET_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* DType ids (include/welvet/dtype.hpp:9-44) */
enum {
  OR_FLOAT64 = 0, OR_FLOAT32 = 1, OR_FLOAT16 = 2, OR_BFLOAT16 = 3, OR_FP8E4M3 = 4,
  OR_FP8E5M2 = 5, OR_INT64 = 6, OR_INT32 = 7, OR_INT16 = 8, OR_INT8 = 9, OR_UINT64 = 10,
  OR_UINT32 = 11, OR_UINT16 = 12, OR_UINT8 = 13, OR_INT4 = 14, OR_UINT4 = 15, OR_FP4 = 16,
  OR_INT2 = 17, OR_UINT2 = 18, OR_TERNARY = 19, OR_BINARY = 20, OR_INT = 21, OR_UINT = 22,
  OR_UINTPTR = 23, OR_COMPLEX64 = 24, OR_COMPLEX128 = 25, OR_NF4 = 26, OR_FP6 = 27,
  OR_INT6 = 28, OR_UINT6 = 29, OR_INT5 = 30, OR_UINT5 = 31, OR_INT3 = 32, OR_UINT3 = 33,
  OR_NUM_DTYPES = 34
};

/* scalar float codecs (src/core/float_codecs.cpp) */
uint16_t or_f32_to_f16(float f);
float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_bf16(float f);
float or_bf16_to_f32(uint16_t h);
uint8_t or_f32_to_e4m3(float f);
float or_e4m3_to_f32(uint8_t b);
uint8_t or_f32_to_e5m2(float f);
float or_e5m2_to_f32(uint8_t b);
uint8_t or_f32_to_fp4(float f);
float or_fp4_to_f32(uint8_t code);

/* native store (src/weights/native_codec.cpp, src/weights/store.cpp) */
int64_t or_native_bytes(int dtype, int64_t n);
int or_pack(int dtype, const float *w, int64_t n, uint8_t *out, float *scale);
int or_decode(int dtype, const uint8_t *raw, int64_t raw_n, float scale, int64_t n, float *out);
int or_decode_f64(int dtype, const uint8_t *raw, int64_t raw_n, float scale, int64_t n,
                  double *out);
int or_set(int dtype, uint8_t *raw, int64_t raw_n, float scale, int64_t i, int64_t n, float v);

/* training (shaders/welvet_dense.metal, shaders/ops_storage.metal) */
int or_native_sgd(int dtype, uint8_t *raw, int64_t raw_n, float scale, int64_t n,
                  const float *dW, double lr);
void or_sgd_f32(float *w, const float *dW, int64_t n, double lr);
double or_mse(const float *pred, const float *target, int64_t n);
void or_mse_grad(const float *pred, const float *target, int64_t n, float *grad);

/* activations (shaders/ops_common.metal:83-138) */
float or_act(float v, int act);
float or_act_prime(float v, int act);

/* Dense (shaders/welvet_dense.metal:54-178) */
void or_dense_forward(int batch, int in, int out, int act, const double *Wd, const double *bias,
                      int64_t bias_len, const float *x, float *pre, float *post);
void or_dense_backward(int batch, int in, int out, int act, const double *Wd, const float *x,
                       const float *pre, const float *gy, float *dpre, float *dX, float *dW);

/* op_swiglu (shaders/ops_common.metal:27-38): forward h = fl32(silu(gate)) * up
 * in f32; backward d_up = gh * fl32(silu(gate)) in f32 and
 * d_gate = fl32(gh * up * fl32(silu'(gate))) with the product kept wide */
void or_swiglu_h(const float *gate, const float *up, int64_t n, float *h);
void or_swiglu_split(const float *gate, const float *up, const float *gh, int64_t n, float *d_up,
                     float *d_gate);

/* whole NormalBP leaf (src/interop/c_abi.cpp:142-207); returns a welvet status code */
int or_normalbp(int batch, int in, int out, int act, int dtype, const float *W_init,
                const double *bias, int64_t bias_len, const float *x, const float *grad_or_target,
                int use_target, double lr, float *pre, float *post, float *dX, float *dW,
                float *W_after, double *loss);

int or_repack(int dt, const float *a, int64_t n, uint8_t *raw, int64_t raw_n, float *scale_out);
void or_decode_many(int kind, const uint32_t *codes, int64_t n, float *out);
void or_encode_many(int kind, const float *in, int64_t n, void *out);

/* CPU baseline: decode each element through the dtype switch, then the f64 dot */
void or_dense_forward_native(int batch, int in, int out, int act, int dtype, const uint8_t *raw,
                             int64_t raw_n, float scale, const double *bias, int64_t bias_len,
                             const float *x, float *pre, float *post, int threads);

#ifdef __cplusplus
}
#endif
#endif
