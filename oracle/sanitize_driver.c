/*
 * sanitize_driver.c — drives every oracle entry point under AddressSanitizer
 * and UndefinedBehaviorSanitizer (TEST INFRASTRUCTURE ONLY; built by
 * `make -C oracle sanitize`, run by tests/test_sanitizers.py).
 *
 * Each call gets heap buffers of exactly the size the function may touch
 * (or_native_bytes for codes, n values for arrays), so one element past the
 * end is a reported overflow.  Inputs cover every dtype, element counts that
 * end inside a packed unit (1, 3, 7, 33, 257, ...), zero-length stores,
 * special values (signed zeros, subnormals, the formats' overflow range,
 * infinities, NaN), non-finite gradients and learning rates, biases shorter
 * and longer than the output, and unknown activation ids.  The driver checks
 * no values: the parity tests do that; it exits 0 when no sanitizer fired
 * (every sanitizer report aborts: -fno-sanitize-recover=all).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static uint64_t g_state = 0x9E3779B97F4A7C15ull;

static uint32_t next_u32(void) {
  /* xorshift64* */
  g_state ^= g_state >> 12;
  g_state ^= g_state << 25;
  g_state ^= g_state >> 27;
  return (uint32_t)((g_state * 0x2545F4914F6CDD1Dull) >> 32);
}

static float uniform(float lo, float hi) { return lo + (hi - lo) * (float)(next_u32() >> 8) / 16777216.0f; }

/* a value of the kind `mode` picks: 0 ordinary, 1 mixed specials */
static float value(int mode) {
  if (mode == 0) return uniform(-2.0f, 2.0f);
  static const float special[] = {0.0f, -0.0f, 1e-40f, -1e-40f, 1e-45f, 65504.0f, 65520.0f, 448.0f,
                                  464.0f, 57344.0f, 61440.0f, 6.0f, 7.0f, 3.4e38f, -3.4e38f, 1e30f};
  const uint32_t r = next_u32() % 24;
  if (r < 16) return special[r];
  if (r == 16) return INFINITY;
  if (r == 17) return -INFINITY;
  if (r == 18) return NAN;
  return uniform(-100.0f, 100.0f);
}

static void *xmalloc(size_t bytes) {
  void *p = malloc(bytes ? bytes : 1);
  if (!p) {
    fprintf(stderr, "out of memory\n");
    exit(3);
  }
  return p;
}

static float *values(int64_t n, int mode) {
  float *v = (float *)xmalloc(sizeof(float) * (size_t)n);
  for (int64_t i = 0; i < n; ++i) v[i] = value(mode);
  return v;
}

static void scalar_codecs(void) {
  for (uint32_t c = 0; c < 65536; ++c) {
    (void)or_f16_to_f32((uint16_t)c);
    (void)or_bf16_to_f32((uint16_t)c);
  }
  for (uint32_t c = 0; c < 256; ++c) {
    (void)or_e4m3_to_f32((uint8_t)c);
    (void)or_e5m2_to_f32((uint8_t)c);
    (void)or_fp4_to_f32((uint8_t)c);
  }
  /* every 65537th f32 bit pattern (all exponents, both signs, NaN payloads) */
  for (uint64_t b = 0; b <= 0xffffffffull; b += 65537) {
    const uint32_t u = (uint32_t)b;
    float f;
    memcpy(&f, &u, 4);
    (void)or_f32_to_f16(f);
    (void)or_f32_to_bf16(f);
    (void)or_f32_to_e4m3(f);
    (void)or_f32_to_e5m2(f);
    (void)or_f32_to_fp4(f);
  }
  for (int kind = 0; kind < 6; ++kind) {
    const int64_t n = 77;
    uint32_t *codes = (uint32_t *)xmalloc(sizeof(uint32_t) * n);
    float *out = (float *)xmalloc(sizeof(float) * n);
    float *in = values(n, 1);
    void *enc = xmalloc((size_t)n * (kind < 2 ? 2 : 1));
    for (int64_t i = 0; i < n; ++i) codes[i] = next_u32() & (kind < 2 ? 0xffffu : 0xffu);
    or_decode_many(kind, codes, n, out);
    or_encode_many(kind, in, n, enc);
    free(codes), free(out), free(in), free(enc);
  }
}

/* pack / decode / set / SGD / repack of one store */
static void store_calls(int dtype, int64_t n, int mode) {
  const int64_t nb = or_native_bytes(dtype, n);
  if (nb < 0) return;
  float *w = values(n, mode);
  uint8_t *raw = (uint8_t *)xmalloc((size_t)nb);
  memset(raw, 0, (size_t)nb);
  float scale = 1.0f;
  if (or_pack(dtype, w, n, raw, &scale) == 0) {
    float *out = (float *)xmalloc(sizeof(float) * (size_t)n);
    double *out64 = (double *)xmalloc(sizeof(double) * (size_t)n);
    (void)or_decode(dtype, raw, nb, scale, n, out);
    (void)or_decode_f64(dtype, raw, nb, scale, n, out64);
    /* a raw buffer one byte short must be refused, not read past */
    if (nb > 0) {
      uint8_t *shorter = (uint8_t *)xmalloc((size_t)nb - 1);
      memcpy(shorter, raw, (size_t)nb - 1);
      (void)or_decode(dtype, shorter, nb - 1, scale, n, out);
      free(shorter);
    }
    for (int k = 0; k < 4 && n > 0; ++k) {
      const int64_t i = (int64_t)(next_u32() % (uint32_t)n);
      (void)or_set(dtype, raw, nb, scale, i, n, value(1));
    }
    (void)or_set(dtype, raw, nb, scale, n, n, 1.0f); /* index past the end: refused */
    float *g = values(n, mode);
    const double rates[] = {1e-3, 0.0, -0.5, 1e30, NAN, INFINITY};
    for (int r = 0; r < 6; ++r) (void)or_native_sgd(dtype, raw, nb, scale, n, g, rates[r]);
    float *w2 = (float *)xmalloc(sizeof(float) * (size_t)n);
    memcpy(w2, w, sizeof(float) * (size_t)n);
    or_sgd_f32(w2, g, n, 1e-2);
    float scale2 = 1.0f;
    (void)or_repack(dtype, w, n, raw, nb, &scale2);
    free(out), free(out64), free(g), free(w2);
  }
  free(w), free(raw);
}

static void dense_calls(int batch, int in, int out, int act, int64_t bias_len, int mode) {
  const int64_t n = (int64_t)out * in, ny = (int64_t)batch * out, nx = (int64_t)batch * in;
  double *Wd = (double *)xmalloc(sizeof(double) * (size_t)n);
  for (int64_t i = 0; i < n; ++i) Wd[i] = value(mode);
  double *bias = bias_len > 0 ? (double *)xmalloc(sizeof(double) * (size_t)bias_len) : NULL;
  for (int64_t i = 0; i < bias_len; ++i) bias[i] = value(0);
  float *x = values(nx, mode), *gy = values(ny, mode), *tgt = values(ny, 0);
  float *pre = (float *)xmalloc(sizeof(float) * (size_t)ny), *post = (float *)xmalloc(sizeof(float) * (size_t)ny);
  float *dpre = (float *)xmalloc(sizeof(float) * (size_t)ny), *dX = (float *)xmalloc(sizeof(float) * (size_t)nx);
  float *dW = (float *)xmalloc(sizeof(float) * (size_t)n), *grad = (float *)xmalloc(sizeof(float) * (size_t)ny);
  or_dense_forward(batch, in, out, act, Wd, bias, bias_len, x, pre, post);
  or_dense_backward(batch, in, out, act, Wd, x, pre, gy, dpre, dX, dW);
  (void)or_mse(post, tgt, ny);
  or_mse_grad(post, tgt, ny, grad);
  for (int dtype = 0; dtype < OR_NUM_DTYPES; dtype += 3) {
    float *W_init = values(n, mode), *W_after = (float *)xmalloc(sizeof(float) * (size_t)n);
    double loss = 0.0;
    (void)or_normalbp(batch, in, out, act, dtype, W_init, bias, bias_len, x, tgt, 1, 1e-2, pre, post, dX, dW,
                      W_after, &loss);
    (void)or_normalbp(batch, in, out, act, dtype, W_init, bias, bias_len, x, gy, 0, 0.0, pre, post, dX, dW,
                      W_after, &loss);
    const int64_t nb = or_native_bytes(dtype, n);
    uint8_t *raw = (uint8_t *)xmalloc((size_t)(nb > 0 ? nb : 1));
    float scale = 1.0f;
    if (nb >= 0 && or_pack(dtype, W_init, n, raw, &scale) == 0)
      for (int threads = 1; threads <= 2; ++threads)
        or_dense_forward_native(batch, in, out, act, dtype, raw, nb, scale, bias, bias_len, x, pre, post,
                                threads);
    free(W_init), free(W_after), free(raw);
  }
  free(Wd), free(bias), free(x), free(gy), free(tgt), free(pre), free(post), free(dpre), free(dX), free(dW),
      free(grad);
}

int main(void) {
  scalar_codecs();
  static const int64_t counts[] = {0, 1, 2, 3, 5, 7, 8, 15, 16, 17, 31, 32, 33, 63, 64, 65, 100, 255, 257, 1031};
  for (int dtype = 0; dtype < OR_NUM_DTYPES; ++dtype)
    for (size_t c = 0; c < sizeof(counts) / sizeof(counts[0]); ++c)
      for (int mode = 0; mode < 2; ++mode) store_calls(dtype, counts[c], mode);
  for (int act = -2; act <= 8; ++act) {
    for (int k = 0; k < 200; ++k) {
      const float v = value(k & 1);
      (void)or_act(v, act);
      (void)or_act_prime(v, act);
    }
  }
  {
    const int64_t n = 129;
    float *gate = values(n, 1), *up = values(n, 1), *gh = values(n, 1);
    float *h = (float *)xmalloc(sizeof(float) * n), *du = (float *)xmalloc(sizeof(float) * n);
    float *dg = (float *)xmalloc(sizeof(float) * n);
    or_swiglu_h(gate, up, n, h);
    or_swiglu_split(gate, up, gh, n, du, dg);
    free(gate), free(up), free(gh), free(h), free(du), free(dg);
  }
  static const int shapes[][3] = {{1, 1, 1}, {1, 7, 3}, {3, 33, 5}, {2, 64, 17}, {4, 5, 70}};
  for (size_t s = 0; s < sizeof(shapes) / sizeof(shapes[0]); ++s) {
    const int batch = shapes[s][0], in = shapes[s][1], out = shapes[s][2];
    for (int act = -1; act <= 6; ++act) {
      dense_calls(batch, in, out, act, 0, 0);
      dense_calls(batch, in, out, act, out > 1 ? out - 1 : 1, 1);
      dense_calls(batch, in, out, act, out + 3, act & 1);
    }
  }
  printf("sanitize_driver: ok\n");
  return 0;
}
