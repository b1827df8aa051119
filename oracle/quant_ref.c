/*
 * Plain-C restatement of per-output-channel symmetric int8 quantization of an
 * fp32 weight matrix, as src/rotalabs_accel/quantization/symmetric.py:126-151
 * (quantize_weight_per_channel -> quantize_symmetric(dim=1), :24-82) computes
 * it on the CPU:
 *
 *   a_r = max_k |W[r,k]|                        (:66, exact)
 *   s_r = fl32(a_r / 127)                       (:67, IEEE true division)
 *   s_r = 1 if s_r == 0                         (:70)
 *   q   = int8(clamp(rne(fl32(W[r,k] / s_r)), -128, 127))   (:73)
 *
 * TEST INFRASTRUCTURE ONLY: an independent second restatement used to
 * cross-check oracle/quant.py. Build with oracle/Makefile (no fast-math).
 */
#include <math.h>
#include <stdint.h>

void oracle_quantize_rows_f32(const float *w, int64_t rows, int64_t cols,
                              int8_t *q, float *scale) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *row = w + r * cols;
    float amax = 0.0f;
    for (int64_t k = 0; k < cols; ++k) {
      float a = fabsf(row[k]);
      if (a > amax) amax = a;
    }
    volatile float s = amax / 127.0f; /* volatile: force one fp32 rounding */
    float sv = s;
    if (sv == 0.0f) sv = 1.0f;
    scale[r] = sv;
    for (int64_t k = 0; k < cols; ++k) {
      volatile float v = row[k] / sv;
      float rv = nearbyintf(v); /* default rounding mode: to nearest even */
      if (rv > 127.0f) rv = 127.0f;
      if (rv < -128.0f) rv = -128.0f;
      q[r * cols + k] = (int8_t)rv;
    }
  }
}

/* Dequantize then one fp32 GEMV row-dot in float64, used for brute-force
 * known-answer checks on tiny shapes: y[m,n] = sum_k x[m,k] * (q[n,k]*s[n]). */
void oracle_w8a16_gemm_f64(const double *x, const int8_t *q, const float *scale,
                           int64_t M, int64_t N, int64_t K, double *y) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0;
      float s = scale[n];
      for (int64_t k = 0; k < K; ++k) {
        float wq = (float)q[n * K + k] * s; /* one fp32 product */
        acc += x[m * K + k] * (double)wq;
      }
      y[m * N + n] = acc;
    }
}
