// Row-wise and elementwise kernels on the decoder-MLP path:
//  * RMSNorm (the prologue of the gate/up projection),
//  * standalone SwiGLU (the fused path folds it into the gate/up epilogue),
//  * per-output-channel int8 weight quantisation, bit-exact with the CPU.
// All are HBM-bound row/byte work: one workgroup per row, coalesced loads,
// wave64 shuffles + LDS for the row reduction, fp32 math.
#include "ra_common.h"
#include "ra_internal.h"

namespace ra {

constexpr int kRowThreads = 256;

template <bool IsMax>
__device__ __forceinline__ float block_reduce(float v, float *smem) {
  v = IsMax ? wave_max(v) : wave_sum(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) smem[wid] = v;
  __syncthreads();
  float r = smem[0];
#pragma unroll
  for (int i = 1; i < kRowThreads / 64; ++i) r = IsMax ? fmaxf(r, smem[i]) : r + smem[i];
  return r;
}

// y = round_y( round_x(x * rsqrt(mean(x^2) + eps)) * w ), as rmsnorm_torch
// (src/rotalabs_accel/kernels/normalization.py:43-45): the normalised value
// is stored in x's dtype, then multiplied by the weight in the promoted dtype.
// rsqrt is 1/sqrt with both operations correctly rounded (no approximation).
__global__ __launch_bounds__(kRowThreads) void rmsnorm_kernel(const void *__restrict__ x, int64_t ldx,
                                                              int x_dt, const void *__restrict__ w,
                                                              int w_dt, void *__restrict__ y,
                                                              int64_t ldy, int y_dt, int hidden,
                                                              float eps) {
  __shared__ float smem[kRowThreads / 64];
  const int64_t row = blockIdx.x;
  float ss = 0.f;
  for (int i = threadIdx.x; i < hidden; i += kRowThreads) {
    const float v = load_as_f32(x, row * ldx + i, x_dt);
    ss += v * v;
  }
  const float total = block_reduce<false>(ss, smem);
  const float r = 1.0f / sqrtf(total / (float)hidden + eps);
  for (int i = threadIdx.x; i < hidden; i += kRowThreads) {
    const float v = round_through(load_as_f32(x, row * ldx + i, x_dt) * r, x_dt);
    store_from_f32(y, row * ldy + i, y_dt, v * load_as_f32(w, i, w_dt));
  }
}

hipError_t rmsnorm_launch(const void *x, int64_t ldx, int x_dt, const void *w, int w_dt, void *y,
                          int64_t ldy, int y_dt, int64_t rows, int64_t hidden, float eps,
                          hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(kRowThreads), 0, s, x, ldx, x_dt, w, w_dt,
                     y, ldy, y_dt, (int)hidden, eps);
  return hipGetLastError();
}

// out = silu(g) * u = g / (1 + exp(-g)) * u in fp32, one rounding
// (the Triton kernel's arithmetic, src/rotalabs_accel/kernels/activations.py:69-80).
__global__ __launch_bounds__(256) void swiglu_kernel(const void *__restrict__ g, const void *__restrict__ u,
                                                     void *__restrict__ o, int64_t n, int dt) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const float gv = load_as_f32(g, i, dt);
    store_from_f32(o, i, dt, gv / (1.0f + expf(-gv)) * load_as_f32(u, i, dt));
  }
}

hipError_t swiglu_launch(const void *g, const void *u, void *o, int64_t n, int dt, hipStream_t s) {
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)blocks), dim3(256), 0, s, g, u, o, n, dt);
  return hipGetLastError();
}

// Per-row symmetric quantisation, the op sequence of quantize_symmetric(dim=1)
// (src/rotalabs_accel/quantization/symmetric.py:66-80) on the CPU:
//   s = round_w(amax / 127)   IEEE division (built without fast-math)
//   s = 1 if s == 0
//   q = int8(clamp(rint(round_w(w / s)), -128, 127))   rint: half to even
// round_w is the rounding to the weight dtype (identity for fp32).
__global__ __launch_bounds__(kRowThreads) void quantize_kernel(const void *__restrict__ w, int64_t ldw,
                                                               int w_dt, int K, int8_t *__restrict__ q,
                                                               int64_t ldq, float *__restrict__ scale) {
  __shared__ float smem[kRowThreads / 64];
  const int64_t row = blockIdx.x;
  float amax = 0.f;
  for (int i = threadIdx.x; i < K; i += kRowThreads)
    amax = fmaxf(amax, fabsf(load_as_f32(w, row * ldw + i, w_dt)));
  amax = block_reduce<true>(amax, smem);
  float s = round_through(amax / 127.0f, w_dt);
  if (s == 0.0f) s = 1.0f;
  for (int i = threadIdx.x; i < K; i += kRowThreads) {
    const float v = round_through(load_as_f32(w, row * ldw + i, w_dt) / s, w_dt);
    const float rq = fminf(fmaxf(rintf(v), -128.0f), 127.0f);
    q[row * ldq + i] = (int8_t)(int)rq;
  }
  if (threadIdx.x == 0) scale[row] = s;
}

hipError_t quantize_launch(const void *w, int64_t ldw, int w_dt, int64_t N, int64_t K, int8_t *q,
                           int64_t ldq, float *scale, hipStream_t s) {
  hipLaunchKernelGGL(quantize_kernel, dim3((unsigned)N), dim3(kRowThreads), 0, s, w, ldw, w_dt, (int)K, q,
                     ldq, scale);
  return hipGetLastError();
}

}  // namespace ra
