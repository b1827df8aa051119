// Generic W8A16 kernels: any M, N, K, leading dimensions, alignment and
// activation dtype (fp16, bf16, fp32). Plain VALU dot products, one wave per
// output channel and four activation rows; used where the MFMA kernels'
// alignment / K % 16 requirements do not hold and for fp32 activations.
// Same arithmetic contract as the fast kernels: exact int8, fp32 accumulation,
// scale (and bias) applied to the fp32 sum, one rounding to the output dtype.
#include "ra_common.h"
#include "ra_internal.h"

namespace ra {

template <int XDT>
__global__ __launch_bounds__(256) void generic_kernel(const void *__restrict__ x, int64_t ldx,
                                                      const int8_t *__restrict__ w, int64_t ldw,
                                                      const float *__restrict__ scale,
                                                      const void *__restrict__ bias, int bias_dt,
                                                      void *__restrict__ y, int64_t ldy, int M, int N,
                                                      int K) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;  // whole wave exits; no barriers below
  const int8_t *wr = w + (int64_t)n * ldw;
  for (int m0 = blockIdx.y * 4; m0 < M; m0 += gridDim.y * 4) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k = lane; k < K; k += 64) {
      const float q = (float)wr[k];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (m0 + i < M) acc[i] += load_as_f32(x, (int64_t)(m0 + i) * ldx + k, XDT) * q;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float s = wave_sum(acc[i]);
      if (lane == i && m0 + i < M)
        store_from_f32(y, (int64_t)(m0 + i) * ldy + n, XDT, epilogue_value(s, scale, bias, bias_dt, n));
    }
  }
}

hipError_t generic_launch(const GemmArgs &a, hipStream_t s) {
  const unsigned gy = (unsigned)(a.M + 3) / 4 < 65535u ? (unsigned)(a.M + 3) / 4 : 65535u;
  dim3 grid((unsigned)((a.N + 3) / 4), gy > 0 ? gy : 1);
  const int M = (int)a.M, N = (int)a.N, K = (int)a.K;
  if (a.x_dt == RA_F16)
    hipLaunchKernelGGL(generic_kernel<RA_F16>, grid, dim3(256), 0, s, a.x, a.ldx, a.w, a.ldw, a.scale,
                       a.bias, a.bias_dt, a.y, a.ldy, M, N, K);
  else if (a.x_dt == RA_BF16)
    hipLaunchKernelGGL(generic_kernel<RA_BF16>, grid, dim3(256), 0, s, a.x, a.ldx, a.w, a.ldw, a.scale,
                       a.bias, a.bias_dt, a.y, a.ldy, M, N, K);
  else
    hipLaunchKernelGGL(generic_kernel<RA_F32>, grid, dim3(256), 0, s, a.x, a.ldx, a.w, a.ldw, a.scale,
                       a.bias, a.bias_dt, a.y, a.ldy, M, N, K);
  return hipGetLastError();
}

// h[m][j] = silu(g) * u, g / u the scaled dot products with weight rows j and I + j.
template <int XDT>
__global__ __launch_bounds__(256) void gateup_generic_kernel(const void *__restrict__ x, int64_t ldx,
                                                             const int8_t *__restrict__ w, int64_t ldw,
                                                             const float *__restrict__ scale,
                                                             void *__restrict__ h, int64_t ldh, int M,
                                                             int I, int K) {
  const int lane = threadIdx.x & 63;
  const int j = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (j >= I) return;
  const int8_t *wg = w + (int64_t)j * ldw;
  const int8_t *wu = w + (int64_t)(I + j) * ldw;
  for (int m0 = blockIdx.y * 4; m0 < M; m0 += gridDim.y * 4) {
    float ag[4] = {0.f, 0.f, 0.f, 0.f}, au[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k = lane; k < K; k += 64) {
      const float qg = (float)wg[k], qu = (float)wu[k];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (m0 + i < M) {
          const float xv = load_as_f32(x, (int64_t)(m0 + i) * ldx + k, XDT);
          ag[i] += xv * qg;
          au[i] += xv * qu;
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float sg = round_through(wave_sum(ag[i]) * scale[j], XDT);
      const float su = round_through(wave_sum(au[i]) * scale[I + j], XDT);
      const float act = round_through(sg / (1.0f + expf(-sg)), XDT);
      if (lane == i && m0 + i < M) store_from_f32(h, (int64_t)(m0 + i) * ldh + j, XDT, act * su);
    }
  }
}

hipError_t gateup_generic_launch(const GateUpArgs &a, hipStream_t s) {
  const unsigned gy = (unsigned)(a.M + 3) / 4 < 65535u ? (unsigned)(a.M + 3) / 4 : 65535u;
  dim3 grid((unsigned)((a.I + 3) / 4), gy > 0 ? gy : 1);
  const int M = (int)a.M, I = (int)a.I, K = (int)a.K;
  if (a.x_dt == RA_F16)
    hipLaunchKernelGGL(gateup_generic_kernel<RA_F16>, grid, dim3(256), 0, s, a.x, a.ldx, a.w, a.ldw,
                       a.scale, a.h, a.ldh, M, I, K);
  else if (a.x_dt == RA_BF16)
    hipLaunchKernelGGL(gateup_generic_kernel<RA_BF16>, grid, dim3(256), 0, s, a.x, a.ldx, a.w, a.ldw,
                       a.scale, a.h, a.ldh, M, I, K);
  else
    hipLaunchKernelGGL(gateup_generic_kernel<RA_F32>, grid, dim3(256), 0, s, a.x, a.ldx, a.w, a.ldw,
                       a.scale, a.h, a.ldh, M, I, K);
  return hipGetLastError();
}

}  // namespace ra
