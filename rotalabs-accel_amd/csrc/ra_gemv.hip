// Decode GEMV (M <= 4) for gfx950: one HBM round trip per wave.
//
// Replaces the reference's Triton tile loop (src/rotalabs_accel/kernels/
// gemm.py:113-138) for decode batches. At M <= 4 the weight stream is the
// whole cost (N*K bytes, 2*M flops per byte), so the kernel is organised
// around keeping HBM busy from the first cycle:
//
//  * A workgroup owns 16 weight rows (32 with the gate/up pair) and all of K;
//    its NW waves split K into NW slices of STEPS x 64 (split-K inside the
//    workgroup). Each wave issues ALL of its weight loads -- STEPS 128-bit
//    loads per lane and row tile -- before doing anything else, so the kernel
//    is a single memory round trip per wave instead of a loop of them.
//  * The activations x[0:M, 0:K] (<= 64 KB) are copied once per workgroup
//    into LDS while the weight loads are in flight; MFMA operands are read
//    from there, so x costs no VGPRs and the weight registers bound occupancy.
//  * Compute: v_mfma_f32_16x16x32_{f16,bf16} on Y^T = W . X^T (MFMA rows are
//    weight rows, columns are activation rows, M padded to 16 with zeros).
//    Lane (r, g) holds 16 contiguous weight bytes of row r at k + 16g; the
//    two 8-byte halves feed two MFMAs with the matching x halves (the same k
//    permutation on both operands). int8 -> fp16/bf16 is exact, in registers.
//  * The NW partial sums are combined through LDS in a fixed order (only the
//    M valid columns are exchanged); the epilogue applies scale (+ bias) or
//    the SwiGLU of the gate/up pair to the fp32 result. No atomics, no
//    workspace, deterministic.
#include "ra_common.h"
#include "ra_internal.h"

namespace ra {

constexpr int kGemvMaxM = 4;
constexpr int kGemvMaxWaves = 16;
constexpr size_t kGemvMaxLdsBytes = 64 * 1024;

template <int DT, int STEPS, bool GU>
__global__ __launch_bounds__(1024) void gemv_kernel(const uint16_t *__restrict__ x, int64_t ldx,
                                                    const int8_t *__restrict__ w, int64_t ldw,
                                                    const float *__restrict__ scale,
                                                    const void *__restrict__ bias, int bias_dt,
                                                    uint16_t *__restrict__ y, int64_t ldy, int M, int N,
                                                    int K) {
  using A = Act<DT>;
  constexpr int NT = GU ? 2 : 1;  // weight row tiles (gate, up)
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint16_t *xs = reinterpret_cast<uint16_t *>(smem);  // [M][K]
  const int kpad = (K + 7) & ~7;
  float *red = reinterpret_cast<float *>(smem + (size_t)M * kpad * 2);  // [NW][NT][M][16]

  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int kb = wid * (STEPS * 64);

  // 1. every weight load of this wave, issued up front
  uint4 wv[NT][STEPS];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int n = n0 + r;
    n = n < N ? n : N - 1;
    if (t == 1) n += N;
    const int8_t *wp = w + (int64_t)n * ldw + 16 * g;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int k = kb + 64 * s;
      wv[t][s] = (k + 16 * g + 16 <= K) ? *reinterpret_cast<const uint4 *>(wp + k) : make_uint4(0, 0, 0, 0);
    }
  }

  // 2. x[0:M, 0:K] -> LDS (16-byte chunks; K % 16 == 0)
  const int chunks_per_row = K >> 3;
  for (int i = threadIdx.x; i < M * chunks_per_row; i += blockDim.x) {
    const int m = i / chunks_per_row, c = i - m * chunks_per_row;
    *reinterpret_cast<uint4 *>(xs + m * kpad + c * 8) =
        *reinterpret_cast<const uint4 *>(x + (int64_t)m * ldx + c * 8);
  }
  __syncthreads();

  // 3. MFMAs over this wave's K slice
  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const bool mv = r < M;
  const uint16_t *xr = xs + (mv ? r : 0) * kpad + 16 * g;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int k = kb + 64 * s;
    if (k >= K) break;  // wave-uniform
    const bool ok = mv && (k + 16 * g + 16 <= K);
    const uint4 xa = ok ? *reinterpret_cast<const uint4 *>(xr + k) : make_uint4(0, 0, 0, 0);
    const uint4 xb = ok ? *reinterpret_cast<const uint4 *>(xr + k + 8) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      acc[t] = A::mfma16(A::dq8(wv[t][s].x, wv[t][s].y), xa, acc[t]);
      acc[t] = A::mfma16(A::dq8(wv[t][s].z, wv[t][s].w), xb, acc[t]);
    }
  }

  // 4. split-K combine: lanes with r < M hold D[4g+q][r] = partial y[r][n0+4g+q]
  if (mv) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q) red[((wid * NT + t) * M + r) * 16 + 4 * g + q] = acc[t][q];
  }
  __syncthreads();
  // 16 rows x M outputs, one thread each
  const int o = threadIdx.x;
  if (o < 16 * M) {
    const int m = o >> 4, i = o & 15;
    const int n = n0 + i;
    if (n < N) {
      float s0 = 0.f, s1 = 0.f;
      for (int v = 0; v < nw; ++v) {
        s0 += red[((v * NT + 0) * M + m) * 16 + i];
        if (GU) s1 += red[((v * NT + 1) * M + m) * 16 + i];
      }
      uint16_t *yrow = y + (int64_t)m * ldy;
      if (GU)
        yrow[n] = swiglu_out<A>(s0 * scale[n], s1 * scale[N + n]);
      else
        yrow[n] = A::out(epilogue_value(s0, scale, bias, bias_dt, n));
    }
  }
}

// STEPS per wave so that one workgroup (<= 16 waves) covers K; only the
// spill-free instantiations (<= 128 VGPRs at 1024 threads) are used:
// STEPS 8 (single or gate/up pair), STEPS 16 (single row tile).
static int gemv_steps(int64_t K, bool gu) {
  if (K <= 8 * 64 * kGemvMaxWaves) return 8;
  if (!gu && K <= 16 * 64 * kGemvMaxWaves) return 16;
  return 0;
}

static size_t gemv_lds_bytes(int64_t M, int64_t K, int nw, bool gu) {
  return (size_t)M * ((K + 7) & ~7) * 2 + (size_t)nw * (gu ? 2 : 1) * M * 16 * 4;
}

static bool gemv_ok(int x_dt, const void *x, int64_t ldx, const int8_t *w, int64_t ldw, int64_t M, int64_t N,
                    int64_t K, bool gu) {
  if (x_dt != RA_F16 && x_dt != RA_BF16) return false;
  if (M < 1 || M > kGemvMaxM || N > ((int64_t)1 << 30) || K < 16 || K % 16 != 0) return false;
  const int steps = gemv_steps(K, gu);
  if (steps == 0) return false;
  const int nw = (int)((K + 64 * steps - 1) / (64 * steps));
  if (gemv_lds_bytes(M, K, nw, gu) > kGemvMaxLdsBytes) return false;
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(w) & 15)) return false;
  return (ldx % 8) == 0 && (ldw % 16) == 0;
}

bool gemv_supported(const GemmArgs &a) { return gemv_ok(a.x_dt, a.x, a.ldx, a.w, a.ldw, a.M, a.N, a.K, false); }

bool gateup_gemv_supported(const GateUpArgs &a) {
  return gemv_ok(a.x_dt, a.x, a.ldx, a.w, a.ldw, a.M, 2 * a.I, a.K, true);
}

template <bool GU>
static hipError_t gemv_launch_impl(const void *x, int64_t ldx, int x_dt, const int8_t *w, int64_t ldw,
                                   const float *scale, const void *bias, int bias_dt, void *y, int64_t ldy,
                                   int64_t M, int64_t N, int64_t K, hipStream_t s) {
  const int steps = gemv_steps(K, GU);
  const int nw = (int)((K + 64 * steps - 1) / (64 * steps));
  const size_t lds = gemv_lds_bytes(M, K, nw, GU);
  const dim3 grid((unsigned)((N + 15) / 16)), block(64 * nw);
  const uint16_t *xp = static_cast<const uint16_t *>(x);
  uint16_t *yp = static_cast<uint16_t *>(y);
  const int Mi = (int)M, Ni = (int)N, Ki = (int)K;
#define RA_GEMV_LAUNCH(DT_, ST_)                                                                            \
  hipLaunchKernelGGL((gemv_kernel<DT_, ST_, GU>), grid, block, lds, s, xp, ldx, w, ldw, scale, bias, bias_dt, \
                     yp, ldy, Mi, Ni, Ki)
  if constexpr (GU) {
    if (x_dt == RA_F16) RA_GEMV_LAUNCH(RA_F16, 8);
    else RA_GEMV_LAUNCH(RA_BF16, 8);
  } else {
    if (x_dt == RA_F16) {
      if (steps == 8) RA_GEMV_LAUNCH(RA_F16, 8);
      else RA_GEMV_LAUNCH(RA_F16, 16);
    } else {
      if (steps == 8) RA_GEMV_LAUNCH(RA_BF16, 8);
      else RA_GEMV_LAUNCH(RA_BF16, 16);
    }
  }
#undef RA_GEMV_LAUNCH
  return hipGetLastError();
}

hipError_t gemv_launch(const GemmArgs &a, hipStream_t s) {
  return gemv_launch_impl<false>(a.x, a.ldx, a.x_dt, a.w, a.ldw, a.scale, a.bias, a.bias_dt, a.y, a.ldy, a.M,
                                 a.N, a.K, s);
}

hipError_t gateup_gemv_launch(const GateUpArgs &a, hipStream_t s) {
  return gemv_launch_impl<true>(a.x, a.ldx, a.x_dt, a.w, a.ldw, a.scale, nullptr, RA_F32, a.h, a.ldh, a.M, a.I,
                                a.K, s);
}

}  // namespace ra
