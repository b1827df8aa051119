// Decode GEMV (M <= 4) for gfx950: line-wide weight loads, one HBM round
// trip per wave.
//
// Replaces the reference's Triton tile loop (src/rotalabs_accel/kernels/
// gemm.py:113-138) for decode batches. At M <= 4 the weight stream is the
// whole cost (N*K bytes, 2*M flops per byte), so the kernel is organised
// around the HBM access pattern:
//
//  * Weight loads cover whole 128-byte lines: one 128-bit wave load reads 8
//    rows x 128 contiguous bytes (lane l: row l/8, bytes 16*(l%8)). On MI355X
//    a wave load spread over 16 rows x 64 bytes (the MFMA operand layout,
//    where lane%16 is the row) streams at ~3.9 TB/s; full lines stream at
//    ~5.4 TB/s for the same 45 MB.
//  * Each wave then transposes its 16-row x 128-byte window through a
//    private 2 KB LDS slot (16-byte chunks XOR-swizzled by row, so both the
//    write and the MFMA-layout read are bank-conflict free) into the
//    v_mfma_f32_16x16x32_{f16,bf16} layout: lane (r, g) reads row r, bytes
//    32g .. 32g+31 of the window, which feed four MFMAs (k-slots of lane
//    group g in MFMA u: window bytes 32g + 8u .. +7). int8 -> fp16 / bf16 is
//    exact, in registers.
//  * A workgroup owns 16 weight rows (32 with the gate/up pair) and all of
//    K. Its NW waves split K; each wave issues the loads of up to STEPS
//    windows at once (its whole slice when K <= NW * STEPS * 128) before
//    consuming any, so there is one memory round trip per wave.
//  * x[0:M, 0:K] is copied once per workgroup into LDS while the weight loads
//    are in flight; the MFMA B operand (x[m][window k]) is read from there.
//  * The NW partial sums are combined through LDS in a fixed order (only the
//    M valid columns), then scale (+ bias) or the gate/up SwiGLU is applied
//    to the fp32 result. No atomics, no workspace, deterministic.
#include "ra_common.h"
#include "ra_internal.h"

namespace ra {

constexpr int kGemvMaxM = 4;
constexpr int kGemvMaxWaves = 8;
constexpr size_t kGemvMaxLdsBytes = 128 * 1024;

template <int DT, int STEPS, int RT, bool GU>
__global__ __launch_bounds__(512) void gemv_kernel(const uint16_t *__restrict__ x, int64_t ldx,
                                                   const int8_t *__restrict__ w, int64_t ldw,
                                                   const float *__restrict__ scale,
                                                   const void *__restrict__ bias, int bias_dt,
                                                   uint16_t *__restrict__ y, int64_t ldy, int M, int N,
                                                   int K) {
  using A = Act<DT>;
  constexpr int NT = GU ? 2 * RT : RT;  // 16-row weight tiles (RT plain / gate, RT up)
  constexpr int NLD = 2 * NT;           // 1 KB loads per 128-byte window
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int nw = blockDim.x >> 6;
  const int kpad = (K + 7) & ~7;
  uint16_t *xs = reinterpret_cast<uint16_t *>(smem);                                  // [M][kpad]
  uint8_t *slots = smem + (((size_t)M * kpad * 2 + 15) & ~(size_t)15);               // [nw][NLD KB]
  float *red = reinterpret_cast<float *>(slots + (size_t)nw * NLD * 1024);            // [nw][NT][M][16]

  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = blockIdx.x * 16 * RT;
  uint8_t *slot = slots + (size_t)wid * NLD * 1024;

  // load instruction i: tile t = i/2 (t < RT plain / gate, t >= RT up),
  // half hh = i%2; lane -> weight row n0 + 16*(t%RT) + 8*hh + lane/8
  // (+N for up), bytes 16*(lane%8)
  const int8_t *wp[NLD];
#pragma unroll
  for (int i = 0; i < NLD; ++i) {
    const int t = i >> 1;
    int n = n0 + 16 * (t % RT) + 8 * (i & 1) + (lane >> 3);
    n = n < N ? n : N - 1;
    if (t >= RT) n += N;
    wp[i] = w + (int64_t)n * ldw + 16 * (lane & 7);
  }
  // Transpose slot of one 16-row tile: row rr (0..15) at 128*rr, its 16-byte
  // chunk c at position c ^ ((rr >> 1) & 7). LDS serves 16 lanes of a 128-bit
  // access per cycle (64 banks): the MFMA-layout read (16 lanes = 16 rows,
  // same chunk) then hits 16 distinct bank groups; the write is 2 rows x 8
  // chunks per 16 lanes, conflict free for any swizzle.
  const int wrow = lane >> 3;  // row within the 8-row half written by this load
  const int w_off0 = wrow * 128 + (((lane & 7) ^ ((wrow >> 1) & 7)) << 4);
  const int w_off1 = (8 + wrow) * 128 + (((lane & 7) ^ (((8 + wrow) >> 1) & 7)) << 4);
  const int r = lane & 15, g = lane >> 4;
  const int r_off0 = r * 128 + (((2 * g) ^ ((r >> 1) & 7)) << 4);
  const int r_off1 = r * 128 + (((2 * g + 1) ^ ((r >> 1) & 7)) << 4);

  const int windows = (K + 127) >> 7;
  const int pass_windows = nw * STEPS;
  const bool mv = r < M;
  const uint16_t *xr = xs + (mv ? r : 0) * kpad + 32 * g;
  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int pass = 0; pass * pass_windows < windows; ++pass) {
    const int win0 = pass * pass_windows + wid * STEPS;
    // 1. all weight loads of this pass, up front (bytes beyond K read as 0)
    uint4 wv[STEPS][NLD];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int k = (win0 + s) * 128;
      const bool ok = k + 16 * (lane & 7) + 16 <= K;
#pragma unroll
      for (int i = 0; i < NLD; ++i)
        wv[s][i] = ok ? *reinterpret_cast<const uint4 *>(wp[i] + k) : make_uint4(0, 0, 0, 0);
    }
    // 2. x -> LDS (first pass only; 16-byte chunks, K % 16 == 0)
    if (pass == 0) {
      const int cpr = K >> 3;
      for (int i = threadIdx.x; i < M * cpr; i += blockDim.x) {
        const int m = i / cpr, c = i - m * cpr;
        *reinterpret_cast<uint4 *>(xs + m * kpad + c * 8) =
            *reinterpret_cast<const uint4 *>(x + (int64_t)m * ldx + c * 8);
      }
      __syncthreads();
    }
    // 3. per window: transpose through the slot, 4 MFMAs per weight tile
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int k = (win0 + s) * 128;
      if (k >= K) break;  // wave-uniform
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        *reinterpret_cast<uint4 *>(slot + t * 2048 + w_off0) = wv[s][2 * t];
        *reinterpret_cast<uint4 *>(slot + t * 2048 + w_off1) = wv[s][2 * t + 1];
      }
      // x[r][k + 32g + 8u .. +7]; zero past K (K % 16 == 0: 8-chunks are all in or all out)
      uint4 xf[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        xf[u] = (mv && k + 32 * g + 8 * u + 8 <= K) ? *reinterpret_cast<const uint4 *>(xr + k + 8 * u)
                                                     : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint4 c0 = *reinterpret_cast<const uint4 *>(slot + t * 2048 + r_off0);
        const uint4 c1 = *reinterpret_cast<const uint4 *>(slot + t * 2048 + r_off1);
        acc[t] = A::mfma16(A::dq8s(c0.x, c0.y), xf[0], acc[t]);
        acc[t] = A::mfma16(A::dq8s(c0.z, c0.w), xf[1], acc[t]);
        acc[t] = A::mfma16(A::dq8s(c1.x, c1.y), xf[2], acc[t]);
        acc[t] = A::mfma16(A::dq8s(c1.z, c1.w), xf[3], acc[t]);
      }
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
  const int o = threadIdx.x;
  if (o < 16 * M) {
    const int m = o >> 4, i = o & 15;
#pragma unroll
    for (int t = 0; t < RT; ++t) {
    const int n = n0 + 16 * t + i;
    if (n < N) {
      float s0 = 0.f, s1 = 0.f;
      for (int v = 0; v < nw; ++v) {
        s0 += red[((v * NT + t) * M + m) * 16 + i];
        if (GU) s1 += red[((v * NT + RT + t) * M + m) * 16 + i];
      }
      uint16_t *yrow = y + (int64_t)m * ldy;
      if (GU)
        yrow[n] = swiglu_out<A>(s0 * scale[n], s1 * scale[N + n]);
      else
        yrow[n] = A::out(epilogue_value(s0, scale, bias, bias_dt, n));
    }
    }
  }
}

// Windows per wave per pass (STEPS) and waves (NW): the smallest STEPS whose
// NW <= 8 covers K in one pass; beyond that, STEPS = 16 (8 with the gate/up
// pair) and several passes. STEPS * loads-per-window <= 32 keeps the
// up-front weight registers at <= 128 VGPRs.
struct GemvCfg {
  int steps, nw;
};

static GemvCfg gemv_config(int64_t K, bool gu) {
  const int64_t windows = (K + 127) / 128;
  const int max_steps = gu ? 8 : 16;
  for (int steps = 4; steps <= max_steps; steps *= 2)
    if ((windows + steps - 1) / steps <= kGemvMaxWaves)
      return GemvCfg{steps, (int)((windows + steps - 1) / steps)};
  return GemvCfg{max_steps, kGemvMaxWaves};
}

static size_t gemv_lds_bytes(int64_t M, int64_t K, int nw, int rt, bool gu) {
  const int nt = (gu ? 2 : 1) * rt;
  const size_t xb = ((size_t)M * ((K + 7) & ~7) * 2 + 15) & ~(size_t)15;
  return xb + (size_t)nw * nt * 2 * 1024 + (size_t)nw * nt * M * 16 * 4;
}

static bool gemv_ok(int x_dt, const void *x, int64_t ldx, const int8_t *w, int64_t ldw, int64_t M, int64_t N,
                    int64_t K, bool gu) {
  if (x_dt != RA_F16 && x_dt != RA_BF16) return false;
  if (M < 1 || M > kGemvMaxM || N > ((int64_t)1 << 30) || K < 16 || K % 16 != 0 || K > ((int64_t)1 << 30))
    return false;
  const GemvCfg c = gemv_config(K, gu);
  if (gemv_lds_bytes(M, K, c.nw, 2, gu) > kGemvMaxLdsBytes) return false;  // fits either RT
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(w) & 15)) return false;
  return (ldx % 8) == 0 && (ldw % 16) == 0;
}

bool gemv_supported(const GemmArgs &a) { return gemv_ok(a.x_dt, a.x, a.ldx, a.w, a.ldw, a.M, a.N, a.K, false); }

bool gateup_gemv_supported(const GateUpArgs &a) {
  return gemv_ok(a.x_dt, a.x, a.ldx, a.w, a.ldw, a.M, a.I, a.K, true);
}

static int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 256;
  return cus;
}

// Workgroups of this kernel that fit on one CU at once (registers, LDS, waves).
template <typename Kern>
static int resident_per_cu(Kern kern, int threads, size_t lds) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void *>(kern), threads, lds) !=
      hipSuccess)
    return 1;
  return n > 0 ? n : 1;
}

template <typename Kern>
static hipError_t set_lds_limit(Kern kern, size_t bytes) {
  // dynamic LDS above 64 KB must be allowed per kernel (gfx950: 160 KB per CU)
  if (bytes <= 64 * 1024) return hipSuccess;
  return hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)kGemvMaxLdsBytes);
}

template <int DT, int STEPS, int RT, bool GU>
static hipError_t gemv_go(const GemvCfg &c, hipStream_t s, const uint16_t *x, int64_t ldx, const int8_t *w,
                          int64_t ldw, const float *scale, const void *bias, int bias_dt, uint16_t *y, int64_t ldy,
                          int M, int N, int K) {
  auto kern = gemv_kernel<DT, STEPS, RT, GU>;
  const size_t lds = gemv_lds_bytes(M, K, c.nw, RT, GU);
  hipError_t e = set_lds_limit(kern, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)((N + 16 * RT - 1) / (16 * RT))), dim3(64 * c.nw), lds, s, x, ldx, w,
                     ldw, scale, bias, bias_dt, y, ldy, M, N, K);
  return hipGetLastError();
}

// Row tiles per workgroup: 1 when every 16-row workgroup fits on the GPU at
// once (one wave of workgroups, no tail), else 2 (half as many workgroups).
template <int DT, int STEPS, bool GU>
static hipError_t gemv_rt(const GemvCfg &c, hipStream_t s, const uint16_t *x, int64_t ldx, const int8_t *w,
                          int64_t ldw, const float *scale, const void *bias, int bias_dt, uint16_t *y, int64_t ldy,
                          int M, int N, int K) {
  // RT = 2 doubles the up-front loads per wave; only instantiated while they
  // stay <= 32 per lane (no spills).
  if constexpr (STEPS * 2 * (GU ? 4 : 2) <= 32) {
    const int wgs1 = (N + 15) / 16;
    const int fit1 =
        resident_per_cu(gemv_kernel<DT, STEPS, 1, GU>, 64 * c.nw, gemv_lds_bytes(M, K, c.nw, 1, GU)) * device_cus();
    if (wgs1 > fit1) return gemv_go<DT, STEPS, 2, GU>(c, s, x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K);
  }
  return gemv_go<DT, STEPS, 1, GU>(c, s, x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K);
}

template <bool GU>
static hipError_t gemv_launch_impl(const void *x, int64_t ldx, int x_dt, const int8_t *w, int64_t ldw,
                                   const float *scale, const void *bias, int bias_dt, void *y, int64_t ldy,
                                   int64_t M, int64_t N, int64_t K, hipStream_t s) {
  const GemvCfg c = gemv_config(K, GU);
  const uint16_t *xp = static_cast<const uint16_t *>(x);
  uint16_t *yp = static_cast<uint16_t *>(y);
  const int Mi = (int)M, Ni = (int)N, Ki = (int)K;
#define RA_GEMV_GO(DT_, ST_) \
  return gemv_rt<DT_, ST_, GU>(c, s, xp, ldx, w, ldw, scale, bias, bias_dt, yp, ldy, Mi, Ni, Ki)
  if (x_dt == RA_F16) {
    if (c.steps == 4) RA_GEMV_GO(RA_F16, 4);
    if (c.steps == 8) RA_GEMV_GO(RA_F16, 8);
    if constexpr (!GU) RA_GEMV_GO(RA_F16, 16);
  } else {
    if (c.steps == 4) RA_GEMV_GO(RA_BF16, 4);
    if (c.steps == 8) RA_GEMV_GO(RA_BF16, 8);
    if constexpr (!GU) RA_GEMV_GO(RA_BF16, 16);
  }
#undef RA_GEMV_GO
  return hipErrorInvalidValue;
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
