// Row GEMV for decode (M <= 2) on gfx950: one weight row per wave, VALU dot
// products, no LDS, no barriers.
//
// Replaces the reference's Triton tile loop (src/rotalabs_accel/kernels/
// gemm.py:113-138) for the decode shapes, where the whole cost is streaming
// N*K weight bytes from HBM. Measured on MI355X, a CU sustains only a bounded
// number of outstanding 128-byte line requests, so the kernel time is set by
// the bytes assigned to the busiest CU: the work must be split into many
// small, equal, independent units that the hardware dispatcher balances
// across CUs as they finish. Here the unit is one weight row per wave:
//
//  * Lane l reads bytes 16l .. 16l+15 of each 1 KB window of its row (one
//    128-bit load per window, the whole wave reading 1 KB contiguous = 8 full
//    128-byte lines); CH windows are loaded at once, with the matching
//    activation chunks x[m][k .. k+15] (two 128-bit loads, L2 resident).
//  * int8 -> fp16 is exact (magic-number conversion) and the products are
//    accumulated with v_dot2_f32_f16 (two fp16 products per instruction, fp32
//    accumulator); bf16 converts through fp32 (exact) and uses
//    v_dot2_f32_bf16. Per weight: 1.75 VALU ops (fp16), 2 (bf16).
//  * A wave64 reduction gives the row's dot product; scale (+ bias), or the
//    SwiGLU of the gate/up pair, is applied to the fp32 sum before the single
//    rounding. Deterministic; no workspace.
#include "ra_common.h"
#include "ra_internal.h"

namespace ra {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kRowsMaxM = 2;
constexpr int kRowsCh = 4;  // windows of 1 KB in flight per wave

// sum += dot(x[0..15], q[0..15]) for 16 weights packed in w (4 dwords) and 16
// activations in xa (elements 0..7) and xb (8..15).
template <int DT>
__device__ __forceinline__ float dot16(const uint4 &w, const uint4 &xa, const uint4 &xb, float sum);

template <>
__device__ __forceinline__ float dot16<RA_F16>(const uint4 &w, const uint4 &xa, const uint4 &xb, float sum) {
  const uint4 lo = dq8_f16_cvt(w.x, w.y), hi = dq8_f16_cvt(w.z, w.w);
  sum = __builtin_amdgcn_fdot2(bitcast<f16x2>(lo.x), bitcast<f16x2>(xa.x), sum, false);
  sum = __builtin_amdgcn_fdot2(bitcast<f16x2>(lo.y), bitcast<f16x2>(xa.y), sum, false);
  sum = __builtin_amdgcn_fdot2(bitcast<f16x2>(lo.z), bitcast<f16x2>(xa.z), sum, false);
  sum = __builtin_amdgcn_fdot2(bitcast<f16x2>(lo.w), bitcast<f16x2>(xa.w), sum, false);
  sum = __builtin_amdgcn_fdot2(bitcast<f16x2>(hi.x), bitcast<f16x2>(xb.x), sum, false);
  sum = __builtin_amdgcn_fdot2(bitcast<f16x2>(hi.y), bitcast<f16x2>(xb.y), sum, false);
  sum = __builtin_amdgcn_fdot2(bitcast<f16x2>(hi.z), bitcast<f16x2>(xb.z), sum, false);
  sum = __builtin_amdgcn_fdot2(bitcast<f16x2>(hi.w), bitcast<f16x2>(xb.w), sum, false);
  return sum;
}

template <>
__device__ __forceinline__ float dot16<RA_BF16>(const uint4 &w, const uint4 &xa, const uint4 &xb, float sum) {
  const uint4 lo = dq8_bf16(w.x, w.y), hi = dq8_bf16(w.z, w.w);
  sum = __builtin_amdgcn_fdot2_f32_bf16(bitcast<bf16x2>(lo.x), bitcast<bf16x2>(xa.x), sum, false);
  sum = __builtin_amdgcn_fdot2_f32_bf16(bitcast<bf16x2>(lo.y), bitcast<bf16x2>(xa.y), sum, false);
  sum = __builtin_amdgcn_fdot2_f32_bf16(bitcast<bf16x2>(lo.z), bitcast<bf16x2>(xa.z), sum, false);
  sum = __builtin_amdgcn_fdot2_f32_bf16(bitcast<bf16x2>(lo.w), bitcast<bf16x2>(xa.w), sum, false);
  sum = __builtin_amdgcn_fdot2_f32_bf16(bitcast<bf16x2>(hi.x), bitcast<bf16x2>(xb.x), sum, false);
  sum = __builtin_amdgcn_fdot2_f32_bf16(bitcast<bf16x2>(hi.y), bitcast<bf16x2>(xb.y), sum, false);
  sum = __builtin_amdgcn_fdot2_f32_bf16(bitcast<bf16x2>(hi.z), bitcast<bf16x2>(xb.z), sum, false);
  sum = __builtin_amdgcn_fdot2_f32_bf16(bitcast<bf16x2>(hi.w), bitcast<bf16x2>(xb.w), sum, false);
  return sum;
}

// One wave per RW consecutive output rows n0 .. n0+RW-1 (with GU: gate rows n
// and up rows N + n). The RW rows are loaded together and share the wave's
// activation loads, which are L2 hits but cost the CU as many line requests
// as the weight loads themselves.
template <int DT, int MR, int RW, bool GU>
__global__ __launch_bounds__(256) void gemv_rows_kernel(const uint16_t *__restrict__ x, int64_t ldx,
                                                        const int8_t *__restrict__ w, int64_t ldw,
                                                        const float *__restrict__ scale,
                                                        const void *__restrict__ bias, int bias_dt,
                                                        uint16_t *__restrict__ y, int64_t ldy, int M, int N,
                                                        int K) {
  using A = Act<DT>;
  constexpr int NR = GU ? 2 * RW : RW;  // weight rows per wave: [r] gate/plain, [RW + r] up
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * RW;
  if (n0 >= N) return;  // whole wave; no barriers in this kernel
  // Rows past N (last wave only) are clamped to N - 1: in bounds, never stored.
  const int8_t *wr[NR];
#pragma unroll
  for (int t = 0; t < NR; ++t) {
    const int n = min(n0 + t % RW, N - 1);
    wr[t] = w + (int64_t)(t < RW ? n : N + n) * ldw + 16 * lane;
  }
  const uint16_t *xr[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) xr[m] = x + (int64_t)(m < M ? m : 0) * ldx + 16 * lane;
  // Epilogue operands are loaded up front, in flight with the weights (a load
  // after the reduction would add a memory round trip to every wave).
  // The bias is kept as raw bits until the end so that no conversion (and no
  // wait) sits in front of the weight loads.
  float sc[RW], su[RW];
  uint32_t bb[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int n = min(n0 + r, N - 1);
    sc[r] = __uint_as_float(vload_b32(scale + n));
    su[r] = GU ? __uint_as_float(vload_b32(scale + N + n)) : 0.f;
    bb[r] = 0;
    if (!GU && bias) {
      if (bias_dt == RA_F32) bb[r] = vload_b32(static_cast<const uint32_t *>(bias) + n);
      else bb[r] = vload_b16(static_cast<const uint16_t *>(bias) + n);
    }
  }

  float acc[NR][MR];
#pragma unroll
  for (int t = 0; t < NR; ++t)
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[t][m] = 0.f;

  // Main loop: kRowsCh whole windows, unconditional 128-bit loads (a guarded
  // load would be split into per-dword loads, each waited on). x rows m >= M
  // alias row 0 and their sums are never stored.
  int k0 = 0;
  for (; k0 + 1024 * kRowsCh <= K; k0 += 1024 * kRowsCh) {
    uint4 wv[kRowsCh][NR], xa[kRowsCh][MR], xb[kRowsCh][MR];
#pragma unroll
    for (int c = 0; c < kRowsCh; ++c)
#pragma unroll
      for (int t = 0; t < NR; ++t) wv[c][t] = load_stream16(wr[t] + k0 + 1024 * c);
#pragma unroll
    for (int c = 0; c < kRowsCh; ++c)
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        xa[c][m] = *reinterpret_cast<const uint4 *>(xr[m] + k0 + 1024 * c);
        xb[c][m] = *reinterpret_cast<const uint4 *>(xr[m] + k0 + 1024 * c + 8);
      }
    __builtin_amdgcn_sched_barrier(0);  // every load of the step is issued before the first wait
#pragma unroll
    for (int c = 0; c < kRowsCh; ++c)
#pragma unroll
      for (int t = 0; t < NR; ++t)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[t][m] = dot16<DT>(wv[c][t], xa[c][m], xb[c][m], acc[t][m]);
  }
  // Tail (fewer than kRowsCh windows left): one step of kRowsCh windows whose
  // loads are all issued before the first use, as in the main loop. K % 16
  // == 0, so a lane's 16-byte chunk is all in or all out; chunks past K
  // re-read the first 16 elements of their rows (offset -16*lane from the
  // lane's own column; K >= 16) and contribute zeros.
  if (k0 < K) {
    uint4 wv[kRowsCh][NR], xa[kRowsCh][MR], xb[kRowsCh][MR];
    bool ok[kRowsCh];
#pragma unroll
    for (int c = 0; c < kRowsCh; ++c) {
      ok[c] = k0 + 1024 * c + 16 * lane + 16 <= K;
      const int k = ok[c] ? k0 + 1024 * c : -16 * lane;
#pragma unroll
      for (int t = 0; t < NR; ++t) wv[c][t] = load_stream16(wr[t] + k);
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        xa[c][m] = *reinterpret_cast<const uint4 *>(xr[m] + k);
        xb[c][m] = *reinterpret_cast<const uint4 *>(xr[m] + k + 8);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the step is issued before the first wait
    const uint4 z = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int c = 0; c < kRowsCh; ++c)
#pragma unroll
      for (int t = 0; t < NR; ++t)
#pragma unroll
        for (int m = 0; m < MR; ++m)
          acc[t][m] = dot16<DT>(ok[c] ? wv[c][t] : z, ok[c] ? xa[c][m] : z, ok[c] ? xb[c][m] : z, acc[t][m]);
  }

  // Reduce over the wave (DPP); lane r stores row n0 + r. Same arithmetic as
  // epilogue_value: acc * scale, + bias only when there is one.
#pragma unroll
  for (int m = 0; m < MR; ++m) {
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const float s0 = wave_sum_dpp(acc[r][m]);
      const float s1 = GU ? wave_sum_dpp(acc[NR - RW + r][m]) : 0.f;
      const int n = n0 + r;
      if (lane == r && m < M && n < N) {
        uint16_t *yrow = y + (int64_t)m * ldy;
        if (GU) {
          yrow[n] = swiglu_out<A>(s0 * sc[r], s1 * su[r]);
        } else {
          float v = s0 * sc[r];
          if (bias)
            v += bias_dt == RA_F32 ? __uint_as_float(bb[r])
                                   : (bias_dt == RA_F16 ? f16_to_f32((uint16_t)bb[r]) : bf16_to_f32((uint16_t)bb[r]));
          yrow[n] = A::out(v);
        }
      }
    }
  }
}

// M = 1 with x staged once per workgroup in LDS: the four waves of a
// workgroup copy x[0:K] into LDS with direct-to-LDS loads (issued before
// their first weight loads), wait for those copies only, meet at a barrier,
// and read their activation chunks from LDS. The L2 line requests of x --
// as many per wave as its weight requests at two rows per wave, and charged
// to the same per-CU budget of outstanding lines -- drop fourfold. The weight
// streaming, the per-wave rows and the epilogue are those of
// gemv_rows_kernel.
constexpr int kRowsLdsMaxK = 32768;  // at most 64 KB of LDS per workgroup (2K bytes, dynamic)

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

template <int DT, int RW, bool GU, int WPG>
__global__ __launch_bounds__(64 * WPG) void gemv_rows_lds_kernel(const uint16_t *__restrict__ x,
                                                            const int8_t *w, int64_t ldw,  // (not restrict: the
                                                            // first loads must stay in front of the copy wait)
                                                            const float *__restrict__ scale,
                                                            const void *__restrict__ bias, int bias_dt,
                                                            int N, int K,  // (ahead of y: preloaded)
                                                            uint16_t *__restrict__ y) {
  using A = Act<DT>;
  constexpr int NR = GU ? 2 * RW : RW;
  constexpr int WLOADS = kRowsCh * NR;  // weight loads of the first step
  extern __shared__ __attribute__((aligned(16))) uint16_t xl[];  // K elements
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = (blockIdx.x * WPG + wid) * RW;
  // Waves past N (last workgroup only) copy, meet the barrier and compute on
  // clamped rows like the others, and store nothing.
  const int8_t *wr[NR];
#pragma unroll
  for (int t = 0; t < NR; ++t) {
    const int n = min(n0 + t % RW, N - 1);
    wr[t] = w + (int64_t)(t < RW ? n : N + n) * ldw + 16 * lane;
  }
  // Epilogue operands first (older than the copies, so the copy wait covers them).
  float sc[RW], su[RW];
  uint32_t bb[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int n = min(n0 + r, N - 1);
    sc[r] = __uint_as_float(vload_b32(scale + n));
    su[r] = GU ? __uint_as_float(vload_b32(scale + N + n)) : 0.f;
    bb[r] = 0;
    if (!GU && bias) {
      if (bias_dt == RA_F32) bb[r] = vload_b32(static_cast<const uint32_t *>(bias) + n);
      else bb[r] = vload_b16(static_cast<const uint16_t *>(bias) + n);
    }
  }
  // x -> LDS: 1 KB chunks, chunk j by wave j % WPG, lane -> bytes 16 lane of
  // the chunk (M0 = the chunk's LDS address; the copy writes M0 + 16 lane).
  const int xbytes = 2 * K;  // K % 16 == 0: whole 16-byte pieces
  const uint32_t lds0 = lds_addr(xl);
  for (int j = wid; 1024 * j < xbytes; j += WPG) {
    const int off = 1024 * j + 16 * lane;
    if (off < xbytes)
      asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds0 + 1024 * j),
                   "v"(reinterpret_cast<const char *>(x) + off)
                   : "memory", "m0");
  }
  float acc[NR];
#pragma unroll
  for (int t = 0; t < NR; ++t) acc[t] = 0.f;
  // First step's weights (K >= 1024 * kRowsCh is required by the host; rows
  // of inactive waves are clamped to N - 1: in bounds, never used).
  const int full = K / (1024 * kRowsCh);  // whole steps of kRowsCh windows, >= 1
  uint4 wv[kRowsCh][NR];
#pragma unroll
  for (int c = 0; c < kRowsCh; ++c)
#pragma unroll
    for (int t = 0; t < NR; ++t) wv[c][t] = load_stream16(wr[t] + 1024 * c);
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(WLOADS) : "memory");  // this wave's copies have landed
  asm volatile("s_barrier" ::: "memory");                         // every wave's copies have landed
  // Nothing that uses the first step's weights may move in front of the
  // barrier (it would bring the wait for them along).
  __builtin_amdgcn_sched_barrier(0);

  const uint16_t *xr = xl + 16 * lane;
  for (int step = 0; step < full; ++step) {
    const int k0 = 1024 * kRowsCh * step;
    if (step > 0) {
#pragma unroll
      for (int c = 0; c < kRowsCh; ++c)
#pragma unroll
        for (int t = 0; t < NR; ++t) wv[c][t] = load_stream16(wr[t] + k0 + 1024 * c);
    }
    // Window by window, each as soon as its weights are in: the compiler
    // would otherwise wait for all of them first, putting every window's dot
    // products behind the step's last load.
#pragma unroll
    for (int c = 0; c < kRowsCh; ++c) {
      const uint4 xa = *reinterpret_cast<const uint4 *>(xr + k0 + 1024 * c);
      const uint4 xb = *reinterpret_cast<const uint4 *>(xr + k0 + 1024 * c + 8);
#pragma unroll
      for (int t = 0; t < NR; ++t) acc[t] = dot16<DT>(wv[c][t], xa, xb, acc[t]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // Tail (fewer than kRowsCh windows left): one step with all its weight
  // loads issued before the first use; chunks past K read the row's first
  // 16 weights and x[0..15] (in bounds) and contribute zeros.
  const int kt = 1024 * kRowsCh * full;
  if (kt < K) {
    uint4 wt[kRowsCh][NR];
    bool ok[kRowsCh];
    int kk[kRowsCh];
#pragma unroll
    for (int c = 0; c < kRowsCh; ++c) {
      ok[c] = kt + 1024 * c + 16 * lane + 16 <= K;
      kk[c] = ok[c] ? kt + 1024 * c : -16 * lane;
#pragma unroll
      for (int t = 0; t < NR; ++t) wt[c][t] = load_stream16(wr[t] + kk[c]);
    }
    const uint4 z = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int c = 0; c < kRowsCh; ++c) {
      const uint4 xa = *reinterpret_cast<const uint4 *>(xr + kk[c]);
      const uint4 xb = *reinterpret_cast<const uint4 *>(xr + kk[c] + 8);
#pragma unroll
      for (int t = 0; t < NR; ++t) acc[t] = dot16<DT>(ok[c] ? wt[c][t] : z, ok[c] ? xa : z, ok[c] ? xb : z, acc[t]);
    }
  }
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const float s0 = wave_sum_dpp(acc[r]);
    const float s1 = GU ? wave_sum_dpp(acc[NR - RW + r]) : 0.f;
    const int n = n0 + r;
    if (lane == r && n < N) {
      if (GU) {
        y[n] = swiglu_out<A>(s0 * sc[r], s1 * su[r]);
      } else {
        float v = s0 * sc[r];
        if (bias)
          v += bias_dt == RA_F32 ? __uint_as_float(bb[r])
                                 : (bias_dt == RA_F16 ? f16_to_f32((uint16_t)bb[r]) : bf16_to_f32((uint16_t)bb[r]));
        y[n] = A::out(v);
      }
    }
  }
}

// M = 1 with one weight row per wave (with the gate/up pair, its gate and up
// rows) and 4096 < K <= 1024 * CH: the wave issues the loads of its whole row
// at once -- CH windows of 1 KB -- instead of stepping through it four
// windows at a time, so every byte of the launch is in flight from the start
// (K=11008 N=4096: three dependent steps before). x is staged in LDS per
// workgroup as in gemv_rows_lds_kernel, rounded up to whole windows with
// zeros: lanes past K read their row's first 16 weights (in bounds, finite)
// against zero activations, so no lane needs a mask and the kernel has no
// divergent branch (masked selects cost registers the resident waves need).
template <int DT, bool GU, int WPG, int CH>
__global__ __launch_bounds__(64 * WPG) void gemv_row1_kernel(const uint16_t *__restrict__ x,
                                                        const int8_t *w, int64_t ldw,  // (not restrict: the
                                                        // loads must stay in front of the copy wait)
                                                        const float *__restrict__ scale,
                                                        const void *__restrict__ bias, int bias_dt,
                                                        int N, int K,  // (ahead of y: preloaded)
                                                        uint16_t *__restrict__ y) {
  using A = Act<DT>;
  constexpr int NR = GU ? 2 : 1;
  constexpr int WLOADS = CH * NR;  // weight loads of the wave
  extern __shared__ __attribute__((aligned(16))) uint16_t xl[];  // 1024 * nwin elements
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = blockIdx.x * WPG + wid;
  const int nc = min(n, N - 1);  // waves past N load row N - 1 and store nothing
  const int nwin = (K + 1023) >> 10;  // windows holding k < K (<= CH)
  const int8_t *wr[NR];
#pragma unroll
  for (int t = 0; t < NR; ++t) wr[t] = w + (int64_t)(t ? N + nc : nc) * ldw + 16 * lane;
  // Epilogue operands first (older than the copies, so the copy wait covers them).
  const float sc = __uint_as_float(vload_b32(scale + nc));
  const float su = GU ? __uint_as_float(vload_b32(scale + N + nc)) : 0.f;
  uint32_t bb = 0;
  if (!GU && bias)
    bb = bias_dt == RA_F32 ? vload_b32(static_cast<const uint32_t *>(bias) + nc)
                           : vload_b16(static_cast<const uint16_t *>(bias) + nc);
  // x -> LDS: 1 KB chunks, chunk j by wave j % WPG (as gemv_rows_lds_kernel);
  // elements K .. 1024 nwin - 1 are zeroed (K % 16 == 0: whole 32-byte pieces).
  const int xbytes = 2 * K;
  const uint32_t lds0 = lds_addr(xl);
  for (int j = wid; 1024 * j < xbytes; j += WPG) {
    const int off = 1024 * j + 16 * lane;
    if (off < xbytes)
      asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds0 + 1024 * j),
                   "v"(reinterpret_cast<const char *>(x) + off)
                   : "memory", "m0");
  }
  for (int p = (K >> 4) + (int)threadIdx.x; p < 64 * nwin; p += 64 * WPG) {
    uint4 *q = reinterpret_cast<uint4 *>(xl + 16 * p);
    q[0] = make_uint4(0, 0, 0, 0);
    q[1] = make_uint4(0, 0, 0, 0);
  }
  // The whole row: window c holds k = 1024 c + 16 lane .. +15. Lanes whose
  // piece starts at or past K read the row's first 16 weights instead.
  uint4 wv[CH][NR];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int kk = 1024 * c + 16 * lane < K ? 1024 * c : -16 * lane;
#pragma unroll
    for (int t = 0; t < NR; ++t) wv[c][t] = load_stream16(wr[t] + kk);
  }
  // This wave's copies have landed (the weight loads are younger), its zero
  // stores are done, then every wave's are.
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(WLOADS) : "memory");
  // Nothing that uses the weights may move in front of the barrier (it would
  // bring the wait for them along).
  __builtin_amdgcn_sched_barrier(0);
  const uint16_t *xr = xl + 16 * lane;
  float acc[NR];
#pragma unroll
  for (int t = 0; t < NR; ++t) acc[t] = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    if (c < nwin) {  // wave-uniform
      const uint4 xa = *reinterpret_cast<const uint4 *>(xr + 1024 * c);
      const uint4 xb = *reinterpret_cast<const uint4 *>(xr + 1024 * c + 8);
#pragma unroll
      for (int t = 0; t < NR; ++t) acc[t] = dot16<DT>(wv[c][t], xa, xb, acc[t]);
    }
    // Window by window: hoisting every window's x reads to the barrier would
    // hold 8 more registers per window.
    __builtin_amdgcn_sched_barrier(0);
  }
  const float s0 = wave_sum_dpp(acc[0]);
  const float s1 = GU ? wave_sum_dpp(acc[NR - 1]) : 0.f;
  if (lane == 0 && n < N) {
    if (GU) {
      y[n] = swiglu_out<A>(s0 * sc, s1 * su);
    } else {
      float v = s0 * sc;
      if (bias)
        v += bias_dt == RA_F32 ? __uint_as_float(bb)
                               : (bias_dt == RA_F16 ? f16_to_f32((uint16_t)bb) : bf16_to_f32((uint16_t)bb));
      y[n] = A::out(v);
    }
  }
}

// Short-K variant (K <= 4096, one step): a wave handles RP consecutive rows
// one after another, loading row r+1 while it reduces row r, so the wave's
// 4 KB of weight loads stay in flight during the dot products; x[0:M, 0:K] is
// loaded once per wave and kept in registers for all RP rows.
template <int DT, int MR, int RP, bool GU>
__global__ __launch_bounds__(256) void gemv_rows_pipe_kernel(const uint16_t *__restrict__ x, int64_t ldx,
                                                             const int8_t *__restrict__ w, int64_t ldw,
                                                             const float *__restrict__ scale,
                                                             const void *__restrict__ bias, int bias_dt,
                                                             uint16_t *__restrict__ y, int64_t ldy, int M,
                                                             int N, int K) {
  using A = Act<DT>;
  constexpr int NT = GU ? 2 : 1;  // weight rows per output row: gate (and up)
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * RP;
  if (n0 >= N) return;  // whole wave; no barriers in this kernel
  // Window c covers k = 1024c + 16*lane .. +15; lanes past K re-read the first
  // 16 elements of the row (offset 0 from the row start; K >= 16) and
  // contribute zeros.
  int off[kRowsCh];
  bool ok[kRowsCh];
#pragma unroll
  for (int c = 0; c < kRowsCh; ++c) {
    ok[c] = 1024 * c + 16 * lane + 16 <= K;
    off[c] = ok[c] ? 1024 * c + 16 * lane : 0;
  }
  uint4 wv[2][kRowsCh][NT];
  auto load_row = [&](int r, uint4(&dst)[kRowsCh][NT]) {
    const int n = min(n0 + r, N - 1);  // rows past N: in bounds, never stored
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int8_t *row = w + (int64_t)(t ? N + n : n) * ldw;
#pragma unroll
      for (int c = 0; c < kRowsCh; ++c) dst[c][t] = load_stream16(row + off[c]);
    }
  };
  load_row(0, wv[0]);
  uint4 xa[kRowsCh][MR], xb[kRowsCh][MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const uint16_t *xrow = x + (int64_t)(m < M ? m : 0) * ldx;  // rows m >= M alias row 0, never stored
#pragma unroll
    for (int c = 0; c < kRowsCh; ++c) {
      xa[c][m] = *reinterpret_cast<const uint4 *>(xrow + off[c]);
      xb[c][m] = *reinterpret_cast<const uint4 *>(xrow + off[c] + 8);
    }
  }
  float sc[RP], su[RP];
  uint32_t bb[RP];
#pragma unroll
  for (int r = 0; r < RP; ++r) {
    const int n = min(n0 + r, N - 1);
    sc[r] = __uint_as_float(vload_b32(scale + n));
    su[r] = GU ? __uint_as_float(vload_b32(scale + N + n)) : 0.f;
    bb[r] = 0;
    if (!GU && bias) {
      if (bias_dt == RA_F32) bb[r] = vload_b32(static_cast<const uint32_t *>(bias) + n);
      else bb[r] = vload_b16(static_cast<const uint16_t *>(bias) + n);
    }
  }
  // Operands of windows past K are replaced by zeros at use (selects into new
  // registers: overwriting a register with a load in flight would wait).
  const uint4 z = make_uint4(0, 0, 0, 0);

#pragma unroll
  for (int r = 0; r < RP; ++r) {
    if (r + 1 < RP) load_row(r + 1, wv[(r + 1) & 1]);
    __builtin_amdgcn_sched_barrier(0);  // next row's loads go out before this row's wait
    float acc[NT][MR];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int m = 0; m < MR; ++m) acc[t][m] = 0.f;
#pragma unroll
    for (int c = 0; c < kRowsCh; ++c)
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint4 wc = ok[c] ? wv[r & 1][c][t] : z;
#pragma unroll
        for (int m = 0; m < MR; ++m)
          acc[t][m] = dot16<DT>(wc, ok[c] ? xa[c][m] : z, ok[c] ? xb[c][m] : z, acc[t][m]);
      }
    const int n = n0 + r;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float s0 = wave_sum_dpp(acc[0][m]);
      const float s1 = GU ? wave_sum_dpp(acc[NT - 1][m]) : 0.f;
      if (lane == 0 && m < M && n < N) {
        uint16_t *yrow = y + (int64_t)m * ldy;
        if (GU) {
          yrow[n] = swiglu_out<A>(s0 * sc[r], s1 * su[r]);
        } else {
          float v = s0 * sc[r];
          if (bias)
            v += bias_dt == RA_F32 ? __uint_as_float(bb[r])
                                   : (bias_dt == RA_F16 ? f16_to_f32((uint16_t)bb[r]) : bf16_to_f32((uint16_t)bb[r]));
          yrow[n] = A::out(v);
        }
      }
    }
  }
}

static bool rows_ok(int x_dt, const void *x, int64_t ldx, const int8_t *w, int64_t ldw, int64_t M, int64_t N,
                    int64_t K) {
  if (x_dt != RA_F16 && x_dt != RA_BF16) return false;
  if (M < 1 || M > kRowsMaxM || N > ((int64_t)1 << 30) || K < 16 || K % 16 != 0 || K > ((int64_t)1 << 30))
    return false;
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(w) & 15)) return false;
  return (ldx % 8) == 0 && (ldw % 16) == 0;
}

bool gemv_rows_supported(const GemmArgs &a) { return rows_ok(a.x_dt, a.x, a.ldx, a.w, a.ldw, a.M, a.N, a.K); }

bool gateup_gemv_rows_supported(const GateUpArgs &a) {
  return rows_ok(a.x_dt, a.x, a.ldx, a.w, a.ldw, a.M, a.I, a.K);
}

// Rows per wave: as many as keep >= kRowsMinWaves waves in the grid (the
// dispatcher balances CUs only with many small units), at most 4.
constexpr int kRowsMinWaves = 4096;

static int rows_per_wave(int64_t M, int64_t N, bool gu) {
  const int cap = (gu || M > 1) ? 2 : 4;
  int rw = cap;
  while (rw > 1 && N / rw < kRowsMinWaves) rw >>= 1;
#ifdef RA_TUNING
  extern int g_rows_rw;  // 0 auto, else forced rows per wave (capped)
  if (g_rows_rw > 0) rw = g_rows_rw < cap ? g_rows_rw : cap;
#endif
  return rw;
}

struct RowsParams {
  const uint16_t *x;
  int64_t ldx;
  const int8_t *w;
  int64_t ldw;
  const float *scale;
  const void *bias;
  int bias_dt;
  uint16_t *y;
  int64_t ldy;
  int M, N, K;
};

template <int DT, int MR, int RW, bool GU>
static void rows_go(const RowsParams &p, hipStream_t s) {
  const int64_t waves = ((int64_t)p.N + RW - 1) / RW;
  hipLaunchKernelGGL((gemv_rows_kernel<DT, MR, RW, GU>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, p.x,
                     p.ldx, p.w, p.ldw, p.scale, p.bias, p.bias_dt, p.y, p.ldy, p.M, p.N, p.K);
}

template <int DT, int RW, bool GU>
static void rows_lds_go(const RowsParams &p, hipStream_t s) {
  const int64_t waves = ((int64_t)p.N + RW - 1) / RW;
  // Waves per workgroup (sharing one copy of x): 8 up to N = 8192 (K=14336
  // N=4096 12.1 -> 11.4 us, K=28672 N=8192 37.2 -> 36.4), 4 above (K=4096
  // N=11008 8.40 vs 8.54 with 8, K=8192 N=57344 65.3 vs 68.5).
  int wpg = p.N <= 8192 ? 8 : 4;
#ifdef RA_TUNING
  extern int g_rows_lds;  // > 0: waves per workgroup
  if (g_rows_lds == 4 || g_rows_lds == 8 || g_rows_lds == 16) wpg = g_rows_lds;
#endif
#define RA_LDS_GO(WPG_)                                                                                       \
  hipLaunchKernelGGL((gemv_rows_lds_kernel<DT, RW, GU, WPG_>), dim3((unsigned)((waves + WPG_ - 1) / WPG_)),  \
                     dim3(64 * WPG_), (size_t)2 * p.K, s, p.x, p.w, p.ldw, p.scale, p.bias, p.bias_dt, p.N, p.K, \
                     p.y)
  if (wpg == 16) RA_LDS_GO(16);
  else if (wpg == 8) RA_LDS_GO(8);
  else RA_LDS_GO(4);
#undef RA_LDS_GO
}

// Windows per wave of gemv_row1_kernel for this K (0: not used): rows of
// 4096 < K <= 16384 (8192 with the gate/up pair, two rows per wave).
static int row1_windows(int64_t K, bool gu) {
  if (K <= 4096 || K > (gu ? 8192 : 16384)) return 0;
  const int64_t win = (K + 1023) / 1024;
  return win <= 8 ? 8 : (win <= 12 ? 12 : 16);
}

template <int DT, bool GU, int CH>
static void row1_go(const RowsParams &p, hipStream_t s) {
  // 4 waves per workgroup at every N (same run, against 8 up to N = 8192:
  // K=11008 N=4096 9.08 vs 9.30 us, K=14336 N=4096 11.1 vs 11.3, K=8192
  // N=8192 11.6 vs 11.8, K=5120 N=5120 6.10 vs 6.35; 16: 6-15 % slower).
  int wpg = 4;
#ifdef RA_TUNING
  extern int g_rows_lds;  // > 0: waves per workgroup
  if (g_rows_lds == 4 || g_rows_lds == 8 || g_rows_lds == 16) wpg = g_rows_lds;
#endif
#define RA_ROW1_GO(WPG_)                                                                                     \
  hipLaunchKernelGGL((gemv_row1_kernel<DT, GU, WPG_, CH>), dim3((unsigned)((p.N + WPG_ - 1) / WPG_)),       \
                     dim3(64 * WPG_), (size_t)2048 * ((p.K + 1023) / 1024), s, p.x, p.w, p.ldw, p.scale, p.bias, p.bias_dt, p.N, p.K, \
                     p.y)
#ifdef RA_TUNING
  if (wpg == 16) { RA_ROW1_GO(16); return; }
#endif
  if (wpg == 8) RA_ROW1_GO(8);
  else RA_ROW1_GO(4);
#undef RA_ROW1_GO
}

template <int DT, int MR, bool GU>
static void rows_go_rw(const RowsParams &p, int rw, hipStream_t s) {
  if constexpr (MR == 1) {
    const int ch = row1_windows(p.K, GU);
    if (ch == 8) return row1_go<DT, GU, 8>(p, s);
    if constexpr (!GU) {
      if (ch == 12) return row1_go<DT, GU, 12>(p, s);
      if (ch == 16) return row1_go<DT, GU, 16>(p, s);
    }
    // x in LDS when it fits (one copy per workgroup instead of per wave) and
    // the first step is whole
    bool lds = p.K <= kRowsLdsMaxK && p.K >= 1024 * kRowsCh;
#ifdef RA_TUNING
    extern int g_rows_lds;  // 0 auto, -1 off
    if (g_rows_lds == -1) lds = false;
#endif
    if (lds) {
      // With x in LDS one row per wave streams fastest up to K = 16384
      // (K=4096 N=11008: 9.2 us vs 9.7 with two rows, 10.2 with four); longer
      // rows keep the count above.
      int r = p.K <= 16384 ? 1 : rw;
#ifdef RA_TUNING
      extern int g_rows_rw;
      if (g_rows_rw > 0) r = rw;
#endif
      if constexpr (!GU) {
        if (r == 4) return rows_lds_go<DT, 4, GU>(p, s);
      }
      if (r >= 2) return rows_lds_go<DT, 2, GU>(p, s);
      return rows_lds_go<DT, 1, GU>(p, s);
    }
  }
  if constexpr (MR == 1 && !GU) {
    if (rw == 4) return rows_go<DT, MR, 4, GU>(p, s);
  }
  if (rw >= 2) return rows_go<DT, MR, 2, GU>(p, s);
  rows_go<DT, MR, 1, GU>(p, s);
}

// Rows per wave of the short-K variant (used for M == 2, where a wave's dot
// products take long enough to be worth overlapping with the next row's
// loads; at M == 1 it measured the same as one row per wave): up to 4 rows
// while >= 2048 waves remain.
static int rows_pipe_rows(int64_t M, int64_t N, int64_t K, bool gu) {
  int rp = 0;
  if (M == 2 && K <= 1024 * kRowsCh) {
    rp = 4;
    while (rp > 1 && N / rp < 2048) rp >>= 1;
  }
#ifdef RA_TUNING
  extern int g_rows_pipe;  // 0 auto, -1 off, else forced rows per wave
  if (g_rows_pipe == -1) rp = 0;
  else if (g_rows_pipe > 0 && K <= 1024 * kRowsCh) rp = g_rows_pipe;
#endif
  return rp;
}

template <int DT, int MR, bool GU>
static void rows_pipe_go(const RowsParams &p, int rp, hipStream_t s) {
  const int64_t waves = ((int64_t)p.N + rp - 1) / rp;
  const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
#define RA_PIPE(RP_)                                                                                      \
  hipLaunchKernelGGL((gemv_rows_pipe_kernel<DT, MR, RP_, GU>), grid, block, 0, s, p.x, p.ldx, p.w, p.ldw, \
                     p.scale, p.bias, p.bias_dt, p.y, p.ldy, p.M, p.N, p.K)
  if (rp >= 4) RA_PIPE(4);
  else if (rp == 3) RA_PIPE(3);
  else if (rp == 2) RA_PIPE(2);
  else RA_PIPE(1);
#undef RA_PIPE
}

template <bool GU>
static hipError_t rows_launch(const void *x, int64_t ldx, int x_dt, const int8_t *w, int64_t ldw,
                              const float *scale, const void *bias, int bias_dt, void *y, int64_t ldy, int64_t M,
                              int64_t N, int64_t K, hipStream_t s) {
  const RowsParams p{static_cast<const uint16_t *>(x), ldx, w, ldw, scale, bias, bias_dt,
                     static_cast<uint16_t *>(y), ldy, (int)M, (int)N, (int)K};
  const int rp = rows_pipe_rows(M, N, K, GU);
  if (rp > 0) {
    if (x_dt == RA_F16) {
      if (M == 1) rows_pipe_go<RA_F16, 1, GU>(p, rp, s);
      else rows_pipe_go<RA_F16, 2, GU>(p, rp, s);
    } else {
      if (M == 1) rows_pipe_go<RA_BF16, 1, GU>(p, rp, s);
      else rows_pipe_go<RA_BF16, 2, GU>(p, rp, s);
    }
    return hipGetLastError();
  }
  const int rw = rows_per_wave(M, N, GU);
  if (x_dt == RA_F16) {
    if (M == 1) rows_go_rw<RA_F16, 1, GU>(p, rw, s);
    else rows_go_rw<RA_F16, 2, GU>(p, rw, s);
  } else {
    if (M == 1) rows_go_rw<RA_BF16, 1, GU>(p, rw, s);
    else rows_go_rw<RA_BF16, 2, GU>(p, rw, s);
  }
  return hipGetLastError();
}

hipError_t gemv_rows_launch(const GemmArgs &a, hipStream_t s) {
  return rows_launch<false>(a.x, a.ldx, a.x_dt, a.w, a.ldw, a.scale, a.bias, a.bias_dt, a.y, a.ldy, a.M, a.N, a.K,
                            s);
}

hipError_t gateup_gemv_rows_launch(const GateUpArgs &a, hipStream_t s) {
  return rows_launch<true>(a.x, a.ldx, a.x_dt, a.w, a.ldw, a.scale, nullptr, RA_F32, a.h, a.ldh, a.M, a.I, a.K,
                           s);
}

}  // namespace ra
