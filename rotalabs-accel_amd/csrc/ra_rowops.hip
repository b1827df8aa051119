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

// Workgroup sum, or NaN-propagating maximum (as torch's amax).
template <bool IsMax>
__device__ __forceinline__ float block_reduce(float v, float *smem) {
  v = IsMax ? wave_maximum(v) : wave_sum(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) smem[wid] = v;
  __syncthreads();
  float r = smem[0];
#pragma unroll
  for (int i = 1; i < kRowThreads / 64; ++i) r = IsMax ? nan_max(r, smem[i]) : r + smem[i];
  return r;
}

// Workgroup sum of fp64 values (fixed order).
__device__ __forceinline__ double block_sum_f64(double v, double *smem) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) smem[wid] = v;
  __syncthreads();
  double r = smem[0];
#pragma unroll
  for (int i = 1; i < kRowThreads / 64; ++i) r += smem[i];
  return r;
}

// y = round_y( round_x(v * rsqrt(mean(v^2) + eps)) * w ) with v = x, as
// rmsnorm_torch (src/rotalabs_accel/kernels/normalization.py:43-45): the
// normalised value is stored in x's dtype, then multiplied by the weight in
// the promoted dtype. With a residual r, v = round_s(x + r) in s, the
// promotion of x's and r's dtypes, as rmsnorm_residual_torch (:60-62)
// computes (x + residual) before .float().
// The fp32 squares (exact for 16-bit v) are summed in fp64 and the sum is
// rounded once to fp32: the exactly rounded fp32 sum, whatever the order
// (the reference's fp32 reduction depends on its order; an order-dependent
// last bit of the sum moves rsqrt by an ulp and can flip the 16-bit
// rounding of an element of the row). mean = sum / hidden, + eps and
// rsqrt = 1 / sqrt are fp32 operations, each correctly rounded.
__global__ __launch_bounds__(kRowThreads) void rmsnorm_kernel(const void *__restrict__ x, int64_t ldx,
                                                              int x_dt, const void *__restrict__ r,
                                                              int64_t ldr, int r_dt, int s_dt,
                                                              const void *__restrict__ w,
                                                              int w_dt, void *__restrict__ y,
                                                              int64_t ldy, int y_dt, int hidden,
                                                              float eps) {
  __shared__ double smem[kRowThreads / 64];
  const int64_t row = blockIdx.x;
  auto in = [&](int i) -> float {
    const float v = load_as_f32(x, row * ldx + i, x_dt);
    return r ? round_through(v + load_as_f32(r, row * ldr + i, r_dt), s_dt) : v;
  };
  double ss = 0.0;
  for (int i = threadIdx.x; i < hidden; i += kRowThreads) {
    const float v = in(i);
    ss += (double)fp32_rounded(v * v);
  }
  const float total = (float)block_sum_f64(ss, smem);
  const float rr = 1.0f / sqrtf(total / (float)hidden + eps);
  for (int i = threadIdx.x; i < hidden; i += kRowThreads) {
    const float v = round_through(in(i) * rr, x_dt);
    store_from_f32(y, row * ldy + i, y_dt, v * load_as_f32(w, i, w_dt));
  }
}

// Same arithmetic for x, (r,) w, y of one 16-bit dtype with hidden % 8 == 0:
// every thread loads its VPT 16-byte chunks of the row (and of r and w) at
// once, keeps them in registers for the normalisation, and stores 16-byte
// chunks -- one pass over memory with all loads in flight, instead of a
// latency-bound loop.
template <int DT, int VPT, bool RES>
__global__ __launch_bounds__(kRowThreads) void rmsnorm_vec_kernel(const uint16_t *__restrict__ x, int64_t ldx,
                                                                  const uint16_t *__restrict__ r, int64_t ldr,
                                                                  const uint16_t *__restrict__ w,
                                                                  uint16_t *__restrict__ y, int64_t ldy,
                                                                  int hidden, float eps) {
  using A = Act<DT>;
  __shared__ double smem[kRowThreads / 64];
  const int64_t row = blockIdx.x;
  const int nch = hidden / 8;
  const uint16_t *xr = x + row * ldx;
  uint4 xv[VPT], rv[VPT], wv[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int c = min((int)threadIdx.x + kRowThreads * j, nch - 1);  // clamped: loads stay unconditional
    xv[j] = *reinterpret_cast<const uint4 *>(xr + 8 * c);
    if (RES) rv[j] = *reinterpret_cast<const uint4 *>(r + row * ldr + 8 * c);
    wv[j] = *reinterpret_cast<const uint4 *>(w + 8 * c);
  }
  // v = x (+ r, rounded to the dtype)
  float v[VPT][8];
  double ss = 0.0;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const uint16_t *h = reinterpret_cast<const uint16_t *>(&xv[j]);
    const uint16_t *hr = reinterpret_cast<const uint16_t *>(&rv[j]);
    const bool live = (int)threadIdx.x + kRowThreads * j < nch;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[j][e] = RES ? A::rnd(A::in(h[e]) + A::in(hr[e])) : A::in(h[e]);
      if (live) ss += (double)(v[j][e] * v[j][e]);  // exact: 16-bit values square exactly in fp32
    }
  }
  const float total = (float)block_sum_f64(ss, smem);
  const float rr = 1.0f / sqrtf(total / (float)hidden + eps);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int c = (int)threadIdx.x + kRowThreads * j;
    if (c >= nch) continue;
    const uint16_t *hw = reinterpret_cast<const uint16_t *>(&wv[j]);
    uint4 o;
    uint16_t *ho = reinterpret_cast<uint16_t *>(&o);
#pragma unroll
    for (int e = 0; e < 8; ++e) ho[e] = A::out(A::rnd(v[j][e] * rr) * A::in(hw[e]));
    *reinterpret_cast<uint4 *>(y + row * ldy + 8 * c) = o;
  }
}

template <int DT, bool RES>
static void rmsnorm_vec_launch(const void *x, int64_t ldx, const void *r, int64_t ldr, const void *w, void *y,
                               int64_t ldy, int64_t rows, int hidden, float eps, hipStream_t s) {
  const int nch = hidden / 8;
  const uint16_t *xp = static_cast<const uint16_t *>(x), *rp = static_cast<const uint16_t *>(r),
                 *wp = static_cast<const uint16_t *>(w);
  uint16_t *yp = static_cast<uint16_t *>(y);
  const dim3 grid((unsigned)rows), block(kRowThreads);
  if (nch <= kRowThreads)
    hipLaunchKernelGGL((rmsnorm_vec_kernel<DT, 1, RES>), grid, block, 0, s, xp, ldx, rp, ldr, wp, yp, ldy, hidden, eps);
  else if (nch <= 2 * kRowThreads)
    hipLaunchKernelGGL((rmsnorm_vec_kernel<DT, 2, RES>), grid, block, 0, s, xp, ldx, rp, ldr, wp, yp, ldy, hidden, eps);
  else if (nch <= 4 * kRowThreads)
    hipLaunchKernelGGL((rmsnorm_vec_kernel<DT, 4, RES>), grid, block, 0, s, xp, ldx, rp, ldr, wp, yp, ldy, hidden, eps);
  else
    hipLaunchKernelGGL((rmsnorm_vec_kernel<DT, 8, RES>), grid, block, 0, s, xp, ldx, rp, ldr, wp, yp, ldy, hidden, eps);
}

hipError_t rmsnorm_launch(const void *x, int64_t ldx, int x_dt, const void *r, int64_t ldr, int r_dt,
                          const void *w, int w_dt, void *y, int64_t ldy, int y_dt, int64_t rows, int64_t hidden,
                          float eps, hipStream_t s) {
  const bool vec = (x_dt == RA_F16 || x_dt == RA_BF16) && w_dt == x_dt && y_dt == x_dt && (!r || r_dt == x_dt) &&
                   hidden % 8 == 0 && hidden >= 8 && hidden <= 8 * 8 * kRowThreads && ldx % 8 == 0 &&
                   ldy % 8 == 0 && (!r || ldr % 8 == 0) &&
                   ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(r) |
                     reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(y)) & 15) == 0;
  if (vec) {
    if (x_dt == RA_F16) {
      if (r) rmsnorm_vec_launch<RA_F16, true>(x, ldx, r, ldr, w, y, ldy, rows, (int)hidden, eps, s);
      else rmsnorm_vec_launch<RA_F16, false>(x, ldx, r, ldr, w, y, ldy, rows, (int)hidden, eps, s);
    } else {
      if (r) rmsnorm_vec_launch<RA_BF16, true>(x, ldx, r, ldr, w, y, ldy, rows, (int)hidden, eps, s);
      else rmsnorm_vec_launch<RA_BF16, false>(x, ldx, r, ldr, w, y, ldy, rows, (int)hidden, eps, s);
    }
    return hipGetLastError();
  }
  const int s_dt = !r ? x_dt : (x_dt == r_dt ? x_dt : RA_F32);  // dtype of x + r
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(kRowThreads), 0, s, x, ldx, x_dt, r, ldr, r_dt,
                     s_dt, w, w_dt, y, ldy, y_dt, (int)hidden, eps);
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

// out = silu(g + bg) * (u + bu) in fp32, one rounding, bias index i % hidden
// (the arithmetic of swiglu_with_bias's Triton kernel,
// src/rotalabs_accel/kernels/swiglu.py:201-218).
__global__ __launch_bounds__(256) void swiglu_bias_kernel(const void *__restrict__ g, const void *__restrict__ u,
                                                          const void *__restrict__ bg, const void *__restrict__ bu,
                                                          int b_dt, void *__restrict__ o, int64_t n, int64_t hidden,
                                                          int dt) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t c = i % hidden;
    const float gv = load_as_f32(g, i, dt) + load_as_f32(bg, c, b_dt);
    const float uv = load_as_f32(u, i, dt) + load_as_f32(bu, c, b_dt);
    store_from_f32(o, i, dt, gv / (1.0f + expf(-gv)) * uv);
  }
}

hipError_t swiglu_bias_launch(const void *g, const void *u, const void *bg, const void *bu, int b_dt, void *o,
                              int64_t n, int64_t hidden, int dt, hipStream_t s) {
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(swiglu_bias_kernel, dim3((unsigned)blocks), dim3(256), 0, s, g, u, bg, bu, b_dt, o, n, hidden,
                     dt);
  return hipGetLastError();
}

// Per-row symmetric quantisation, the op sequence of quantize_symmetric(dim=1)
// (src/rotalabs_accel/quantization/symmetric.py:66-80) on the CPU:
//   s = round_w(amax / 127)   IEEE division (built without fast-math)
//   s = 1 if s == 0
//   q = int8(clamp(rint(round_w(w / s)), -128, 127))   rint: half to even
// round_w is the rounding to the weight dtype (identity for fp32). amax
// propagates NaN (torch's amax) and a NaN quotient converts to 0, as the CPU
// conversion does.
__global__ __launch_bounds__(kRowThreads) void quantize_kernel(const void *__restrict__ w, int64_t ldw,
                                                               int w_dt, int K, int8_t *__restrict__ q,
                                                               int64_t ldq, float *__restrict__ scale) {
  __shared__ float smem[kRowThreads / 64];
  const int64_t row = blockIdx.x;
  float amax = 0.f;
  for (int i = threadIdx.x; i < K; i += kRowThreads)
    amax = nan_max(amax, fabsf(load_as_f32(w, row * ldw + i, w_dt)));
  amax = block_reduce<true>(amax, smem);
  float s = round_through(amax / 127.0f, w_dt);
  if (s == 0.0f) s = 1.0f;
  for (int i = threadIdx.x; i < K; i += kRowThreads) {
    const float v = rintf(round_through(load_as_f32(w, row * ldw + i, w_dt) / s, w_dt));
    q[row * ldq + i] = v != v ? (int8_t)0 : (int8_t)(int)fminf(fmaxf(v, -128.0f), 127.0f);
  }
  if (threadIdx.x == 0) scale[row] = s;
}

hipError_t quantize_launch(const void *w, int64_t ldw, int w_dt, int64_t N, int64_t K, int8_t *q,
                           int64_t ldq, float *scale, hipStream_t s) {
  hipLaunchKernelGGL(quantize_kernel, dim3((unsigned)N), dim3(kRowThreads), 0, s, w, ldw, w_dt, (int)K, q,
                     ldq, scale);
  return hipGetLastError();
}

// Per-row symmetric quantisation of a KV-cache tensor, as QuantizedTensor
// (src/rotalabs_accel/speculative/kv_compression.py:51-78, per_channel) on
// the CPU, with every intermediate in the tensor's dtype t:
//   s = round_t(max(round_t(amax / qmax), 1e-8))      qmax = 2^(bits-1) - 1
//   q = int8(clamp(rint(round_t(x / s)), -qmax-1, qmax)), NaN -> 0
// (fp16 rounds the 1e-8 floor to 0, so an all-zero row gives 0/0 = NaN, which
// the CPU's float -> int8 conversion turns into 0). The scale is stored in t.
__global__ __launch_bounds__(kRowThreads) void quantize_rows_kernel(const void *__restrict__ t, int64_t ldt,
                                                                    int t_dt, int cols, int qmax,
                                                                    int8_t *__restrict__ q, int64_t ldq,
                                                                    void *__restrict__ scale) {
  __shared__ float smem[kRowThreads / 64];
  const int64_t row = blockIdx.x;
  float amax = 0.f;
  for (int i = threadIdx.x; i < cols; i += kRowThreads)
    amax = nan_max(amax, fabsf(load_as_f32(t, row * ldt + i, t_dt)));
  amax = block_reduce<true>(amax, smem);
  const float s = round_through(nan_max(round_through(amax / (float)qmax, t_dt), 1e-8f), t_dt);
  for (int i = threadIdx.x; i < cols; i += kRowThreads) {
    const float v = round_through(load_as_f32(t, row * ldt + i, t_dt) / s, t_dt);
    const float r = rintf(v);
    q[row * ldq + i] = r != r ? (int8_t)0 : (int8_t)(int)fminf(fmaxf(r, (float)(-qmax - 1)), (float)qmax);
  }
  if (threadIdx.x == 0) store_from_f32(scale, row, t_dt, s);
}

// Same arithmetic for short 16-bit rows (cols % 8 == 0, cols <= 512, 16-byte
// aligned rows; e.g. head_dim-wide KV rows): L = cols / 8 lanes per row
// (rounded up to a power of two), 64 / L rows per wave, each lane one 16-byte
// chunk of 8 values (4 rows' chunks loaded at once), the row maximum by lane
// shuffles within the group, 8-byte stores of the 8 quantised values -- no
// per-row workgroup.
template <int DT, int L>
__global__ __launch_bounds__(256) void quantize_rows_short_kernel(const uint16_t *__restrict__ t, int64_t ldt,
                                                                  int64_t rows, int cols, int qmax,
                                                                  int8_t *__restrict__ q, int64_t ldq,
                                                                  uint16_t *__restrict__ scale) {
  using A = Act<DT>;
  constexpr int U = 4;                       // rows per lane group, loads in flight together
  constexpr int RPW = 64 / L;                // rows per wave and pass
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int c = lane % L;                    // 16-byte chunk of this lane
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + wid) * (RPW * U) + lane / L;
  const int cc = 8 * c < cols ? c : 0;       // clamped: loads stay unconditional
  const float qf = (float)qmax, rq = 1.0f / qf, qlo = -qf - 1.0f, qhi = qf;
  uint4 v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    int64_t rr = row0 + (int64_t)u * RPW;
    rr = rr < rows ? rr : rows - 1;
    v[u] = load_stream16(t + rr * ldt + 8 * cc);  // read once: non-temporal (72 -> 66 us on 256 MiB)
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t row = row0 + (int64_t)u * RPW;
    const bool live = row < rows && 8 * c < cols;
    const uint16_t *h = reinterpret_cast<const uint16_t *>(&v[u]);
    float x[8], amax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] = A::in(h[e]);
      amax = nan_max(amax, fabsf(x[e]));  // NaN propagates, as torch's amax
    }
    if (!live) amax = 0.f;
#pragma unroll
    for (int off = L / 2; off >= 1; off >>= 1) amax = nan_max(amax, __shfl_xor(amax, off, 64));
    // amax / qmax by the same correction (exact for every finite 16-bit amax
    // and qmax = 127 or 7, checked exhaustively; inf and NaN pass through)
    const float d0 = amax * rq;
    const float d = __builtin_isfinite(d0) ? __builtin_fmaf(__builtin_fmaf(-d0, qf, amax), rq, d0) : d0;
    const float sc = A::rnd(nan_max(A::rnd(fp32_rounded(d)), 1e-8f));
    if (!live) continue;
    // x / sc correctly rounded to fp32 without a division per element:
    // Markstein's correction of x * RN(1/sc) by one residual FMA. For every
    // 16-bit x and 16-bit sc >= 1e-8 with |x / sc| <= 256 (the codec's range:
    // |x| <= amax, sc ~ amax / qmax) it rounds to the same 16-bit value as the
    // IEEE quotient (checked exhaustively on the CPU, both formats). A zero
    // scale (fp16 rounds the 1e-8 floor to 0) or an infinite one (a row
    // holding inf) keeps the plain product x * (1 / sc): +-inf / NaN for
    // x / 0, 0 / NaN for x / inf, as the quotient.
    const float rinv = 1.0f / sc;
    uint32_t lo = 0, hi = 0;
    if (sc != 0.0f && __builtin_isfinite(sc)) {
      // Finite, nonzero scale: every element is finite (a NaN or inf element
      // makes amax, hence sc, NaN or inf), so the clamped integers plus 128
      // lie in [0, 255]; convert and pack them four at a time, then flip the
      // sign bits.
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float q0 = x[e] * rinv;
        const float q1 = __builtin_fmaf(__builtin_fmaf(-q0, sc, x[e]), rinv, q0);
        // (the rounded value goes through a register again: otherwise the
        // compiler re-rounds the integral rint result to 16 bits)
        const float r = rintf(fp32_rounded(A::rnd(fp32_rounded(q1))));
        const float b = __builtin_amdgcn_fmed3f(r, qlo, qhi) + 128.0f;
        if (e < 4) lo = __builtin_amdgcn_cvt_pk_u8_f32(b, e, lo);
        else hi = __builtin_amdgcn_cvt_pk_u8_f32(b, e - 4, hi);
      }
      lo ^= 0x80808080u;
      hi ^= 0x80808080u;
    } else {
      // Zero scale (fp16 rounds the 1e-8 floor to 0), infinite or NaN: the
      // plain product x * (1 / sc) is the quotient's +-inf / NaN / 0; NaN
      // converts to 0.
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float r = rintf(A::rnd(fp32_rounded(x[e] * rinv)));
        const int qi = r != r ? 0 : (int)__builtin_amdgcn_fmed3f(r, qlo, qhi);
        const uint32_t b = (uint32_t)(uint8_t)(int8_t)qi;
        if (e < 4) lo |= b << (8 * e);
        else hi |= b << (8 * (e - 4));
      }
    }
    store8(q + row * ldq + 8 * c, lo, hi);
    if (c == 0) scale[row] = A::out(sc);
  }
}

template <int DT>
static void quantize_rows_short_launch(const void *t, int64_t ldt, int64_t rows, int cols, int qmax, int8_t *q,
                                       int64_t ldq, void *scale, hipStream_t s) {
  const uint16_t *tp = static_cast<const uint16_t *>(t);
  uint16_t *sp = static_cast<uint16_t *>(scale);
  const int need = cols / 8;
#define RA_QROWS(L_)                                                                                \
  if (need <= L_) {                                                                                 \
    const int64_t blocks = (rows + 4 * 4 * (64 / L_) - 1) / (4 * 4 * (64 / L_));                  \
    hipLaunchKernelGGL((quantize_rows_short_kernel<DT, L_>), dim3((unsigned)blocks), dim3(256), 0, s, tp, ldt, \
                       rows, cols, qmax, q, ldq, sp);                                               \
    return;                                                                                         \
  }
  RA_QROWS(1) RA_QROWS(2) RA_QROWS(4) RA_QROWS(8) RA_QROWS(16) RA_QROWS(32) RA_QROWS(64)
#undef RA_QROWS
}

hipError_t quantize_rows_launch(const void *t, int64_t ldt, int t_dt, int64_t rows, int64_t cols, int bits,
                                int8_t *q, int64_t ldq, void *scale, hipStream_t s) {
  const int qmax = (1 << (bits - 1)) - 1;
  const bool short_rows = (t_dt == RA_F16 || t_dt == RA_BF16) && cols % 8 == 0 && cols <= 512 && ldt % 8 == 0 &&
                          ldq % 8 == 0 && !(reinterpret_cast<uintptr_t>(t) & 15) &&
                          !(reinterpret_cast<uintptr_t>(q) & 7) && rows * 64 < ((int64_t)1 << 31);
  if (short_rows) {
    if (t_dt == RA_F16) quantize_rows_short_launch<RA_F16>(t, ldt, rows, (int)cols, qmax, q, ldq, scale, s);
    else quantize_rows_short_launch<RA_BF16>(t, ldt, rows, (int)cols, qmax, q, ldq, scale, s);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(quantize_rows_kernel, dim3((unsigned)rows), dim3(kRowThreads), 0, s, t, ldt, t_dt, (int)cols,
                     qmax, q, ldq, scale);
  return hipGetLastError();
}

}  // namespace ra
