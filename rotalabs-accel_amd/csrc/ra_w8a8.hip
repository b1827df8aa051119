// W8A8 GEMM on the int8 matrix cores of gfx950 (opt-in path):
//   y[m,n] = ((float)sum_k xq[m,k] * w[n,k] * xs[m]) * s[n] (+ bias[n])
// with xq, xs the per-row dynamically quantised activations.
//
// Replaces the reference's W8A8 route of int8_gemm(..., use_cublas=True)
// (src/rotalabs_accel/kernels/quantized_matmul.py:441-447 -> _int8_gemm_cublas
// :43-102: per-row absmax activation quantisation :85-87, torch._int_mm :93,
// dequantisation :99-100; its fused Triton variant :162-264 dequantises in
// fp32 as done here). The int32 sums are exact; the reference's
// _dequantize_output converts them to fp16 before scaling, which overflows
// once |sum| > 65504 (K = 4096 reaches that for typical data), so the scaling
// here is the fused kernel's: fp32 (acc * xs) * s, one rounding.
//
// Kernels:
//  * quantize_act_kernel: one workgroup per activation row, the reference's
//    ops in the activation dtype t, each rounded to t as torch does:
//      a = max(amax, round_t(1e-5)); xs = round_t(a / c);
//      mult = round_t(round_t(1 / a) * c)   (torch evaluates c / a so)
//    with c = act_scale (127 by default), an fp32 value
//      xq = int8(clamp(rint(round_t(x * mult)), -128, 127)), NaN -> 0
//  * w8a8_gemm_kernel: the direct-to-LDS pipeline of the W8A16 prefill kernel
//    with both operands int8 in LDS (128-byte rows = 128 k per K tile, 8 rows
//    per 1 KB copy, 16-byte chunks XOR-swizzled by (row>>1)&7) and
//    v_mfma_i32_32x32x32_i8 (32 k per MFMA, twice the fp16 rate): no
//    dequantisation, int32 accumulators in AGPRs.
//  * w8a8_generic_kernel: any K (one output per thread); slow, correct.
#include <algorithm>
#include <type_traits>

#include "ra_common.h"
#include "ra_internal.h"

namespace ra {

#ifdef RA_TUNING
extern int g_w8a8_mode;  // 0 auto; i forces configuration kCfgs[i - 1]
#endif

namespace w8a8 {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kRowThreads = 256;

template <int DT>
__global__ __launch_bounds__(kRowThreads) void quantize_act_kernel(const uint16_t *__restrict__ x, int64_t ldx,
                                                                   int K, int8_t *__restrict__ q, int64_t ldq,
                                                                   uint16_t *__restrict__ xs, float c) {
  using A = Act<DT>;
  __shared__ float smem[kRowThreads / 64];
  const int64_t row = blockIdx.x;
  const uint16_t *xr = x + row * ldx;
  float amax = 0.f;  // NaN propagates, as torch's amax
  for (int i = threadIdx.x; i < K; i += kRowThreads) amax = nan_max(amax, fabsf(A::in(xr[i])));
  amax = wave_maximum(amax);
  if ((threadIdx.x & 63) == 0) smem[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = nan_max(nan_max(smem[0], smem[1]), nan_max(smem[2], smem[3]));
  // clamp(min=1e-5) compares against the bound rounded to the tensor dtype
  // (and keeps NaN); c / a is torch's reciprocal(a) * c, each rounded.
  const float a = nan_max(amax, A::rnd(1e-5f));
  const float mult = A::rnd(A::rnd(1.0f / a) * c);
  for (int i = threadIdx.x; i < K; i += kRowThreads) {
    const float r = rintf(A::rnd(A::in(xr[i]) * mult));
    q[row * ldq + i] = r != r ? (int8_t)0 : (int8_t)(int)fminf(fmaxf(r, -128.0f), 127.0f);
  }
  if (threadIdx.x == 0) xs[row] = A::out(A::rnd(a / c));
}

// The same for rows of K % 8 == 0, K <= 2048 * NC elements, 16-byte aligned:
// each thread keeps NC chunks of 8 elements in registers (one 16-byte load
// each), so the row is read once; 8-byte stores of the int8 values.
template <int DT, int NC>
__global__ __launch_bounds__(kRowThreads) void quantize_act_vec_kernel(const uint16_t *__restrict__ x, int64_t ldx,
                                                                       int K, int8_t *__restrict__ q, int64_t ldq,
                                                                       uint16_t *__restrict__ xs, float c) {
  using A = Act<DT>;
  __shared__ float smem[kRowThreads / 64];
  const int64_t row = blockIdx.x;
  const uint4 *xr = reinterpret_cast<const uint4 *>(x + row * ldx);
  const int chunks = K >> 3;
  uint4 v[NC];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = threadIdx.x + j * kRowThreads;
    v[j] = c < chunks ? xr[c] : uint4{0, 0, 0, 0};
    const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
    for (int h = 0; h < 8; ++h) {
      amax = nan_max(amax, fabsf(A::in((uint16_t)(w[h >> 1] >> (16 * (h & 1))))));
    }
  }
  amax = wave_maximum(amax);
  if ((threadIdx.x & 63) == 0) smem[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = nan_max(nan_max(smem[0], smem[1]), nan_max(smem[2], smem[3]));
  const float a = nan_max(amax, A::rnd(1e-5f));
  const float mult = A::rnd(A::rnd(1.0f / a) * c);
  int8_t *qr = q + row * ldq;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = threadIdx.x + j * kRowThreads;
    if (c >= chunks) break;
    const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
    uint32_t packed[2] = {0, 0};
#pragma unroll
    for (int h = 0; h < 8; ++h) {
      const float r = rintf(A::rnd(A::in((uint16_t)(w[h >> 1] >> (16 * (h & 1)))) * mult));
      const int qi = r != r ? 0 : (int)fminf(fmaxf(r, -128.0f), 127.0f);
      packed[h >> 2] |= (uint32_t)(qi & 0xFF) << (8 * (h & 3));
    }
    store8(qr + 8 * c, packed[0], packed[1]);
  }
  if (threadIdx.x == 0) xs[row] = A::out(A::rnd(a / c));
}

// One output per thread, exact int32 sums; any K and layout.
template <int DT>
__global__ __launch_bounds__(256) void w8a8_generic_kernel(const int8_t *__restrict__ xq, int64_t ldxq,
                                                           const uint16_t *__restrict__ xs,
                                                           const int8_t *__restrict__ w, int64_t ldw,
                                                           const float *__restrict__ scale,
                                                           const void *__restrict__ bias, int bias_dt,
                                                           uint16_t *__restrict__ y, int64_t ldy, int M, int N,
                                                           int K) {
#pragma clang fp contract(off)
  using A = Act<DT>;
  const int n = blockIdx.x * 256 + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N) return;
  int acc = 0;
  for (int k = 0; k < K; ++k) acc += (int)xq[(int64_t)m * ldxq + k] * (int)w[(int64_t)n * ldw + k];
  float v = ((float)acc * A::in(xs[m])) * scale[n];
  if (bias) v += load_as_f32(bias, n, bias_dt);
  y[(int64_t)m * ldy + n] = A::out(fp32_rounded(v));
}

// Tile of BM x BN outputs over 2 x 2 waves; K tiles of BK int8 (BK-byte LDS
// rows of 16-byte chunks). With 64 LDS banks (256 bytes), P = 256 / BK rows
// share a bank window, so chunk c of row r sits at position c ^ ((r / P) % CPR):
// the 16 lanes a ds_read_b128 serves per cycle (16 consecutive rows, one
// chunk each) then hit 64 distinct banks.
template <int BMB, int BNB, int BK_, int OCC_>
struct Tile {
  static constexpr int WM = 32 * BMB, WN = 32 * BNB;  // per-wave sub-tile
  static constexpr int BM = 2 * WM, BN = 2 * WN, BK = BK_;
  static constexpr int CPR = BK / 16, RPC = 64 / CPR, P = 256 / BK;  // chunks per row, rows per 1 KB copy
  static constexpr int NSUB = BK / 32;                                // k32 MFMA steps per K tile
  static constexpr int A_BYTES = BM * BK, B_BYTES = BN * BK;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int A_COPIES = A_BYTES / 4096, B_COPIES = B_BYTES / 4096;  // 1 KB copies per wave
  static constexpr int COPIES = A_COPIES + B_COPIES;
  static constexpr int OCC = OCC_;  // workgroups per CU (they share the 160 KB of LDS)
  static constexpr int S = (160 * 1024 / OCC) / STAGE < 6 ? (160 * 1024 / OCC) / STAGE : 6;
  static_assert(BK == 64 || BK == 128, "K tile");
  static_assert(A_BYTES % 4096 == 0 && B_BYTES % 4096 == 0, "copies must split evenly over 4 waves");
  static_assert(S >= 2 && (S - 1) * COPIES <= 63, "pipeline depth");
};

template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Wait until at most `younger` (<= MAXY) K tiles' copies (COPIES each) are
// in flight.
template <int COPIES, int MAXY, int Y = MAXY>
__device__ __forceinline__ void wait_tiles(int younger) {
  if constexpr (Y == 0) {
    wait_vm<0>();
  } else {
    if (younger >= Y) wait_vm<Y * COPIES>();
    else wait_tiles<COPIES, MAXY, Y - 1>(younger);
  }
}

__device__ __forceinline__ uint32_t lds_off(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// 16 bytes per lane from SGPR base + 32-bit lane offset + OFS to LDS at
// M0 + OFS + 16 * lane (OFS applies to both sides); M0 written first when
// NEW_M0 (one wait state before the copy reads it).
template <int OFS, bool NEW_M0>
__device__ __forceinline__ void copy16(const void *sbase, uint32_t voff, uint32_t m0v) {
  if (NEW_M0)
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 offset:%3" ::"s"(m0v), "v"(voff),
                 "s"(sbase), "n"(OFS)
                 : "memory", "m0");
  else
    asm volatile("global_load_lds_dwordx4 %0, %1 offset:%2" ::"v"(voff), "s"(sbase), "n"(OFS) : "memory");
}

constexpr int COPY_BIAS = 3072;
constexpr uint64_t COPY_SPAN = (uint64_t)0x7FFFFFFF - 2 * COPY_BIAS;  // per-lane offsets stay below 2^31

// Lane (l32, g) holds, for block (bi, bj), column l32 of rows
// 32*bi + r(e) + 4g, r(e) = (e & 3) + 8 * (e >> 2). The lane's activation
// scales are loaded into registers before any store (y may alias nothing, but
// the compiler cannot know that), the bias test and the row guard (only tiles
// that reach past M need it) are hoisted out of the store loops, and addresses
// are a uniform base plus 32-bit per-lane offsets (BM * ldy < 2^31 is checked
// on the host).
template <int DT, int BMB, int BNB>
__device__ __forceinline__ void epilogue(const i32x16 (&acc)[BMB][BNB], const uint16_t *__restrict__ xs,
                                         const float *__restrict__ scale, const void *__restrict__ bias,
                                         int bias_dt, uint16_t *__restrict__ y, int64_t ldy, int M, int N,
                                         int row0, int g, int col_w, int l32) {
#pragma clang fp contract(off)
  using Ac = Act<DT>;
  const int row_l = row0 + 4 * g;
  const int rows_left = M - row_l;  // rows r < rows_left are in range
  float xsv[BMB][16];
#pragma unroll
  for (int bi = 0; bi < BMB; ++bi)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int r = bi * 32 + (e & 3) + 8 * (e >> 2);
      xsv[bi][e] = Ac::in(xs[min(row_l + r, M - 1)]);
    }
  uint16_t *const yw = y + (int64_t)row0 * ldy + col_w;
  const uint32_t ldy32 = (uint32_t)ldy;
  const uint32_t lane_off = 4u * (uint32_t)g * ldy32 + (uint32_t)l32;
  auto store_blocks = [&](auto guard_c, auto bias_c) __attribute__((always_inline)) {
#pragma clang fp contract(off)  // (a lambda body does not inherit the pragma)
    constexpr bool GUARD = decltype(guard_c)::value, HAS_BIAS = decltype(bias_c)::value;
#pragma unroll
    for (int bj = 0; bj < BNB; ++bj) {
      const int n = col_w + bj * 32 + l32;
      if (n >= N) continue;
      const float sn = scale[n];
      const float bn = HAS_BIAS ? load_as_f32(bias, n, bias_dt) : 0.f;
#pragma unroll
      for (int bi = 0; bi < BMB; ++bi)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = bi * 32 + (e & 3) + 8 * (e >> 2);
          if (!GUARD || r < rows_left) {
            float v = ((float)acc[bi][bj][e] * xsv[bi][e]) * sn;
            if (HAS_BIAS) v += bn;
            // non-temporal: written once, not read back by this launch
            // (M=2048 K=4096 N=11008: 91.2 -> 89.8 us, same-box A/B)
            __builtin_nontemporal_store((uint16_t)Ac::out(fp32_rounded(v)),
                                        &yw[lane_off + (uint32_t)r * ldy32 + 32u * bj]);
          }
        }
    }
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  const bool guard = rows_left < 32 * BMB - 4;  // some row r <= 32 * BMB - 5 of this lane is past M
  if (bias) {
    if (guard) store_blocks(T_{}, T_{});
    else store_blocks(F_{}, T_{});
  } else {
    if (guard) store_blocks(T_{}, F_{});
    else store_blocks(F_{}, F_{});
  }
}

template <int DT, int BMB, int BNB, int BK_, int OCC_>
__global__ __launch_bounds__(256, OCC_) void w8a8_gemm_kernel(const int8_t *__restrict__ xq, int64_t ldxq,
                                                           const uint16_t *__restrict__ xs,
                                                           const int8_t *__restrict__ w, int64_t ldw,
                                                           const float *__restrict__ scale,
                                                           const void *__restrict__ bias, int bias_dt,
                                                           uint16_t *__restrict__ y, int64_t ldy, int M, int N,
                                                           int K, int tiles_m, int tiles_n) {
  using G = Tile<BMB, BNB, BK_, OCC_>;
  constexpr int BM = G::BM, BN = G::BN, BK = G::BK, WM = G::WM, WN = G::WN, S = G::S;
  constexpr int CPR = G::CPR, RPC = G::RPC, P = G::P, NSUB = G::NSUB;
  constexpr int A_COPIES = G::A_COPIES, B_COPIES = G::B_COPIES, COPIES = G::COPIES;
  constexpr int STAGE = G::STAGE, A_BYTES = G::A_BYTES;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[S * STAGE];

  // ---- tile coordinates (XCD-aware, grouped along M), as the W8A16 kernel
  const int T = tiles_m * tiles_n;
  const int b = blockIdx.x;
  const int xcd = b & 7, idx = b >> 3;
  const int per = T >> 3, rem = T & 7;
  const int t = xcd * per + (xcd < rem ? xcd : rem) + idx;
  constexpr int GM = 8;
  const int span = GM * tiles_n;
  const int first_m = (t / span) * GM;
  const int gm = min(tiles_m - first_m, GM);
  const int m0 = (first_m + (t % span) % gm) * BM, n0 = ((t % span) / gm) * BN;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wid >> 1, wn = wid & 1;
  const int l32 = lane & 31, g = lane >> 5;

  // ---- copy sources: copy i of an operand covers tile rows RPC*(COPIES_OF_OPERAND*wid + i) ..
  // + RPC-1, lane -> row + lane/CPR, LDS chunk lane%CPR <- global chunk (lane%CPR) ^ ((row/P)%CPR);
  // rows past M / N are clamped (loaded, never stored). Per-lane byte offsets from the bases
  // moved down by COPY_BIAS (the instruction offset of copy i is (i%4) KB).
  uint32_t a_voff[A_COPIES], b_voff[B_COPIES];
#pragma unroll
  for (int i = 0; i < A_COPIES; ++i) {
    const int row = RPC * (A_COPIES * wid + i) + lane / CPR;
    const int c = (lane % CPR) ^ ((row / P) % CPR);
    const int gr = min(m0 + row, M - 1);
    a_voff[i] = (uint32_t)((int64_t)gr * ldxq + c * 16) + (uint32_t)(COPY_BIAS - (i % 4) * 1024);
  }
#pragma unroll
  for (int i = 0; i < B_COPIES; ++i) {
    const int row = RPC * (B_COPIES * wid + i) + lane / CPR;
    const int c = (lane % CPR) ^ ((row / P) % CPR);
    const int gr = min(n0 + row, N - 1);
    b_voff[i] = (uint32_t)((int64_t)gr * ldw + c * 16) + (uint32_t)(COPY_BIAS - (i % 4) * 1024);
  }
  const char *const ab = reinterpret_cast<const char *>(xq) - COPY_BIAS;
  const char *const bb = reinterpret_cast<const char *>(w) - COPY_BIAS;
  const uint32_t lds0 = lds_off(lds);
  const uint32_t a_dst = lds0 + (uint32_t)(A_COPIES * wid) * 1024;
  const uint32_t b_dst = lds0 + A_BYTES + (uint32_t)(B_COPIES * wid) * 1024;

// Copies [LO_, HI_) of K tile kt_ into stage st_ (A copies first, then B).
#define RW_ISSUE_PART(kt_, st_, LO_, HI_)                                                           \
  {                                                                                                 \
    const char *sa_ = ab + (int64_t)(kt_) * BK;                                                     \
    const char *sb_ = bb + (int64_t)(kt_) * BK;                                                     \
    const uint32_t so_ = (uint32_t)(st_) * STAGE;                                                   \
    static_for_int<LO_, HI_>([&](auto ic_) {                                                        \
      constexpr int i = decltype(ic_)::value;                                                       \
      constexpr bool isA = i < A_COPIES;                                                            \
      constexpr int li = isA ? i : i - A_COPIES;                                                    \
      constexpr bool fresh = i == (LO_) || i == A_COPIES || li % 4 == 0;                            \
      const uint32_t m0v = (isA ? a_dst : b_dst) + so_ + (uint32_t)(li / 4) * 4096;                 \
      if constexpr (isA)                                                                            \
        copy16<(li % 4) * 1024, fresh>(sa_, a_voff[li], m0v);                                       \
      else                                                                                          \
        copy16<(li % 4) * 1024, fresh>(sb_, b_voff[li], m0v);                                       \
    });                                                                                             \
  }

  i32x16 acc[BMB][BNB];
#pragma unroll
  for (int i = 0; i < BMB; ++i)
#pragma unroll
    for (int j = 0; j < BNB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

  // Fragment rows: A row wm*WM + 32*bi + l32, B row wn*WN + 32*bj + l32 (both
  // swizzles reduce to (l32/P)%CPR). Sub-step ss (0..NSUB-1) of a K tile is the
  // k32 block ss: lane group g supplies chunk 2ss+g of both operands.
  const int a_row_off = (wm * WM + l32) * BK;
  const int b_row_off = A_BYTES + (wn * WN + l32) * BK;
  const int sw = (l32 / P) % CPR;
  i32x4 fa[2][BMB], fb[2][BNB];
  auto read = [&](int st, int ss, i32x4 (&FA)[BMB], i32x4 (&FB)[BNB]) __attribute__((always_inline)) {
    const uint8_t *base = lds + st * STAGE;
    const int ch = ((2 * ss + g) ^ sw) << 4;
#pragma unroll
    for (int bi = 0; bi < BMB; ++bi)
      FA[bi] = *reinterpret_cast<const i32x4 *>(base + a_row_off + bi * 32 * BK + ch);
#pragma unroll
    for (int bj = 0; bj < BNB; ++bj)
      FB[bj] = *reinterpret_cast<const i32x4 *>(base + b_row_off + bj * 32 * BK + ch);
  };
  auto mma = [&](const i32x4 (&FA)[BMB], const i32x4 (&FB)[BNB]) __attribute__((always_inline)) {
#pragma unroll
    for (int bi = 0; bi < BMB; ++bi)
#pragma unroll
      for (int bj = 0; bj < BNB; ++bj)
        acc[bi][bj] = __builtin_amdgcn_mfma_i32_32x32x32_i8(FA[bi], FB[bj], acc[bi][bj], 0, 0, 0);
  };
  // One LDS read after each of the first BMB+BNB MFMAs of a sub-step.
  auto interleave = [&]() __attribute__((always_inline)) {
    static_for_int<0, BMB * BNB>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if constexpr (i < BMB + BNB) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    });
    __builtin_amdgcn_sched_barrier(0);
  };
  // The K tile in stage STC: sub-steps 0..NSUB-2 (reads of the next sub-step
  // under the MFMAs; with ISSUE, the copies of K tile ikt into stage IST
  // spread over them), then the boundary -- wait until only the copies of K
  // tiles younger than the next one are in flight, barrier (next K tile
  // visible, this stage free) -- and the last sub-step with the next K tile's
  // first reads under its MFMAs (LAST: no next K tile).
  // (st is a constant where the copies are issued: the steady state is
  // unrolled by S; the drain passes it at run time.)
  auto ktile = [&](int st, auto issue, int ikt, int younger, auto last) __attribute__((always_inline)) {
    constexpr bool ISSUE = decltype(issue)::value, LAST = decltype(last)::value;
    static_for_int<0, NSUB - 1>([&](auto ssc) __attribute__((always_inline)) {
      constexpr int ss = decltype(ssc)::value;
      if constexpr (ISSUE)
        RW_ISSUE_PART(ikt, (st + S - 1) % S, ss * COPIES / (NSUB - 1), (ss + 1) * COPIES / (NSUB - 1));
      __builtin_amdgcn_sched_barrier(0);
      read(st, ss + 1, fa[(ss + 1) & 1], fb[(ss + 1) & 1]);
      mma(fa[ss & 1], fb[ss & 1]);
      interleave();
    });
    if constexpr (LAST) {
      __builtin_amdgcn_sched_barrier(0);
      mma(fa[(NSUB - 1) & 1], fb[(NSUB - 1) & 1]);
    } else {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      wait_tiles<COPIES, S - 2>(younger);
      asm volatile("s_barrier" ::: "memory");
      read((st + 1) % S, 0, fa[0], fb[0]);
      mma(fa[(NSUB - 1) & 1], fb[(NSUB - 1) & 1]);
      interleave();
    }
  };
  using T0 = std::false_type;
  using T1 = std::true_type;

  const int KT = K / BK;
#pragma unroll
  for (int s = 0; s < S; ++s)
    if (s < KT) RW_ISSUE_PART(s, s, 0, COPIES);
#undef RW_ISSUE_PART
  wait_tiles<COPIES, S - 2>(min(KT, S) - 1);
  asm volatile("s_barrier" ::: "memory");
  read(0, 0, fa[0], fb[0]);
  int kt = 0;
  if (KT > 1) {
    // K tile 0: its stage's refill (K tile S) is issued by K tile 1.
    ktile(0, T0{}, 0, min(KT - 2, S - 2), T0{});
    // Steady state, unrolled by S so that stages are compile-time: K tile kt
    // refills the stage of K tile kt - 1 with K tile kt + S - 1.
    for (kt = 1; kt + S <= KT - S + 1; kt += S) {
      static_for_int<0, S>([&](auto jc) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value;
        ktile((1 + j) % S, T1{}, kt + j + S - 1, S - 2, T0{});
      });
    }
    static_for_int<0, S - 1>([&](auto jc) __attribute__((always_inline)) {
      constexpr int j = decltype(jc)::value;
      if (kt <= KT - S) {
        ktile((1 + j) % S, T1{}, kt + S - 1, S - 2, T0{});
        ++kt;
      }
    });
    // Drain: no more copies to issue.
    for (; kt < KT - 1; ++kt) ktile(kt % S, T0{}, 0, KT - 2 - kt, T0{});
  }
  ktile(kt % S, T0{}, 0, 0, T1{});

  // ---- epilogue: ((float)acc * xs[m]) * s[n] (+ bias[n]) in fp32, each op
  // rounded (no fused multiply-add), then one rounding to the output dtype.
  epilogue<DT, BMB, BNB>(acc, xs, scale, bias, bias_dt, y, ldy, M, N, m0 + wm * WM, g, n0 + wn * WN, l32);
}

// Tile configurations: 2 x 2 waves of (32 BMB) x (32 BNB) outputs, BK-k
// stages, OCC workgroups per CU. `cost` is the relative time per output
// when every CU is busy (measured at prefill shapes, M = 512..8192). Two
// workgroups per CU (to overlap one's epilogue with the other's loop) and
// 64-k stages measured slower; the 64-k configuration serves K % 128 == 64.
struct Cfg {
  int bmb, bnb, bk, occ;
  double cost;
};
constexpr Cfg kCfgs[] = {
    {4, 4, 128, 1, 1.00}, {4, 3, 128, 1, 1.05}, {4, 2, 128, 1, 1.10}, {4, 2, 64, 1, 1.10},
};
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

template <int DT, int BMB, int BNB, int BK, int OCC>
static void launch_tiles(const W8A8Args &a, hipStream_t s) {
  using G = Tile<BMB, BNB, BK, OCC>;
  // Rows of xq (multiple of BM) and of w (multiple of BN) per launch, so that
  // the 31-bit copy offsets never overflow.
  const int64_t mc = std::max<int64_t>(G::BM, ((int64_t)((COPY_SPAN - a.K) / a.ldxq) + 1) / G::BM * G::BM);
  const int64_t nc = std::max<int64_t>(G::BN, ((int64_t)((COPY_SPAN - a.K) / a.ldw) + 1) / G::BN * G::BN);
  const size_t bias_sz = a.bias_dt == RA_F32 ? 4 : 2;
  for (int64_t ms = 0; ms < a.M; ms += mc)
    for (int64_t ns = 0; ns < a.N; ns += nc) {
      const int64_t Mi = std::min(mc, a.M - ms), Ni = std::min(nc, a.N - ns);
      const int tiles_m = (int)((Mi + G::BM - 1) / G::BM), tiles_n = (int)((Ni + G::BN - 1) / G::BN);
      const void *bi = a.bias ? static_cast<const void *>(static_cast<const char *>(a.bias) + ns * bias_sz) : nullptr;
      hipLaunchKernelGGL((w8a8_gemm_kernel<DT, BMB, BNB, BK, OCC>), dim3((unsigned)(tiles_m * tiles_n)), dim3(256),
                         0, s, a.xq + ms * a.ldxq, a.ldxq, static_cast<const uint16_t *>(a.xs) + ms,
                         a.w + ns * a.ldw, a.ldw, a.scale + ns, bi, a.bias_dt,
                         static_cast<uint16_t *>(a.y) + ms * a.ldy + ns, a.ldy, (int)Mi, (int)Ni, (int)a.K, tiles_m,
                         tiles_n);
    }
}

static int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 256;
  return cus;
}

template <int DT, int I = 0>
static void launch_cfg(int idx, const W8A8Args &a, hipStream_t s) {
  if constexpr (I < kNumCfgs) {
    constexpr Cfg c = kCfgs[I];
    if (idx == I) return launch_tiles<DT, c.bmb, c.bnb, c.bk, c.occ>(a, s);
    launch_cfg<DT, I + 1>(idx, a, s);
  }
}

// Tiles run in rounds of (CUs x workgroups per CU); the configuration with
// the least (rounds x tile area x relative cost) wins.
template <int DT>
static void launch_dt(const W8A8Args &a, hipStream_t s) {
  const int cus = device_cus();
  int pick = -1;
  double best_t = 0;
  for (int i = 0; i < kNumCfgs; ++i) {
    const Cfg &c = kCfgs[i];
    if (a.K % c.bk != 0 || (c.bk == 64 && a.K % 128 == 0)) continue;
    const int64_t bm = 64 * c.bmb, bn = 64 * c.bnb, slots = (int64_t)cus * c.occ;
    const int64_t tiles = ((a.M + bm - 1) / bm) * ((a.N + bn - 1) / bn);
    const double t = (double)((tiles + slots - 1) / slots) * (double)(bm * bn) * c.cost / c.occ;
    if (pick < 0 || t < best_t) pick = i, best_t = t;
  }
#ifdef RA_TUNING
  if (g_w8a8_mode > 0 && g_w8a8_mode <= kNumCfgs) pick = g_w8a8_mode - 1;
#endif
  launch_cfg<DT>(pick, a, s);
}

}  // namespace w8a8

namespace w8a8 {
template <int DT>
static bool quantize_act_vec(const uint16_t *x, int64_t ldx, int64_t M, int64_t K, int8_t *q, int64_t ldq,
                             uint16_t *xs, float c, hipStream_t s) {
  if (K % 8 != 0 || ldx % 8 != 0 || ldq % 8 != 0 || (reinterpret_cast<uintptr_t>(x) & 15) ||
      (reinterpret_cast<uintptr_t>(q) & 7))
    return false;
  const dim3 grid((unsigned)M), block(kRowThreads);
  const int64_t per = 8 * kRowThreads;  // elements per chunk slot
  if (K <= per) hipLaunchKernelGGL((quantize_act_vec_kernel<DT, 1>), grid, block, 0, s, x, ldx, (int)K, q, ldq, xs, c);
  else if (K <= 2 * per)
    hipLaunchKernelGGL((quantize_act_vec_kernel<DT, 2>), grid, block, 0, s, x, ldx, (int)K, q, ldq, xs, c);
  else if (K <= 4 * per)
    hipLaunchKernelGGL((quantize_act_vec_kernel<DT, 4>), grid, block, 0, s, x, ldx, (int)K, q, ldq, xs, c);
  else if (K <= 8 * per)
    hipLaunchKernelGGL((quantize_act_vec_kernel<DT, 8>), grid, block, 0, s, x, ldx, (int)K, q, ldq, xs, c);
  else
    return false;
  return true;
}
}  // namespace w8a8

hipError_t quantize_act_launch(const void *x, int64_t ldx, int x_dt, int64_t M, int64_t K, int8_t *q, int64_t ldq,
                               void *xs, float c, hipStream_t s) {
  const dim3 grid((unsigned)M), block(w8a8::kRowThreads);
  const uint16_t *xp = static_cast<const uint16_t *>(x);
  uint16_t *sp = static_cast<uint16_t *>(xs);
  const bool vec = x_dt == RA_F16 ? w8a8::quantize_act_vec<RA_F16>(xp, ldx, M, K, q, ldq, sp, c, s)
                                  : w8a8::quantize_act_vec<RA_BF16>(xp, ldx, M, K, q, ldq, sp, c, s);
  if (vec) return hipGetLastError();
  if (x_dt == RA_F16)
    hipLaunchKernelGGL((w8a8::quantize_act_kernel<RA_F16>), grid, block, 0, s, xp, ldx, (int)K, q, ldq, sp, c);
  else
    hipLaunchKernelGGL((w8a8::quantize_act_kernel<RA_BF16>), grid, block, 0, s, xp, ldx, (int)K, q, ldq, sp, c);
  return hipGetLastError();
}

bool w8a8_tiled_supported(const W8A8Args &a) {
  if (a.K % 64 != 0 || a.K == 0) return false;
  if ((reinterpret_cast<uintptr_t>(a.xq) & 15) || (reinterpret_cast<uintptr_t>(a.w) & 15)) return false;
  if (a.ldxq % 16 != 0 || a.ldw % 16 != 0) return false;
  if ((uint64_t)(255 * a.ldxq + a.K) > w8a8::COPY_SPAN || (uint64_t)(255 * a.ldw + a.K) > w8a8::COPY_SPAN)
    return false;
  if (a.ldy > ((int64_t)1 << 22)) return false;  // 32-bit epilogue offsets: 256 * ldy < 2^31
  return a.M <= ((int64_t)1 << 30) && a.N <= ((int64_t)1 << 30);
}

hipError_t w8a8_launch(const W8A8Args &a, hipStream_t s) {
  if (w8a8_tiled_supported(a)) {
    if (a.y_dt == RA_F16) w8a8::launch_dt<RA_F16>(a, s);
    else w8a8::launch_dt<RA_BF16>(a, s);
    return hipGetLastError();
  }
  const dim3 grid((unsigned)((a.N + 255) / 256), (unsigned)a.M);
  const uint16_t *xs = static_cast<const uint16_t *>(a.xs);
  uint16_t *y = static_cast<uint16_t *>(a.y);
  if (a.y_dt == RA_F16)
    hipLaunchKernelGGL((w8a8::w8a8_generic_kernel<RA_F16>), grid, dim3(256), 0, s, a.xq, a.ldxq, xs, a.w, a.ldw,
                       a.scale, a.bias, a.bias_dt, y, a.ldy, (int)a.M, (int)a.N, (int)a.K);
  else
    hipLaunchKernelGGL((w8a8::w8a8_generic_kernel<RA_BF16>), grid, dim3(256), 0, s, a.xq, a.ldxq, xs, a.w, a.ldw,
                       a.scale, a.bias, a.bias_dt, y, a.ldy, (int)a.M, (int)a.N, (int)a.K);
  return hipGetLastError();
}

}  // namespace ra
