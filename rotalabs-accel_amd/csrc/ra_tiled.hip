// LDS-staged, double-buffered W8A16 MFMA GEMM for prefill (large M) on gfx950.
//
// Replaces the reference's Triton kernel (src/rotalabs_accel/kernels/
// gemm.py:53-138) for large M: C[M,N] = A[M,K](fp16|bf16) . dq(W[N,K])^T * s[N].
// The reference feeds tl.dot a [K,N]-transposed int8 copy made on every call
// (gemm.py:157-160); this kernel reads W in its [N,K] layout.
//
// Tile 256(M) x 128(N) x 64(K), 256 threads = 4 waves in a 2x2 grid, each
// wave owns a 128x64 sub-tile = 4x2 blocks of v_mfma_f32_32x32x16_{f16,bf16}
// (128 fp32 accumulators per lane).
//  * Global -> registers -> LDS, double buffered: tile k+1 is fetched into
//    registers while tile k is multiplied out of LDS, then written to the
//    other buffer; one barrier per K tile.
//  * A (activations) in LDS: 256 rows x 128 B, 16-byte chunks XOR-swizzled by
//    ((row >> 1) & 7). LDS serves a 128-bit access 16 lanes per cycle (64
//    banks x 4 B), so the MFMA operand reads (16 consecutive rows, same
//    chunk) must land in 16 distinct 16-byte bank groups: rows alternate
//    between the two 128-byte halves of a 256-byte bank row, and the swizzle
//    separates the 8 rows within each half.
//  * B (weights) stays int8 in LDS (8 KB per stage: half the LDS traffic of
//    fp16), 128 rows x 64 B, 8-byte chunks swizzled by ((row >> 2) & 7); each
//    wave dequantises its 32x16 B fragments in registers right before the
//    MFMA (exact int8 -> fp16/bf16).
//  * K permutation: in sub-step s (0..3) lane group g (0,1) supplies the 8
//    consecutive k's of chunk 2s+g to both operands, so every MFMA operand is
//    one 16-byte (A) or 8-byte (B) LDS read.
//  * Scale (and bias, or the SwiGLU of a gate/up pair) are applied to the
//    fp32 accumulators in the epilogue, one rounding to the output dtype.
//  * XCD-aware tile order: hardware deals workgroups round-robin over the 8
//    XCDs; workgroup b is remapped so each XCD owns a contiguous range of the
//    grouped (8 M-tiles per group) tile order and its L2 keeps the shared
//    weight columns and activation rows.
// GU (gate/up + SwiGLU): the 128 B rows of a tile are 64 gate rows and the
// 64 matching up rows, arranged so that each wave's two 32-column blocks are
// the gate and up values of the same 32 output columns.
#include "ra_common.h"
#include "ra_internal.h"

namespace ra {

#ifndef RA_TILED_STAGES
#define RA_TILED_STAGES 4
#endif

namespace tiled {
constexpr int BM = 256, BN = 128, BK = 64;
constexpr int A_BYTES = BM * BK * 2;  // 32 KB
constexpr int B_BYTES = BN * BK;      // 8 KB
constexpr int STAGE = A_BYTES + B_BYTES;
}  // namespace tiled

template <int DT, bool GU>
__global__ __launch_bounds__(256, 2) void tiled_kernel(const uint16_t *__restrict__ x, int64_t ldx,
                                                       const int8_t *__restrict__ w, int64_t ldw,
                                                       const float *__restrict__ scale,
                                                       const void *__restrict__ bias, int bias_dt,
                                                       uint16_t *__restrict__ y, int64_t ldy, int M, int N,
                                                       int K, int tiles_m, int tiles_n) {
  using namespace tiled;
  using Ac = Act<DT>;
  constexpr int OUTN = GU ? BN / 2 : BN;  // output columns per tile
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * STAGE];

  // ---- tile coordinates (XCD-aware, grouped along M) ----
  const int T = tiles_m * tiles_n;
  const int b = blockIdx.x;
  const int xcd = b & 7, idx = b >> 3;
  const int per = T >> 3, rem = T & 7;
  const int t = xcd * per + (xcd < rem ? xcd : rem) + idx;
  constexpr int GM = 8;
  const int span = GM * tiles_n;
  const int first_m = (t / span) * GM;
  const int gm = min(tiles_m - first_m, GM);
  const int tm = first_m + (t % span) % gm;
  const int tn = (t % span) / gm;
  const int m0 = tm * BM, n0 = tn * OUTN;

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  const int l32 = lane & 31, g = lane >> 5;

  // ---- global load assignment ----
  // A: 8 x 16 B per thread: rows i*32 + tid/8, chunk tid%8.
  const int ac = tid & 7;
  const uint16_t *ap[8];
  int a_off[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = i * 32 + (tid >> 3);
    int gr = m0 + row;
    gr = gr < M ? gr : M - 1;
    ap[i] = x + (int64_t)gr * ldx + ac * 8;
    a_off[i] = row * 128 + ((ac ^ ((row >> 1) & 7)) << 4);
  }
  // B: 2 x 16 B per thread: rows i*64 + tid/4, bytes 16*(tid%4) .. +15
  // (= 8-byte chunks 2q and 2q+1).
  const int bq = tid & 3;
  const int8_t *bp[2];
  int b_off0[2], b_off1[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = i * 64 + (tid >> 2);
    int wr;
    if (GU) {
      // tile row = wn*64 + half*32 + jj  ->  weight row (half ? N : 0) + n0 + wn*32 + jj
      const int half = (row >> 5) & 1, jj = row & 31;
      int j = n0 + (row >> 6) * 32 + jj;
      j = j < N ? j : N - 1;
      wr = half ? N + j : j;
    } else {
      wr = n0 + row;
      wr = wr < N ? wr : N - 1;
    }
    bp[i] = w + (int64_t)wr * ldw + bq * 16;
    const int sw = (row >> 2) & 7;
    b_off0[i] = A_BYTES + row * 64 + (((2 * bq) ^ sw) << 3);
    b_off1[i] = A_BYTES + row * 64 + (((2 * bq + 1) ^ sw) << 3);
  }

  uint4 ra[8], rb[2];
// Fully unrolled statement repetition (constant indices keep ra / rb in VGPRs).
#define RA_UNROLL2(i, stmt) { { constexpr int i = 0; stmt } { constexpr int i = 1; stmt } }
#define RA_UNROLL8(i, stmt) { RA_UNROLL2(i##_, { constexpr int i = 0 + i##_; stmt }) \
                              RA_UNROLL2(i##_, { constexpr int i = 2 + i##_; stmt }) \
                              RA_UNROLL2(i##_, { constexpr int i = 4 + i##_; stmt }) \
                              RA_UNROLL2(i##_, { constexpr int i = 6 + i##_; stmt }) }
// Global loads of K tile starting at k0 into ra / rb (zero past K).
#define RA_TILED_GLOAD(k0)                                                                    \
  {                                                                                          \
    const bool av_ = (k0) + ac * 8 + 8 <= K;                                                 \
    RA_UNROLL8(i, ra[i] = av_ ? *reinterpret_cast<const uint4 *>(ap[i] + (k0)) : make_uint4(0, 0, 0, 0);)       \
    const bool bv_ = (k0) + bq * 16 + 16 <= K;                                               \
    RA_UNROLL2(i, rb[i] = bv_ ? *reinterpret_cast<const uint4 *>(bp[i] + (k0)) : make_uint4(0, 0, 0, 0);)       \
  }
// Store ra / rb into LDS stage buf.
#define RA_TILED_SSTORE(buf)                                                                  \
  {                                                                                          \
    uint8_t *base_ = lds + (buf) * STAGE;                                                    \
    RA_UNROLL8(i, *reinterpret_cast<uint4 *>(base_ + a_off[i]) = ra[i];)                    \
    RA_UNROLL2(i, *reinterpret_cast<uint2 *>(base_ + b_off0[i]) = make_uint2(rb[i].x, rb[i].y);  \
                  *reinterpret_cast<uint2 *>(base_ + b_off1[i]) = make_uint2(rb[i].z, rb[i].w);) \
  }

  // ---- MFMA operand read offsets (row bases are multiples of 32) ----
  const int a_row_base = (wm * 128 + l32) * 128;
  const int b_row_base = A_BYTES + (wn * 64 + l32) * 64;
  const int a_sw = (l32 >> 1) & 7;
  const int b_sw = (l32 >> 2) & 7;

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // K tiles: the loop body always prefetches the next tile (no branches, so
  // the staging registers stay in VGPRs); the last tile is peeled.
#define RA_TILED_COMPUTE(buf)                                                                       \
  {                                                                                                 \
    const uint8_t *base = lds + (buf) * STAGE;                                                      \
    _Pragma("unroll") for (int s = 0; s < 4; ++s) {                                                 \
      const int c = 2 * s + g;                                                                      \
      uint4 af[4], bf[2];                                                                           \
      _Pragma("unroll") for (int bi = 0; bi < 4; ++bi) af[bi] =                                     \
          *reinterpret_cast<const uint4 *>(base + a_row_base + bi * 32 * 128 + ((c ^ a_sw) << 4)); \
      _Pragma("unroll") for (int bj = 0; bj < 2; ++bj) {                                            \
        const uint2 raw =                                                                           \
            *reinterpret_cast<const uint2 *>(base + b_row_base + bj * 32 * 64 + ((c ^ b_sw) << 3)); \
        bf[bj] = Ac::dq8(raw.x, raw.y);                                                             \
      }                                                                                             \
      _Pragma("unroll") for (int bi = 0; bi < 4; ++bi)                                              \
          _Pragma("unroll") for (int bj = 0; bj < 2; ++bj) acc[bi][bj] =                            \
              Ac::mfma32(af[bi], bf[bj], acc[bi][bj]);                                              \
    }                                                                                               \
  }
  const int KT = (K + BK - 1) / BK;
  if (KT > 0) {
    RA_TILED_GLOAD(0);
    RA_TILED_SSTORE(0);
    __syncthreads();
    int kt = 0;
    for (; kt + 1 < KT; ++kt) {
      RA_TILED_GLOAD((kt + 1) * BK);
      RA_TILED_COMPUTE(kt & 1);
      RA_TILED_SSTORE((kt + 1) & 1);
      __syncthreads();
    }
    RA_TILED_COMPUTE(kt & 1);
  }

#undef RA_TILED_GLOAD
#undef RA_TILED_SSTORE
#undef RA_UNROLL8
#undef RA_UNROLL2
#undef RA_TILED_COMPUTE

  // ---- epilogue ----
  if (GU) {
    const int j = n0 + wn * 32 + l32;
    if (j < N) {
      const float sg = scale[j], su = scale[N + j];
#pragma unroll
      for (int bi = 0; bi < 4; ++bi)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m0 + wm * 128 + bi * 32 + (e & 3) + 8 * (e >> 2) + 4 * g;
          if (m < M) {
            y[(int64_t)m * ldy + j] = swiglu_out<Ac>(acc[bi][0][e] * sg, acc[bi][1][e] * su);
          }
        }
    }
  } else {
#pragma unroll
    for (int bj = 0; bj < 2; ++bj) {
      const int n = n0 + wn * 64 + bj * 32 + l32;
      if (n >= N) continue;
      const float sn = scale[n];
      const float bn = bias ? load_as_f32(bias, n, bias_dt) : 0.f;
#pragma unroll
      for (int bi = 0; bi < 4; ++bi)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m0 + wm * 128 + bi * 32 + (e & 3) + 8 * (e >> 2) + 4 * g;
          if (m < M) y[(int64_t)m * ldy + n] = Ac::out(acc[bi][bj][e] * sn + bn);
        }
    }
  }
}

// ---------------------------------------------------------------------------
// Multi-stage variant for K % 64 == 0: the global -> LDS copies are gfx950
// direct-to-LDS loads (global_load_lds_dwordx4: each lane's 16 bytes land at
// M0 + 16 * lane, no VGPR round trip), S K-tiles deep, so S-1 tiles are in
// flight while one is multiplied. The XOR swizzles are applied on the global
// side (lane l of a copy fetches the chunk that belongs at its LDS slot).
// The copies are issued with inline asm so that the waits are explicit:
// before tile kt is read, each wave waits until only the copies of the
// younger tiles are outstanding (s_waitcnt vmcnt), then one s_barrier makes
// every wave's copies of tile kt visible and frees the stage that the next
// copy overwrites.
// K permutation of the MFMA sub-steps: B is read as 16 bytes (k = 16q ..
// 16q + 15, q = 2p + g) once per pair p of sub-steps; sub-step s = 2p + h
// uses its 8-byte half h, and A supplies the same k's (8-half chunk
// 4p + 2g + h), so the B read is shared by two MFMA sub-steps.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t lds_offset(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// 16 bytes per lane from global memory to LDS at m0 + 16 * lane.
__device__ __forceinline__ void dma16(const void *g, uint32_t lds_wave_base) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_wave_base), "v"(g)
               : "memory", "m0");
}

template <int DT, bool GU, int S>
__global__ __launch_bounds__(256, 1) void tiled_dma_kernel(const uint16_t *__restrict__ x, int64_t ldx,
                                                           const int8_t *__restrict__ w, int64_t ldw,
                                                           const float *__restrict__ scale,
                                                           const void *__restrict__ bias, int bias_dt,
                                                           uint16_t *__restrict__ y, int64_t ldy, int M, int N,
                                                           int K, int tiles_m, int tiles_n) {
  using namespace tiled;
  using Ac = Act<DT>;
  constexpr int OUTN = GU ? BN / 2 : BN;
  constexpr int A_COPIES = A_BYTES / 1024 / 4;  // per wave per tile: 8
  constexpr int B_COPIES = B_BYTES / 1024 / 4;  // 2
  constexpr int COPIES = A_COPIES + B_COPIES;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[S * STAGE];

  // ---- tile coordinates (XCD-aware, grouped along M; as tiled_kernel) ----
  const int T = tiles_m * tiles_n;
  const int b = blockIdx.x;
  const int xcd = b & 7, idx = b >> 3;
  const int per = T >> 3, rem = T & 7;
  const int t = xcd * per + (xcd < rem ? xcd : rem) + idx;
  constexpr int GM = 8;
  const int span = GM * tiles_n;
  const int first_m = (t / span) * GM;
  const int gm = min(tiles_m - first_m, GM);
  const int tm = first_m + (t % span) % gm;
  const int tn = (t % span) / gm;
  const int m0 = tm * BM, n0 = tn * OUTN;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wid >> 1, wn = wid & 1;
  const int l32 = lane & 31, g = lane >> 5;

  // ---- copy sources: A copy i covers tile rows 8*ai .. +7 (ai = 8*wid + i),
  // lane -> row 8*ai + lane/8, LDS chunk lane%8 <- global chunk
  // (lane%8) ^ ((row>>1)&7)
  const uint16_t *a_src[A_COPIES];
#pragma unroll
  for (int i = 0; i < A_COPIES; ++i) {
    const int row = 8 * (A_COPIES * wid + i) + (lane >> 3);
    const int c = (lane & 7) ^ ((row >> 1) & 7);
    int gr = m0 + row;
    gr = gr < M ? gr : M - 1;
    a_src[i] = x + (int64_t)gr * ldx + c * 8;
  }
  // B copy i covers tile rows 16*bi .. +15 (bi = 2*wid + i), lane -> row
  // 16*bi + lane/4, LDS chunk lane%4 <- global chunk (lane%4)^((row>>2)&3)
  const int8_t *b_src[B_COPIES];
#pragma unroll
  for (int i = 0; i < B_COPIES; ++i) {
    const int row = 16 * (B_COPIES * wid + i) + (lane >> 2);
    const int c = (lane & 3) ^ ((row >> 2) & 3);
    int wr;
    if (GU) {
      const int half = (row >> 5) & 1, jj = row & 31;
      int j = n0 + (row >> 6) * 32 + jj;
      j = j < N ? j : N - 1;
      wr = half ? N + j : j;
    } else {
      wr = n0 + row;
      wr = wr < N ? wr : N - 1;
    }
    b_src[i] = w + (int64_t)wr * ldw + c * 16;
  }
  const uint32_t lds0 = lds_offset(lds);
  const uint32_t a_dst = lds0 + (uint32_t)(A_COPIES * wid) * 1024;
  const uint32_t b_dst = lds0 + A_BYTES + (uint32_t)(B_COPIES * wid) * 1024;

#define RA_ISSUE(kt_, st_)                                                                  \
  {                                                                                         \
    const int kofs_ = (kt_) * BK;                                                           \
    const uint32_t so_ = (uint32_t)(st_) * STAGE;                                           \
    _Pragma("unroll") for (int i = 0; i < A_COPIES; ++i)                                    \
        dma16(a_src[i] + kofs_, a_dst + so_ + (uint32_t)i * 1024);                         \
    _Pragma("unroll") for (int i = 0; i < B_COPIES; ++i)                                    \
        dma16(b_src[i] + kofs_, b_dst + so_ + (uint32_t)i * 1024);                         \
  }

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int a_row_off = (wm * 128 + l32) * 128;
  const int b_row_off = A_BYTES + (wn * 64 + l32) * 64;
  const int a_sw = (l32 >> 1) & 7;
  const int b_sw = (l32 >> 2) & 3;

  // Software pipeline at sub-step granularity. A fragments ping-pong between
  // two sets (sub-step ss+1 is read while ss is multiplied); B (both pairs of
  // the tile, 4 x 16 B) is read once per tile into the set of the tile after.
  // The tile boundary (wait for the next tile's copies, barrier, next copy,
  // first reads of the next tile) sits before the last sub-step's MFMAs.
  uint4 fa0[4], fa1[4], fbA[2][2], fbB[2][2];
#define RA_READ_A(st_, ss_, FA)                                                                     \
  {                                                                                                 \
    const uint8_t *base_ = lds + (st_) * STAGE;                                                     \
    _Pragma("unroll") for (int bi = 0; bi < 4; ++bi) FA[bi] = *reinterpret_cast<const uint4 *>(     \
        base_ + a_row_off + bi * 32 * 128 + (((4 * ((ss_) >> 1) + 2 * g + ((ss_) & 1)) ^ a_sw) << 4)); \
  }
#define RA_READ_B(st_, FB)                                                                          \
  {                                                                                                 \
    const uint8_t *base_ = lds + (st_) * STAGE;                                                     \
    _Pragma("unroll") for (int p = 0; p < 2; ++p)                                                   \
        _Pragma("unroll") for (int bj = 0; bj < 2; ++bj) FB[p][bj] = *reinterpret_cast<const uint4 *>( \
            base_ + b_row_off + bj * 32 * 64 + (((2 * p + g) ^ b_sw) << 4));                        \
  }
#define RA_MMA(ss_, FA, FB)                                                                         \
  {                                                                                                 \
    uint4 bf_[2];                                                                                   \
    _Pragma("unroll") for (int bj = 0; bj < 2; ++bj) bf_[bj] = ((ss_) & 1)                          \
        ? Ac::dq8(FB[(ss_) >> 1][bj].z, FB[(ss_) >> 1][bj].w)                                        \
        : Ac::dq8(FB[(ss_) >> 1][bj].x, FB[(ss_) >> 1][bj].y);                                       \
    _Pragma("unroll") for (int bi = 0; bi < 4; ++bi)                                                \
        _Pragma("unroll") for (int bj = 0; bj < 2; ++bj) acc[bi][bj] =                              \
            Ac::mfma32(FA[bi], bf_[bj], acc[bi][bj]);                                               \
  }
// One K tile kt_ from B set FBC (A sub-step 0 already in fa0). Before the last
// sub-step: complete this tile's LDS reads, wait until this wave's copies of
// tile kt_+1 are done (only younger tiles in flight), barrier (tile kt_+1 is
// visible to all; stage kt_ % S is free), copy tile kt_+S into it, and start
// reading tile kt_+1 (A sub-step 0 into fa0, B into FBN).
#define RA_TILE(kt_, FBC, FBN)                                                                        \
  {                                                                                                   \
    const int st_ = (kt_) % S;                                                                        \
    RA_READ_A(st_, 1, fa1);                                                                           \
    RA_MMA(0, fa0, FBC);                                                                              \
    RA_READ_A(st_, 2, fa0);                                                                           \
    RA_MMA(1, fa1, FBC);                                                                              \
    RA_READ_A(st_, 3, fa1);                                                                           \
    RA_MMA(2, fa0, FBC);                                                                              \
    if ((kt_) + 1 < KT) {                                                                             \
      const int younger_ = min(KT - 2 - (kt_), S - 2);                                                \
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");                                              \
      if (younger_ >= 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * COPIES) : "memory");            \
      else if (younger_ == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(COPIES) : "memory");           \
      else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");                                           \
      asm volatile("s_barrier" ::: "memory");                                                         \
      if ((kt_) + S < KT) RA_ISSUE((kt_) + S, st_);                                                   \
      RA_READ_A(((kt_) + 1) % S, 0, fa0);                                                             \
      RA_READ_B(((kt_) + 1) % S, FBN);                                                                \
    }                                                                                                 \
    RA_MMA(3, fa1, FBC);                                                                              \
  }

  const int KT = K / BK;
#pragma unroll
  for (int s = 0; s < S; ++s)
    if (s < KT) RA_ISSUE(s, s);
  {
    const int younger0 = min(KT, S) - 1;  // tiles issued after tile 0
    if (younger0 >= 3) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * COPIES) : "memory");
    else if (younger0 == 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * COPIES) : "memory");
    else if (younger0 == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(COPIES) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("s_barrier" ::: "memory");
  }
  RA_READ_A(0, 0, fa0);
  RA_READ_B(0, fbA);
  for (int kt = 0; kt < KT; kt += 2) {
    RA_TILE(kt, fbA, fbB);
    if (kt + 1 < KT) RA_TILE(kt + 1, fbB, fbA);
  }
#undef RA_TILE
#undef RA_MMA
#undef RA_READ_B
#undef RA_READ_A
#undef RA_ISSUE

  // ---- epilogue (as tiled_kernel) ----
  if (GU) {
    const int j = n0 + wn * 32 + l32;
    if (j < N) {
      const float sg = scale[j], su = scale[N + j];
#pragma unroll
      for (int bi = 0; bi < 4; ++bi)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m0 + wm * 128 + bi * 32 + (e & 3) + 8 * (e >> 2) + 4 * g;
          if (m < M) y[(int64_t)m * ldy + j] = swiglu_out<Ac>(acc[bi][0][e] * sg, acc[bi][1][e] * su);
        }
    }
  } else {
#pragma unroll
    for (int bj = 0; bj < 2; ++bj) {
      const int n = n0 + wn * 64 + bj * 32 + l32;
      if (n >= N) continue;
      const float sn = scale[n];
      const float bn = bias ? load_as_f32(bias, n, bias_dt) : 0.f;
#pragma unroll
      for (int bi = 0; bi < 4; ++bi)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m0 + wm * 128 + bi * 32 + (e & 3) + 8 * (e >> 2) + 4 * g;
          if (m < M) y[(int64_t)m * ldy + n] = Ac::out(acc[bi][bj][e] * sn + bn);
        }
    }
  }
}

static bool tiled_shape_ok(int x_dt, const void *x, int64_t ldx, const int8_t *w, int64_t ldw, int64_t M,
                           int64_t N, int64_t K) {
  if (x_dt != RA_F16 && x_dt != RA_BF16) return false;
  if (M > ((int64_t)1 << 30) || N > ((int64_t)1 << 30) || K > ((int64_t)1 << 30)) return false;
  if (K % 16 != 0) return false;
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(w) & 15)) return false;
  if ((ldx % 8) != 0 || (ldw % 16) != 0) return false;
  const int64_t tiles = ((M + tiled::BM - 1) / tiled::BM) * ((N + tiled::BN - 1) / tiled::BN);
  return tiles < ((int64_t)1 << 31);
}

bool tiled_supported(const GemmArgs &a) { return tiled_shape_ok(a.x_dt, a.x, a.ldx, a.w, a.ldw, a.M, a.N, a.K); }

template <bool GU>
static hipError_t launch(const void *x, int64_t ldx, int x_dt, const int8_t *w, int64_t ldw,
                         const float *scale, const void *bias, int bias_dt, void *y, int64_t ldy,
                         int64_t M, int64_t N, int64_t K, hipStream_t s) {
  constexpr int OUTN = GU ? tiled::BN / 2 : tiled::BN;
  const int tiles_m = (int)((M + tiled::BM - 1) / tiled::BM);
  const int tiles_n = (int)((N + OUTN - 1) / OUTN);
  const dim3 grid((unsigned)(tiles_m * tiles_n));
#ifdef RA_TUNING
  extern int g_tiled_mode;  // 0 auto, 1 register-staged kernel, 2 direct-to-LDS kernel
  const bool use_dma = g_tiled_mode == 2 || (g_tiled_mode == 0 && K % tiled::BK == 0);
#else
  const bool use_dma = K % tiled::BK == 0;
#endif
  if (use_dma) {
    constexpr int S = RA_TILED_STAGES;
    if (x_dt == RA_F16)
      hipLaunchKernelGGL((tiled_dma_kernel<RA_F16, GU, S>), grid, dim3(256), 0, s,
                         static_cast<const uint16_t *>(x), ldx, w, ldw, scale, bias, bias_dt,
                         static_cast<uint16_t *>(y), ldy, (int)M, (int)N, (int)K, tiles_m, tiles_n);
    else
      hipLaunchKernelGGL((tiled_dma_kernel<RA_BF16, GU, S>), grid, dim3(256), 0, s,
                         static_cast<const uint16_t *>(x), ldx, w, ldw, scale, bias, bias_dt,
                         static_cast<uint16_t *>(y), ldy, (int)M, (int)N, (int)K, tiles_m, tiles_n);
    return hipGetLastError();
  }
  if (x_dt == RA_F16)
    hipLaunchKernelGGL((tiled_kernel<RA_F16, GU>), grid, dim3(256), 0, s, static_cast<const uint16_t *>(x), ldx,
                       w, ldw, scale, bias, bias_dt, static_cast<uint16_t *>(y), ldy, (int)M, (int)N, (int)K,
                       tiles_m, tiles_n);
  else
    hipLaunchKernelGGL((tiled_kernel<RA_BF16, GU>), grid, dim3(256), 0, s, static_cast<const uint16_t *>(x),
                       ldx, w, ldw, scale, bias, bias_dt, static_cast<uint16_t *>(y), ldy, (int)M, (int)N,
                       (int)K, tiles_m, tiles_n);
  return hipGetLastError();
}

hipError_t tiled_launch(const GemmArgs &a, hipStream_t s) {
  return launch<false>(a.x, a.ldx, a.x_dt, a.w, a.ldw, a.scale, a.bias, a.bias_dt, a.y, a.ldy, a.M, a.N, a.K,
                       s);
}

bool gateup_tiled_supported(const GateUpArgs &a) {
  return tiled_shape_ok(a.x_dt, a.x, a.ldx, a.w, a.ldw, a.M, 2 * a.I, a.K);
}

hipError_t gateup_tiled_launch(const GateUpArgs &a, hipStream_t s) {
  return launch<true>(a.x, a.ldx, a.x_dt, a.w, a.ldw, a.scale, nullptr, RA_F32, a.h, a.ldh, a.M, a.I, a.K, s);
}

}  // namespace ra
