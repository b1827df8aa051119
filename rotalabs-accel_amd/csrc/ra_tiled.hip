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
//    grouped (8 M-tiles per group; 4 in the direct-to-LDS kernel) tile order
//    and its L2 keeps the shared weight columns and activation rows.
// GU (gate/up + SwiGLU): the 128 B rows of a tile are 64 gate rows and the
// 64 matching up rows, arranged so that each wave's two 32-column blocks are
// the gate and up values of the same 32 output columns.
#include <type_traits>

#include "ra_common.h"
#include "ra_internal.h"

namespace ra {

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
// Largest byte offset the 32-bit per-lane copy offsets may reach. The copy
// bases are moved down by DMA_BIAS so that offsets minus the instruction
// offset stay non-negative, and offsets stay below 2^31 so that they mean
// the same whether the address unit reads them as signed or unsigned.
constexpr int DMA_BIAS = 3072;
constexpr uint64_t DMA_SPAN = (uint64_t)0x7FFFFFFF - 2 * DMA_BIAS;

// Tile geometry of the direct-to-LDS kernel: 4 waves in a WR x (4/WR) grid,
// each owning BMB x BNB blocks of 32 x 32 outputs (one v_mfma_f32_32x32x16 per
// block and 16-deep K sub-step). Bigger per-wave tiles need fewer LDS bytes
// per MFMA: (4,2) reads 0.625 KB per MFMA, (3,4) 0.417, (4,4) 0.375. With one
// wave row (WR = 1) every weight column is dequantised by one wave instead
// of two, for 50 % more activation reads: 256x256 as (8,2) in 1 x 4 measured
// 1-2 % faster than (4,4) in 2 x 2.
template <int BMB, int BNB, int WR, int SMAX_SMALL = 4>
struct DmaTile {
  static constexpr int WM = 32 * BMB, WN = 32 * BNB;  // per-wave sub-tile
  static constexpr int BM = WR * WM, BN = (4 / WR) * WN, BK = 64;
  static constexpr int A_BYTES = BM * BK * 2;  // fp16/bf16 rows of 128 B
  static constexpr int B_BYTES = BN * BK;      // int8 rows of 64 B
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int A_COPIES = A_BYTES / 4096;  // 1 KB copies per wave per K tile
  static constexpr int B_COPIES = B_BYTES / 4096;
  static constexpr int COPIES = A_COPIES + B_COPIES;
  // pipeline depth: up to 4 stages, up to SMAX for small tiles
  static constexpr int SMAX = STAGE <= 24 * 1024 ? SMAX_SMALL : 4;
  static constexpr int S = (160 * 1024) / STAGE < SMAX ? (160 * 1024) / STAGE : SMAX;
  static_assert(A_BYTES % 4096 == 0 && B_BYTES % 4096 == 0, "copies must split evenly over 4 waves");
  static_assert(S >= 2 && S <= 13, "2 to 13 stages");
  static_assert((S - 1) * COPIES <= 63, "vmcnt is a 6-bit counter");
};


// Wait until at most `younger` K tiles of copies (COPIES loads each) are
// still in flight for this wave; younger <= Y = S - 1 <= 7.
template <int COPIES, int Y>
__device__ __forceinline__ void wait_tiles(int younger) {
  if constexpr (Y == 0) {
    wait_vmcnt<0>();
  } else {
    if (younger >= Y) wait_vmcnt<Y * COPIES>();
    else wait_tiles<COPIES, Y - 1>(younger);
  }
}

// The K-tile byte offset of the copies' SGPR base: the 128-row split tiles
// need it marked uniform (else it can land in VGPRs, which the copy's SGPR
// operand cannot take).
template <bool RFL>
__device__ __forceinline__ int uniform_if(int v) {
  if constexpr (RFL) return __builtin_amdgcn_readfirstlane(v);
  else return v;
}

// SPLIT (M <= 1024, one or more rows of tiles): K is split over nsplit workgroups per
// tile, ksplit K tiles each (the last may have fewer); workgroup b runs split
// b % nsplit of tile b / nsplit. With nsplit > 1 each writes its fp32 sums
// to the workspace with device-scope stores, waits for them and counts
// itself in on the tile's counter (device-scope atomic); the workgroup that
// completes the count adds the nsplit partial sums in split order
// (deterministic), runs the epilogue and resets the counter. No workgroup
// waits for another. Partial sums: [tile][split][wave][BMB*BNB*4 chunks of
// 4][64 lanes][4 floats]; counters: one int per tile at cnt.
constexpr int kMaxTileSplits = 4;  // K splits per tile of the SPLIT form
constexpr int kMaxTileBmb = 2;     // 32x32 row blocks per wave of the SPLIT form (tiles of 64 or 128 rows)

template <int DT, bool GU, int BMB, int BNB, int WR, int SM = 4, bool SPLIT = false>
__global__ __launch_bounds__(256, 1) void tiled_dma_kernel(const uint16_t *__restrict__ x, int64_t ldx,
                                                           const int8_t *__restrict__ w, int64_t ldw,
                                                           const float *__restrict__ scale,
                                                           const void *__restrict__ bias, int bias_dt,
                                                           uint16_t *__restrict__ y, int64_t ldy, int M, int N,
                                                           int K, int tiles_m, int tiles_n, int nsplit, int ksplit,
                                                           float *__restrict__ part, int *__restrict__ cnt) {
  using G = DmaTile<BMB, BNB, WR, SM>;
  using Ac = Act<DT>;
  constexpr int BM = G::BM, BN = G::BN, BK = G::BK, WM = G::WM, WN = G::WN, S = G::S;
  constexpr int A_COPIES = G::A_COPIES, B_COPIES = G::B_COPIES, COPIES = G::COPIES;
  constexpr int STAGE = G::STAGE, A_BYTES = G::A_BYTES;
  // GU: each wave's WN weight rows are WN/2 gate rows followed by the WN/2
  // matching up rows, so block bj (< BNB/2) pairs with block bj + BNB/2.
  static_assert(!GU || BNB % 2 == 0, "gate/up pairing needs an even number of column blocks");
  constexpr int OUTN = GU ? BN / 2 : BN;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[S * STAGE];
#ifdef RA_TRACE
  // Trace builds only: per-workgroup timestamps (constant 100 MHz clock) of
  // entry, first tile ready, end of the K loop and end of the epilogue's
  // stores, written to `part` (unused by the non-split kernel).
  const uint64_t tr_entry = __builtin_amdgcn_s_memrealtime();
  const uint64_t tr_entry_clk = __builtin_amdgcn_s_memtime();
  uint64_t tr_ready = 0, tr_kend = 0;
#endif

  // ---- tile coordinates (XCD-aware, grouped along M as in tiled_kernel) ----
  const int T = tiles_m * tiles_n;
  const int b = SPLIT ? (int)blockIdx.x / nsplit : (int)blockIdx.x;
  const int sp = SPLIT ? (int)blockIdx.x - b * nsplit : 0;  // K split of this workgroup
  const int kt0 = sp * ksplit;                               // its first K tile
  const int xcd = b & 7, idx = b >> 3;
  const int per = T >> 3, rem = T & 7;
  const int t = xcd * per + (xcd < rem ? xcd : rem) + idx;
  // Groups of 4 M-tiles: an XCD's 32 concurrent tiles are 4 M-tiles x 8
  // weight-column tiles, whose per-K-tile operands (4 x 256 fp16 rows, 8 x BN
  // int8 rows) are fewer bytes than 8 x 4 (M=2048 K=4096 N=11008: 153.7 ->
  // 152.4-153.4 us, same-box A/B).
  constexpr int GM = 4;
  const int span = GM * tiles_n;
  const int first_m = (t / span) * GM;
  const int gm = min(tiles_m - first_m, GM);
  const int tm = first_m + (t % span) % gm;
  const int tn = (t % span) / gm;
  const int m0 = tm * BM, n0 = tn * OUTN;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wid / (4 / WR), wn = wid % (4 / WR);
  const int l32 = lane & 31, g = lane >> 5;

  // ---- copy sources: A copy i covers tile rows 8*ai .. +7 (ai = A_COPIES*wid
  // + i), lane -> row 8*ai + lane/8, LDS chunk lane%8 <- global chunk
  // (lane%8) ^ ((row>>1)&7). Rows past M are clamped (loaded, never stored).
  // Per-lane byte offsets from the copy bases xb / wb (moved down by
  // DMA_BIAS; the host keeps every offset below 2^32).
  uint32_t a_voff[A_COPIES];
#pragma unroll
  for (int i = 0; i < A_COPIES; ++i) {
    const int row = 8 * (A_COPIES * wid + i) + (lane >> 3);
    const int c = (lane & 7) ^ ((row >> 1) & 7);
    int gr = m0 + row;
    gr = gr < M ? gr : M - 1;
    a_voff[i] = (uint32_t)(((int64_t)gr * ldx + c * 8) * 2) + (uint32_t)(DMA_BIAS - (i % 4) * 1024);
  }
  // B copy i covers tile rows 16*bi .. +15 (bi = B_COPIES*wid + i), lane ->
  // row 16*bi + lane/4, LDS chunk lane%4 <- global chunk (lane%4)^((row>>2)&3).
  uint32_t b_voff[B_COPIES];
#pragma unroll
  for (int i = 0; i < B_COPIES; ++i) {
    const int row = 16 * (B_COPIES * wid + i) + (lane >> 2);
    const int c = (lane & 3) ^ ((row >> 2) & 3);
    int wr;
    if (GU) {
      const int rr = row % WN, half = rr / (WN / 2);
      int j = n0 + (row / WN) * (WN / 2) + rr % (WN / 2);
      j = j < N ? j : N - 1;
      wr = half ? N + j : j;
    } else {
      wr = n0 + row;
      wr = wr < N ? wr : N - 1;
    }
    b_voff[i] = (uint32_t)((int64_t)wr * ldw + c * 16) + (uint32_t)(DMA_BIAS - (i % 4) * 1024);
  }
  const char *const xb = reinterpret_cast<const char *>(x) - DMA_BIAS;
  const char *const wb = reinterpret_cast<const char *>(w) - DMA_BIAS;
  const uint32_t lds0 = lds_offset(lds);
  const uint32_t a_dst = lds0 + (uint32_t)(A_COPIES * wid) * 1024;
  const uint32_t b_dst = lds0 + A_BYTES + (uint32_t)(B_COPIES * wid) * 1024;

// Copies [LO_, HI_) of K tile kt_ into stage st_ (copies 0..A_COPIES-1 are
// the A copies, the rest the B copies).
// A copy's local index li (within A or B) selects M0 group li/4 and
// instruction offset (li%4)*1024; the per-lane offsets are stored
// pre-adjusted by -(li%4)*1024 bytes. M0 is written at the first copy of a
// part and of each group. The K tile's byte offset goes into the SGPR base.
#define RA_ISSUE_PART(kt_, st_, LO_, HI_)                                                   \
  {                                                                                         \
    const int ko_ = uniform_if<SPLIT && (BMB > 1)>((kt0 + (kt_)) * BK);                     \
    const char *sa_ = xb + (int64_t)ko_ * 2;                                                \
    const char *sb_ = wb + (int64_t)ko_;                                                    \
    const uint32_t so_ = (uint32_t)(st_) * STAGE;                                           \
    static_for_int<LO_, HI_>([&](auto ic_) {                                                    \
      constexpr int i = decltype(ic_)::value;                                               \
      constexpr bool isA = i < A_COPIES;                                                    \
      constexpr int li = isA ? i : i - A_COPIES;                                            \
      constexpr bool fresh = i == (LO_) || i == A_COPIES || li % 4 == 0;                    \
      const uint32_t m0v = (isA ? a_dst : b_dst) + so_ + (uint32_t)(li / 4) * 4096;         \
      if constexpr (isA)                                                                    \
        dma16s<(li % 4) * 1024, fresh>(sa_, a_voff[li], m0v);                              \
      else                                                                                  \
        dma16s<(li % 4) * 1024, fresh>(sb_, b_voff[li], m0v);                              \
    });                                                                                     \
  }
#define RA_ISSUE(kt_, st_) RA_ISSUE_PART(kt_, st_, 0, COPIES)
// In the steady state a tile's copies are spread over the first three
// sub-steps of the following tile: issued in one burst they stall the wave
// behind the address unit (measured: ~17% of the MFMA rate).
constexpr int P1 = (COPIES + 2) / 3, P2 = (2 * COPIES + 2) / 3;

  f32x16 acc[BMB][BNB];
#pragma unroll
  for (int i = 0; i < BMB; ++i)
#pragma unroll
    for (int j = 0; j < BNB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Rows of this lane's fragments: A row wm*WM + 32*bi + l32, B row
  // wn*WN + 32*bj + l32; the swizzle terms reduce to l32 because WM/2 and
  // WN/4 are multiples of 8 and 4.
  const int a_row_off = (wm * WM + l32) * 128;
  const int b_row_off = A_BYTES + (wn * WN + l32) * 64;
  const int a_sw = (l32 >> 1) & 7;
  const int b_sw = (l32 >> 2) & 3;

  // Software pipeline at sub-step granularity (4 sub-steps of 16 k per K
  // tile), with the order pinned by scheduling groups so that LDS latency and
  // dequantisation hide under the MFMAs. Sub-step ss issues its copies, then
  // its 16-ish MFMAs with the LDS reads for ss+1 slotted one after each of
  // the first MFMAs (a burst of reads stalls the wave behind the LDS queue)
  // and three dequantisation VALU instructions after each MFMA.
  // A fragments ping-pong in fa[2]; the raw 16-byte B fragments of sub-step
  // pair p sit in fbr[p] (pair 1 is read during sub-step 0, pair 0 of the
  // next tile during sub-step 3); dequantised B ping-pongs in bq[2]. The tile
  // boundary (wait for the next tile's copies, barrier, first reads of the
  // next tile) opens sub-step 3. Stage indices are compile-time constants in
  // the steady state, so every LDS address is a base register plus an
  // immediate offset.
  uint4 fa[2][BMB], fbr[2][BNB], bq[2][BNB];
#define RA_READ_A(st_, ss_, FA)                                                                     \
  {                                                                                                 \
    const uint8_t *base_ = lds + (st_) * STAGE;                                                     \
    _Pragma("unroll") for (int bi = 0; bi < BMB; ++bi) FA[bi] = *reinterpret_cast<const uint4 *>(   \
        base_ + a_row_off + bi * 32 * 128 + (((4 * ((ss_) >> 1) + 2 * g + ((ss_) & 1)) ^ a_sw) << 4)); \
  }
#define RA_READ_B(st_, p_, FB)                                                                      \
  {                                                                                                 \
    const uint8_t *base_ = lds + (st_) * STAGE;                                                     \
    _Pragma("unroll") for (int bj = 0; bj < BNB; ++bj) FB[bj] = *reinterpret_cast<const uint4 *>(   \
        base_ + b_row_off + bj * 32 * 64 + (((2 * (p_) + g) ^ b_sw) << 4));                         \
  }
// The 64-row tiles (one 32-row block per wave; M <= 64 and the split plans)
// spend more VALU than MFMA cycles per sub-step on dequantisation and take
// the 1-VALU-per-value conversion (M=64 K=4096 N=11008: 19.7 -> 18.9 us);
// the large tiles keep the magic-number form, which their scheduling groups
// interleave with the MFMAs (the opaque asm form measured 2 % slower there).
#define RA_DQ_(a_, b_) (BMB == 1 ? Ac::dq8s(a_, b_) : Ac::dq8(a_, b_))
#define RA_DEQ(h_, FB, BQ)                                                                          \
  _Pragma("unroll") for (int bj = 0; bj < BNB; ++bj) BQ[bj] =                                       \
      (h_) ? RA_DQ_(FB[bj].z, FB[bj].w) : RA_DQ_(FB[bj].x, FB[bj].y);
#define RA_MMA(FA, BQ)                                                                              \
  _Pragma("unroll") for (int bi = 0; bi < BMB; ++bi)                                                \
      _Pragma("unroll") for (int bj = 0; bj < BNB; ++bj) acc[bi][bj] = Ac::mfma32(FA[bi], BQ[bj], acc[bi][bj]);
// The BMB*BNB MFMAs of a sub-step: one LDS read after each of the first NR_,
// three VALU instructions after each.
#define RA_INTERLEAVE(NR_)                                                                          \
  static_for_int<0, BMB * BNB>([&](auto ic_) {                                                      \
    constexpr int i_ = decltype(ic_)::value;                                                        \
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                              \
    if constexpr (i_ < (NR_)) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                    \
    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);                                              \
  });                                                                                               \
  __builtin_amdgcn_sched_barrier(0);
// Sub-steps 0..2 of the tile in stage st_; with ISSUE_, the copies of tile
// ikt_ into stage ist_ are issued in three parts.
#define RA_SUBSTEPS_012(st_, ISSUE_, ikt_, ist_)                                                    \
  if (ISSUE_) RA_ISSUE_PART(ikt_, ist_, 0, P1);                                                     \
  __builtin_amdgcn_sched_barrier(0);                                                                \
  RA_READ_A(st_, 1, fa[1]);                                                                         \
  RA_READ_B(st_, 1, fbr[1]);                                                                        \
  RA_MMA(fa[0], bq[0]);                                                                             \
  RA_DEQ(1, fbr[0], bq[1]);                                                                         \
  RA_INTERLEAVE(BMB + BNB);                                                                         \
  if (ISSUE_) RA_ISSUE_PART(ikt_, ist_, P1, P2);                                                    \
  __builtin_amdgcn_sched_barrier(0);                                                                \
  RA_READ_A(st_, 2, fa[0]);                                                                         \
  RA_MMA(fa[1], bq[1]);                                                                             \
  RA_DEQ(0, fbr[1], bq[0]);                                                                         \
  RA_INTERLEAVE(BMB);                                                                               \
  if (ISSUE_) RA_ISSUE_PART(ikt_, ist_, P2, COPIES);                                                \
  __builtin_amdgcn_sched_barrier(0);                                                                \
  RA_READ_A(st_, 3, fa[1]);                                                                         \
  RA_MMA(fa[0], bq[0]);                                                                             \
  RA_DEQ(1, fbr[1], bq[1]);                                                                         \
  RA_INTERLEAVE(BMB);
// Tile boundary + sub-step 3: this tile's LDS reads are complete; wait until
// only the copies of tiles younger than kt_+1 are in flight, then the barrier
// makes tile kt_+1 visible and frees stage st_ (for tile kt_+S, copied during
// the next tile); then the last MFMAs of tile kt_ with the first reads of
// tile kt_+1 (B first: the dequantisation of its first B fragments, after
// half the MFMAs, needs them).
#define RA_BOUNDARY_SUBSTEP3(kt_, st_, YOUNGER_)                                                    \
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");                                                \
  wait_tiles<COPIES, S - 1>(YOUNGER_);                                                                     \
  asm volatile("s_barrier" ::: "memory");                                                           \
  {                                                                                                 \
    const int sn_ = ((kt_) + 1) % S;                                                                \
    RA_READ_B(sn_, 0, fbr[0]);                                                                      \
    RA_READ_A(sn_, 0, fa[0]);                                                                       \
  }                                                                                                 \
  RA_MMA(fa[1], bq[1]);                                                                             \
  RA_DEQ(0, fbr[0], bq[0]);                                                                         \
  static_for_int<0, BMB * BNB>([&](auto ic_) {                                                      \
    constexpr int i_ = decltype(ic_)::value;                                                        \
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                              \
    if constexpr (i_ < BMB + BNB) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                \
    if constexpr (i_ >= (BMB * BNB) / 2) __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);         \
  });                                                                                               \
  __builtin_amdgcn_sched_barrier(0);

  const int KT = SPLIT ? min(K / BK - kt0, ksplit) : K / BK;  // K tiles of this workgroup (>= 1)
#pragma unroll
  for (int s = 0; s < S; ++s)
    if (s < KT) RA_ISSUE(s, s);
  wait_tiles<COPIES, S - 1>(min(KT, S) - 1);
  asm volatile("s_barrier" ::: "memory");
#ifdef RA_TRACE
  tr_ready = __builtin_amdgcn_s_memrealtime();
#endif
  RA_READ_A(0, 0, fa[0]);
  RA_READ_B(0, 0, fbr[0]);
  RA_DEQ(0, fbr[0], bq[0]);
  int kt = 0;
  if (KT > 1) {
    // Tile 0: tiles 1 .. min(KT, S)-1 are in flight (prologue copies).
    RA_SUBSTEPS_012(0, false, 0, 0);
    RA_BOUNDARY_SUBSTEP3(0, 0, min(KT - 2, S - 2));
    // Steady state: tile kt copies tile kt+S-1 into the stage freed at the
    // last boundary; at its own boundary S-2 younger tiles are in flight.
    // Unrolled by S (stage kt % S known at compile time).
    auto steady = [&](auto stc, int ktv) __attribute__((always_inline)) {
      constexpr int st = decltype(stc)::value;
      RA_SUBSTEPS_012(st, true, ktv + S - 1, (st + S - 1) % S);
      RA_BOUNDARY_SUBSTEP3(ktv, st, S - 2);
    };
    for (kt = 1; kt + S <= KT - S + 1; kt += S) {
      static_for_int<0, S>([&](auto jc) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value;
        steady(std::integral_constant<int, (1 + j) % S>{}, kt + j);
      });
    }
    static_for_int<0, S - 1>([&](auto jc) __attribute__((always_inline)) {
      constexpr int j = decltype(jc)::value;
      if (kt <= KT - S) {
        steady(std::integral_constant<int, (1 + j) % S>{}, kt);
        ++kt;
      }
    });
    // Drain: every copy is issued.
    for (; kt < KT - 1; ++kt) {
      const int st = kt % S;
      RA_SUBSTEPS_012(st, false, 0, 0);
      RA_BOUNDARY_SUBSTEP3(kt, st, KT - 2 - kt);
    }
  }
  // Last tile.
  {
    const int st = kt % S;
    RA_SUBSTEPS_012(st, false, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    RA_MMA(fa[1], bq[1]);
  }
#undef RA_BOUNDARY_SUBSTEP3
#undef RA_SUBSTEPS_012
#undef RA_INTERLEAVE
#undef RA_DEQ
#undef RA_DQ_
#undef RA_MMA
#undef RA_READ_B
#undef RA_READ_A
#undef RA_ISSUE
#undef RA_ISSUE_PART

#ifdef RA_TRACE
  tr_kend = __builtin_amdgcn_s_memrealtime();
#endif
  if constexpr (SPLIT) {
    if (nsplit > 1) {
      // Partial sums through the level all XCDs share (sc1 stores / loads).
      __shared__ int s_last;
      constexpr int CH = BMB * BNB * 4;  // 16-byte chunks per lane
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          part + (size_t)t * nsplit * 4 * CH * 256, 0, nsplit * 4 * CH * 256 * (int)sizeof(float), kRsrcWord3);
      auto off = [&](int split, int c) { return (uint32_t)((((split * 4 + wid) * CH + c) * 64 + lane) * 16); };
#pragma unroll
      for (int bi = 0; bi < BMB; ++bi)
#pragma unroll
        for (int bj = 0; bj < BNB; ++bj)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x16 &a = acc[bi][bj];
            store_dev16(rs, off(sp, (bi * BNB + bj) * 4 + q), f32x4{a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]});
          }
      wait_vmcnt<0>();  // this wave's partial sums are stored
      __syncthreads();  // and every wave's
      if (tid == 0) s_last = __hip_atomic_fetch_add(&cnt[t], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nsplit - 1;
      __syncthreads();
      if (!s_last) return;
      // Sum the splits in order 0..nsplit-1 (this workgroup's from
      // registers): every other split's chunks are loaded at once (one
      // round trip; loading split by split cost a round trip each), then
      // added in order; above 12 chunks per lane (128-row tiles) in groups
      // of 8, one round trip each, to bound the registers they take.
      constexpr int NC = BMB * BNB * 4;
      constexpr int CG = NC <= 12 ? NC : 8;
#pragma unroll
      for (int g0 = 0; g0 < NC; g0 += CG) {
        f32x4 o[kMaxTileSplits][CG];
#pragma unroll
        for (int s2 = 0; s2 < kMaxTileSplits; ++s2)
#pragma unroll
          for (int c = 0; c < CG; ++c)
            if (g0 + c < NC && s2 < nsplit && s2 != sp) o[s2][c] = load_dev16(rs, off(s2, g0 + c));
#pragma unroll
        for (int c = 0; c < CG; ++c) {
          if (g0 + c >= NC) break;
          const int bi = (g0 + c) / (BNB * 4), bj = (g0 + c) / 4 % BNB, q = (g0 + c) % 4;
          const f32x16 &a = acc[bi][bj];
          const f32x4 own{a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]};
          f32x4 v = sp == 0 ? own : o[0][c];
#pragma unroll
          for (int s2 = 1; s2 < kMaxTileSplits; ++s2)
            if (s2 < nsplit) v += s2 == sp ? own : o[s2][c];
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[bi][bj][4 * q + e] = v[e];
        }
      }
      if (tid == 0) __hip_atomic_store(&cnt[t], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // ---- epilogue: scale (+ bias) or the gate/up SwiGLU on the fp32 sums ----
  // Lane (l32, g) holds, for block (bi, bj), column l32 of rows
  // 32*bi + r(e) + 4g, r(e) = (e & 3) + 8 * (e >> 2). The row offsets
  // r(e) * ldy are uniform; the bias test and the row guard (only tiles that
  // reach past M need it) are hoisted out of the store loops.
  // Addresses: a uniform base (wave's first row and column) plus a 32-bit
  // per-lane element offset (BM * ldy < 2^31 is checked on the host).
  const int row_l = m0 + wm * WM + 4 * g;
  const int rows_left = M - row_l;  // rows r < rows_left are in range
  const int col_w = n0 + wn * (GU ? WN / 2 : WN);  // wave's first output column
  uint16_t *const yw = y + (int64_t)(m0 + wm * WM) * ldy + col_w;
  const uint32_t ldy32 = (uint32_t)ldy;
  const uint32_t lane_off = 4u * (uint32_t)g * ldy32 + (uint32_t)l32;
  // Non-temporal stores: the tile is written once and not read back by this
  // launch (M=2048 K=4096 N=11008: 153.3 -> 152.4 us, same-box A/B).
  auto store_blocks = [&](auto guard_c, auto bias_c) {
    constexpr bool GUARD = decltype(guard_c)::value, HAS_BIAS = decltype(bias_c)::value;
    if constexpr (GU) {
#pragma unroll
      for (int bj = 0; bj < BNB / 2; ++bj) {
        const int j = n0 + wn * (WN / 2) + bj * 32 + l32;
        if (j >= N) continue;
        const float sg = scale[j], su = scale[N + j];
#pragma unroll
        for (int bi = 0; bi < BMB; ++bi)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int r = bi * 32 + (e & 3) + 8 * (e >> 2);
            if (!GUARD || r < rows_left)
              __builtin_nontemporal_store((uint16_t)swiglu_out<Ac>(acc[bi][bj][e] * sg, acc[bi][bj + BNB / 2][e] * su),
                                          &yw[lane_off + (uint32_t)r * ldy32 + 32u * bj]);
          }
      }
    } else {
#pragma unroll
      for (int bj = 0; bj < BNB; ++bj) {
        const int n = n0 + wn * WN + bj * 32 + l32;
        if (n >= N) continue;
        const float sn = scale[n];
        const float bn = HAS_BIAS ? load_as_f32(bias, n, bias_dt) : 0.f;
#pragma unroll
        for (int bi = 0; bi < BMB; ++bi)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int r = bi * 32 + (e & 3) + 8 * (e >> 2);
            if (!GUARD || r < rows_left) {
              float v = acc[bi][bj][e] * sn;
              if (HAS_BIAS) v += bn;
              __builtin_nontemporal_store((uint16_t)Ac::out(v), &yw[lane_off + (uint32_t)r * ldy32 + 32u * bj]);
            }
          }
      }
    }
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  const bool guard = m0 + BM > M;
  if (bias) {
    if (guard) store_blocks(T_{}, T_{});
    else store_blocks(F_{}, T_{});
  } else {
    if (guard) store_blocks(T_{}, F_{});
    else store_blocks(F_{}, F_{});
  }
#ifdef RA_TRACE
  if constexpr (!SPLIT) {
    if (part != nullptr) {
      wait_vmcnt<0>();
      const uint64_t tr_end = __builtin_amdgcn_s_memrealtime();
      const uint64_t tr_end_clk = __builtin_amdgcn_s_memtime();
      const uint32_t hwid = __builtin_amdgcn_s_getreg((31 << 11) | 4);
      const uint32_t xcc = __builtin_amdgcn_s_getreg((31 << 11) | 20);
      if (lane == 0) {
        uint64_t *rec = reinterpret_cast<uint64_t *>(part) + ((size_t)blockIdx.x * 4 + wid) * 8;
        rec[0] = tr_entry; rec[1] = tr_ready; rec[2] = tr_kend; rec[3] = tr_end;
        rec[4] = ((uint64_t)xcc << 32) | hwid; rec[5] = tr_entry_clk; rec[6] = tr_end_clk; rec[7] = (uint64_t)t;
      }
    }
  }
#endif
}

static bool tiled_shape_ok(int x_dt, const void *x, int64_t ldx, const int8_t *w, int64_t ldw, int64_t ldy,
                           int64_t M, int64_t N, int64_t K) {
  if (x_dt != RA_F16 && x_dt != RA_BF16) return false;
  if (M > ((int64_t)1 << 30) || N > ((int64_t)1 << 30) || K > ((int64_t)1 << 30)) return false;
  if (K % 16 != 0) return false;
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(w) & 15)) return false;
  if ((ldx % 8) != 0 || (ldw % 16) != 0) return false;
  if (ldy > ((int64_t)1 << 22)) return false;  // 32-bit epilogue offsets: 256 * ldy < 2^31
  const int64_t tiles = ((M + tiled::BM - 1) / tiled::BM) * ((N + tiled::BN - 1) / tiled::BN);
  return tiles < ((int64_t)1 << 31);
}

bool tiled_supported(const GemmArgs &a) {
  return tiled_shape_ok(a.x_dt, a.x, a.ldx, a.w, a.ldw, a.ldy, a.M, a.N, a.K);
}

// M <= 64 (not gate/up): 64 x 64 tiles with a six-stage copy pipeline. For
// M = 33..64 with at least 8192 weight rows they are ahead of the
// small-batch kernel, whose activation tiles are padded to 64 rows (M=64
// K=4096 N=11008: 19.7 vs 23.6 us; N=4096 level); for M <= 32 behind (M=32
// 19.6 vs 15.3, M=17 18.6 vs 12.5): the 64 x 64 tile costs about the same
// from M = 17 to 64.
constexpr int64_t kSmallTileMaxM = 64;
constexpr int64_t kSmallTileMinM = 33;
constexpr int64_t kSmallTileMinN = 8192;

// The copies address x and w through 31-bit per-lane byte offsets: a launch
// covers at most DMA_SPAN bytes of each. Larger operands are split into row
// chunks of x (and, without the gate/up pairing, of w), one launch each.
static bool dma_span_ok(bool gu, int64_t ldx, int64_t ldw, int64_t N, int64_t K, int bm) {
  if ((uint64_t)((bm - 1) * ldx + K) * 2 > DMA_SPAN) return false;  // one row tile of x
  const int64_t wrows = gu ? 2 * N : 256;                            // gate/up: both halves in one launch
  return (uint64_t)((wrows - 1) * ldw + K) <= DMA_SPAN;
}

bool tiled_small_selected(const GemmArgs &a) {
  return a.M >= kSmallTileMinM && a.M <= kSmallTileMaxM && a.N >= kSmallTileMinN && a.K > 0 &&
         a.K % tiled::BK == 0 && tiled_supported(a) && dma_span_ok(false, a.ldx, a.ldw, a.N, a.K, 256);
}

// M = 65..1024: the large tiles leave most CUs idle where N is small (M=128
// K=11008 N=4096: 16 tiles of 256 x 256), so these run the split tiles too
// (64 or 128 rows each; up to M = kSplitTileMaxM).

static bool tiled_split_eligible(const GemmArgs &a) {
  if (tiled_small_selected(a)) return true;
  // One launch covers all rows of x (its copies' 31-bit offsets).
  return a.M > kSmallTileMaxM && a.M <= kSplitTileMaxM && a.K > 0 && a.K % tiled::BK == 0 &&
         tiled_supported(a) && dma_span_ok(false, a.ldx, a.ldw, a.N, a.K, (int)std::max<int64_t>(a.M, 256));
}

static int device_cus();

// Split-K plans for the small tile (M = 33..64): 64-row tiles of 64*bnb
// weight rows (2 x 2 waves of bnb 32x32 blocks), K split over nsplit
// workgroups per tile. Time model fitted to the same-run times of every
// (bnb, nsplit) at 15 shapes (M = 33..64, K = 2048..14336, N = 8192..28672):
// a workgroup takes a_bnb + 16 us per MB it copies (64*bnb weight rows and 64
// activation rows of 128 B per K tile), a = 6 / 10 / 12 us for bnb = 1 / 2
// / 3, in rounds of one workgroup per CU, plus 2 us for the combine when
// nsplit > 1. It picks the fastest measured configuration at 13 of the 15
// and is within 0.6 us at the other two; e.g. M=64 K=11008 N=8192 27.6 us
// (bnb 2, 4 splits) against 51.3 for the 64 x 64 tile over all of K, K=8192
// N=11008 28.9 against 35.0, K=4096 N=28672 32.7 against 38.4; K=4096
// N=11008 keeps the 64 x 64 tile (19.6 us; the best split 19.4).
constexpr double kTileUs[4] = {0.0, 6.0, 10.0, 12.0};  // a_bnb
constexpr double kTileUsPerMB = 16.0;
constexpr double kTileCombineUs = 2.0;
// M = 65..256 (rows of 64-row tiles, or of 128-row tiles, bmb = 2): the
// same form refitted (least squares on relative error) to the
// same-run times of all 24 (bmb, bnb, nsplit) at M = 65 / 96 / 128 over 7
// (K, N) from K=2048 N=8192 to K=28672 N=8192: a = 1.9 / 7.9 / 10.3 us for
// bmb = 1 and 5.8 / 12.3 / 18.6 for bmb = 2 (bnb = 1 / 2 / 3), 18.8 us per
// MB, 4.5 us for the combine. Its pick is the fastest at 12 of the 21 and
// 4 % off on average (worst 18 %, K=8192 N=8192 at M=128); e.g. M=128
// K=28672 N=8192 83.1 us (128 x 128 tiles in 4 splits) against 97.5 for the
// 64-row tiles' plan, K=4096 N=28672 44.4 against 57.8.
constexpr double kTile2Us[3][4] = {{0, 0, 0, 0}, {0.0, 1.9, 7.9, 10.3}, {0.0, 5.8, 12.3, 18.6}};
constexpr double kTile2UsPerMB = 18.8;
constexpr double kTile2CombineUs = 4.5;
#ifdef RA_TUNING
extern int g_tiled_split;  // tuning builds: -1 never split, 10*bnb + nsplit forced
#endif

static int64_t large_tile_count(int64_t M, int64_t N, int cus);

TiledSplitPlan tiled_split_plan(const GemmArgs &a) {
  TiledSplitPlan best{};
  if (!tiled_split_eligible(a)) return best;
  if ((uint64_t)((a.N - 1) * a.ldw + a.K) > DMA_SPAN) return best;  // one launch covers all of W
  const int cus = device_cus();
  // M > 128: the large tiles where they fill at least half of the CUs, and
  // at M = 257..384 where they fill a whole round or N > 16384 (same-run
  // times, bf16; M=320 K=4096 N=28672, 224 tiles of 192 x 256: 99.1 us
  // against 118.2 for the split plan;
  // M=256 K=4096 N=28672, 224 tiles of 256 x 128: 59.8 us against 61.2 for
  // the split plan, N=13824, 108 tiles: 58.7 against 45.5; M=384 K=8192
  // N=8192, 128 tiles: 90.8 against 64.8, K=28672 N=8192 271.6 against
  // 220.0, K=5120 N=13824, 216 tiles: 78.0 against 61.9; M=512 K=5120
  // N=13824, 216 tiles: 67.8 against 89.4; M=768: the large tiles ahead at
  // every N >= 8192 measured).
  bool guard = true;
#ifdef RA_TUNING
  guard = g_tiled_split != -2;  // tuning builds: -2 plans past this rule
#endif
  if (guard && a.M > 2 * kSmallTileMaxM) {
    const int64_t lt = large_tile_count(a.M, a.N, cus);
    const bool mid = a.M > 4 * kSmallTileMaxM && a.M <= 6 * kSmallTileMaxM;
    if (mid ? (lt >= cus || a.N > 16384) : 2 * lt >= cus) return best;
  }
  const int64_t KT = a.K / tiled::BK;
  const int64_t tiles_m = (a.M + 63) / 64;
  auto cost = [&](int bmb, int bnb, int nsplit, int64_t ksplit) {
    const int64_t tiles = (tiles_m + bmb - 1) / bmb * ((a.N + 64 * bnb - 1) / (64 * bnb));
    const int64_t rounds = (tiles * nsplit + cus - 1) / cus;
    const double mb = (double)(64 * bnb + 128 * bmb) * 64 * ksplit * 1e-6;
    if (tiles_m > 1)
      return (double)rounds * (kTile2Us[bmb][bnb] + kTile2UsPerMB * mb) + (nsplit > 1 ? kTile2CombineUs : 0.0);
    return (double)rounds * (kTileUs[bnb] + kTileUsPerMB * mb) + (nsplit > 1 ? kTileCombineUs : 0.0);
  };
  // Up to 64 rows the split plans compete with the 64 x 64 tile over all of
  // K (the launch without a workspace); above, the best plan is taken.
  const bool one_row = tiles_m == 1;
  double best_t = one_row ? cost(1, 1, 1, KT) : 0.0;
  int force = 0;
#ifdef RA_TUNING
  force = g_tiled_split == -2 ? 0 : g_tiled_split;
  if (force < 0) return best;
#endif
  for (int bmb = 1; bmb <= kMaxTileBmb; ++bmb) {
    if (bmb > 1 && one_row) break;
    for (int bnb = 1; bnb <= 3; ++bnb) {
      for (int nsplit = 1; nsplit <= kMaxTileSplits; ++nsplit) {
        if (one_row && bnb == 1 && nsplit == 1) continue;
        if (bmb == 2 && bnb == 1 && force == 0) continue;  // 128 x 64: never the model's pick where measured
        if (force > 0 && force != 100 * (bmb - 1) + 10 * bnb + nsplit) continue;
        const int64_t tiles = (tiles_m + bmb - 1) / bmb * ((a.N + 64 * bnb - 1) / (64 * bnb));
        const int64_t ksplit = (KT + nsplit - 1) / nsplit;
        if ((nsplit - 1) * ksplit >= KT) continue;  // a split would be empty
        if (nsplit > 1 && tiles > (int64_t)(kSplitkCounterBytes / sizeof(int))) continue;
        const double t = cost(bmb, bnb, nsplit, ksplit);
        if (force > 0 || (!best.ok && !one_row) || t < best_t) {
          best.ok = true;
          best.bmb = bmb;
          best.bnb = bnb;
          best.nsplit = nsplit;
          best.ksplit = (int)ksplit;
          best.ws_bytes = nsplit > 1 ? kSplitkCounterBytes + (size_t)tiles * nsplit * 4 * (bmb * bnb * 4) * 256 * sizeof(float) : 0;
          best_t = t;
        }
      }
    }
  }
  return best;
}

template <int DT, int BMB, int BNB>
static void launch_dma_split(const GemmArgs &a, const TiledSplitPlan &p, void *ws, hipStream_t s) {
  using G = DmaTile<BMB, BNB, 2, 6>;
  const int tiles_n = (int)((a.N + G::BN - 1) / G::BN);
  const int tiles_m = (int)((a.M + G::BM - 1) / G::BM);
  int *cnt = static_cast<int *>(ws);
  float *part = p.nsplit > 1 ? reinterpret_cast<float *>(static_cast<char *>(ws) + kSplitkCounterBytes) : nullptr;
  hipLaunchKernelGGL((tiled_dma_kernel<DT, false, BMB, BNB, 2, 6, true>), dim3((unsigned)(tiles_m * tiles_n * p.nsplit)),
                     dim3(256), 0, s, static_cast<const uint16_t *>(a.x), a.ldx, a.w, a.ldw, a.scale, a.bias,
                     a.bias_dt, static_cast<uint16_t *>(a.y), a.ldy, (int)a.M, (int)a.N, (int)a.K, tiles_m, tiles_n,
                     p.nsplit, p.ksplit, part, cnt);
}

#ifdef RA_TRACE
extern void *g_trace_buf;
#endif

template <int DT, bool GU, int BMB, int BNB, int WR, int SM = 4>
static void launch_dma(const void *x, int64_t ldx, const int8_t *w, int64_t ldw, const float *scale,
                       const void *bias, int bias_dt, void *y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                       hipStream_t s) {
  using G = DmaTile<BMB, BNB, WR, SM>;
  constexpr int OUTN = GU ? G::BN / 2 : G::BN;
  // Rows of x (multiple of BM) and rows of w (multiple of OUTN) per launch.
  const int64_t mc = std::max<int64_t>(G::BM, ((int64_t)((DMA_SPAN / 2 - K) / ldx) + 1) / G::BM * G::BM);
  const int64_t nc = GU ? N : std::max<int64_t>(OUTN, ((int64_t)((DMA_SPAN - K) / ldw) + 1) / OUTN * OUTN);
  const size_t bias_sz = bias_dt == RA_F32 ? 4 : 2;
  for (int64_t ms = 0; ms < M; ms += mc) {
    for (int64_t ns = 0; ns < N; ns += nc) {
      const int64_t Mi = std::min(mc, M - ms), Ni = std::min(nc, N - ns);
      const uint16_t *xi = static_cast<const uint16_t *>(x) + ms * ldx;
      uint16_t *yi = static_cast<uint16_t *>(y) + ms * ldy + ns;
      const float *si = scale + ns;
      const void *bi = bias ? static_cast<const void *>(static_cast<const char *>(bias) + ns * bias_sz) : nullptr;
      const int tiles_m = (int)((Mi + G::BM - 1) / G::BM);
      const int tiles_n = (int)((Ni + OUTN - 1) / OUTN);
#ifdef RA_TRACE
      float *trace = reinterpret_cast<float *>(g_trace_buf);  // trace builds: per-workgroup timestamps
#else
      float *trace = nullptr;
#endif
      hipLaunchKernelGGL((tiled_dma_kernel<DT, GU, BMB, BNB, WR, SM>), dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, s,
                         xi, ldx, w + ns * ldw, ldw, si, bi, bias_dt, yi, ldy, (int)Mi, (int)Ni, (int)K, tiles_m,
                         tiles_n, 1, 0, trace, nullptr);
    }
  }
}

// Direct-to-LDS tile shapes, (BMB, BNB, WR) = per-wave 32x32 blocks and wave
// rows, and a relative cost per output element of a full tile, measured on
// MI355X with whole rounds of tiles (M=8192 K=4096 N=4096 and the 70B MLP
// shapes): 256x256 reaches ~1330 TFLOP/s, 256x192 ~1240, 192x256 ~1180,
// 256x128 ~1040.
struct DmaShape {
  int bmb, bnb, wr;
  double cost;
  int64_t bm() const { return 32 * bmb * wr; }
  int64_t bn() const { return 32 * bnb * (4 / wr); }
};
constexpr DmaShape kDmaShapes[] = {{8, 2, 1, 1.00}, {4, 3, 2, 1.10}, {3, 4, 2, 1.13}, {4, 2, 2, 1.28}};

// One workgroup per CU (160 KB LDS), so tiles run in rounds of `cus`; pick
// the shape with the least (rounds x tile area x cost).
static DmaShape pick_dma_shape(int64_t M, int64_t N, bool gu, int cus) {
  DmaShape best = kDmaShapes[3];
  double best_t = 0;
  bool first = true;
  for (const DmaShape &c : kDmaShapes) {
    if (gu && c.bnb % 2) continue;
    const int64_t bm = c.bm(), bn = c.bn(), outn = gu ? bn / 2 : bn;
    const int64_t tiles = ((M + bm - 1) / bm) * ((N + outn - 1) / outn);
    const int64_t rounds = (tiles + cus - 1) / cus;
    const double t = (double)rounds * (double)(bm * bn) * c.cost;
    if (first || t < best_t) best = c, best_t = t, first = false;
  }
  return best;
}

static int64_t large_tile_count(int64_t M, int64_t N, int cus) {
  const DmaShape c = pick_dma_shape(M, N, false, cus);
  return ((M + c.bm() - 1) / c.bm()) * ((N + c.bn() - 1) / c.bn());
}

static int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 256;
  return cus;
}

template <int DT, bool GU>
static void launch_dma_auto(const void *x, int64_t ldx, const int8_t *w, int64_t ldw, const float *scale,
                            const void *bias, int bias_dt, void *y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                            hipStream_t s, int forced) {
  DmaShape c = pick_dma_shape(M, N, GU, device_cus());
#ifdef RA_TUNING
  // Tuning builds only: forced tile shapes.
  if (forced == 3) c = {4, 2, 2, 0};
  if (forced == 4) c = {3, 4, 2, 0};
  if (forced == 5) c = {8, 2, 1, 0};
  if (forced == 6 && !GU) c = {4, 3, 2, 0};
  if (forced == 7) return launch_dma<DT, GU, 4, 4, 2>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
  if constexpr (!GU) {
    if (forced == 8) return launch_dma<DT, GU, 6, 2, 1>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
    if (forced == 9) return launch_dma<DT, GU, 7, 2, 1>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
  }
#else
  (void)forced;
#endif
  // Up to 64 rows: 64 x 64 tiles (2 x 2 waves of one 32 x 32 block each),
  // six K tiles of copies in flight.
  if constexpr (!GU) {
#ifdef RA_TUNING
    // Tuning builds only: the small tile with deeper copy pipelines.
    if (M <= kSmallTileMaxM && forced >= 10 && forced <= 13) {
      if (forced == 10) return launch_dma<DT, GU, 1, 1, 2, 8>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
      if (forced == 11) return launch_dma<DT, GU, 1, 1, 2, 10>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
      if (forced == 12) return launch_dma<DT, GU, 1, 1, 2, 12>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
      return launch_dma<DT, GU, 1, 1, 2, 4>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
    }
#endif
    if (M <= kSmallTileMaxM)
      return launch_dma<DT, GU, 1, 1, 2, 6>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
  }
  if (c.wr == 1) return launch_dma<DT, GU, 8, 2, 1>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
  if (c.bmb == 3 && c.bnb == 4)
    return launch_dma<DT, GU, 3, 4, 2>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
  if constexpr (!GU) {
    if (c.bmb == 4 && c.bnb == 3)
      return launch_dma<DT, GU, 4, 3, 2>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
  }
  launch_dma<DT, GU, 4, 2, 2>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
}

template <bool GU>
static hipError_t launch(const void *x, int64_t ldx, int x_dt, const int8_t *w, int64_t ldw,
                         const float *scale, const void *bias, int bias_dt, void *y, int64_t ldy,
                         int64_t M, int64_t N, int64_t K, hipStream_t s) {
  int forced = 0;
#ifdef RA_TUNING
  extern int g_tiled_mode;  // 0 auto, 1 register-staged kernel, 2 direct-to-LDS auto, 3.. forced shapes (5 = 256x256 1x4, 7 = 256x256 2x2)
  forced = g_tiled_mode;
  const bool use_dma = (g_tiled_mode >= 2 || (g_tiled_mode == 0 && K % tiled::BK == 0)) &&
                       dma_span_ok(GU, ldx, ldw, N, K, 256);
#else
  const bool use_dma = K % tiled::BK == 0 && dma_span_ok(GU, ldx, ldw, N, K, 256);
#endif
  if (use_dma) {
    if (x_dt == RA_F16)
      launch_dma_auto<RA_F16, GU>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s, forced);
    else
      launch_dma_auto<RA_BF16, GU>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s, forced);
    return hipGetLastError();
  }
  constexpr int OUTN = GU ? tiled::BN / 2 : tiled::BN;
  const int tiles_m = (int)((M + tiled::BM - 1) / tiled::BM);
  const int tiles_n = (int)((N + OUTN - 1) / OUTN);
  const dim3 grid((unsigned)(tiles_m * tiles_n));
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

hipError_t tiled_launch_ws(const GemmArgs &a, void *ws, size_t ws_bytes, hipStream_t s) {
  const TiledSplitPlan p = tiled_split_plan(a);
  if (!p.ok || (p.nsplit > 1 && (!ws || ws_bytes < p.ws_bytes))) return tiled_launch(a, s);
#define RA_SPLIT_GO(BMB_, BNB_)                                                    \
  if (p.bmb == BMB_ && p.bnb == BNB_) {                                            \
    if (a.x_dt == RA_F16) launch_dma_split<RA_F16, BMB_, BNB_>(a, p, ws, s);       \
    else launch_dma_split<RA_BF16, BMB_, BNB_>(a, p, ws, s);                       \
    return hipGetLastError();                                                      \
  }
  RA_SPLIT_GO(1, 1)
  RA_SPLIT_GO(1, 2)
  RA_SPLIT_GO(1, 3)
#ifdef RA_TUNING
  RA_SPLIT_GO(2, 1)
#endif
  RA_SPLIT_GO(2, 2)
  RA_SPLIT_GO(2, 3)
#undef RA_SPLIT_GO
  return tiled_launch(a, s);
}

bool gateup_tiled_supported(const GateUpArgs &a) {
  return tiled_shape_ok(a.x_dt, a.x, a.ldx, a.w, a.ldw, a.ldh, a.M, 2 * a.I, a.K);
}

hipError_t gateup_tiled_launch(const GateUpArgs &a, hipStream_t s) {
  return launch<true>(a.x, a.ldx, a.x_dt, a.w, a.ldw, a.scale, nullptr, RA_F32, a.h, a.ldh, a.M, a.I, a.K, s);
}

}  // namespace ra
