// Small-batch W8A16 GEMM (3 <= M <= 64) on gfx950.
//
// Replaces the reference's Triton tile loop (src/rotalabs_accel/kernels/
// gemm.py:113-138) for small batches. Like the decode kernels the cost is the
// weight stream (N*K bytes, 2*M flops per byte), but M is large enough that
// the dot products belong on the matrix cores:
//
//  * Y^T = W . X^T with v_mfma_f32_16x16x32_{f16,bf16}: MFMA rows are weight
//    rows, MFMA columns activation rows (M padded to 16*MT).
//  * A workgroup owns 16*RT weight rows (32*RT with the gate/up pair); its NW
//    waves split K into slices and combine their partial sums through LDS in a
//    fixed order (deterministic, no workspace).
//  * Weights are streamed in stages of 128 k: one stage of a wave's 16*NTW rows
//    is loaded with 128-bit loads covering 8 rows x 128 contiguous bytes per
//    wave instruction (full cache lines; the MFMA operand layout, 16 rows x 64
//    bytes per instruction, streams HBM markedly slower), D stages in flight.
//    Each stage is transposed through a wave-private LDS slot (16-byte chunks
//    XOR-swizzled by (row >> 1) & 7, conflict-free both ways) into the MFMA
//    layout, then dequantised exactly in registers.
//  * Activation fragments are read from global memory (L2-resident) in the
//    MFMA layout, in flight together with the stage's weights.
//  * Scale (+ bias) or the gate/up SwiGLU is applied to the fp32 sums, one
//    rounding.
// batch_xlds_kernel (below) takes M <= 16 with 2048 <= K <= 4096: the
// activation rows stay in LDS and the weights stream in full cache lines.
#include "ra_common.h"
#include "ra_internal.h"

namespace ra {

namespace batch {
constexpr int KS = 128;  // k per stage
constexpr int kMaxM = 64;
}  // namespace batch

template <int DT, int MT, int RT, int NW, int D, bool GU>
__global__ __launch_bounds__(NW * 64) void batch_kernel(const uint16_t *__restrict__ x, int64_t ldx,
                                                       const int8_t *__restrict__ w, int64_t ldw,
                                                       const float *__restrict__ scale,
                                                       const void *__restrict__ bias, int bias_dt,
                                                       uint16_t *__restrict__ y, int64_t ldy, int M, int N, int K,
                                                       int kslice) {
  using A = Act<DT>;
  constexpr int KS = batch::KS;
  // GU: N is the intermediate size I; tile t < RT holds gate rows, tile RT + t
  // the matching up rows (weight rows N + n).
  constexpr int NTW = GU ? 2 * RT : RT;  // 16-row weight tiles per wave
  constexpr int WROWS = 16 * NTW;
  constexpr int WL = WROWS / 8;  // 1 KB loads per stage (8 rows x 128 B each)
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar loop control
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * (16 * RT);
  const int m0 = blockIdx.y * (16 * MT);

  // LDS: the waves' transposition slots during the K loop, then their
  // partial sums for the split-K combine.
  constexpr int NACC = NTW * MT;
  constexpr int SLOT_BYTES = NW * WROWS * KS;
  constexpr int RED_BYTES = NW > 1 ? NW * NACC * 64 * 16 : 16;
  __shared__ __attribute__((aligned(16))) uint8_t smem[SLOT_BYTES > RED_BYTES ? SLOT_BYTES : RED_BYTES];

  // Stage loads: load j covers wave rows 8j .. 8j+7; lane -> row 8j + lane/8,
  // 16-byte chunk lane%8 of the row's 128-byte stage segment. Rows past N are
  // clamped (loaded, never stored).
  const int8_t *wsrc[WL];
  uint32_t wdst[WL];
#pragma unroll
  for (int j = 0; j < WL; ++j) {
    const int row = 8 * j + (lane >> 3);
    const int t = row >> 4;
    int n = n0 + 16 * (t % RT) + (row & 15);
    n = n < N ? n : N - 1;
    if (t >= RT) n += N;
    const int c = lane & 7;
    wsrc[j] = w + (int64_t)n * ldw + 16 * c;
    wdst[j] = (uint32_t)row * KS + (uint32_t)((c ^ ((row >> 1) & 7)) << 4);
  }
  // Activation fragment of lane (r, g): x[m0 + 16mt + r][k + 8g .. +7]; rows
  // past M alias row 0 (their columns are never stored).
  const uint16_t *xp[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = m0 + 16 * mt + r;
    xp[mt] = x + (int64_t)(m < M ? m : 0) * ldx + 8 * g;
  }
  uint8_t *const slot = smem + wid * (WROWS * KS);

  const int kb = wid * kslice;
  const int ke = min(K, kb + kslice);
  const int nst = ke > kb ? (ke - kb) / KS : 0;

  f32x4 acc[NTW][MT];
#pragma unroll
  for (int t = 0; t < NTW; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Ring of D stages in flight; stage st's weights and activation fragments
  // sit in slot st % D (loaded D stages ahead).
  uint4 wreg[D][WL];
  uint4 xf[D][4][MT];
#define RA_LOAD_STAGE(st_, SLOT_)                                                                   \
  {                                                                                                 \
    const int k_ = kb + KS * (st_);                                                                 \
    const int slot_ = (SLOT_);                                                                      \
    _Pragma("unroll") for (int j_ = 0; j_ < WL; ++j_) wreg[slot_][j_] =                             \
        load_stream16(wsrc[j_] + k_);                                                               \
    _Pragma("unroll") for (int s_ = 0; s_ < 4; ++s_)                                                \
        _Pragma("unroll") for (int mt_ = 0; mt_ < MT; ++mt_) xf[slot_][s_][mt_] =                   \
            *reinterpret_cast<const uint4 *>(xp[mt_] + k_ + 32 * s_);                               \
  }

#pragma unroll
  for (int p = 0; p < D; ++p)
    if (p < nst) RA_LOAD_STAGE(p, p);

  // Stage st_ in ring slot DP_ (= st_ % D; a literal after unrolling):
  // transpose its weights through the wave's LDS slot (LDS executes a wave's
  // accesses in order, so the reads see these writes and the next stage's
  // writes cannot overtake the reads), multiply, then reload the slot with
  // stage st_ + D.
#define RA_BODY(st_, DP_)                                                                           \
  {                                                                                                 \
    _Pragma("unroll") for (int j = 0; j < WL; ++j)                                                  \
        store16(slot + wdst[j], wreg[DP_][j]);                                                     \
    _Pragma("unroll") for (int s = 0; s < 4; ++s) {                                                 \
      _Pragma("unroll") for (int t = 0; t < NTW; ++t) {                                             \
        const int row = 16 * t + r;                                                                 \
        const int chunk = 2 * s + (g >> 1);                                                         \
        const uint2 q = *reinterpret_cast<const uint2 *>(                                           \
            slot + row * KS + ((chunk ^ ((row >> 1) & 7)) << 4) + 8 * (g & 1));                     \
        const uint4 a = A::dq8s(q.x, q.y);                                                           \
        _Pragma("unroll") for (int mt = 0; mt < MT; ++mt) acc[t][mt] =                              \
            A::mfma16(a, xf[DP_][s][mt], acc[t][mt]);                                               \
      }                                                                                             \
    }                                                                                               \
    if ((st_) + D < nst) RA_LOAD_STAGE((st_) + D, DP_);                                             \
  }

  int st = 0;
  for (; st + D <= nst; st += D) {
#pragma unroll
    for (int i = 0; i < D; ++i) RA_BODY(st + i, i);
  }
#pragma unroll
  for (int i = 0; i < D; ++i)
    if (st + i < nst) RA_BODY(st + i, i);
#undef RA_BODY
#undef RA_LOAD_STAGE

  // Combine the NW split-K partial sums in a fixed order, then the epilogue.
  // Output tile i = t*MT + mt (t < RT) is finished by wave i % NW.
  constexpr int NOUT = RT * MT;
  f32x4(*red)[NACC][64] = reinterpret_cast<f32x4(*)[NACC][64]>(smem);
  if (NW > 1) {
    __syncthreads();  // every wave is done with its transposition slot
#pragma unroll
    for (int t = 0; t < NTW; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) red[wid][t * MT + mt][lane] = acc[t][mt];
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < NOUT; ++i) {
    if (NW > 1 && (i % NW) != wid) continue;
    const int t = i / MT, mt = i % MT;
    f32x4 s = acc[t][mt];
    f32x4 su = acc[GU ? RT + t : t][mt];
    if (NW > 1) {
      s = red[0][i][lane];
      if (GU) su = red[0][(RT + t) * MT + mt][lane];
#pragma unroll
      for (int v = 1; v < NW; ++v) {
        s += red[v][i][lane];
        if (GU) su += red[v][(RT + t) * MT + mt][lane];
      }
    }
    const int m = m0 + 16 * mt + r;
    if (m >= M) continue;
    uint16_t *yrow = y + (int64_t)m * ldy;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n0 + 16 * t + 4 * g + q;
      if (n >= N) continue;
      if (GU)
        yrow[n] = swiglu_out<A>(s[q] * scale[n], su[q] * scale[N + n]);
      else
        yrow[n] = A::out(epilogue_value(s[q], scale, bias, bias_dt, n));
    }
  }
}

// ----------------------------------------------------------------------------
// Small batch with the activation rows resident in LDS: M <= 16,
// K % 512 == 0, 2048 <= K <= 4096.
//
// batch_kernel loads the activation fragments from L2 beside every weight
// stage, in the MFMA operand layout (16 rows x 64 bytes per load
// instruction), and holds them in registers. Here:
//  * the workgroup (K / 512 waves, 16*RT weight rows) first copies the M
//    activation rows into LDS with direct-to-LDS copies, one 1 KB row
//    segment per copy (wave w copies segment w of every row; 16-byte chunk c
//    of row j lands at chunk c ^ (j & 15), so the 16 rows an MFMA operand
//    read touches sit in 16 distinct bank groups);
//  * wave w owns 16-row tile t = w % RT and k in [512 RT kp, 512 RT (kp + 1))
//    (kp = w / RT) and streams it in 4 RT stages of 128 k, each 2 loads of
//    8 rows x 128 contiguous bytes (full cache lines), D stages in flight
//    (stage s + D is loaded once stage s is consumed). Loads return to a
//    wave in issue order, so with every stage in flight at once a wave's work
//    waits for its oldest load and piles up behind the stream (measured
//    M=16 K=4096 N=11008: 15.3 us with all 16 stages in flight, 10.9 with 2);
//  * transposes each stage through a 2 KB wave-private LDS slot into the
//    MFMA layout (load h gives lane l row 8h + (l >> 3), 16-byte chunk l & 7,
//    eight lanes per cache line; the address unit takes markedly longer when
//    consecutive lanes hit different lines, measured 9.1 vs 8.1 us for the
//    same 45 MB): lane (p = l & 15, g = l >> 4) reads chunks 2g and 2g + 1 of
//    row p, k in [32g, 32g + 32) of the stage, which feed 4 MFMA sub-steps of
//    8 k; chunks XOR-swizzled by (row >> 1) & 7 (conflict-free both ways);
//    the activation fragment of sub-step j is k = 32g + 8j .. +7 of its row
//    (the same permutation of k on both operands);
//  * combines the K parts of each tile through LDS in a fixed order.
// ----------------------------------------------------------------------------
namespace batchx {
constexpr int kMaxM = 16;
constexpr int kSeg = 512;                                 // k per copy segment (1 KB of fp16)
constexpr int kMinWaves = 4;                              // K >= 2048
constexpr int kMaxWaves = 8;                              // K <= 4096
constexpr int kXBytes = kMaxM * kSeg * kMaxWaves * 2;     // 128 KB of activation rows
constexpr int kSlot = 16 * 128;                           // one stage of a wave's tile
constexpr int kLdsBytes = kXBytes + kMaxWaves * kSlot;    // 144 KB
}  // namespace batchx

template <int DT, int RT, int D>
__global__ __launch_bounds__(512) void batch_xlds_kernel(const uint16_t *__restrict__ x, int64_t ldx,
                                                         const int8_t *__restrict__ w, int64_t ldw,
                                                         const float *__restrict__ scale,
                                                         const void *__restrict__ bias, int bias_dt, int M, int N,
                                                         uint16_t *__restrict__ y, int64_t ldy) {
  using A = Act<DT>;
  constexpr int ST = 4 * RT;  // 128-k stages per wave
  __shared__ __attribute__((aligned(1024))) uint8_t xs[batchx::kLdsBytes];
  const int nw = (int)(blockDim.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int p = lane & 15, g = lane >> 4;
  const int tile = wid % RT, kp = wid / RT;
  const int n0 = blockIdx.x * (16 * RT) + 16 * tile;
  const int k0 = kp * (batchx::kSeg * RT);
  const int row_bytes = nw * (batchx::kSeg * 2);  // LDS bytes of one activation row (2K)
  // The wave's stage s is stage (s + rot) mod ST of its K part, rot set per
  // workgroup from its XCD (b & 7) and place there (b >> 3), so the
  // workgroups in flight stream different k windows instead of one (same
  // run: M=4 K=4096 N=11008 9.9 -> 9.6 us, M=8 10.2 -> 9.95, M=16 10.85 ->
  // 10.7; N=4096 and K=2048 level).
  const int rot = (((int)blockIdx.x >> 3) ^ ((int)blockIdx.x & 7)) % ST;
  auto kst = [&](int q) __attribute__((always_inline)) { return q >= ST ? q - ST : q; };

  // Activation rows: segment wid of row j -> LDS j * row_bytes + 1024 wid.
  {
    const uint32_t base = lds_offset(xs) + (uint32_t)wid * 1024u;
    const uint16_t *src = x + batchx::kSeg * wid + 8 * lane;
    for (int j = 0; j < M; ++j)
      dma16<0, true>(src + (int64_t)j * ldx + 8 * ((lane ^ (j & 15)) - lane),
                     base + (uint32_t)(j * row_bytes));
  }

  // Weight loads, oldest first: stage s (K stage s' = (s + rot) mod ST),
  // half h covers rows n0 + 8h + (lane >> 3), bytes k0 + 128s' + 16 (lane &
  // 7) .. +15. Rows past N are clamped (loaded, never stored).
  const int8_t *wp[2];
  uint32_t wdst[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int r = 8 * h + (lane >> 3), c = lane & 7;
    int n = n0 + r;
    n = n < N ? n : N - 1;
    wp[h] = w + (int64_t)n * ldw + k0 + 16 * c;
    wdst[h] = (uint32_t)(r * 128 + ((c ^ ((r >> 1) & 7)) << 4));
  }
  uint8_t *const slot = xs + batchx::kXBytes + wid * batchx::kSlot;
  const int xr_off = p * 128, xsw = (p >> 1) & 7;
  // D stages in flight; stage s + D is loaded once stage s is consumed.
  uint4 wr[ST][2];
#pragma unroll
  for (int s = 0; s < D; ++s)
#pragma unroll
    for (int h = 0; h < 2; ++h) wr[s][h] = load_stream16(wp[h] + 128 * kst(s + rot));

  // The copies are older than the 2*D weight loads: once at most 2*D loads
  // are outstanding, this wave's copies are in LDS; the barrier makes every
  // wave's copies visible.
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * D) : "memory");

  // Activation fragments: lane (p, g) reads row min(p, M - 1) (rows past M
  // repeat row M - 1; their output columns are never stored).
  const int rr = p < M ? p : M - 1;
  const uint8_t *const xrow = xs + rr * row_bytes;
  const int sw = rr & 15;
  const int c0 = k0 / 8 + 4 * g;  // 16-byte chunk of k0 + 32g in the row

  // Two accumulators (sub-steps 0-1 and 2-3) shorten the MFMA dependency chain.
  f32x4 acc0 = f32x4{0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
#pragma unroll
  for (int s = 0; s < ST; ++s) {
    // LDS executes a wave's accesses in order: the reads see these writes,
    // and the next stage's writes cannot overtake them.
    store16(slot + wdst[0], wr[s][0]);
    store16(slot + wdst[1], wr[s][1]);
    uint4 xf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      xf[j] = *reinterpret_cast<const uint4 *>(xrow + (((c0 + 16 * kst(s + rot) + j) ^ sw) << 4));
    const uint4 X = *reinterpret_cast<const uint4 *>(slot + xr_off + (((2 * g) ^ xsw) << 4));
    const uint4 Y = *reinterpret_cast<const uint4 *>(slot + xr_off + (((2 * g + 1) ^ xsw) << 4));
    acc0 = A::mfma16(A::dq8s(X.x, X.y), xf[0], acc0);
    acc1 = A::mfma16(A::dq8s(Y.x, Y.y), xf[2], acc1);
    acc0 = A::mfma16(A::dq8s(X.z, X.w), xf[1], acc0);
    acc1 = A::mfma16(A::dq8s(Y.z, Y.w), xf[3], acc1);
    if (s + D < ST) {
#pragma unroll
      for (int h = 0; h < 2; ++h) wr[s + D][h] = load_stream16(wp[h] + 128 * kst(s + D + rot));
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  const f32x4 acc = acc0 + acc1;

  // Combine the K parts of each tile in part order; wave `tile` (kp = 0)
  // finishes it.
  const int parts = nw / RT;
  f32x4 *const red = reinterpret_cast<f32x4 *>(xs);
  f32x4 sum = acc;
  if (parts > 1) {
    __syncthreads();  // every wave is done reading the activation rows
    red[wid * 64 + lane] = acc;
    __syncthreads();
    if (kp != 0) return;
    sum = red[tile * 64 + lane];
    for (int v = 1; v < parts; ++v) sum += red[(v * RT + tile) * 64 + lane];
  }
  if (p >= M) return;
  uint16_t *yrow = y + (int64_t)p * ldy;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int n = n0 + 4 * g + q;
    if (n < N) yrow[n] = A::out(epilogue_value(sum[q], scale, bias, bias_dt, n));
  }
}

// ----------------------------------------------------------------------------
// Gate/up pair with the SwiGLU epilogue, small batch (M <= 32), the
// activation rows resident in LDS one K chunk at a time (the MLP's gate/up
// GEMM at H=8192, 2 x 28672 weight rows).
//  * Each wave owns 16 output columns: gate rows n0 .. n0+15 and up rows
//    I + n0 .. I + n0 + 15, over the whole of K (no combine between waves);
//    the workgroup's 4 waves take consecutive column blocks.
//  * K is walked in chunks of kc (a multiple of 512 dividing K, M rows x kc
//    fp16 <= 34 KB; 1024 k at M=16): the workgroup copies the chunk's M
//    activation rows into LDS with direct-to-LDS copies (1 KB row segments,
//    16-byte chunks XOR-swizzled by the row) between two barriers, then
//    streams the chunk's weights. Three workgroups share a CU (42 KB of LDS
//    each), so the others stream while one waits for its next chunk. Each
//    workgroup starts at its own chunk and wraps round, so the workgroups in
//    flight read different k windows.
//  * Weights in 128-k stages, per tile 2 loads of 8 rows x 128 contiguous
//    bytes, D stages in flight (D divides the stages of a chunk), each
//    tile's stage transposed through the wave's 2 KB LDS slot into the
//    16x16x32 MFMA layout (as in batch_xlds_kernel); the activation
//    fragments of a stage (MT = 1 or 2 16-row activation tiles) are read
//    once for both weight tiles.
// ----------------------------------------------------------------------------
namespace gux {
constexpr int kMaxM = 32;                                 // two 16-row activation tiles
constexpr int kWaves = 4;                                 // per workgroup
constexpr int kSlot = 16 * 128;
constexpr int kXBytes = 34 * 1024;                        // activation chunk
constexpr int kLdsBytes = kXBytes + kWaves * kSlot;       // 42 KB: three workgroups per CU
}  // namespace gux

template <int DT, int D, int MT = 1>
__global__ __launch_bounds__(64 * gux::kWaves) void gateup_xlds_kernel(
    const uint16_t *__restrict__ x, int64_t ldx, const int8_t *__restrict__ w, int64_t ldw,
    const float *__restrict__ scale, int M, int I, int K, int kc, uint16_t *__restrict__ h, int64_t ldh) {
  using A = Act<DT>;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[gux::kLdsBytes];
  const int nw = (int)(blockDim.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int p = lane & 15, g = lane >> 4;
  const int n0 = (blockIdx.x * nw + wid) * 16;
  const int row_bytes = 2 * kc;  // LDS bytes of one activation row of a chunk
  const int nseg = kc / 512;     // 1 KB copy segments per row and chunk
  const int spc = kc / 128;      // stages per chunk (a multiple of D)
  const int nst = K / 128;       // stages in all
  // Workgroup b walks the chunks starting at chunk ((b >> 3) ^ (b & 7)) mod
  // nch, wrapping (b & 7 is the XCD the hardware deals it to, b >> 3 its
  // place there): the workgroups in flight then stream different k windows,
  // on one XCD and across XCDs. In lockstep they all read one window, at
  // addresses equal in their low log2(ldw) bits, which gathers the weight
  // stream on fewer memory channels. Gate/up H=8192 I=28672 (same run):
  // M=8 81.4 -> 73.7 us, M=16 82.5 -> 75.2, M=17 85.4 -> 78.5, M=32 94.0 ->
  // 84.3; H=4096 I=11008 level to 5 % faster. Starting at b mod nch (XCD
  // only) or (b >> 3) mod nch (place only) was 10-20 % slower than no
  // rotation at M=5-8 (nch = 4).
  const int nch = nst / spc;
  const int rc = (((int)blockIdx.x >> 3) ^ ((int)blockIdx.x & 7)) % nch;
  const int rs = rc * spc;  // first stage
  auto wrap = [&](int q) __attribute__((always_inline)) { return q >= nst ? q - nst : q; };

  // Weight loads: the workgroup's stage s (K stage s' = (s + rs) mod nst) of
  // tile t (0 gate, 1 up), half hh covers rows n0 + 8hh + (lane >> 3) (+ I
  // for up), bytes 128s' + 16 (lane & 7) .. +15. Rows past I are clamped
  // (loaded, never stored).
  const int8_t *wp[2][2];
  uint32_t wdst[2];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int r = 8 * hh + (lane >> 3), c = lane & 7;
    int n = n0 + r;
    n = n < I ? n : I - 1;
    wp[0][hh] = w + (int64_t)n * ldw + 16 * c;
    wp[1][hh] = w + (int64_t)(I + n) * ldw + 16 * c;
    wdst[hh] = (uint32_t)(r * 128 + ((c ^ ((r >> 1) & 7)) << 4));
  }
  uint8_t *const slot = lds + gux::kXBytes + wid * gux::kSlot;
  const int xr_off = p * 128, xsw = (p >> 1) & 7;

  // Copies of the workgroup's chunk c (chunk (c + rc) mod nch of K): segment
  // sg of row m -> LDS m * row_bytes + 1024 sg, dealt to the waves in turn.
  auto copy_chunk = [&](int c) __attribute__((always_inline)) {
    c = c + rc < nch ? c + rc : c + rc - nch;
    for (int i = wid; i < M * nseg; i += nw) {
      const int m = i / nseg, sg = i - m * nseg;
      dma16<0, true>(x + (int64_t)m * ldx + (int64_t)c * kc + 512 * sg + 8 * (lane ^ (m & 15)),
                     lds_offset(lds) + (uint32_t)(m * row_bytes + 1024 * sg));
    }
  };

  copy_chunk(0);
  uint4 wr[D][2][2];
#pragma unroll
  for (int d = 0; d < D; ++d)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) wr[d][t][hh] = load_stream16(wp[t][hh] + 128 * wrap(d + rs));
  // The copies are older than the 4*D weight loads.
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(4 * D) : "memory");

  // Activation fragments: lane (p, g) of 16-row activation tile mt reads row
  // min(16 mt + p, M - 1) (rows past M repeat row M - 1; their outputs are
  // never stored); sub-step j of stage s (within the chunk) is the 16-byte
  // chunk 16s + 4g + j of the row, swizzled in its low 4 bits.
  const uint8_t *xo[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int rr = 16 * mt + p < M ? 16 * mt + p : M - 1;
#pragma unroll
    for (int j = 0; j < 4; ++j) xo[mt][j] = lds + rr * row_bytes + (((4 * g + j) ^ (rr & 15)) << 4);
  }

  f32x4 acc[2][MT];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto stage = [&](int sc, const uint4 (&wt)[2][2]) __attribute__((always_inline)) {
    uint4 xf[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) xf[mt][j] = *reinterpret_cast<const uint4 *>(xo[mt][j] + 256 * sc);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      // LDS executes a wave's accesses in order: the reads see these writes,
      // and the next writes cannot overtake them.
      store16(slot + wdst[0], wt[t][0]);
      store16(slot + wdst[1], wt[t][1]);
      const uint4 X = *reinterpret_cast<const uint4 *>(slot + xr_off + (((2 * g) ^ xsw) << 4));
      const uint4 Y = *reinterpret_cast<const uint4 *>(slot + xr_off + (((2 * g + 1) ^ xsw) << 4));
      const uint4 a0 = A::dq8s(X.x, X.y), a1 = A::dq8s(X.z, X.w), a2 = A::dq8s(Y.x, Y.y), a3 = A::dq8s(Y.z, Y.w);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[t][mt] = A::mfma16(a0, xf[mt][0], acc[t][mt]);
        acc[t][mt] = A::mfma16(a1, xf[mt][1], acc[t][mt]);
        acc[t][mt] = A::mfma16(a2, xf[mt][2], acc[t][mt]);
        acc[t][mt] = A::mfma16(a3, xf[mt][3], acc[t][mt]);
      }
    }
  };

  // Every iteration consumes D stages and loads the next D (the same loads
  // each time, so the waits count them exactly); the last D stages follow
  // the loop. A chunk starts at a multiple of D stages: every wave has
  // finished reading the previous chunk (LDS reads done, barrier) before its
  // copies are issued, and all copies have landed (wait, barrier) before the
  // chunk is read.
  int s0 = 0;
  for (; s0 < nst - D; s0 += D) {
    if (s0 > 0 && s0 % spc == 0) {
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      copy_chunk(s0 / spc);
      asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
      stage(s0 % spc + d, wr[d]);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) wr[d][t][hh] = load_stream16(wp[t][hh] + 128 * wrap(s0 + d + D + rs));
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (s0 > 0 && s0 % spc == 0) {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    copy_chunk(s0 / spc);
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  }
#pragma unroll
  for (int d = 0; d < D; ++d) {
    stage(s0 % spc + d, wr[d]);
    __builtin_amdgcn_sched_barrier(0);
  }

  // SwiGLU of the gate/up sums: lane (p, g) holds rows 4g + q of the tile
  // (output columns n0 + 4g + q) for activation rows 16 mt + p.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + p;
    if (m >= M) continue;
    uint16_t *hrow = h + (int64_t)m * ldh;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n0 + 4 * g + q;
      if (n < I) hrow[n] = swiglu_out<A>(acc[0][mt][q] * scale[n], acc[1][mt][q] * scale[I + n]);
    }
  }
}

// ----------------------------------------------------------------------------
// Host side.
// ----------------------------------------------------------------------------
static bool batch_shape_ok(int x_dt, const void *x, int64_t ldx, const int8_t *w, int64_t ldw, int64_t M,
                           int64_t N, int64_t K) {
  if (x_dt != RA_F16 && x_dt != RA_BF16) return false;
  if (M < 1 || M > batch::kMaxM || N > ((int64_t)1 << 30) || K > ((int64_t)1 << 30)) return false;
  if (K < batch::KS || K % batch::KS != 0) return false;
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(w) & 15)) return false;
  return (ldx % 8) == 0 && (ldw % 16) == 0;
}

bool batch_supported(const GemmArgs &a) { return batch_shape_ok(a.x_dt, a.x, a.ldx, a.w, a.ldw, a.M, a.N, a.K); }

bool gateup_batch_supported(const GateUpArgs &a) {
  return batch_shape_ok(a.x_dt, a.x, a.ldx, a.w, a.ldw, a.M, a.I, a.K);
}

template <int DT, int MT, int RT, int NW, bool GU>
static void batch_go(const void *x, int64_t ldx, const int8_t *w, int64_t ldw, const float *scale, const void *bias,
                     int bias_dt, void *y, int64_t ldy, int64_t M, int64_t N, int64_t K, hipStream_t s) {
  // stages in flight per wave (registers: D * (8 + 16 MT) per lane); halved
  // with 8 or more waves per workgroup (two or more waves per SIMD)
  constexpr int D4 = MT == 1 ? 4 : (MT == 2 ? 3 : 2);
  constexpr int D = NW >= 8 ? (D4 > 2 ? D4 / 2 : 1) : D4;
  const int kslice = (int)(((K + NW - 1) / NW + batch::KS - 1) / batch::KS * batch::KS);
  const dim3 grid((unsigned)((N + 16 * RT - 1) / (16 * RT)), (unsigned)((M + 16 * MT - 1) / (16 * MT)));
  hipLaunchKernelGGL((batch_kernel<DT, MT, RT, NW, D, GU>), grid, dim3(NW * 64), 0, s,
                     static_cast<const uint16_t *>(x), ldx, w, ldw, scale, bias, bias_dt, static_cast<uint16_t *>(y),
                     ldy, (int)M, (int)N, (int)K, kslice);
}

// M tiles per workgroup: one 16-row activation tile up to M = 16, then the
// whole batch in one workgroup (activations re-read once per weight tile).
// LDS bytes of batch_kernel<., MT, RT, NW, ., GU> (the larger of the
// transposition slots and the split-K partial sums).
template <int MT, int RT, int NW, bool GU>
constexpr int batch_lds_bytes() {
  constexpr int ntw = GU ? 2 * RT : RT;
  constexpr int slots = NW * 16 * ntw * batch::KS, red = NW * ntw * MT * 64 * 16;
  return slots > red ? slots : red;
}

template <int DT, int MT, int RT, int NW, bool GU>
static void batch_go_nw(const void *x, int64_t ldx, const int8_t *w, int64_t ldw, const float *scale, const void *bias,
                        int bias_dt, void *y, int64_t ldy, int64_t M, int64_t N, int64_t K, hipStream_t s) {
  if constexpr (batch_lds_bytes<MT, RT, NW, GU>() <= 160 * 1024)
    batch_go<DT, MT, RT, NW, GU>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
  else
    batch_go<DT, MT, RT, 4, GU>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
}

template <int DT, int RT, int NW, bool GU>
static void batch_dispatch_mt(const void *x, int64_t ldx, const int8_t *w, int64_t ldw, const float *scale,
                              const void *bias, int bias_dt, void *y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                              hipStream_t s) {
  if (M <= 16) batch_go_nw<DT, 1, RT, NW, GU>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
  else if (M <= 32) batch_go_nw<DT, 2, RT, NW, GU>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
  else batch_go_nw<DT, 4, RT, NW, GU>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
}

template <int DT, int RT, bool GU>
static void batch_dispatch_rt(const void *x, int64_t ldx, const int8_t *w, int64_t ldw, const float *scale,
                              const void *bias, int bias_dt, void *y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                              hipStream_t s) {
#ifdef RA_TUNING
  extern int g_batch_nw;
  if (g_batch_nw == 4) return batch_dispatch_mt<DT, RT, 4, GU>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
  if (g_batch_nw == 16) return batch_dispatch_mt<DT, RT, 16, GU>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
#endif
  // Eight waves (each half of the K slice of four, two waves per SIMD, half
  // the stages in flight) measured faster for RT >= 2 (M=4 K=4096 N=11008
  // 12.6 -> 11.4 us, M=17 K=8192 N=57344 106 -> 88) and mixed for RT = 1.
  if constexpr (RT >= 2)
    batch_dispatch_mt<DT, RT, 8, GU>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
  else
    batch_dispatch_mt<DT, RT, 4, GU>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
}

static int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 256;
  return cus;
}

// Weight tiles per workgroup. Each workgroup streams its 16*RT rows (times 2
// with the gate/up pair) and reads the whole activation block once, so the
// cost per CU is the rows of its busiest share plus the activation bytes of
// its workgroups (L2 hits, weighted 1/4 against HBM weight bytes):
//   cost(RT) = max rows per CU + 1/4 * workgroups per CU * 2 * Mpad.
// Measured on MI355X (K=4096 N=11008): M=16 15.0 us with RT=3 vs 18.5 with
// RT=1; M=64 24.7 vs 52.6; (K=28672 N=8192 M=17) RT=2 56 us vs 66 with RT=3.
static int batch_pick_rt(int64_t M, int64_t N, bool gu, int cus) {
  const int64_t mpad = M <= 16 ? 16 : (M <= 32 ? 32 : 64);
  int best = 1;
  double best_c = 0;
  for (int rt = 1; rt <= (gu ? 2 : 3); ++rt) {
    if (gu && rt == 2 && mpad > 32) continue;  // register budget
    const int64_t wgs = (N + 16 * rt - 1) / (16 * rt);
    const int64_t per_cu = (wgs + cus - 1) / cus;
    const double c = (double)(per_cu * 16 * rt * (gu ? 2 : 1)) + 0.25 * (double)(per_cu * 2 * mpad);
    if (rt == 1 || c <= best_c) best = rt, best_c = c;
  }
  return best;
}

template <int DT, bool GU>
static void batch_dispatch(const void *x, int64_t ldx, const int8_t *w, int64_t ldw, const float *scale,
                           const void *bias, int bias_dt, void *y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                           hipStream_t s) {
  int rt = batch_pick_rt(M, N, GU, device_cus());
#ifdef RA_TUNING
  extern int g_batch_rt;
  if (g_batch_rt > 0) rt = g_batch_rt;
#endif
  if constexpr (!GU) {
    if (rt == 3) return batch_dispatch_rt<DT, 3, GU>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
  }
  if (rt == 2 && !(GU && M > 32))
    return batch_dispatch_rt<DT, 2, GU>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
  batch_dispatch_rt<DT, 1, GU>(x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, s);
}

// batch_xlds_kernel takes M <= 16 and K = 2048 .. 4096 in steps of 512
// (K / 512 = 4 .. 8 waves) when its workgroups fit in one round of the CUs
// (one per CU: 144 KB of LDS). Measured on MI355X against batch_kernel
// (us, K=4096): M=16 N=11008 10.9 vs 13.4, M=4 9.8 vs 11.5, M=16 N=4096 6.5
// vs 8.4, M=16 N=14336 12.5 vs 19.3; with fewer waves (K < 2048) the one
// workgroup per CU leaves the weight stream short of loads in flight (K=512:
// 2x slower), and batch_kernel stays.
// Tiles per workgroup: a divisor of the wave count (each tile takes an equal
// share of the waves), the fewest whose workgroups fit in one round; 0 if
// none does.
static int batch_xlds_rt(const GemmArgs &a, int cus) {
  if (a.M < 1 || a.M > batchx::kMaxM || a.K % batchx::kSeg != 0) return 0;
  const int64_t nw = a.K / batchx::kSeg;
  if (nw < batchx::kMinWaves || nw > batchx::kMaxWaves) return 0;
  for (int rt : {1, 2, 3, 4, 6, 8})  // the instantiated tile counts
    if (nw % rt == 0 && (a.N + 16 * rt - 1) / (16 * rt) <= cus) return rt;
  return 0;
}

// Stages in flight per wave: two with six or more waves (two per SIMD),
// four with fewer (measured best of 1 / 2 / 3 / 4 / all).
template <int DT, int RT, int D>
static void batch_xlds_launch(const GemmArgs &a, hipStream_t s) {
  const int nw = (int)(a.K / batchx::kSeg);
  const dim3 grid((unsigned)((a.N + 16 * RT - 1) / (16 * RT)));
  hipLaunchKernelGGL((batch_xlds_kernel<DT, RT, D>), grid, dim3(64 * nw), 0, s, static_cast<const uint16_t *>(a.x),
                     a.ldx, a.w, a.ldw, a.scale, a.bias, a.bias_dt, (int)a.M, (int)a.N,
                     static_cast<uint16_t *>(a.y), a.ldy);
}

template <int DT, int RT>
static void batch_xlds_go(const GemmArgs &a, hipStream_t s) {
  if (a.K / batchx::kSeg >= 6)
    batch_xlds_launch<DT, RT, 2>(a, s);
  else
    batch_xlds_launch<DT, RT, 4>(a, s);
}

template <int DT>
static void batch_xlds_dispatch(const GemmArgs &a, int rt, hipStream_t s) {
  if (rt == 1) return batch_xlds_go<DT, 1>(a, s);
  if (rt == 2) return batch_xlds_go<DT, 2>(a, s);
  if (rt == 3) return batch_xlds_go<DT, 3>(a, s);
  if (rt == 4) return batch_xlds_go<DT, 4>(a, s);
  if (rt == 6) return batch_xlds_go<DT, 6>(a, s);
  batch_xlds_go<DT, 8>(a, s);
}

hipError_t batch_launch(const GemmArgs &a, hipStream_t s) {
  int xrt = batch_xlds_rt(a, device_cus());
#ifdef RA_TUNING
  extern int g_batch_xlds;  // 1: never the LDS-resident kernel
  if (g_batch_xlds == 1) xrt = 0;
#endif
  if (xrt > 0) {
    if (a.x_dt == RA_F16)
      batch_xlds_dispatch<RA_F16>(a, xrt, s);
    else
      batch_xlds_dispatch<RA_BF16>(a, xrt, s);
    return hipGetLastError();
  }
  if (a.x_dt == RA_F16)
    batch_dispatch<RA_F16, false>(a.x, a.ldx, a.w, a.ldw, a.scale, a.bias, a.bias_dt, a.y, a.ldy, a.M, a.N, a.K, s);
  else
    batch_dispatch<RA_BF16, false>(a.x, a.ldx, a.w, a.ldw, a.scale, a.bias, a.bias_dt, a.y, a.ldy, a.M, a.N, a.K,
                                   s);
  return hipGetLastError();
}

// gateup_xlds_kernel: M <= 32, K % 512 == 0; workgroups of 4 waves (42 KB
// of LDS, so three share a CU and one streams while another copies its next
// chunk); the K chunk is the largest multiple of 512 that divides K, is at
// most 2048 and whose M activation rows fit in 34 KB, except that a
// 1024-k chunk becomes 512 when there are more workgroups than CUs.
// Measured (gate/up M=16 H=8192 I=28672, same run, before the chunk
// rotation): 81.0 us against 89.9 with 7 waves and 4096-k chunks (one
// workgroup per CU), 83.0 with 2048-k chunks (two per CU); 2 or 3 waves per
// workgroup 87-94. With the rotation (same run, three weight copies cycled;
// chunk k 4096 / 2048 / 1024 / 512): H=8192 I=28672 (448 workgroups) M=3-4
// 79 / 72.7 / - / 74, M=6-8 - / 73.4-74.8 / 80 / 73.9, M=12-16 - / - /
// 81-81.5 / 75-76, M=17 - / - / 84.9 / 79.9; H=4096 I=11008 (172
// workgroups) M=4 21.4 / 18.1 / - / 22.3, M=16 - / - / 21.0 / 23.7;
// H=8192 I=8192 M=16 - / - / 35.9 / 40.0.
struct GuxCfg {
  int nw = 0, kc = 0;  // waves per workgroup, k per chunk (0: not this kernel)
};

static GuxCfg gateup_xlds_cfg(const GateUpArgs &a) {
  GuxCfg c;
  if (a.M < 1 || a.M > gux::kMaxM || a.K < 512 || a.K % 512 != 0) return c;
  int64_t kc = std::min<int64_t>(std::min<int64_t>(a.K, 2048), gux::kXBytes / (2 * a.M)) / 512 * 512;
  while (kc >= 512 && a.K % kc != 0) kc -= 512;
  if (kc < 512) return c;
  const int64_t blocks = (a.I + 15) / 16;
  c.nw = (int)std::min<int64_t>(gux::kWaves, blocks);
  if (kc == 1024 && (blocks + c.nw - 1) / c.nw > device_cus()) kc = 512;
  c.kc = (int)kc;
  return c;
}

template <int DT, int D = 4, int MT = 1>
static void gateup_xlds_launch(const GateUpArgs &a, GuxCfg c, hipStream_t s) {
#ifdef RA_TUNING
  extern int g_batch_xd;  // forced stages in flight
  if constexpr (D == 4) {
    if (g_batch_xd == 2) return gateup_xlds_launch<DT, 2, MT>(a, c, s);
    if (g_batch_xd == 8 && (c.kc / 128) % 8 == 0) return gateup_xlds_launch<DT, 8, MT>(a, c, s);
  }
#endif
  const int64_t blocks = (a.I + 15) / 16;
  const dim3 grid((unsigned)((blocks + c.nw - 1) / c.nw));
  hipLaunchKernelGGL((gateup_xlds_kernel<DT, D, MT>), grid, dim3(64 * c.nw), 0, s,
                     static_cast<const uint16_t *>(a.x), a.ldx, a.w, a.ldw, a.scale, (int)a.M, (int)a.I, (int)a.K,
                     c.kc, static_cast<uint16_t *>(a.h), a.ldh);
}

hipError_t gateup_batch_launch(const GateUpArgs &a, hipStream_t s) {
  GuxCfg gc = gateup_xlds_cfg(a);
#ifdef RA_TUNING
  extern int g_batch_xlds;  // 1: never the LDS-resident kernels
  if (g_batch_xlds == 1) gc.nw = 0;
#endif
  if (gc.nw > 0) {
    if (a.x_dt == RA_F16) {
      if (a.M <= 16) gateup_xlds_launch<RA_F16, 4, 1>(a, gc, s);
      else gateup_xlds_launch<RA_F16, 4, 2>(a, gc, s);
    } else {
      if (a.M <= 16) gateup_xlds_launch<RA_BF16, 4, 1>(a, gc, s);
      else gateup_xlds_launch<RA_BF16, 4, 2>(a, gc, s);
    }
    return hipGetLastError();
  }
  if (a.x_dt == RA_F16)
    batch_dispatch<RA_F16, true>(a.x, a.ldx, a.w, a.ldw, a.scale, nullptr, RA_F32, a.h, a.ldh, a.M, a.I, a.K, s);
  else
    batch_dispatch<RA_BF16, true>(a.x, a.ldx, a.w, a.ldw, a.scale, nullptr, RA_F32, a.h, a.ldh, a.M, a.I, a.K, s);
  return hipGetLastError();
}

}  // namespace ra
