// Small-batch W8A16 GEMM with split K (3 <= M <= 64) on gfx950.
//
// Replaces the reference's Triton tile loop (src/rotalabs_accel/kernels/
// gemm.py:113-138) for small batches, where the cost is streaming the N*K
// weight bytes and every CU must also read the activation block. With one
// workgroup per CU owning R of the N rows over all of K, each CU reads the
// whole activation block (M*K*2 bytes, 512 KB at M=64 K=4096) through its
// address unit for R*K weight bytes (~176 KB): at M=64 activation reads are
// 2.7x the weight stream. Splitting K over S workgroups lets a workgroup own
// S times more rows for the same weight bytes, so it reads S times fewer
// activation bytes; the S partial sums are combined in a fixed order.
//
//  * Unit = (row block rb, K split s); a workgroup of NW = 4 or 8 waves owns
//    R = NW*TW*16 output columns (with the gate/up pair, TW gate tiles and
//    the TW matching up tiles per wave) over K range [s*kc, min(K, (s+1)*kc)).
//    With 8 waves two share each SIMD, so one wave's dequantisation, MFMAs
//    and LDS reads overlap the other's waits.
//  * Y^T = W . X^T with v_mfma_f32_16x16x32_{f16,bf16}: MFMA rows are weight
//    rows, MFMA columns activation rows (M padded to 16*MT).
//  * Both operands reach LDS through direct-to-LDS copies
//    (global_load_lds_dwordx4), staged 128 k at a time, D stages in flight:
//    - weights: each wave streams its own 16*NTW rows, 8 rows x 128 bytes per
//      1 KB copy (full lines, non-temporal), into a wave-private ring. The
//      16-byte chunks land XOR-swizzled by (row >> 1) & 7 (the swizzle is
//      applied on the global side: lane l fetches the chunk that belongs at
//      its LDS slot), so the MFMA operand reads (16 rows, same chunk) are
//      conflict-free; the int8 values are dequantised exactly in registers.
//    - activations: the stage's [16*MT, 128] fp16/bf16 block is copied once
//      per workgroup (4 rows x 256 bytes per copy, 2 rows when 8 waves share
//      16 rows; chunks swizzled by row & 15) into a ring of D+1 slots shared
//      by the waves; one barrier per stage.
//    No VGPR holds data in flight, so the pipeline depth is set by LDS alone.
//  * S = 1: the epilogue applies scale (+ bias) or the gate/up SwiGLU to the
//    fp32 sums and rounds once. S > 1: every unit stores its fp32 partial
//    sums (fragment order) in the workspace with device-scope stores, waits
//    for them, then increments its row block's counter (device-scope
//    atomic); the unit that finds the other S-1 arrived reads their partial
//    sums with device-scope loads, sums the S partials in split order
//    0..S-1 (deterministic), runs the epilogue and resets the counter to
//    zero for the next call. No unit waits for another.
#include "ra_common.h"
#include "ra_internal.h"

namespace ra {
#ifdef RA_TUNING
extern int g_sk_s, g_sk_dmax, g_sk_x1, g_sk_tw, g_sk_nw, g_sk_mt3;  // tuning builds: forced split count, depth cap, extra-row form, tiles per wave, waves, no 48-row tile
#endif

namespace sk {
constexpr int KS = 128;       // k per stage
constexpr int NW = 4;         // waves per workgroup
constexpr int kMaxM = 64;
constexpr int kLds = 159 * 1024;  // rings; the rest holds the reduction flag
// At most 3 stages in flight (<= 80 KB of LDS): measured against the deepest
// ring that fits (6): M=17 K=28672 N=8192 48.1 vs 49.6 us, K=16384 N=4096
// 22.4 vs 24.2, M=4 K=28672 level, M=64 K=28672 63.7 vs 62.9.
constexpr int kMaxD = 3;
// Counters of the split combine sit at the start of every workspace, one
// per row block, in a fixed region (a call never writes partial sums where
// another plan keeps a counter); plans with more row blocks do not split.
constexpr size_t kCounterBytes = kSplitkCounterBytes;
constexpr int kMaxCounters = (int)(kCounterBytes / sizeof(int));

constexpr int ntw(int tw, bool gu) { return gu ? 2 * tw : tw; }
constexpr int x_slot(int mt) { return mt * 4096; }            // [16*MT rows][256 bytes]
constexpr int w_slot(int tw, bool gu) { return ntw(tw, gu) * 2048; }  // per wave: [16*NTW rows][128 bytes]
constexpr int x1_slot = 256;                                  // the extra row: [128 k] of 2 bytes
constexpr int lds_bytes(int mt, int tw, bool gu, int d, int x1 = 0, int nw = NW) {
  return (d + 1) * (x_slot(mt) + x1 * x1_slot) + d * nw * w_slot(tw, gu);
}
// Activation copies per wave per stage and rows per copy: the stage's 16*MT
// rows of 256 bytes are copied by the nw waves, 4 rows (64 lanes x 16 bytes)
// per copy where the 4*MT copies divide evenly among the waves, else 2 rows
// (lanes 0..31) per copy (8 waves sharing 16 or 48 rows).
constexpr int xcw(int mt, int nw) { return (4 * mt) % nw == 0 ? 4 * mt / nw : 8 * mt / nw; }
constexpr int rpc(int mt, int nw) { return 16 * mt / (nw * xcw(mt, nw)); }
constexpr int copies(int mt, int tw, bool gu, int x1 = 0, int nw = NW) {  // per wave per stage
  return 2 * ntw(tw, gu) + xcw(mt, nw) + x1;
}
// Deepest pipeline that fits LDS and the 6-bit vmcnt.
constexpr int depth(int mt, int tw, bool gu, int dmax = kMaxD, int x1 = 0, int nw = NW) {
  int d = dmax;
  while (d > 2 && (lds_bytes(mt, tw, gu, d, x1, nw) > kLds || (d - 1) * copies(mt, tw, gu, x1, nw) > 63)) --d;
  return d;
}
// fp32 partial sums of one wave per split: NTW x MT fragments of 64 lanes x 4,
// then (extra row) the NTW row sums per lane, packed 4 to a 16-byte group.
constexpr int x1_groups(int tw, bool gu) { return (ntw(tw, gu) + 3) / 4; }
constexpr int wave_floats(int mt, int tw, bool gu, int x1) { return (ntw(tw, gu) * mt + x1 * x1_groups(tw, gu)) * 256; }
constexpr int part_floats(int mt, int tw, bool gu, int x1 = 0, int nw = NW) { return nw * wave_floats(mt, tw, gu, x1); }
// The rings fit LDS at the depth chosen.
constexpr bool fits(int mt, int tw, bool gu, int x1, int nw) {
  return lds_bytes(mt, tw, gu, depth(mt, tw, gu, kMaxD, x1, nw), x1, nw) <= kLds;
}
}  // namespace sk

// Non-temporal direct-to-LDS copy (the weight rows are read once per call).
__device__ __forceinline__ void dma16s_nt(const void *sbase, uint32_t voff, uint32_t m0_value) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt" ::"s"(m0_value), "v"(voff),
               "s"(sbase)
               : "memory", "m0");
}

// Wait until at most `younger` stages of CP copies are in flight for this wave.
template <int CP, int D>
__device__ __forceinline__ void wait_stages(int younger) {
  static_assert((D - 1) * CP <= 63, "vmcnt is a 6-bit counter");
  if constexpr (D > 5) if (younger >= 5) { wait_vmcnt<5 * CP>(); return; }
  if constexpr (D > 4) if (younger >= 4) { wait_vmcnt<4 * CP>(); return; }
  if constexpr (D > 3) if (younger >= 3) { wait_vmcnt<3 * CP>(); return; }
  if constexpr (D > 2) if (younger >= 2) { wait_vmcnt<2 * CP>(); return; }
  if (younger >= 1) { wait_vmcnt<CP>(); return; }
  wait_vmcnt<0>();
}

// X1 = 1: M = 16*MT + 1. The MFMA tiles cover rows 0 .. 16*MT-1 and the last
// row is a dot product on the VALU (v_dot2 over the weights the MFMA tiles
// already dequantised), instead of a second, almost empty 16-row MFMA tile
// (whose activation copies, LDS reads and MFMAs cost as much as a full one).
template <int DT, int MT, int TW, bool GU, int X1, int DMAX = sk::kMaxD, int NWT = sk::NW>
__global__ __launch_bounds__(64 * NWT, 1) void splitk_kernel(const char *__restrict__ xb, int64_t ldx,
                                                        const char *__restrict__ wb, int64_t ldw,
                                                        const float *__restrict__ scale,
                                                        const void *__restrict__ bias, int bias_dt,
                                                        uint16_t *__restrict__ y, int64_t ldy, int M, int N, int K,
                                                        int kc, int S, int NB, int spread,
                                                        float *__restrict__ part, int *__restrict__ cnt) {
  using A = Act<DT>;
  using namespace sk;
  constexpr int NTW = ntw(TW, GU);
  constexpr int WL = 2 * NTW;                              // weight copies per stage per wave
  constexpr int XCW = xcw(MT, NWT), RPC = rpc(MT, NWT);    // activation copies per wave, rows per copy
  constexpr int CP = WL + XCW + X1;                        // copies per stage per wave
  constexpr int D = depth(MT, TW, GU, DMAX, X1, NWT);
  constexpr int XS = x_slot(MT), WS = w_slot(TW, GU);
  constexpr int XRING = 0, WRING = (D + 1) * XS, X1RING = WRING + D * NWT * WS;
  constexpr int R = NWT * TW * 16;  // output columns per unit
  constexpr int X1L = 16 / NWT;     // lanes per wave copying the extra row (16 bytes each)
  static_assert(X1 == 0 || X1 == 1, "at most one row past the MFMA tiles");
  static_assert(NWT == 4 || NWT == 8, "4 or 8 waves per workgroup");
  static_assert(XCW * RPC * NWT == 16 * MT && (RPC == 2 || RPC == 4), "activation copies cover the tile rows");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[lds_bytes(MT, TW, GU, D, X1, NWT)];
  __shared__ int s_last;

  // Unit -> (row block, split). Units of one row block are dealt to one XCD
  // (hardware hands workgroup b to XCD b % 8), so the partial sums they
  // exchange stay close; grid slots past the last row block exit at once.
  // With `spread` (a test mode) they go to consecutive workgroups instead,
  // i.e. to different XCDs.
  const int b = blockIdx.x;
  int rb, s;
  if (spread) {
    rb = b / S;
    s = b % S;
  } else {
    const int xcd = b & 7, idx = b >> 3;
    rb = (idx / S) * 8 + xcd;
    s = idx % S;
  }
  if (rb >= NB) return;  // whole workgroup, before any barrier
  const int n0 = rb * R;
  const int kb = s * kc;
  const int ke = min(K, kb + kc);
  const int nst = (ke - kb) / KS;  // >= 1 (host)
  // Row block rb walks its stages starting at stage rb % nst (wrapping), so
  // the units in flight read different k windows. In lockstep they would all
  // read the same window, addresses equal in their low log2(ldw) bits, which
  // at ldw = 16384 gathers the weight stream on a few memory channels
  // (measured M=8 K=16384 N=16384: 44.0 us against 68.2, M=16 K=32768 N=8192
  // 43.3 against 61.3, M=8 K=8192 N=16384 26.8 against 36.7). Fixed per row
  // block: the sums stay deterministic.
  const int rot = rb % nst;

  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;

  // Weight copy j: wave rows 8j .. 8j+7; lane -> row 8j + lane/8, LDS slot
  // lane%8 <- global chunk (lane%8) ^ ((row>>1)&7). Tile t of the wave: output
  // columns n0 + 16*(wid*TW + t%TW) + i (t >= TW: the up rows N + column).
  // Columns past N are clamped (loaded, never stored).
  uint32_t wvoff[WL];
#pragma unroll
  for (int j = 0; j < WL; ++j) {
    const int row = 8 * j + (lane >> 3);
    const int t = row >> 4, i = row & 15;
    int col = n0 + 16 * (wid * TW + t % TW) + i;
    col = col < N ? col : N - 1;
    const int wrow = (GU && t >= TW) ? N + col : col;
    const int chunk = (lane & 7) ^ ((row >> 1) & 7);
    wvoff[j] = (uint32_t)((int64_t)wrow * ldw + 16 * chunk);
  }
  // Activation copy c of this wave covers block rows RPC*i .. RPC*i+RPC-1,
  // i = wid*XCW + c (RPC = 4, or 2 with lanes 0..31 when 8 waves share 16
  // rows); lane -> row RPC*i + lane/16, LDS slot lane%16 <- global chunk
  // (lane%16) ^ (row & 15). Rows past M read row M-1 (never stored).
  uint32_t xvoff[XCW];
#pragma unroll
  for (int c = 0; c < XCW; ++c) {
    const int row = RPC * (wid * XCW + c) + min(lane >> 4, RPC - 1);
    const int xrow = row < M ? row : M - 1;
    const int chunk = (lane & 15) ^ (row & 15);
    xvoff[c] = (uint32_t)(((int64_t)xrow * ldx + 8 * chunk) * 2);
  }
  const uint32_t lds0 = lds_offset(lds);
  const uint32_t wdst = lds0 + WRING + (uint32_t)wid * WS;
  const uint32_t xdst = lds0 + XRING + (uint32_t)(wid * XCW * RPC) * 256;
  // Extra row (X1): the stage's 256 bytes of row 16*MT, 256/NWT per wave,
  // copied by lanes 0..X1L-1 (16 bytes each).
  const uint32_t x1voff =
      (uint32_t)(((int64_t)(16 * MT) * ldx) * 2 + (256 / NWT) * wid + 16 * (lane & (X1L - 1)));
  const uint32_t x1dst = lds0 + X1RING + (uint32_t)((256 / NWT) * wid);

  auto issue = [&](int st) __attribute__((always_inline)) {
    const int sr = st + rot < nst ? st + rot : st + rot - nst;
    const int k = kb + sr * KS;
    const char *sw = wb + k;
    const char *sx = xb + (int64_t)k * 2;
    const uint32_t wd = wdst + (uint32_t)((st % D) * NWT * WS);
    const uint32_t xd = xdst + (uint32_t)((st % (D + 1)) * XS);
#pragma unroll
    for (int j = 0; j < WL; ++j) dma16s_nt(sw, wvoff[j], wd + 1024u * j);
#pragma unroll
    for (int c = 0; c < XCW; ++c) {
      if constexpr (RPC == 4) {
        dma16s<0, true>(sx, xvoff[c], xd + 1024u * c);
      } else {
        if (lane < 16 * RPC) dma16s<0, true>(sx, xvoff[c], xd + (uint32_t)(RPC * 256) * c);
      }
    }
    if constexpr (X1 != 0) {
      if (lane < X1L) dma16s<0, true>(sx, x1voff, x1dst + (uint32_t)((st % (D + 1)) * x1_slot));
    }
  };

  f32x4 acc[NTW][MT];
#pragma unroll
  for (int t = 0; t < NTW; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Extra row: lane (r, g) sums weight row 16t + r against row 16*MT over
  // its k = 8g .. 8g+7 of every 32; the four g are added after the loop.
  float acc1[NTW];
#pragma unroll
  for (int t = 0; t < NTW; ++t) acc1[t] = 0.f;

  for (int p = 0; p < D; ++p)
    if (p < nst) issue(p);

  const int wsw = (r >> 1) & 7;  // weight-row swizzle of this lane's rows (16t + r)
  for (int st = 0; st < nst; ++st) {
    wait_stages<CP, D>(min(D - 1, nst - 1 - st));
    __syncthreads();  // every wave's copies of stage st have landed
    const uint8_t *ws = lds + WRING + ((st % D) * NWT + wid) * WS;
    const uint8_t *xs = lds + XRING + (st % (D + 1)) * XS;
    const uint8_t *x1s = lds + X1RING + (st % (D + 1)) * x1_slot;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint4 xf[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        xf[mt] = *reinterpret_cast<const uint4 *>(xs + (16 * mt + r) * 256 + (((4 * q + g) ^ r) << 4));
      uint4 x1f;
      if constexpr (X1 != 0) x1f = *reinterpret_cast<const uint4 *>(x1s + 64 * q + 16 * g);  // 16-lane broadcast
#pragma unroll
      for (int t = 0; t < NTW; ++t) {
        const uint2 a8 = *reinterpret_cast<const uint2 *>(ws + (16 * t + r) * 128 +
                                                          (((2 * q + (g >> 1)) ^ wsw) << 4) + 8 * (g & 1));
        // The compiler-visible dequantiser (for fp16 the magic-number form):
        // same run, us, against the SDWA form with its wait state, M=17
        // K=28672 N=8192 41.4 against 43.3, other shapes within +-3 %.
        const uint4 a = A::dq8(a8.x, a8.y);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[t][mt] = A::mfma16(a, xf[mt], acc[t][mt]);
        if constexpr (X1 != 0) acc1[t] = A::dot8(a, x1f, acc1[t]);
      }
    }
    if (st + D < nst) {
      // this wave's reads of weight slot st % D are done before the slot is
      // refilled; activation slot (st + D) % (D + 1) held stage st - 1, which
      // every wave finished before the barrier above
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      issue(st + D);
    }
  }

  if constexpr (X1 != 0) {
    // the four k groups g (lanes r, r+16, r+32, r+48); every lane gets the row sum
#pragma unroll
    for (int t = 0; t < NTW; ++t) {
      acc1[t] += __shfl_xor(acc1[t], 16, 64);
      acc1[t] += __shfl_xor(acc1[t], 32, 64);
    }
  }

  if (S > 1) {
    // The partial sums are exchanged with device-scope stores and loads
    // (sc1), which write through to / read from the level shared by all
    // XCDs; a release / acquire fence would instead write back and
    // invalidate the whole L2 of the XCD, a cost every unit would pay.
    constexpr int FR = wave_floats(MT, TW, GU, X1);  // floats per wave and split
    constexpr int G1 = x1_groups(TW, GU);
    // this row block's partial sums: [S][NWT][NTW * MT fragments + G1 groups][64 lanes][4]
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        part + (size_t)rb * S * NWT * FR, 0, (int)(S * NWT * FR * sizeof(float)), kRsrcWord3);
    const uint32_t lo = (uint32_t)(wid * FR + lane * 4) * 4u;  // byte offset of this lane in split 0
#pragma unroll
    for (int t = 0; t < NTW; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        store_dev16(rs, lo + (uint32_t)(s * NWT * FR + (t * MT + mt) * 256) * 4u, acc[t][mt]);
    if constexpr (X1 != 0) {
#pragma unroll
      for (int q1 = 0; q1 < G1; ++q1) {
        f32x4 e;
#pragma unroll
        for (int i = 0; i < 4; ++i) e[i] = 4 * q1 + i < NTW ? acc1[4 * q1 + i] : 0.f;
        store_dev16(rs, lo + (uint32_t)(s * NWT * FR + (NTW * MT + q1) * 256) * 4u, e);
      }
    }
    wait_vmcnt<0>();  // this wave's partial sums are stored
    __syncthreads();  // and every wave's
    if (threadIdx.x == 0)
      s_last = __hip_atomic_fetch_add(&cnt[rb], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1;
    __syncthreads();
    if (!s_last) return;
    // Sum the splits in order 0..S-1 (this unit's from registers). The
    // fragments of CHK splits at a time are loaded together (one round trip
    // per CHK splits, at most 16 fragments in flight), then added in order.
    constexpr int CHK = NTW * MT >= 16 ? 1 : (16 / (NTW * MT) >= 4 ? 4 : 16 / (NTW * MT));
    f32x4 sum[NTW][MT];
    for (int s0 = 0; s0 < S; s0 += CHK) {
      f32x4 v[CHK][NTW][MT];
#pragma unroll
      for (int j = 0; j < CHK; ++j) {
        const int s2 = s0 + j;
        if (s2 < S && s2 != s) {
#pragma unroll
          for (int t = 0; t < NTW; ++t)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              v[j][t][mt] = load_dev16(rs, lo + (uint32_t)(s2 * NWT * FR + (t * MT + mt) * 256) * 4u);
        }
      }
#pragma unroll
      for (int j = 0; j < CHK; ++j) {
        const int s2 = s0 + j;
        if (s2 < S) {
#pragma unroll
          for (int t = 0; t < NTW; ++t)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              const f32x4 cur = s2 == s ? acc[t][mt] : v[j][t][mt];
              sum[t][mt] = s2 == 0 ? cur : sum[t][mt] + cur;
            }
        }
      }
    }
#pragma unroll
    for (int t = 0; t < NTW; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[t][mt] = sum[t][mt];
    if constexpr (X1 != 0) {
      // the extra row's sums, in split order 0..S-1 as above (one round trip per split)
#pragma unroll
      for (int q1 = 0; q1 < G1; ++q1) {
        f32x4 tot = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int s2 = 0; s2 < S; ++s2) {
          f32x4 cur;
          if (s2 == s) {
#pragma unroll
            for (int i = 0; i < 4; ++i) cur[i] = 4 * q1 + i < NTW ? acc1[4 * q1 + i] : 0.f;
          } else {
            cur = load_dev16(rs, lo + (uint32_t)(s2 * NWT * FR + (NTW * MT + q1) * 256) * 4u);
          }
          tot = s2 == 0 ? cur : tot + cur;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (4 * q1 + i < NTW) acc1[4 * q1 + i] = tot[i];
      }
    }
    if (threadIdx.x == 0) __hip_atomic_store(&cnt[rb], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // Epilogue: lane (r, g) of tile t, m-tile mt holds columns 4g .. 4g+3 of
  // the tile for activation row 16*mt + r.
#pragma unroll
  for (int t = 0; t < TW; ++t) {
    const int nb = n0 + 16 * (wid * TW + t % TW) + 4 * g;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = 16 * mt + r;
      if (m >= M) continue;
      uint16_t *yrow = y + (int64_t)m * ldy;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int n = nb + e;
        if (n >= N) continue;
        if (GU)
          yrow[n] = swiglu_out<A>(acc[t][mt][e] * scale[n], acc[TW + t][mt][e] * scale[N + n]);
        else
          yrow[n] = A::out(epilogue_value(acc[t][mt][e], scale, bias, bias_dt, n));
      }
    }
    if constexpr (X1 != 0) {
      // row 16*MT, column 16*(wid*TW + t) + r, stored by the lanes of group g == t % 4
      const int n = n0 + 16 * (wid * TW + t % TW) + r;
      if (g == (t & 3) && n < N) {
        uint16_t *yrow = y + (int64_t)(16 * MT) * ldy;
        if (GU)
          yrow[n] = swiglu_out<A>(acc1[t] * scale[n], acc1[TW + t] * scale[N + n]);
        else
          yrow[n] = A::out(epilogue_value(acc1[t], scale, bias, bias_dt, n));
      }
    }
  }
}

// ----------------------------------------------------------------------------
// Host side.
// ----------------------------------------------------------------------------
namespace {

// 16-row MFMA tiles per activation block: M = 33..48 in three.
int sk_mt(int64_t M) {
#ifdef RA_TUNING
  if (g_sk_mt3 && M > 32) return 4;  // tuning builds: pad M = 33..48 to four tiles
#endif
  return M <= 16 ? 1 : (M <= 32 ? 2 : (M <= 48 ? 3 : 4));
}

bool sk_shape_ok(int x_dt, const void *x, int64_t ldx, const int8_t *w, int64_t ldw, int64_t M, int64_t wrows,
                 int64_t K) {
  if (x_dt != RA_F16 && x_dt != RA_BF16) return false;
  if (M < 1 || M > sk::kMaxM || K < sk::KS || K % sk::KS != 0 || wrows < 1) return false;
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(w) & 15)) return false;
  if (ldx % 8 != 0 || ldw % 16 != 0) return false;
  // 32-bit per-lane copy offsets (the stage's k offset is in the SGPR base)
  if ((uint64_t)((wrows - 1) * ldw + 16 * 8) >= ((uint64_t)1 << 31)) return false;
  if ((uint64_t)((M - 1) * ldx + 8 * 16) * 2 >= ((uint64_t)1 << 31)) return false;
  return true;
}

// The extra-row form (M = 17 or 33: one 16-row MFMA tile fewer, the last row
// on the VALU), where it is measured ahead (same run, bf16, us, split-K
// kernel with the padded tile -> extra row): at M = 33 (M=33 K=4096 N=28672
// 31.0 -> 27.1, K=8192 N=8192 22.8 -> 21.1, gate/up K=8192 I=28672 92.6 ->
// 82.3), for the gate/up product at M = 17 (K=8192 I=28672 75.2 -> 73.5,
// K=4096 I=11008 28.1 -> 22.2) and for the GEMM at M = 17 from K = 16384
// (K=28672 N=8192 49.5 -> 45.6); the GEMM at M = 17 below K = 16384 is level
// over many rows and behind over few (K=4096 N=6144 11.4 against 13.0,
// K=11008 N=4096 15.5 against 16.1).
bool x1_wanted(int64_t M, int64_t K, bool gu) {
#ifdef RA_TUNING
  if (g_sk_x1 == 1) return false;  // tuning builds: 1 turns the extra-row form off, 2 on at any K
  if (g_sk_x1 == 2) return M == 17 || M == 33 || M == 49;
#endif
  return M == 33 || (M == 17 && (gu || K >= 16384));
}

int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 256;
  return cus;
}

}  // namespace

// Plan: waves per workgroup NW, tiles per wave TW and splits S minimising a
// time model of the busiest CU. Every split of a row block runs on the row
// block's XCD (workgroup b on XCD b % 8), so the busiest XCD holds
// ceil(nb / 8) * S units and its busiest CU n = ceil(that / (CUs / 8)) of
// them, up to `cap` resident at a time (LDS per workgroup). The CU streams at
// a fixed share of HBM (~28 GB/s with 4 waves per workgroup, ~36 GB/s with 8,
// whose waves hide each other's issue and waits) unless its j = min(n, cap)
// resident units keep too few weight bytes in flight (D stages of weight
// copies each) to cover the memory latency; its time is n x the unit's bytes
// (weight rows x kc, activation rows x kc x 2 at about 0.6 weight (they come
// from L2), the fp32 partial sums written and read back when S > 1) over that
// rate, plus a fixed cost per round of resident units (pipeline fill and
// drain: ~1.2 us with 4 waves, ~3.8 us with 8), plus the combining unit's
// serial read of the other S - 1 splits' partial sums. The constants are a
// least-squares fit to 2422 timed plans (every NW x TW x S at 38 shapes,
// M = 2..64, K = 2048..28672, N = 2048..57344; relative rms error 10 %):
// the model's pick is 0.7 % slower than the fastest plan on average (9 % at
// worst); the best 4-wave plans
// alone are 7 % slower on average, and the former bytes-per-round model's
// picks 29 % (it counted rounds over all CUs instead of the busiest XCD's:
// nb = 27, S = 9, 243 units for 256 CUs, but 36 on the 32 CUs of three XCDs).
// Splits whose partial sums exceed kSplitkMaxWorkspace are not considered
// (at M=32 K=28672 N=32768 a 5-way split of 192-row blocks, 21 MB of partial
// sums, measured 196.7 us against 171.7 unsplit).
SplitkPlan splitk_plan(int64_t M, int64_t N, int64_t K, bool gu, bool allow_split) {
  SplitkPlan best{};
  best.ok = false;
  if (M < 1 || M > sk::kMaxM || K < sk::KS || K % sk::KS != 0 || N < 1) return best;
  int mt = sk_mt(M), x1 = 0;
  if (x1_wanted(M, K, gu)) {
    mt = (int)(M / 16);
    x1 = 1;
  }
  const int cus = device_cus();
  const int64_t xcd_cus = std::max(cus / 8, 1);
  const int64_t stages = K / sk::KS;
  constexpr int kCuLds = 160 * 1024;
  // Fitted: CU share of HBM (bytes/us), memory latency (us), cost per round
  // (us), activation and partial-sum byte weights, and the combining unit's
  // read of the other splits' partial sums (us per byte).
  constexpr double kCuRate4 = 28.49e3, kCuRate8 = 35.69e3, kLatency = 1.055, kRound4 = 1.236, kRound8 = 3.78,
                   kActW = 0.592, kPartW = 1.708, kCombine4 = 0.037e-3, kCombine8 = 0.0176e-3;
  double best_t = 0;
  int force_s = 0, force_tw = 0, force_nw = 0;
#ifdef RA_TUNING
  force_s = g_sk_s;
  force_tw = g_sk_tw;
  force_nw = g_sk_nw;
#endif
  for (int nw = 4; nw <= 8; nw += 4)
  for (int tw = 1; tw <= 3; ++tw) {
    if (force_nw > 0 && nw != force_nw) continue;
    if (force_tw > 0 && tw != force_tw) continue;
    const int ntw = gu ? 2 * tw : tw;
    const int64_t R = (int64_t)nw * tw * 16;
    const int64_t nb = (N + R - 1) / R;
    const int smax = (allow_split && nb <= sk::kMaxCounters) ? (int)std::min<int64_t>(stages, 16) : 1;
    if (!sk::fits(mt, tw, gu, x1, nw)) continue;
    const int d = sk::depth(mt, tw, gu, sk::kMaxD, x1, nw);
    const int lds = sk::lds_bytes(mt, tw, gu, d, x1, nw) + 4;  // + the flag
    const int64_t cap = std::max(kCuLds / ((lds + 511) / 512 * 512), 1);  // resident units per CU
    const double inflight = (double)d * ntw * 16 * nw * sk::KS;  // weight bytes in flight per unit
    for (int S = 1; S <= smax; ++S) {
      if (force_s > 0 && S != force_s) continue;
      const int64_t kst = (stages + S - 1) / S;  // stages per split
      const int64_t se = (stages + kst - 1) / kst;
      if (se != S) continue;                     // a split would be empty
      const int64_t kc = kst * sk::KS;
      if (S > 1 && sk::kCounterBytes + (size_t)S * nb * sk::part_floats(mt, tw, gu, x1, nw) * 4 > kSplitkMaxWorkspace)
        continue;  // partial sums beyond the workspace limit
      const int64_t slots = ((nb + 7) / 8) * 8 * S;  // grid (XCD-grouped row blocks)
      const int64_t n = (((nb + 7) / 8) * S + xcd_cus - 1) / xcd_cus;  // units on the busiest CU
      const int64_t rounds = (n + cap - 1) / cap;
      const double wbytes = (double)(ntw * 16 * nw) * kc;
      const double xbytes = (double)std::min<int64_t>(M, 16 * mt + x1) * kc * 2;
      const double pbytes = S > 1 ? (double)sk::part_floats(mt, tw, gu, x1, nw) * 4 * (1.0 + 1.0) : 0.0;
      const double rate = std::min(nw == 8 ? kCuRate8 : kCuRate4, (double)std::min(n, cap) * inflight / kLatency);
      const double t = (double)n * (wbytes + kActW * xbytes + kPartW * pbytes) / rate +
                       (double)rounds * (nw == 8 ? kRound8 : kRound4) +
                       (nw == 8 ? kCombine8 : kCombine4) * (S - 1) * sk::part_floats(mt, tw, gu, x1, nw) * 4 +
                       1e-6 * (double)slots;
      if (!best.ok || t < best_t) {
        best = SplitkPlan{true, mt, tw, S, (int)kc, (int)nb, false, 0, 0, x1, nw};
        best_t = t;
      }
    }
  }
  if (best.ok && best.S > 1) {
    best.cnt_bytes = sk::kCounterBytes;
    best.ws_bytes =
        best.cnt_bytes + (size_t)best.S * best.nb * sk::part_floats(best.mt, best.tw, gu, best.x1, best.nw) * 4;
  }
  return best;
}

namespace {

template <int DT, int MT, int TW, bool GU, int X1, int NWT = sk::NW>
void splitk_go(const SplitkPlan &p, const void *x, int64_t ldx, const int8_t *w, int64_t ldw, const float *scale,
               const void *bias, int bias_dt, void *y, int64_t ldy, int64_t M, int64_t N, int64_t K, void *ws,
               hipStream_t s) {
  const unsigned grid = (unsigned)(p.spread ? (int64_t)p.nb * p.S : ((p.nb + 7) / 8) * 8 * p.S);
  int *cnt = static_cast<int *>(ws);
  float *part = ws ? reinterpret_cast<float *>(static_cast<char *>(ws) + p.cnt_bytes) : nullptr;
  if (NWT != sk::NW) {  // 8 waves per workgroup
    hipLaunchKernelGGL((splitk_kernel<DT, MT, TW, GU, X1, sk::kMaxD, NWT>), dim3(grid), dim3(64 * NWT), 0, s,
                       static_cast<const char *>(x), ldx, reinterpret_cast<const char *>(w), ldw, scale, bias,
                       bias_dt, static_cast<uint16_t *>(y), ldy, (int)M, (int)N, (int)K, p.kc, p.S, p.nb,
                       p.spread ? 1 : 0, part, cnt);
    return;
  }
#ifdef RA_TUNING
  if (g_sk_dmax == 2 || g_sk_dmax == 3) {  // forced pipeline depth cap
    auto k = g_sk_dmax == 2 ? splitk_kernel<DT, MT, TW, GU, X1, 2> : splitk_kernel<DT, MT, TW, GU, X1, 3>;
    hipLaunchKernelGGL(k, dim3(grid), dim3(256), 0, s, static_cast<const char *>(x), ldx,
                       reinterpret_cast<const char *>(w), ldw, scale, bias, bias_dt, static_cast<uint16_t *>(y), ldy,
                       (int)M, (int)N, (int)K, p.kc, p.S, p.nb, p.spread ? 1 : 0, part, cnt);
    return;
  }
#endif
  hipLaunchKernelGGL((splitk_kernel<DT, MT, TW, GU, X1>), dim3(grid), dim3(256), 0, s,
                     static_cast<const char *>(x), ldx, reinterpret_cast<const char *>(w), ldw, scale, bias,
                     bias_dt, static_cast<uint16_t *>(y), ldy, (int)M, (int)N, (int)K, p.kc, p.S, p.nb, p.spread ? 1 : 0,
                     part, cnt);
}

template <int DT, bool GU>
void splitk_dispatch(const SplitkPlan &p, const void *x, int64_t ldx, const int8_t *w, int64_t ldw,
                     const float *scale, const void *bias, int bias_dt, void *y, int64_t ldy, int64_t M, int64_t N,
                     int64_t K, void *ws, hipStream_t s) {
#define RA_SK8(MT_, TW_, X1_)                                                                                    \
  if constexpr (sk::fits(MT_, TW_, GU, X1_, 8))                                                               \
    if (p.nw == 8 && p.mt == MT_ && p.tw == TW_ && p.x1 == X1_)                                                \
      return splitk_go<DT, MT_, TW_, GU, X1_, 8>(p, x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, ws, s);
  RA_SK8(1, 1, 0) RA_SK8(1, 2, 0) RA_SK8(1, 3, 0)
  RA_SK8(2, 1, 0) RA_SK8(2, 2, 0) RA_SK8(2, 3, 0)
  RA_SK8(3, 1, 0) RA_SK8(3, 2, 0) RA_SK8(3, 3, 0)
  RA_SK8(4, 1, 0) RA_SK8(4, 2, 0) RA_SK8(4, 3, 0)
  RA_SK8(1, 1, 1) RA_SK8(1, 2, 1) RA_SK8(1, 3, 1)
  RA_SK8(2, 1, 1) RA_SK8(2, 2, 1) RA_SK8(2, 3, 1)
  RA_SK8(3, 1, 1) RA_SK8(3, 2, 1) RA_SK8(3, 3, 1)
#undef RA_SK8
#define RA_SK(MT_, TW_, X1_)                                                                                     \
  if (p.mt == MT_ && p.tw == TW_ && p.x1 == X1_)                                                               \
    return splitk_go<DT, MT_, TW_, GU, X1_>(p, x, ldx, w, ldw, scale, bias, bias_dt, y, ldy, M, N, K, ws, s);
  RA_SK(1, 1, 0) RA_SK(1, 2, 0) RA_SK(1, 3, 0)
  RA_SK(2, 1, 0) RA_SK(2, 2, 0) RA_SK(2, 3, 0)
  RA_SK(3, 1, 0) RA_SK(3, 2, 0) RA_SK(3, 3, 0)
  RA_SK(4, 1, 0) RA_SK(4, 2, 0) RA_SK(4, 3, 0)
  RA_SK(1, 1, 1) RA_SK(1, 2, 1) RA_SK(1, 3, 1)
  RA_SK(2, 1, 1) RA_SK(2, 2, 1) RA_SK(2, 3, 1)
  RA_SK(3, 1, 1) RA_SK(3, 2, 1) RA_SK(3, 3, 1)
#undef RA_SK
}

}  // namespace

bool splitk_supported(const GemmArgs &a) { return sk_shape_ok(a.x_dt, a.x, a.ldx, a.w, a.ldw, a.M, a.N, a.K); }

bool gateup_splitk_supported(const GateUpArgs &a) {
  return sk_shape_ok(a.x_dt, a.x, a.ldx, a.w, a.ldw, a.M, 2 * a.I, a.K);
}

hipError_t splitk_launch(const GemmArgs &a, const SplitkPlan &p, void *ws, hipStream_t s) {
  if (a.x_dt == RA_F16)
    splitk_dispatch<RA_F16, false>(p, a.x, a.ldx, a.w, a.ldw, a.scale, a.bias, a.bias_dt, a.y, a.ldy, a.M, a.N,
                                   a.K, ws, s);
  else
    splitk_dispatch<RA_BF16, false>(p, a.x, a.ldx, a.w, a.ldw, a.scale, a.bias, a.bias_dt, a.y, a.ldy, a.M, a.N,
                                    a.K, ws, s);
  return hipGetLastError();
}

hipError_t gateup_splitk_launch(const GateUpArgs &a, const SplitkPlan &p, void *ws, hipStream_t s) {
  if (a.x_dt == RA_F16)
    splitk_dispatch<RA_F16, true>(p, a.x, a.ldx, a.w, a.ldw, a.scale, nullptr, RA_F32, a.h, a.ldh, a.M, a.I, a.K,
                                  ws, s);
  else
    splitk_dispatch<RA_BF16, true>(p, a.x, a.ldx, a.w, a.ldw, a.scale, nullptr, RA_F32, a.h, a.ldh, a.M, a.I,
                                   a.K, ws, s);
  return hipGetLastError();
}

}  // namespace ra
