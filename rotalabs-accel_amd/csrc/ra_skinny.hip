// Split-K skinny W8A16 GEMM for decode and small batches (M <= 64) on gfx950.
//
// Replaces the reference's Triton tile loop (src/rotalabs_accel/kernels/
// gemm.py:113-138) for small M, where that kernel launches only cdiv(N, BN)
// programs with BLOCK_M >= 32 and is latency bound. Here the problem is
// memory bound (each weight byte is used for 2*M flops, far below the
// MI355X ridge of ~315 flop/B), so the design streams the int8 weight once
// at HBM speed:
//
//  * The product is computed transposed, Y^T[N,M] = W[N,K] . X^T[K,M], with
//    v_mfma_f32_16x16x32_{f16,bf16}: MFMA rows are weight rows (output
//    channels), MFMA columns are activation rows (M padded to 16*MT).
//  * Lane (r = lane%16, g = lane/16) loads 16 contiguous weight bytes
//    W[n0+r][k+16g .. k+16g+15] per 64-wide K step with one 128-bit load and
//    16 matching activations x[m][k+16g ..] with two 128-bit loads; the two
//    halves feed two MFMAs. The same k permutation is used for both operands,
//    so the dot products are unchanged.
//  * int8 -> fp16/bf16 happens in registers (exact); the per-channel scale
//    and bias are applied to the fp32 result in the epilogue.
//  * A workgroup owns 16*RT weight rows; its NW waves split K into NW slices
//    (split-K) and combine their partial sums through LDS in a fixed order, so
//    results are deterministic and no workspace or atomics are needed.
#include "ra_common.h"
#include "ra_internal.h"

namespace ra {

template <int DT, int MT, int RT, int NW, int U, bool GU>
__global__ __launch_bounds__(NW * 64) void skinny_kernel(
    const uint16_t *__restrict__ x, int64_t ldx, const int8_t *__restrict__ w, int64_t ldw,
    const float *__restrict__ scale, const void *__restrict__ bias, int bias_dt,
    uint16_t *__restrict__ y, int64_t ldy, int M, int N, int K, int kslice) {
  using A = Act<DT>;
  // GU: fused gate/up + SwiGLU. N is then the intermediate size I, weight rows
  // [0, I) are the gate projection and [I, 2I) the up projection; tile t and
  // tile RT + t hold matching gate / up rows.
  constexpr int NTW = GU ? 2 * RT : RT;
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar loop control
  const int r = lane & 15;
  const int g = lane >> 4;
  const int n0 = blockIdx.x * (16 * RT);
  const int m0 = blockIdx.y * (16 * MT);

  // Out-of-range weight rows are clamped to row N-1 (loads stay in bounds,
  // results for those rows are never stored).
  const int8_t *wp[NTW];
#pragma unroll
  for (int t = 0; t < NTW; ++t) {
    int n = n0 + 16 * (t % RT) + r;
    n = n < N ? n : N - 1;
    if (t >= RT) n += N;
    wp[t] = w + (int64_t)n * ldw + 16 * g;
  }
  const uint16_t *xp[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = m0 + 16 * mt + r;
    xp[mt] = x + (int64_t)(m < M ? m : 0) * ldx + 16 * g;
  }

  f32x4 acc[NTW][MT];
#pragma unroll
  for (int t = 0; t < NTW; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int kb = wid * kslice;
  const int ke = min(K, kb + kslice);
  const uint4 zero4 = make_uint4(0, 0, 0, 0);
  int k = kb;

  // Main loop: U full 64-wide steps per iteration, all loads issued first.
  for (; k + 64 * U <= ke; k += 64 * U) {
    uint4 wv[U][NTW], xa[U][MT], xb[U][MT];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int t = 0; t < NTW; ++t) wv[u][t] = *reinterpret_cast<const uint4 *>(wp[t] + k + 64 * u);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        // Unconditional: rows m >= M alias row 0 and only feed MFMA columns
        // that are never stored (a guarded load would be split into waited
        // per-dword loads).
        xa[u][mt] = *reinterpret_cast<const uint4 *>(xp[mt] + k + 64 * u);
        xb[u][mt] = *reinterpret_cast<const uint4 *>(xp[mt] + k + 64 * u + 8);
      }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int t = 0; t < NTW; ++t) {
        const uint4 a0 = A::dq8s(wv[u][t].x, wv[u][t].y);
        const uint4 a1 = A::dq8s(wv[u][t].z, wv[u][t].w);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc[t][mt] = A::mfma16(a0, xa[u][mt], acc[t][mt]);
          acc[t][mt] = A::mfma16(a1, xb[u][mt], acc[t][mt]);
        }
      }
  }
  // Remaining steps, one at a time; a lane group whose 16 k's lie beyond K
  // (only possible in the last step, K % 16 == 0) re-reads the first 16
  // elements of its rows (offset -16*g from its own column; K >= 16) and
  // contributes zeros.
  for (; k < ke; k += 64) {
    const bool gv = k + 16 * g + 16 <= K;
    const int kk = gv ? k : -16 * g;
    uint4 wv[NTW], xa[MT], xb[MT];
#pragma unroll
    for (int t = 0; t < NTW; ++t) {
      wv[t] = *reinterpret_cast<const uint4 *>(wp[t] + kk);
      if (!gv) wv[t] = zero4;
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      xa[mt] = *reinterpret_cast<const uint4 *>(xp[mt] + kk);
      xb[mt] = *reinterpret_cast<const uint4 *>(xp[mt] + kk + 8);
      if (!gv) xa[mt] = xb[mt] = zero4;
    }
#pragma unroll
    for (int t = 0; t < NTW; ++t) {
      const uint4 a0 = A::dq8s(wv[t].x, wv[t].y);
      const uint4 a1 = A::dq8s(wv[t].z, wv[t].w);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[t][mt] = A::mfma16(a0, xa[mt], acc[t][mt]);
        acc[t][mt] = A::mfma16(a1, xb[mt], acc[t][mt]);
      }
    }
  }

  // Combine the NW split-K partial sums in a fixed order, then the epilogue.
  // Output tile i = t*MT + mt (t < RT) is finished by wave i % NW.
  constexpr int NACC = NTW * MT;
  constexpr int NOUT = RT * MT;
  __shared__ f32x4 red[NW > 1 ? NW : 1][NACC][64];
  if (NW > 1) {
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
      if (GU) {
        yrow[n] = swiglu_out<A>(s[q] * scale[n], su[q] * scale[N + n]);
      } else {
        yrow[n] = A::out(epilogue_value(s[q], scale, bias, bias_dt, n));
      }
    }
  }
}

// ----------------------------------------------------------------------------
// Host-side configuration and launch.
// ----------------------------------------------------------------------------
template <int DT, int MT, int RT, int NW, bool GU>
static hipError_t launch_cfg(const GemmArgs &a, hipStream_t stream) {
  constexpr int U = (MT >= 4 || (GU && RT >= 2)) ? 2 : 4;
  const int kslice = (int)(((a.K + NW - 1) / NW + 63) / 64 * 64);
  dim3 grid((unsigned)((a.N + 16 * RT - 1) / (16 * RT)), (unsigned)((a.M + 16 * MT - 1) / (16 * MT)));
  hipLaunchKernelGGL((skinny_kernel<DT, MT, RT, NW, U, GU>), grid, dim3(NW * 64), 0, stream,
                     static_cast<const uint16_t *>(a.x), a.ldx, a.w, a.ldw, a.scale, a.bias, a.bias_dt,
                     static_cast<uint16_t *>(a.y), a.ldy, (int)a.M, (int)a.N, (int)a.K, kslice);
  return hipGetLastError();
}

template <int DT, bool GU>
static hipError_t launch_dt(const GemmArgs &a, const SkinnyCfg &c, hipStream_t s) {
  // Instantiated (MT, RT, NW) combinations; the selector only picks these.
#define RA_SKINNY_CASE(MT_, RT_, NW_) \
  if (c.mt == MT_ && c.rt == RT_ && c.nw == NW_) return launch_cfg<DT, MT_, RT_, NW_, GU>(a, s);
  RA_SKINNY_CASE(1, 1, 4)
  RA_SKINNY_CASE(1, 1, 8)
  RA_SKINNY_CASE(1, 2, 4)
  RA_SKINNY_CASE(1, 2, 8)
  RA_SKINNY_CASE(2, 1, 4)
  RA_SKINNY_CASE(2, 1, 8)
  RA_SKINNY_CASE(2, 2, 4)
  RA_SKINNY_CASE(4, 1, 4)
  RA_SKINNY_CASE(4, 2, 4)
#undef RA_SKINNY_CASE
  return hipErrorInvalidValue;
}

static bool skinny_shape_ok(int x_dt, const void *x, int64_t ldx, const int8_t *w, int64_t ldw, int64_t M,
                            int64_t N, int64_t K) {
  if (x_dt != RA_F16 && x_dt != RA_BF16) return false;
  if (M > 16 * 4 * 65535 || N > ((int64_t)1 << 30) || K > ((int64_t)1 << 30)) return false;
  if (K % 16 != 0) return false;
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(w) & 15)) return false;
  if ((ldx % 8) != 0 || (ldw % 16) != 0) return false;
  return true;
}

bool skinny_supported(const GemmArgs &a) {
  return skinny_shape_ok(a.x_dt, a.x, a.ldx, a.w, a.ldw, a.M, a.N, a.K);
}

SkinnyCfg skinny_select(int64_t M, int64_t N, int64_t K) {
  SkinnyCfg c;
  c.mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  const int64_t ntile = (N + 15) / 16;
  if (c.mt == 1) {
    c.rt = ntile >= 1024 ? 2 : 1;
    c.nw = 8;
  } else if (c.mt == 2) {
    c.rt = ntile >= 1024 ? 2 : 1;
    c.nw = c.rt == 2 ? 4 : 8;
  } else {
    c.rt = ntile >= 512 ? 2 : 1;
    c.nw = 4;
  }
  (void)K;
  return c;
}

hipError_t skinny_launch(const GemmArgs &a, const SkinnyCfg &c, hipStream_t s) {
  if (a.x_dt == RA_F16) return launch_dt<RA_F16, false>(a, c, s);
  return launch_dt<RA_BF16, false>(a, c, s);
}

bool gateup_skinny_supported(const GateUpArgs &a) {
  return skinny_shape_ok(a.x_dt, a.x, a.ldx, a.w, a.ldw, a.M, a.I, a.K);
}

hipError_t gateup_skinny_launch(const GateUpArgs &g, hipStream_t s) {
  GemmArgs a{g.x, g.ldx, g.x_dt, g.w, g.ldw, g.scale, nullptr, RA_F32, g.h, g.ldh, g.M, g.I, g.K};
  SkinnyCfg c = skinny_select(g.M, 2 * g.I, g.K);
  if (c.rt == 2 && c.mt == 4) c.rt = 1;
  if (a.x_dt == RA_F16) return launch_dt<RA_F16, true>(a, c, s);
  return launch_dt<RA_BF16, true>(a, c, s);
}

}  // namespace ra
