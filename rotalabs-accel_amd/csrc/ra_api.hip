// C ABI of librotaccel.so (declared in include/rotaccel.h): argument checks,
// kernel selection and error mapping. No device memory is allocated here.
#include "ra_internal.h"

namespace {

using namespace ra;

bool valid_act(int dt) { return dt == RA_F16 || dt == RA_BF16 || dt == RA_F32; }

int to_status(hipError_t e) { return e == hipSuccess ? RA_OK : RA_ERR_LAUNCH; }

#ifdef RA_TUNING
// Tuning builds only (-DRA_TUNING): force the skinny configuration.
SkinnyCfg g_skinny_override{0, 0, 0};
#endif

}  // namespace

#ifdef RA_TUNING
namespace ra {
int g_tiled_mode = 0;
int g_rows_rw = 0;
int g_rows_pipe = 0;
int g_batch_rt = 0;
int g_batch_nw = 0;
int g_batch_xlds = 0;
int g_batch_xd = 0;
int g_sk_s = 0;
int g_sk_dmax = 0;
int g_sk_x1 = 0;
int g_sk_tw = 0;
int g_sk_nw = 0;
int g_sk_mt3 = 0;
int g_tiled_split = 0;
int g_w8a8_mode = 0;
int g_gu_splitk = 0;
int g_gu_rows = 0;
int g_rows_lds = 0;
}
#endif
#ifdef RA_TRACE
namespace ra {
void *g_trace_buf = nullptr;
}
#endif

namespace {

SkinnyCfg skinny_config(int64_t M, int64_t N, int64_t K) {
  SkinnyCfg c = skinny_select(M, N, K);
#ifdef RA_TUNING
  if (g_skinny_override.mt) c = g_skinny_override;
#endif
  return c;
}

// M above which the tiled kernel is used (below it the weight stream dominates
// and the skinny split-K kernel is faster).
constexpr int64_t kSkinnyMaxM = 64;

// K from which the small-batch GEMM splits K over workgroups (given a
// workspace). Measured on MI355X (graph replay, weights streamed from HBM):
// M=17 K=28672 N=8192 47.4 us split vs 50.0 us for the one-pass batch kernel;
// at K=4096 N=11008 the one-pass kernel is ahead (M=4..64: 11.2-23.5 us vs
// 15.6-30.2), and at K=8192 N=57344 (88.6 vs 115.6).
constexpr int64_t kSplitkMinK = 16384;

// M = 1 at K <= 2048 over at least 4096 weight rows: the row GEMV's short
// rows keep too few bytes in flight per wave, and the small-batch kernel
// (at K = 2048 its activation-resident form) is ahead, or the skinny
// split-K kernel at K <= 1536 over 16384+ rows. Same run, bf16, us, row
// GEMV -> pick: K=2048 N=16384 9.61 -> 7.48, N=11008 7.80 -> 6.45, N=4096
// 4.45 -> 4.21; K=1024 N=8192 5.57 -> 4.44, N=16384 8.41 -> 6.60 (skinny);
// K=512 N=4096 4.21 -> 3.25. N=2048 and K >= 3072 stay with the row GEMV
// (K=3072 N=16384 10.59 against 11.15 for the small-batch kernel).
int one_row_short_k(const GemmArgs &a) {
  if (a.M != 1 || a.K > 2048 || a.N < 4096) return 0;
  if (a.K <= 1536 && a.N >= 16384 && skinny_supported(a)) return RA_VARIANT_SKINNY;
  return batch_supported(a) ? RA_VARIANT_BATCH : 0;
}

// M = 33..56 at short K over at most ~12K weight rows: the small-batch
// kernel is ahead of the 64-row tiles. Same run, bf16, us, tile -> small
// batch: M=33 K=2048 N=8192 12.24 -> 9.76, K=3072 N=12288 16.58 -> 16.03;
// M=40 K=1024 N=8192 9.40 -> 7.19, K=2048 N=12288 12.92 -> 12.84; M=48
// K=1024 N=11008 9.63 -> 9.38, K=2048 N=8192 12.51 -> 11.12; M=56 K=2048
// N=8192 12.54 -> 11.74. The tiles stay ahead at M=48 K=2048 N=9216 (12.85
// against 13.07), M=48 K=3072, M=56 K=1024 N=9216, M=64, K >= 4096 (M=33
// K=4096 N=11008 18.1 against 19.6) and N >= 13824 (M=33 K=2048 12.98
// against 17.89).
bool short_k_batch(const GemmArgs &a) {
  if (a.M < 33 || a.M > 56 || !batch_supported(a)) return false;
  return (a.M <= 40 && a.K <= 3072 && a.N <= 12288) || (a.K <= 2048 && a.N <= 8192) ||
         (a.M <= 48 && a.K <= 1024 && a.N <= 12288);
}

// Where the split-K kernel (4- or 8-wave plans) is measured ahead (same run,
// bf16, us, graph replay of cold weights; the other kernel -> split K):
//  * M = 2..32: K >= 16384 (M=16 K=28672 N=28672 197.0 -> 148.7, M=32
//    N=14336 131.0 -> 83.1); from K = 5120 over 14336+ weight rows (M=16
//    K=5120 N=28672 43.3 -> 27.4, M=2 K=11008 N=28672 61.5 -> 53.8); from
//    K = 11008 (M=8 K=14336 N=4096 16.0 -> 14.7, M=4 K=11008 N=8192 19.6 ->
//    18.7; M = 2..4 at K=14336 N=8192 2 % behind); M >= 16 from K = 8192
//    (M=16 K=8192 N=4096 12.6 -> 11.5, N=8192 17.1 -> 16.4); M >= 24 from
//    K = 5120 (M=24 K=5120 N=8192 14.6 -> 14.2, K=8192 N=8192 19.0 -> 17.5).
//    The small-batch kernel stays ahead below those (M=8 K=8192 N=8192 15.4
//    against 15.8, M=16 K=5120 N=8192 12.4 against 13.5), except from 28
//    rows at K = 3072..4096 over at most 4096 rows, where it has too few
//    workgroups (M=32 K=4096 N=2048 11.2 -> 9.6, K=3072 N=1024 9.6 -> 8.9;
//    M=24 K=3072 level, K=4096 N=4096 10.0 against 10.5), and from 20 rows
//    at K = 4096 over 14336-20480 rows, between the small-batch kernel's
//    even rounds at 12288 and 24576 rows (M=32 N=14336 +29 %, M=24 N=16384
//    +12 %, M=20 N=14336 +10 %; N=12288 7-15 % behind), and from K = 8192
//    over at most 2048 rows, where the small-batch kernel has too few
//    workgroups (M=8 K=8192 N=512 9.9 -> 8.1, N=2048 10.2 -> 9.0).
//  * M = 33 (one 16-row tile fewer, the extra row on the VALU): over 28672+
//    rows (M=33 K=3072 N=28672 28.1 -> 21.4, K=1024 N=57344 28.7 -> 19.3),
//    over 11008+ rows from K = 4096 (K=4096 N=11008 20.4 -> 18.4), over
//    6144+ rows from K = 5120 (K=5120 N=6144 19.7 -> 15.5); the 64-row tiles
//    and the small-batch kernel stay ahead below those (K=4096 N=8192 16.1
//    against 17.5, K=2048 N=8192 9.9 against 11.3).
//  * M = 34..48 (three 16-row tiles): over 28672+ rows (M=40 K=3072 N=57344
//    +25 %, K=4096 N=28672 +23 %; level at K=1024 N=28672), from K = 4096
//    over 6144+ rows (M=40 K=5120 N=11008 +19 %, K=4096 N=6144 +15 %; level
//    at K=4096 N=8192-16384), at K = 3072 over at most 2048 rows (M=40 +9 %);
//    the tiles and the small-batch kernel stay ahead at K <= 2048 below 28672
//    rows (M=48 K=2048 N=11008 24 % behind) and at K = 3072 over 4096-16384.
//  * M = 49..64 (four 16-row tiles): below 8192 rows from K = 4096 and
//    below 6144 from K = 3072, where the small-batch kernel runs (M=64
//    K=8192 N=6144 35.4 -> 21.7, K=3584 N=4608 18.4 -> 15.6; M=52 K=3072
//    N=6144 7.8 % behind); over 57344+ rows (M=52 K=1024 +23 %; at M=64 from
//    K = 3072); over 28672-32768 rows from K = 2048 up to M = 56 (M=56 K=2048
//    +6 %), from K = 4096 at M = 57..64 (M=64 K=11008 +12 %; over 37888
//    rows the plan's 192-row units leave CUs idle: M=52 K=3584 39.7 against
//    48.7 for the tiles); over 16384+ rows from
//    K = 5120 (M=64 K=11008 N=16384 +7 %); up to M = 56 over 8192 rows from
//    K = 8192 (M=52 K=11008 +10 %). The 64-row tiles stay ahead over
//    8192-16384 rows at K <= 4096 (M=64 K=4096 N=11008 11 % behind) and over
//    11008 rows at any K (M=56 K=8192 5 % behind).
//    With a long K: from K = 14336 except M > 56 over at most 8192 rows,
//    where the two are level (M=64 K=16384 N=16384 67.9 -> 63.9; M=64
//    K=16384 N=8192 38.8 against 39.9).
//  * M = 33..48, beside the rules above: from K = 8192 (M=33 K=8192 N=8192
//    25.5 -> 22.7, N=16384 41.2 -> 33.0); over 32768+ rows from K = 4096
//    (M=40 K=4096 N=32768 39.6 -> 33.1); at most 4096 rows from K = 4096,
//    against the small-batch kernel (M=64 K=8192 N=4096 32.8 -> 19.8, M=64
//    K=4096 N=4096 18.4 -> 14.8, the same at M = 33..48).
bool splitk_wanted(const GemmArgs &a) {
  if (a.M < 2 || a.M > kSkinnyMaxM) return false;
  if (a.M <= 32) {
    if (a.K >= kSplitkMinK) return true;
    if (a.M >= 28 && a.K >= 3072 && a.N <= 4096) return true;
    if (a.M >= 20 && a.K == 4096 && a.N >= 14336 && a.N <= 20480) return true;
    if (a.K >= 8192 && a.N <= 2048) return true;
    if (a.K < 5120) return false;
    return a.N >= 14336 || a.K >= 11008 || (a.M >= 16 && a.K >= 8192) || a.M >= 24;
  }
  if (a.M > 48) {
    if (a.N < 8192) return a.K >= 4096 || (a.K >= 3072 && a.N < 6144);
    if (a.N >= 57344) return a.M <= 56 || a.K >= 3072;
    if (a.N >= 28672 && a.N <= 32768) return a.K >= (a.M <= 56 ? 2048 : 4096);
    if (a.N >= 16384 && a.K >= 5120) return true;
    if (a.M <= 56 && a.K >= 8192 && a.N <= 8192) return true;
    return a.K >= 14336 && (a.N > 8192 || a.M <= 56);
  }
  // M = 33..48
  if (a.N >= 28672) return true;
  if (a.M == 33) {
    if ((a.K >= 4096 && a.N >= 11008) || (a.K >= 5120 && a.N >= 6144)) return true;
  } else if ((a.K >= 4096 && a.N >= 6144) || (a.K >= 3072 && a.N <= 2048)) {
    return true;
  }
  if (a.N <= 4096) return a.K >= 4096;
  if (a.K >= 8192) return true;
  if (a.N >= 32768) return a.K >= 4096;
  return false;
}

// The split-K kernel runs where it is wanted and its plan either does not
// split (S = 1: no workspace, the same kernel with or without one given) or
// a workspace is given.
bool splitk_selected(const GemmArgs &a, bool have_ws) {
  if (!splitk_wanted(a) || !splitk_supported(a)) return false;
  const SplitkPlan p = splitk_plan(a.M, a.N, a.K, false, true);
  return p.ok && (p.S == 1 || have_ws);
}

// The gate/up + SwiGLU product through the split-K kernel (same run, bf16,
// us, the one-pass gate/up kernels -> split K): K >= 16384; M = 33..64,
// where the one-pass kernels take two passes over the rows (M=33 K=8192
// I=28672 169.1 -> 109.2, M=64 235.9 -> 115.9, M=40 K=4096 I=14336 60.8 ->
// 34.0), except below M = 48 over at most 4096 gate rows at K < 8192 (M=33
// K=4096 I=1792 14.9 against 16.7); from K = 8192 over at most 4096 gate
// rows, where the one-pass kernels leave CUs idle (M=2 K=8192 I=3584 29.3 ->
// 16.1, M=32 K=12288 I=4096 71.2 -> 25.5); with 8-wave plans also from
// M = 24 (M=32 K=4096 I=14336 31.7 -> 27.2, M=24 K=5120 I=13824 35.3 ->
// 31.2), from 16 rows at K = 8192 (M=17 K=8192 I=28672 79.0 -> 73.1, M=32
// I=14336 53.6 -> 42.9) and where K is not a multiple of 1024, so the
// one-pass kernels' K chunks are 512 (M=16 K=3584 I=18944 35.2 -> 29.5).
// The one-pass kernels stay ahead below M = 24 at K = 4096 (M=2 K=4096
// I=11008 18.2 against 24.7; M=17 I=14336 26.3 against 28.7), level at
// K=5120 I=13824, and ahead below 16 rows at K = 8192 (M=2 K=8192 I=14336
// 38.1 against 40.5). Over few gate rows the one-pass kernels have too few
// workgroups: split K from K = 2048 over at most 4096 gate rows and from
// K = 3072 over at most 8192 (M=8 K=4096 I=2048 16.8 -> 9.4, M=16 K=6144
// I=4096 27.1 -> 13.6, M=2 K=3072 I=8192 14.1 -> 13.4; at K = 1024 the
// one-pass kernels stay ahead, M=2 I=4096 6.8 against 7.9). At M = 17 the
// extra-row form makes split K the faster at any K and I (K=4096 I=4096
// 22.3 -> 12.8, K=4096 I=11008 23.7 -> 22.2, K=2048 I=28672 26.9 -> 22.6;
// at most 4 % behind at K=2048-6144 I=11008). At M = 18..23 (two 16-row
// tiles either way) from K = 5120 (M=20 K=5120 I=11008 33.2 -> 29.6, I=28672
// 59.2 -> 55.0) and at K <= 3072 over 14336+ gate rows (M=22 K=2048 I=28672
// 27.3 -> 23.1); the one-pass kernels stay ahead at K <= 4096 over 11008
// gate rows (M=18 K=2048 16.2 against 17.2). At M = 33..47 over at most
// 4096 gate rows from K = 6144, and from 40 rows at K = 4096 (M=40 K=6144
// I=2048 21.9 -> 16.7, M=44 K=4096 I=2048 16.6 -> 15.4; M=36 K=4096 level,
// K <= 3072 behind: M=40 K=2048 I=4096 10.8 against 13.3).
bool gateup_splitk_wanted(int64_t M, int64_t I, int64_t K) {
  if (M < 2 || M > kSkinnyMaxM) return false;
  if (K >= kSplitkMinK || (K >= 8192 && I <= 4096)) return true;
  if (M > 32) return I > 4096 || M >= 48 || K >= 6144 || (K >= 4096 && M >= 40);
  if (M == 17 || (K >= 2048 && I <= 4096) || (K >= 3072 && I <= 8192)) return true;
  if (M >= 18 && (K >= 5120 || (K <= 3072 && I >= 14336))) return true;
  return M >= 24 || (M >= 16 && K >= 8192) || K % 1024 != 0;
}

// The gate/up product at M = 2 over few gate rows runs the row GEMV (same
// run, bf16, us, previous pick -> row GEMV: K=4096 I=1024 9.4 -> 4.7,
// I=4096 11.6 -> 9.6, K=8192 I=8192 29.5 -> 26.8, K=16384 I=1024 14.6 ->
// 9.5; behind from I = 3584 at K = 16384 and at I = 14336).
bool gateup_two_rows_few(int64_t M, int64_t I, int64_t K) {
  return M == 2 && K % 16 == 0 && (I <= 2048 || (I <= 8192 && K <= 8192));
}

int select_variant(const GemmArgs &a, bool have_ws) {
  if (a.K == 0) return RA_VARIANT_GENERIC;
  // M = 2 runs the small-batch kernels where they apply: the row GEMV
  // streams each weight row once per activation row pair no faster than
  // the MFMA kernels (same run: K=4096 N=11008 9.6 vs 11.3 us, K=28672
  // N=8192 40.3 split K / 38.9 small batch vs 50.0, K=16384 N=16384 44.4 /
  // 47.4 vs 56.2, K=8192 N=57344 81.1 small batch vs 95.0), except over few
  // rows, where the MFMA kernels' 16-row units leave most CUs idle: up to
  // 1024 rows, and 2048 at K = 8192..16384 (K=8192 N=512 8.8 -> 4.2, N=2048
  // 9.1 -> 6.9, K=28672 N=1024 13.2 -> 9.4 against split K, K=4096 N=1024
  // 4.4 -> 3.9; K=28672 N=2048 12 % behind). M = 1 stays with the row GEMV
  // (8.5 vs 9.8 at K=4096 N=11008, 37.3 vs 39.0 at K=28672).
  const bool two_rows_few =
      a.M == 2 && (a.N <= 1024 || (a.N <= 2048 && a.K >= 8192 && a.K <= 16384));
  if (gemv_rows_supported(a) && (a.M == 1 || two_rows_few || !batch_supported(a))) {
    const int v = one_row_short_k(a);
    return v ? v : RA_VARIANT_ROWS;
  }
  // Split K where it is measured ahead (see splitk_wanted), then at M =
  // 33..64 with at least 8192 weight rows the 64-row tiles (K split over
  // workgroups where that pays).
  if (splitk_selected(a, have_ws)) return RA_VARIANT_SPLITK;
  if (tiled_small_selected(a) && !short_k_batch(a)) return RA_VARIANT_TILED;
  // The split-K kernel (a plan that splits needs the workspace, an unsplit
  // one runs either way) at M = 17..32, K = 2048..4096 over 28672+ weight
  // rows, where the small-batch kernel needs a second round of workgroups
  // (same run, bf16, us: M=32 K=4096 N=28672 37.9 -> 29.8, M=24 K=3072
  // N=40960 36.3 -> 31.4, M=20 K=2048 N=28672 18.3 -> 17.5, M=17 K=4096
  // N=28672 29.8 -> 28.7; at N=24576 and at K=5120 N=27648 the small-batch
  // kernel stays ahead).
  if (a.M >= 17 && a.M <= 32 && a.K >= 2048 && a.K <= 4096 && a.N >= 28672 && splitk_supported(a)) {
    const SplitkPlan p = splitk_plan(a.M, a.N, a.K, false, true);
    if (p.ok && (p.S == 1 || have_ws)) return RA_VARIANT_SPLITK;
  }
  // M = 3..64: the small-batch kernel (line-wide weight loads, activations
  // read once per 48 rows) where K % 128 == 0, else the split-K MFMA kernel;
  // both measured faster than the LDS GEMV, which stays as a fallback.
  if (a.M <= kSkinnyMaxM && batch_supported(a)) return RA_VARIANT_BATCH;
  if (a.M <= kSkinnyMaxM && skinny_supported(a)) return RA_VARIANT_SKINNY;
  if (gemv_supported(a)) return RA_VARIANT_GEMV;
  if (tiled_supported(a)) return RA_VARIANT_TILED;
  if (skinny_supported(a)) return RA_VARIANT_SKINNY;
  return RA_VARIANT_GENERIC;
}

// A caller workspace must start on an RA_WORKSPACE_ALIGN boundary (the
// kernels use 4-byte atomics on its counters and 16-byte stores and loads of
// its partial sums).
bool ws_misaligned(const void *ws, size_t bytes) {
  return ws != nullptr && bytes > 0 && reinterpret_cast<uintptr_t>(ws) % RA_WORKSPACE_ALIGN != 0;
}

int check_gemm(const GemmArgs &a) {
  if (a.M < 0 || a.N < 0 || a.K < 0) return RA_ERR_ARG;
  if (a.M > INT32_MAX || a.N > INT32_MAX || a.K > INT32_MAX) return RA_ERR_ARG;
  if (!valid_act(a.x_dt)) return RA_ERR_DTYPE;
  if (a.bias && !valid_act(a.bias_dt)) return RA_ERR_DTYPE;
  if (a.M == 0 || a.N == 0) return RA_OK;
  if (!a.y || !a.scale || !a.w || (a.K > 0 && !a.x)) return RA_ERR_ARG;
  if (a.ldx < a.K || a.ldw < a.K || a.ldy < a.N) return RA_ERR_ARG;
  return RA_OK;
}

}  // namespace

namespace ra {
// Workspace bytes the automatic selection uses for this GEMM (0: none).
bool auto_workspace_optional(const GemmArgs &a) {
  return a.M > 0 && a.N > 0 && select_variant(a, true) == RA_VARIANT_TILED;
}

size_t auto_workspace_bytes(const GemmArgs &a) {
  if (a.M == 0 || a.N == 0) return 0;
  const int v = select_variant(a, true);
  if (v == RA_VARIANT_TILED) return tiled_split_plan(a).ws_bytes;
  if (v != RA_VARIANT_SPLITK) return 0;
  const SplitkPlan p = splitk_plan(a.M, a.N, a.K, false, true);
  return p.ok ? p.ws_bytes : 0;
}
}  // namespace ra

extern "C" {

#ifdef RA_TUNING
void ra_tune_skinny(int mt, int rt, int nw) { g_skinny_override = SkinnyCfg{mt, rt, nw}; }
void ra_tune_tiled(int mode) { ra::g_tiled_mode = mode; }
void ra_tune_rows(int rw) { ra::g_rows_rw = rw; }
void ra_tune_rows_pipe(int rp) { ra::g_rows_pipe = rp; }
void ra_tune_batch_rt(int rt) { ra::g_batch_rt = rt; }
void ra_tune_batch_nw(int nw) { ra::g_batch_nw = nw; }
void ra_tune_batch_xlds(int v) { ra::g_batch_xlds = v; }
void ra_tune_batch_xd(int v) { ra::g_batch_xd = v; }
void ra_tune_sk(int s, int dmax) { ra::g_sk_s = s; ra::g_sk_dmax = dmax; }
void ra_tune_sk_x1(int off) { ra::g_sk_x1 = off; }
void ra_tune_sk_tw(int tw) { ra::g_sk_tw = tw; }
void ra_tune_sk_nw(int nw) { ra::g_sk_nw = nw; }
void ra_tune_sk_mt3(int off) { ra::g_sk_mt3 = off; }
void ra_tune_tiled_split(int v) { ra::g_tiled_split = v; }
void ra_tune_w8a8(int mode) { ra::g_w8a8_mode = mode; }
void ra_tune_rows_lds(int v) { ra::g_rows_lds = v; }
void ra_tune_gu_splitk(int v) { ra::g_gu_splitk = v; }
void ra_tune_gu_rows(int v) { ra::g_gu_rows = v; }
#endif
#ifdef RA_TRACE
// Trace builds only: device buffer for the tiled kernel's per-workgroup timestamps (NULL: none).
void ra_tune_trace(void *buf) { ra::g_trace_buf = buf; }
#endif

int ra_abi_version(void) { return RA_ABI_VERSION; }

const char *ra_strerror(int code) {
  switch (code) {
    case RA_OK: return "success";
    case RA_ERR_ARG: return "rotaccel: invalid argument (size, leading dimension or null pointer)";
    case RA_ERR_DTYPE: return "rotaccel: unsupported dtype";
    case RA_ERR_LAUNCH: return "rotaccel: kernel launch failed";
    case RA_ERR_VARIANT: return "rotaccel: the requested kernel variant cannot run this problem";
    case RA_ERR_DEVICE: return "rotaccel: no usable gfx950 device";
    case RA_ERR_WORKSPACE: return "rotaccel: workspace smaller than the size the problem needs";
    default: return "rotaccel: unknown error";
  }
}

size_t ra_w8a16_gemm_workspace_size(int64_t M, int64_t N, int64_t K, int x_dtype) {
  if (x_dtype != RA_F16 && x_dtype != RA_BF16) return 0;
  if (M < 2 || M > kSplitTileMaxM) return 0;  // the row GEMV (M = 1) and the large-M tiled GEMM need none
  // The split-K kernel's plan (M <= 64; where it is not selected only a
  // forced RA_VARIANT_SPLITK launch uses it) or, at M = 33..128, the 64-row
  // tiles' split plan, whichever needs more (contiguous, aligned operands).
  const SplitkPlan p = splitk_plan(M, N, K, false, true);
  const GemmArgs a{reinterpret_cast<const void *>(256), K, x_dtype, reinterpret_cast<const int8_t *>(256),
                   K, nullptr, nullptr, RA_F32, nullptr, N, M, N, K};
  const size_t tiled = tiled_split_plan(a).ws_bytes;
  const size_t sk = p.ok ? p.ws_bytes : 0;
  return sk > tiled ? sk : tiled;
}

int ra_w8a16_gemm_ex(const void *x, int64_t ldx, int x_dtype, const int8_t *w, int64_t ldw,
                     const float *scale, const void *bias, int bias_dtype, void *y, int64_t ldy, int64_t M,
                     int64_t N, int64_t K, int variant, void *workspace, size_t workspace_bytes, void *stream) {
  const GemmArgs a{x, ldx, x_dtype, w, ldw, scale, bias, bias_dtype, y, ldy, M, N, K};
  int st = check_gemm(a);
  if (st != RA_OK) return st;
  if (ws_misaligned(workspace, workspace_bytes)) return RA_ERR_ARG;
  if (M == 0 || N == 0) return RA_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool have_ws = workspace != nullptr && workspace_bytes > 0;
  int v = variant == RA_VARIANT_AUTO ? select_variant(a, have_ws) : variant;
  switch (v) {
    case RA_VARIANT_SPLITK:
    case RA_VARIANT_SPLITK_SPREAD: {
      if (!splitk_supported(a) || M > kSkinnyMaxM) return RA_ERR_VARIANT;
      SplitkPlan p = splitk_plan(M, N, K, false, have_ws);
      p.spread = v == RA_VARIANT_SPLITK_SPREAD;
      if (!p.ok) return RA_ERR_VARIANT;
      if (p.ws_bytes > 0 && workspace_bytes < p.ws_bytes) return RA_ERR_WORKSPACE;
      return to_status(splitk_launch(a, p, workspace, s));
    }
    case RA_VARIANT_SKINNY:
      if (!skinny_supported(a) || K == 0) return RA_ERR_VARIANT;
      return to_status(skinny_launch(a, skinny_config(M, N, K), s));
    case RA_VARIANT_ROWS:
      if (!gemv_rows_supported(a)) return RA_ERR_VARIANT;
      return to_status(gemv_rows_launch(a, s));
    case RA_VARIANT_GEMV:
      if (!gemv_supported(a)) return RA_ERR_VARIANT;
      return to_status(gemv_launch(a, s));
    case RA_VARIANT_BATCH:
      if (!batch_supported(a)) return RA_ERR_VARIANT;
      return to_status(batch_launch(a, s));
    case RA_VARIANT_TILED:
      if (!tiled_supported(a) || K == 0) return RA_ERR_VARIANT;
      return to_status(tiled_launch_ws(a, have_ws ? workspace : nullptr, workspace_bytes, s));
    case RA_VARIANT_GENERIC:
      return to_status(generic_launch(a, s));
    default:
      return RA_ERR_ARG;
  }
}

int ra_w8a16_gemm(const void *x, int64_t ldx, int x_dtype, const int8_t *w, int64_t ldw, const float *scale,
                  const void *bias, int bias_dtype, void *y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                  void *stream) {
  return ra_w8a16_gemm_ex(x, ldx, x_dtype, w, ldw, scale, bias, bias_dtype, y, ldy, M, N, K, RA_VARIANT_AUTO,
                          nullptr, 0, stream);
}

int ra_w8a16_gemm_ws(const void *x, int64_t ldx, int x_dtype, const int8_t *w, int64_t ldw, const float *scale,
                     const void *bias, int bias_dtype, void *y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                     void *workspace, size_t workspace_bytes, void *stream) {
  return ra_w8a16_gemm_ex(x, ldx, x_dtype, w, ldw, scale, bias, bias_dtype, y, ldy, M, N, K, RA_VARIANT_AUTO,
                          workspace, workspace_bytes, stream);
}

int ra_w8a16_gemm_select(int64_t M, int64_t N, int64_t K, int x_dtype) {
  // Alignment is assumed satisfied (contiguous, 16-byte aligned operands)
  // and a workspace of ra_w8a16_gemm_workspace_size bytes given.
  const GemmArgs a{reinterpret_cast<const void *>(256), K, x_dtype, reinterpret_cast<const int8_t *>(256),
                   K, nullptr, nullptr, RA_F32, nullptr, N, M, N, K};
  return select_variant(a, true);
}

size_t ra_w8a16_gateup_workspace_size(int64_t M, int64_t I, int64_t K, int x_dtype) {
  if (x_dtype != RA_F16 && x_dtype != RA_BF16) return 0;
  // Only the split-K gate/up kernel uses a workspace, where it is selected.
  if (!gateup_splitk_wanted(M, I, K) || gateup_two_rows_few(M, I, K) || K < 128 || K % 128 != 0) return 0;
  const SplitkPlan p = splitk_plan(M, I, K, true, true);
  return p.ok ? p.ws_bytes : 0;
}

int ra_w8a16_gateup_swiglu(const void *x, int64_t ldx, int x_dtype, const int8_t *w, int64_t ldw,
                           const float *scale, void *h, int64_t ldh, int64_t M, int64_t I, int64_t K,
                           void *stream) {
  return ra_w8a16_gateup_swiglu_ws(x, ldx, x_dtype, w, ldw, scale, h, ldh, M, I, K, nullptr, 0, stream);
}

int ra_w8a16_gateup_swiglu_ws(const void *x, int64_t ldx, int x_dtype, const int8_t *w, int64_t ldw,
                              const float *scale, void *h, int64_t ldh, int64_t M, int64_t I, int64_t K,
                              void *workspace, size_t workspace_bytes, void *stream) {
  if (M < 0 || I < 0 || K < 0 || M > INT32_MAX || 2 * I > INT32_MAX || K > INT32_MAX) return RA_ERR_ARG;
  if (x_dtype != RA_F16 && x_dtype != RA_BF16 && x_dtype != RA_F32) return RA_ERR_DTYPE;
  if (M == 0 || I == 0) return RA_OK;
  if (!h || !w || !scale || (K > 0 && !x)) return RA_ERR_ARG;
  if (ldx < K || ldw < K || ldh < I) return RA_ERR_ARG;
  if (ws_misaligned(workspace, workspace_bytes)) return RA_ERR_ARG;
  const GateUpArgs a{x, ldx, x_dtype, w, ldw, scale, h, ldh, M, I, K};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool have_ws = workspace != nullptr && workspace_bytes > 0;
  bool gu_rows = M == 1 || !gateup_batch_supported(a) || gateup_two_rows_few(M, I, K);
#ifdef RA_TUNING
  if (g_gu_rows) gu_rows = true;  // tuning builds: the row GEMV wherever it applies
#endif
  if (K > 0 && gateup_gemv_rows_supported(a) && gu_rows) return to_status(gateup_gemv_rows_launch(a, s));
  bool gu_split = gateup_splitk_wanted(M, I, K);
#ifdef RA_TUNING
  if (g_gu_splitk) gu_split = g_gu_splitk > 0;  // tuning builds: 1 forces, -1 forbids the split-K kernel
#endif
  // A plan that splits needs the workspace; an unsplit one runs either way.
  if (gu_split && gateup_splitk_supported(a)) {
    const SplitkPlan p = splitk_plan(M, I, K, true, true);
    if (p.ok && (p.S == 1 || have_ws)) {
      if (p.ws_bytes > 0 && workspace_bytes < p.ws_bytes) return RA_ERR_WORKSPACE;
      return to_status(gateup_splitk_launch(a, p, workspace, s));
    }
  }
  if (K > 0 && M <= kSkinnyMaxM && gateup_batch_supported(a)) return to_status(gateup_batch_launch(a, s));
  if (K > 0 && M <= kSkinnyMaxM && gateup_skinny_supported(a)) return to_status(gateup_skinny_launch(a, s));
  if (K > 0 && gateup_gemv_supported(a)) return to_status(gateup_gemv_launch(a, s));
  if (K > 0 && gateup_tiled_supported(a)) return to_status(gateup_tiled_launch(a, s));
  return to_status(gateup_generic_launch(a, s));
}

int ra_stream_capture_info(void *stream, int *capturing, unsigned long long *capture_id) {
  if (!capturing || !capture_id) return RA_ERR_ARG;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  unsigned long long id = 0;
  if (hipStreamGetCaptureInfo(static_cast<hipStream_t>(stream), &st, &id) != hipSuccess) return RA_ERR_DEVICE;
  *capturing = st == hipStreamCaptureStatusActive ? 1 : 0;
  *capture_id = *capturing ? id : 0;
  return RA_OK;
}

int ra_rmsnorm(const void *x, int64_t ldx, int x_dtype, const void *weight, int w_dtype, void *y, int64_t ldy,
               int y_dtype, int64_t rows, int64_t hidden, float eps, void *stream) {
  if (rows < 0 || hidden < 0 || rows > INT32_MAX || hidden > INT32_MAX) return RA_ERR_ARG;
  if (!valid_act(x_dtype) || !valid_act(w_dtype) || !valid_act(y_dtype)) return RA_ERR_DTYPE;
  const int promoted = x_dtype == w_dtype ? x_dtype : RA_F32;
  if (y_dtype != promoted) return RA_ERR_DTYPE;
  if (rows == 0 || hidden == 0) return RA_OK;
  if (!x || !weight || !y || ldx < hidden || ldy < hidden) return RA_ERR_ARG;
  return to_status(rmsnorm_launch(x, ldx, x_dtype, nullptr, 0, x_dtype, weight, w_dtype, y, ldy, y_dtype, rows,
                                  hidden, eps, static_cast<hipStream_t>(stream)));
}

int ra_rmsnorm_residual(const void *x, int64_t ldx, int x_dtype, const void *residual, int64_t ldr, int r_dtype,
                        const void *weight, int w_dtype, void *y, int64_t ldy, int y_dtype, int64_t rows,
                        int64_t hidden, float eps, void *stream) {
  if (rows < 0 || hidden < 0 || rows > INT32_MAX || hidden > INT32_MAX) return RA_ERR_ARG;
  if (!valid_act(x_dtype) || !valid_act(r_dtype) || !valid_act(w_dtype) || !valid_act(y_dtype)) return RA_ERR_DTYPE;
  const int promoted = x_dtype == w_dtype ? x_dtype : RA_F32;
  if (y_dtype != promoted) return RA_ERR_DTYPE;
  if (rows == 0 || hidden == 0) return RA_OK;
  if (!x || !residual || !weight || !y || ldx < hidden || ldr < hidden || ldy < hidden) return RA_ERR_ARG;
  return to_status(rmsnorm_launch(x, ldx, x_dtype, residual, ldr, r_dtype, weight, w_dtype, y, ldy, y_dtype, rows,
                                  hidden, eps, static_cast<hipStream_t>(stream)));
}

int ra_swiglu(const void *gate, const void *up, void *out, int64_t n, int dtype, void *stream) {
  if (n < 0) return RA_ERR_ARG;
  if (!valid_act(dtype)) return RA_ERR_DTYPE;
  if (n == 0) return RA_OK;
  if (!gate || !up || !out) return RA_ERR_ARG;
  return to_status(swiglu_launch(gate, up, out, n, dtype, static_cast<hipStream_t>(stream)));
}

int ra_swiglu_bias(const void *gate, const void *up, const void *bias_gate, const void *bias_up, int bias_dtype,
                   void *out, int64_t n, int64_t hidden, int dtype, void *stream) {
  if (n < 0 || hidden <= 0 || n % hidden != 0) return RA_ERR_ARG;
  if (!valid_act(dtype) || !valid_act(bias_dtype)) return RA_ERR_DTYPE;
  if (n == 0) return RA_OK;
  if (!gate || !up || !out || !bias_gate || !bias_up) return RA_ERR_ARG;
  return to_status(swiglu_bias_launch(gate, up, bias_gate, bias_up, bias_dtype, out, n, hidden, dtype,
                                      static_cast<hipStream_t>(stream)));
}

int ra_quantize_per_channel(const void *w, int64_t ldw, int w_dtype, int64_t N, int64_t K, int8_t *q,
                            int64_t ldq, float *scale, void *stream) {
  if (N < 0 || K < 0 || N > INT32_MAX || K > INT32_MAX) return RA_ERR_ARG;
  if (!valid_act(w_dtype)) return RA_ERR_DTYPE;
  if (N == 0) return RA_OK;
  if (!w || !q || !scale || ldw < K || ldq < K) return RA_ERR_ARG;
  return to_status(quantize_launch(w, ldw, w_dtype, N, K, q, ldq, scale, static_cast<hipStream_t>(stream)));
}

int ra_quantize_rows(const void *t, int64_t ldt, int t_dtype, int64_t rows, int64_t cols, int bits, int8_t *q,
                     int64_t ldq, void *scale, void *stream) {
  if (rows < 0 || cols < 0 || rows > INT32_MAX || cols > INT32_MAX) return RA_ERR_ARG;
  if (bits != 8 && bits != 4) return RA_ERR_ARG;
  if (!valid_act(t_dtype)) return RA_ERR_DTYPE;
  if (rows == 0 || cols == 0) return RA_OK;
  if (!t || !q || !scale || ldt < cols || ldq < cols) return RA_ERR_ARG;
  return to_status(quantize_rows_launch(t, ldt, t_dtype, rows, cols, bits, q, ldq, scale,
                                        static_cast<hipStream_t>(stream)));
}

int ra_quantize_act_rows(const void *x, int64_t ldx, int x_dtype, int64_t M, int64_t K, int8_t *q, int64_t ldq,
                         void *xs, float act_scale, void *stream) {
  if (M < 0 || K < 0 || M > INT32_MAX || K > INT32_MAX) return RA_ERR_ARG;
  if (x_dtype != RA_F16 && x_dtype != RA_BF16) return RA_ERR_DTYPE;
  if (M == 0) return RA_OK;
  if (K == 0 || !x || !q || !xs || ldx < K || ldq < K) return RA_ERR_ARG;  // torch's amax rejects K = 0
  return to_status(
      quantize_act_launch(x, ldx, x_dtype, M, K, q, ldq, xs, act_scale, static_cast<hipStream_t>(stream)));
}

int ra_w8a8_gemm(const int8_t *xq, int64_t ldxq, const void *xs, const int8_t *w, int64_t ldw, const float *scale,
                 const void *bias, int bias_dtype, void *y, int64_t ldy, int y_dtype, int64_t M, int64_t N,
                 int64_t K, void *stream) {
  const W8A8Args a{xq, ldxq, xs, w, ldw, scale, bias, bias_dtype, y, ldy, y_dtype, M, N, K};
  if (M < 0 || N < 0 || K < 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return RA_ERR_ARG;
  if (y_dtype != RA_F16 && y_dtype != RA_BF16) return RA_ERR_DTYPE;
  if (bias && !valid_act(bias_dtype)) return RA_ERR_DTYPE;
  if (M == 0 || N == 0) return RA_OK;
  if (!y || !xs || !scale || !w || (K > 0 && !xq)) return RA_ERR_ARG;
  if (ldxq < K || ldw < K || ldy < N) return RA_ERR_ARG;
  return to_status(w8a8_launch(a, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
