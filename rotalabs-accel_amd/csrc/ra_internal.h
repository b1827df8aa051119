// Host-side declarations shared by the kernel translation units and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <algorithm>

#include "rotaccel.h"

namespace ra {

struct GemmArgs {
  const void *x;
  int64_t ldx;
  int x_dt;
  const int8_t *w;
  int64_t ldw;
  const float *scale;
  const void *bias;  // may be null
  int bias_dt;
  void *y;
  int64_t ldy;
  int64_t M, N, K;
};

// Skinny (split-K MFMA) kernel: MT 16-wide activation tiles, RT 16-row weight
// tiles per workgroup, NW waves splitting K.
struct SkinnyCfg {
  int mt, rt, nw;
};
bool skinny_supported(const GemmArgs &a);
SkinnyCfg skinny_select(int64_t M, int64_t N, int64_t K);
hipError_t skinny_launch(const GemmArgs &a, const SkinnyCfg &c, hipStream_t s);

// Tiled (LDS-staged MFMA) kernel for large M.
bool tiled_supported(const GemmArgs &a);
// Whether the automatic choice runs the tiled kernel with its 64 x 64 tile
// (M = 33..64, at least 8192 weight rows, K % 64 == 0).
bool tiled_small_selected(const GemmArgs &a);
hipError_t tiled_launch(const GemmArgs &a, hipStream_t s);
// M = 33..64 (where tiled_small_selected): the small tile with K split over
// workgroups, when the plan beats the 64 x 64 tile over all of K; M =
// 65..1024: rows of these tiles or of 128-row tiles, the best plan (above
// M = 128 only where the large tiles fill less than half of the CUs).
// nsplit > 1 needs ws_bytes of workspace, laid out as the split-K kernel's:
// the counter block first. tiled_launch_ws runs it when it applies and the
// workspace suffices, else tiled_launch.
struct TiledSplitPlan {
  bool ok = false;
  int bmb = 1, bnb = 0, nsplit = 1, ksplit = 0;  // tiles of 64*bmb x 64*bnb
  size_t ws_bytes = 0;
};
TiledSplitPlan tiled_split_plan(const GemmArgs &a);
constexpr int64_t kSplitTileMaxM = 1024;  // largest M the split plans run
hipError_t tiled_launch_ws(const GemmArgs &a, void *ws, size_t ws_bytes, hipStream_t s);

// Generic kernel: any shape, alignment and activation dtype.
hipError_t generic_launch(const GemmArgs &a, hipStream_t s);

// Fused gate/up + SwiGLU.
struct GateUpArgs {
  const void *x;
  int64_t ldx;
  int x_dt;
  const int8_t *w;
  int64_t ldw;
  const float *scale;
  void *h;
  int64_t ldh;
  int64_t M, I, K;
};
bool gateup_skinny_supported(const GateUpArgs &a);
hipError_t gateup_skinny_launch(const GateUpArgs &a, hipStream_t s);
bool gateup_tiled_supported(const GateUpArgs &a);
hipError_t gateup_tiled_launch(const GateUpArgs &a, hipStream_t s);
hipError_t gateup_generic_launch(const GateUpArgs &a, hipStream_t s);

// Row GEMV (M <= 2): one weight row per wave, VALU dot products.
bool gemv_rows_supported(const GemmArgs &a);
hipError_t gemv_rows_launch(const GemmArgs &a, hipStream_t s);
bool gateup_gemv_rows_supported(const GateUpArgs &a);
hipError_t gateup_gemv_rows_launch(const GateUpArgs &a, hipStream_t s);

// Small-batch MFMA GEMM (M <= 64, K % 128 == 0): line-wide weight loads
// transposed through LDS, split-K across the workgroup's waves.
bool batch_supported(const GemmArgs &a);
hipError_t batch_launch(const GemmArgs &a, hipStream_t s);
bool gateup_batch_supported(const GateUpArgs &a);
hipError_t gateup_batch_launch(const GateUpArgs &a, hipStream_t s);

// Small-batch GEMM with split K (M <= 64, K % 128 == 0): weights and
// activations staged by direct-to-LDS copies; S > 1 needs a workspace of
// ws_bytes (a zeroed counter block of cnt_bytes, then the partial sums).
// Bytes of the counter block at the start of every split-K workspace (must
// be zero before the first use; each call leaves it zero).
constexpr size_t kSplitkCounterBytes = RA_WORKSPACE_COUNTER_BYTES;  // 4096 counters
// Largest split-K workspace a plan may use (counters + partial sums); plans
// that would need more split less.
constexpr size_t kSplitkMaxWorkspace = (size_t)16 << 20;
struct SplitkPlan {
  bool ok;
  int mt, tw, S, kc, nb;
  bool spread;  // a row block's splits on different XCDs (test mode)
  size_t cnt_bytes, ws_bytes;
  int x1;  // 1: M = 16*mt + 1, the last row summed on the VALU
  int nw;  // waves per workgroup (4)
};
SplitkPlan splitk_plan(int64_t M, int64_t N, int64_t K, bool gu, bool allow_split);
bool splitk_supported(const GemmArgs &a);
hipError_t splitk_launch(const GemmArgs &a, const SplitkPlan &p, void *ws, hipStream_t s);
bool gateup_splitk_supported(const GateUpArgs &a);
hipError_t gateup_splitk_launch(const GateUpArgs &a, const SplitkPlan &p, void *ws, hipStream_t s);

// Workspace bytes the automatic kernel selection of ra_w8a16_gemm_ws uses
// for this problem (0: the selected kernel needs none), and whether that
// kernel also runs without it (the tiled kernel's split plan is optional:
// with less workspace it runs its tile over all of K).
size_t auto_workspace_bytes(const GemmArgs &a);
bool auto_workspace_optional(const GemmArgs &a);

// Decode GEMV (M <= 4, x staged in LDS, one HBM round trip per wave).
bool gemv_supported(const GemmArgs &a);
hipError_t gemv_launch(const GemmArgs &a, hipStream_t s);
bool gateup_gemv_supported(const GateUpArgs &a);
hipError_t gateup_gemv_launch(const GateUpArgs &a, hipStream_t s);

hipError_t rmsnorm_launch(const void *x, int64_t ldx, int x_dt, const void *r, int64_t ldr, int r_dt,
                          const void *w, int w_dt, void *y, int64_t ldy, int y_dt, int64_t rows, int64_t hidden,
                          float eps, hipStream_t s);
hipError_t swiglu_launch(const void *g, const void *u, void *o, int64_t n, int dt, hipStream_t s);
hipError_t swiglu_bias_launch(const void *g, const void *u, const void *bg, const void *bu, int b_dt, void *o,
                              int64_t n, int64_t hidden, int dt, hipStream_t s);
hipError_t quantize_launch(const void *w, int64_t ldw, int w_dt, int64_t N, int64_t K, int8_t *q,
                           int64_t ldq, float *scale, hipStream_t s);
hipError_t quantize_rows_launch(const void *t, int64_t ldt, int t_dt, int64_t rows, int64_t cols, int bits,
                                int8_t *q, int64_t ldq, void *scale, hipStream_t s);

// W8A8 (int8 activations x int8 weights on the int8 matrix cores).
struct W8A8Args {
  const int8_t *xq;  // [M, K] quantised activations, row stride ldxq
  int64_t ldxq;
  const void *xs;  // [M] activation scales, dtype y_dt
  const int8_t *w;
  int64_t ldw;
  const float *scale;
  const void *bias;  // may be null
  int bias_dt;
  void *y;
  int64_t ldy;
  int y_dt;
  int64_t M, N, K;
};
hipError_t quantize_act_launch(const void *x, int64_t ldx, int x_dt, int64_t M, int64_t K, int8_t *q, int64_t ldq,
                               void *xs, float act_scale, hipStream_t s);
bool w8a8_tiled_supported(const W8A8Args &a);
hipError_t w8a8_launch(const W8A8Args &a, hipStream_t s);

}  // namespace ra
