/*
 * rotaccel.h -- C ABI of librotaccel.so, the MI355X (gfx950) W8A16 INT8 GEMM
 * library behind the rotalabs_accel Python API.
 *
 * Conventions
 *  - Every pointer is a device pointer (HBM) unless stated otherwise. The
 *    library never allocates, frees or retains device memory: callers own
 *    inputs, outputs and streams.
 *  - Matrices are row-major with an explicit leading dimension in ELEMENTS.
 *    Weights are int8 [N, K] (nn.Linear layout: one row per output channel),
 *    scales fp32 [N] (one per output channel).
 *  - `stream` is a hipStream_t passed as void* (NULL = the default stream).
 *    Every entry point only enqueues work; none synchronises the host.
 *  - Every entry point returns RA_OK (0) or an ra_status code; the C side
 *    never aborts or throws. ra_strerror() turns a code into text.
 *  - dtype codes: RA_F16, RA_BF16, RA_F32 (see enum ra_dtype).
 */
#ifndef ROTACCEL_H
#define ROTACCEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RA_ABI_VERSION 7

/* Caller workspaces (ra_w8a16_gemm_ws, ra_w8a16_gateup_swiglu_ws) start on
 * this byte boundary (RA_ERR_ARG otherwise). Their first
 * RA_WORKSPACE_COUNTER_BYTES bytes are the counter block, which must be zero
 * before the first use; the rest needs no initialisation. */
#define RA_WORKSPACE_ALIGN 256
#define RA_WORKSPACE_COUNTER_BYTES 16384

enum ra_dtype { RA_F16 = 0, RA_BF16 = 1, RA_F32 = 2 };

enum ra_status {
  RA_OK = 0,
  RA_ERR_ARG = 1,       /* bad size / leading dimension / null pointer       */
  RA_ERR_DTYPE = 2,     /* unsupported dtype combination                      */
  RA_ERR_LAUNCH = 3,    /* kernel launch failed (hipGetLastError != success)  */
  RA_ERR_VARIANT = 4,   /* a forced kernel variant cannot run this shape      */
  RA_ERR_DEVICE = 5,    /* no usable device / not a gfx950 device             */
  RA_ERR_WORKSPACE = 6  /* workspace smaller than the problem needs           */
};

/* Kernel variants for ra_w8a16_gemm_ex. RA_VARIANT_AUTO picks by shape. */
enum ra_variant {
  RA_VARIANT_AUTO = 0,
  RA_VARIANT_SKINNY = 1,  /* split-K MFMA skinny GEMM (decode, small M)        */
  RA_VARIANT_TILED = 2,   /* LDS-staged double-buffered MFMA GEMM (prefill)   */
  RA_VARIANT_GENERIC = 3, /* any shape / alignment / dtype, VALU, slow        */
  RA_VARIANT_GEMV = 4,    /* decode GEMV, M <= 4, x staged in LDS             */
  RA_VARIANT_ROWS = 5,    /* decode row GEMV, M <= 2, one weight row per wave */
  RA_VARIANT_BATCH = 6,   /* small batch, M <= 64, K % 128 == 0, MFMA + LDS */
  RA_VARIANT_SPLITK = 7,  /* small batch, M <= 64, K % 128 == 0, split K      */
  RA_VARIANT_SPLITK_SPREAD = 8 /* the same with a row block's K splits run on
                                  different XCDs (tests the exchange of the
                                  partial sums across XCDs)                  */
};

/* Version of this ABI (RA_ABI_VERSION of the built library). */
int ra_abi_version(void);

/* Static text for an ra_status code. Never NULL. */
const char *ra_strerror(int code);

/*
 * y[M,N] = x[M,K] @ (w[N,K] * scale[N,None]).T (+ bias[N])
 *
 * Replaces the reference's GPU branch of int8_gemm:
 *   src/rotalabs_accel/kernels/gemm.py:234-235 (dispatch) ->
 *   _int8_gemm_triton gemm.py:140-186 -> _int8_gemm_kernel gemm.py:53-138.
 * Same arithmetic as the kernel there: exact int8 -> fp16/bf16 conversion,
 * fp32 accumulation, per-output-channel scale applied to the fp32 accumulator
 * (gemm.py:133); bias is added to the fp32 value before the single rounding to
 * the output dtype (the reference adds it after rounding, gemm.py:181-182).
 * Differences by design: w is read in its [N,K] layout (no per-call
 * transpose, gemm.py:157-160), and y has the activation dtype (the reference
 * fallback's output dtype, gemm.py:46) instead of always fp16 (gemm.py:162).
 *
 * x_dtype: RA_F16 | RA_BF16 | RA_F32 (y has the same dtype).
 * bias: NULL or [N] of bias_dtype (RA_F16 | RA_BF16 | RA_F32).
 * ldx >= K, ldw >= K, ldy >= N. M, N, K >= 0 (M == 0 or N == 0: no-op;
 * K == 0: y = bias or 0).
 */
int ra_w8a16_gemm(const void *x, int64_t ldx, int x_dtype,
                  const int8_t *w, int64_t ldw, const float *scale,
                  const void *bias, int bias_dtype,
                  void *y, int64_t ldy,
                  int64_t M, int64_t N, int64_t K, void *stream);

/*
 * ra_w8a16_gemm with a caller-owned device workspace, which lets the small-
 * batch kernels (2 <= M <= 1024) split K over several workgroups and combine
 * their fp32 partial sums there in a fixed order (deterministic). Same
 * parity as ra_w8a16_gemm; it replaces the same reference call.
 * workspace_bytes must be at least ra_w8a16_gemm_workspace_size(M, N, K,
 * x_dtype) (RA_ERR_WORKSPACE otherwise); workspace may be NULL (or the size
 * 0), which runs the kernels that need none, as ra_w8a16_gemm does.
 * The workspace starts on an RA_WORKSPACE_ALIGN boundary (RA_ERR_ARG
 * otherwise). Its counter block (the first RA_WORKSPACE_COUNTER_BYTES) must
 * be zero before its first use; every call leaves it ready for the next one
 * (its counters back at zero). Calls that may run concurrently (other
 * streams, graphs replayed on other streams) need workspaces of their own.
 * Under HIP graph capture a call records the workspace's address: keep the
 * buffer alive, and its counter block zero before each replay, for as long
 * as the graph may be replayed.
 */
int ra_w8a16_gemm_ws(const void *x, int64_t ldx, int x_dtype,
                     const int8_t *w, int64_t ldw, const float *scale,
                     const void *bias, int bias_dtype,
                     void *y, int64_t ldy,
                     int64_t M, int64_t N, int64_t K,
                     void *workspace, size_t workspace_bytes, void *stream);

/* Workspace bytes ra_w8a16_gemm_ws may use for this problem (0: none). */
size_t ra_w8a16_gemm_workspace_size(int64_t M, int64_t N, int64_t K, int x_dtype);

/*
 * ra_w8a16_gemm_ws without a caller workspace and without any allocation:
 * the split-K kernel's workspace is a fixed 16 MiB device array of the
 * library (one per GPU, held until the process ends), so the call allocates
 * and frees nothing -- for callers that cannot allocate: code under HIP
 * graph capture, serving loops and harnesses that forbid allocation. No
 * counterpart in the reference. Same kernels and results as
 * ra_w8a16_gemm_ws with a workspace (split-K plans never need more than
 * 16 MiB; a tiled split plan that needs more runs its tile over all of K
 * instead, as ra_w8a16_gemm_ws does with too small a workspace;
 * RA_ERR_WORKSPACE if a plan ever needed more than the array holds).
 * Every call on a GPU shares that GPU's array: calls that may
 * overlap on one GPU (several streams) race.
 */
int ra_w8a16_gemm_noalloc(const void *x, int64_t ldx, int x_dtype,
                          const int8_t *w, int64_t ldw, const float *scale,
                          const void *bias, int bias_dtype,
                          void *y, int64_t ldy,
                          int64_t M, int64_t N, int64_t K, void *stream);

/* ra_w8a16_gemm_ws with an explicit kernel variant (enum ra_variant); used by
 * tests to run every kernel on the same inputs. Returns RA_ERR_VARIANT if the
 * forced variant cannot handle the shape, dtype or alignment. */
int ra_w8a16_gemm_ex(const void *x, int64_t ldx, int x_dtype,
                     const int8_t *w, int64_t ldw, const float *scale,
                     const void *bias, int bias_dtype,
                     void *y, int64_t ldy,
                     int64_t M, int64_t N, int64_t K, int variant,
                     void *workspace, size_t workspace_bytes, void *stream);

/* Which variant RA_VARIANT_AUTO runs for this problem (enum ra_variant),
 * given a workspace of ra_w8a16_gemm_workspace_size bytes. */
int ra_w8a16_gemm_select(int64_t M, int64_t N, int64_t K, int x_dtype);

/*
 * Fused gate/up projection with SwiGLU epilogue:
 *   g = x @ (w[0:I]  * s[0:I]).T,   u = x @ (w[I:2I] * s[I:2I]).T
 *   h[M,I] = silu(g) * u            (fp32 math, one rounding to x_dtype)
 * w is the row-concatenation [Wg; Wu] of two per-channel-quantized [I,K]
 * weights (per-row quantization makes this identical to quantizing [2I,K]).
 * Replaces int8_gemm (gemm.py:189-238) twice followed by swiglu_fused
 * (src/rotalabs_accel/kernels/activations.py:108-138, kernel :51-80).
 * x_dtype: RA_F16 | RA_BF16. ldh >= I.
 */
int ra_w8a16_gateup_swiglu(const void *x, int64_t ldx, int x_dtype,
                           const int8_t *w, int64_t ldw, const float *scale,
                           void *h, int64_t ldh,
                           int64_t M, int64_t I, int64_t K, void *stream);

/* ra_w8a16_gateup_swiglu with a caller-owned workspace (contract as for
 * ra_w8a16_gemm_ws; size from ra_w8a16_gateup_workspace_size). */
int ra_w8a16_gateup_swiglu_ws(const void *x, int64_t ldx, int x_dtype,
                              const int8_t *w, int64_t ldw, const float *scale,
                              void *h, int64_t ldh,
                              int64_t M, int64_t I, int64_t K,
                              void *workspace, size_t workspace_bytes, void *stream);

size_t ra_w8a16_gateup_workspace_size(int64_t M, int64_t I, int64_t K, int x_dtype);

/*
 * Whether `stream` is being captured into a HIP graph (*capturing = 1, and
 * *capture_id = the capture's id, unique within the process) or not
 * (*capturing = 0, *capture_id = 0). Host plumbing with no counterpart in the
 * reference: the Python layer gives every graph capture a workspace of its
 * own, so that graphs never share one and a replay never depends on state
 * another graph or an eager call left behind.
 */
int ra_stream_capture_info(void *stream, int *capturing, unsigned long long *capture_id);

/*
 * y[r,:] = (x[r,:] * rsqrt(mean(x[r,:]^2) + eps)) rounded to x_dtype, times
 * weight, rounded to y_dtype -- the two roundings of rmsnorm_torch
 * (src/rotalabs_accel/kernels/normalization.py:32-45); math in fp32.
 * Replaces the GPU branch of rmsnorm (normalization.py:208-213 ->
 * _rmsnorm_triton :141-160 -> _rmsnorm_kernel :67-101).
 * x_dtype, w_dtype, y_dtype: RA_F16 | RA_BF16 | RA_F32; y_dtype must be the
 * promotion of x_dtype and w_dtype (as torch promotes x.to(x.dtype) * w).
 */
int ra_rmsnorm(const void *x, int64_t ldx, int x_dtype,
               const void *weight, int w_dtype,
               void *y, int64_t ldy, int y_dtype,
               int64_t rows, int64_t hidden, float eps, void *stream);

/*
 * ra_rmsnorm of v = x + residual, the sum rounded to the promotion of x_dtype
 * and r_dtype (as rmsnorm_residual_torch computes (x + residual).float(),
 * src/rotalabs_accel/kernels/normalization.py:48-64); the normalised value
 * is rounded to x_dtype, then multiplied by weight into y_dtype (the
 * promotion of x_dtype and w_dtype). Only y is written.
 * Replaces the GPU branch of rmsnorm_residual_fused (normalization.py:
 * 219-255 -> _rmsnorm_residual_triton :162-183 -> _rmsnorm_residual_kernel
 * :103-139).
 */
int ra_rmsnorm_residual(const void *x, int64_t ldx, int x_dtype,
                        const void *residual, int64_t ldr, int r_dtype,
                        const void *weight, int w_dtype,
                        void *y, int64_t ldy, int y_dtype,
                        int64_t rows, int64_t hidden, float eps, void *stream);

/*
 * out[i] = silu(gate[i]) * up[i] over n contiguous elements, fp32 math, one
 * rounding. Replaces swiglu_fused's GPU branch
 * (src/rotalabs_accel/kernels/activations.py:131-135 -> _swiglu_kernel :51-80).
 */
int ra_swiglu(const void *gate, const void *up, void *out, int64_t n,
              int dtype, void *stream);

/*
 * out = silu(gate + bias_gate[i % hidden]) * (up + bias_up[i % hidden]) over
 * n = rows * hidden contiguous elements (dtype), biases [hidden] in
 * bias_dtype; fp32 math, one rounding. Replaces swiglu_with_bias
 * (src/rotalabs_accel/kernels/swiglu.py:221-260 -> _swiglu_fused_kernel_with_bias
 * :180-218).
 */
int ra_swiglu_bias(const void *gate, const void *up,
                   const void *bias_gate, const void *bias_up, int bias_dtype,
                   void *out, int64_t n, int64_t hidden, int dtype, void *stream);

/*
 * Per-output-channel symmetric int8 quantization of w[N,K] (w_dtype RA_F32,
 * RA_F16 or RA_BF16), bit-exact with quantize_weight_per_channel on the CPU
 * (src/rotalabs_accel/quantization/symmetric.py:126-151 ->
 * quantize_symmetric(dim=1) :24-82): s = max|w_row| / 127 with IEEE division
 * (rounded to w_dtype for fp16/bf16), s = 1 for all-zero rows,
 * q = clamp(round_half_even(w / s), -128, 127); scale written as fp32.
 */
int ra_quantize_per_channel(const void *w, int64_t ldw, int w_dtype,
                            int64_t N, int64_t K,
                            int8_t *q, int64_t ldq, float *scale, void *stream);

/*
 * Per-row symmetric quantisation of a tensor viewed as [rows, cols] (the
 * last dimension is the row), as the KV-cache codec QuantizedTensor(t, bits,
 * per_channel=True) computes it on the CPU
 * (src/rotalabs_accel/speculative/kv_compression.py:51-78): with every
 * intermediate rounded to t_dtype, s = max(amax / qmax, 1e-8) with
 * qmax = 2^(bits-1) - 1, q = clamp(round_half_even(t / s), -qmax-1, qmax)
 * (an all-zero fp16 row, whose floor rounds to 0, gives q = 0).
 * q: int8 [rows, ldq]; scale: [rows] in t_dtype. bits: 8 or 4 (4-bit values
 * are stored one per int8, as the reference does).
 * No counterpart on the reference's GPU: it runs torch ops on any device.
 */
int ra_quantize_rows(const void *t, int64_t ldt, int t_dtype,
                     int64_t rows, int64_t cols, int bits,
                     int8_t *q, int64_t ldq, void *scale, void *stream);

/*
 * W8A8 route, step 1: per-row dynamic int8 quantisation of the activations
 * x[M,K] (fp16 or bf16), as _int8_gemm_cublas computes it
 * (src/rotalabs_accel/kernels/quantized_matmul.py:85-87), every op rounded to
 * x_dtype as torch does on the CPU, with c = act_scale (the reference's
 * default is 127) taken as an fp32 value: a = max(max_k |x[m,k]|, 1e-5) (NaN
 * propagates), xs[m] = a / c (true division), mult = reciprocal(a) * c
 * (torch's evaluation of c / a), q[m,k] = clamp(round_half_even(x[m,k] *
 * mult), -128, 127) (NaN -> 0).
 * q: int8 [M, ldq]; xs: [M] in x_dtype. K = 0 is an error (as torch's
 * amax over an empty row is).
 */
int ra_quantize_act_rows(const void *x, int64_t ldx, int x_dtype,
                         int64_t M, int64_t K,
                         int8_t *q, int64_t ldq, void *xs, float act_scale,
                         void *stream);

/*
 * W8A8 route, step 2: int8 x int8 GEMM on the int8 matrix cores,
 *   y[m,n] = (float(sum_k xq[m,k] * w[n,k]) * xs[m]) * scale[n] (+ bias[n])
 * with exact int32 sums and fp32 scaling rounded once to y_dtype. Replaces
 * torch._int_mm (quantized_matmul.py:93) and _dequantize_output (:38-40,
 * :99-100), which converts the int32 sums to fp16 first (|sum| > 65504
 * becomes inf there); the fp32 scaling is that of the reference's fused
 * int8 kernel (:259). bias (added as in :474-476) is optional.
 * xq: int8 [M, ldxq]; xs: [M] in y_dtype (fp16 or bf16, the activation
 * dtype); w: int8 [N, ldw]; scale: fp32 [N]; y: [M, ldy] in y_dtype.
 * K % 64 == 0 with 16-byte aligned rows and row strides runs the MFMA
 * kernel, anything else a slow VALU kernel.
 */
int ra_w8a8_gemm(const int8_t *xq, int64_t ldxq, const void *xs,
                 const int8_t *w, int64_t ldw, const float *scale,
                 const void *bias, int bias_dtype,
                 void *y, int64_t ldy, int y_dtype,
                 int64_t M, int64_t N, int64_t K, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* ROTACCEL_H */
