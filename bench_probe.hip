// Measurement probe (not part of the GEMM library): plain streaming reads of
// an int8 [N, K] matrix with the decode kernels' access pattern -- one row
// per wave, lane l reading bytes 16l .. 16l+15 of each 1 KB window of the
// row, every window of the row in flight at once, non-temporal loads -- and
// no arithmetic beyond folding the loaded words into one register. Two
// modes:
//  * read: the weight bytes only;
//  * io: also the GEMV's other traffic -- each workgroup copies x[0:K] (fp16
//    or bf16) into LDS with the kernels' direct-to-LDS copy and barrier, and
//    each wave stores one 16-bit word y[n] -- without the dequantisation and
//    dot products.
// Their durations are the single-launch floors the M=1 GEMV kernels are
// compared with (bench.py --only ceiling). bench.py builds it into
// bench_probe.so beside itself, with the library's compile flags.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int CH, bool IO>
__global__ __launch_bounds__(512) void stream_rows_kernel(const int8_t *w, int64_t ldw, int N, int K,  // (w not
                                                          // restrict: its loads stay in front of the copy wait)
                                                          int wpg, const uint16_t *__restrict__ x,
                                                          uint16_t *__restrict__ y, unsigned *__restrict__ sink) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xl[];
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = blockIdx.x * wpg + wid;  // < N: the host launches N / wpg whole workgroups in io mode
  if (!IO && n >= N) return;
  if (IO) {
    const uint32_t lds0 = (uint32_t)(uintptr_t)xl;
    for (int j = wid; 1024 * j < 2 * K; j += wpg) {
      const int off = 1024 * j + 16 * lane;
      if (off < 2 * K)
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds0 + 1024 * j),
                     "v"(reinterpret_cast<const char *>(x) + off)
                     : "memory", "m0");
    }
  }
  const int8_t *row = w + (int64_t)n * ldw + 16 * lane;
  u32x4 v[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int k = 1024 * c + 16 * lane < K ? 1024 * c : -16 * lane;  // past K: the row's first chunk
    v[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(row + k));
  }
  if (IO) {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(CH) : "memory");
    __builtin_amdgcn_sched_barrier(0);  // no use of the weights in front of the barrier
  }
  unsigned a = 0;
#pragma unroll
  for (int c = 0; c < CH; ++c) a ^= v[c].x ^ v[c].y ^ v[c].z ^ v[c].w;
  // Every lane tests its own words (a test in one lane only would let the
  // compiler load one lane's share); the store reads the copy.
  if (a == 0x9e3779b9u) sink[0] = a;  // keeps the loads; (practically) never taken
  if (IO && lane == 0) y[n] = xl[n & 1023];
}

}  // namespace

// Streams rows [0, N) of w (ldw >= K bytes per row, K % 16 == 0, 16 <= K <=
// 32768, 16-byte aligned) with `wpg` waves (rows) per workgroup (1..8).
// io = 0: read mode (x and y unused, may be null); io = 1: io mode (x: K
// 16-bit words, y: N 16-bit words, N % wpg == 0). sink: one device word.
// Returns a hipError_t value (0 on success), 1 for arguments out of range.
extern "C" int rap_stream_rows(const int8_t *w, int64_t ldw, int64_t N, int64_t K, int wpg, int io,
                               const uint16_t *x, uint16_t *y, unsigned *sink, void *stream) {
  if (!w || !sink || N <= 0 || K < 16 || K % 16 || K > 32768 || ldw < K || wpg < 1 || wpg > 8) return 1;
  if (io && (!x || !y || N % wpg)) return 1;
  const int ch = (int)((K + 1023) / 1024);
  const dim3 grid((unsigned)((N + wpg - 1) / wpg)), block(64 * wpg);
  const size_t lds = io ? (size_t)2048 * ch : 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
#define RAP(CH_)                                                                                            \
  if (ch <= CH_) {                                                                                        \
    if (io)                                                                                               \
      hipLaunchKernelGGL((stream_rows_kernel<CH_, true>), grid, block, lds, s, w, ldw, (int)N, (int)K, wpg, x, \
                         y, sink);                                                                        \
    else                                                                                                  \
      hipLaunchKernelGGL((stream_rows_kernel<CH_, false>), grid, block, 0, s, w, ldw, (int)N, (int)K, wpg, x, \
                         y, sink);                                                                        \
    return (int)hipGetLastError();                                                                        \
  }
  RAP(4) RAP(8) RAP(12) RAP(16) RAP(32)
#undef RAP
  return 1;
}
