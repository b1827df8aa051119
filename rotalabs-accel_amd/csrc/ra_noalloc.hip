// ra_w8a16_gemm_noalloc: ra_w8a16_gemm_ws for callers that cannot allocate
// (code under HIP graph capture, serving loops that forbid allocation). The
// workspace of the small-batch kernels that split K (the split-K kernel,
// the tiled kernel's split plan) is a fixed device array of this library
// instead of a caller buffer; nothing is allocated or freed.
//
//  * `scratch` is a file-scope device array, one per GPU the library runs on
//    (each holds its own copy at its own address until the process ends).
//    Host code uses the address hipGetSymbolAddress returns for the current
//    device, looked up once per device on that device's first call; the
//    array's name is only a host-side stand-in.
//  * The split-K kernel needs the counter block at the start of its
//    workspace to be zero and leaves it zero after every call; the first
//    call on a device clears it with a fill kernel (not a memset, so the
//    call may be captured into a graph).
//  * Every call on a GPU shares that GPU's array: calls that may overlap on
//    one GPU (several streams, or graph replays beside eager calls) race.
#include <mutex>

#include "ra_internal.h"

namespace {

constexpr size_t kScratchBytes = (size_t)16 << 20;  // largest workspace a call may need
static_assert(kScratchBytes >= ra::kSplitkMaxWorkspace, "every split-K plan fits the array");
constexpr int kMaxDevices = 64;

}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

std::mutex g_mutex;
void *g_scratch[kMaxDevices];  // device address of `scratch`, per device

__global__ void clear_words(uint32_t *p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Device address of `scratch` on the current device (looked up, and its
// counter block cleared, on the device's first call).
int scratch_address(void **out, hipStream_t s) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return RA_ERR_DEVICE;
  std::lock_guard<std::mutex> lock(g_mutex);
  if (g_scratch[dev] == nullptr) {
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return RA_ERR_DEVICE;
    constexpr int words = (int)(ra::kSplitkCounterBytes / sizeof(uint32_t));
    hipLaunchKernelGGL(clear_words, dim3((words + 255) / 256), dim3(256), 0, s, static_cast<uint32_t *>(p), words);
    if (hipGetLastError() != hipSuccess) return RA_ERR_LAUNCH;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return RA_OK;
}

}  // namespace

extern "C" int ra_w8a16_gemm_noalloc(const void *x, int64_t ldx, int x_dtype, const int8_t *w, int64_t ldw,
                                     const float *scale, const void *bias, int bias_dtype, void *y, int64_t ldy,
                                     int64_t M, int64_t N, int64_t K, void *stream) {
  const ra::GemmArgs a{x, ldx, x_dtype, w, ldw, scale, bias, bias_dtype, y, ldy, M, N, K};
  // Argument errors first (ra_w8a16_gemm_ws reports them the same way).
  if (M < 0 || N < 0 || K < 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return RA_ERR_ARG;
  if (M == 0 || N == 0) return ra_w8a16_gemm_ws(x, ldx, x_dtype, w, ldw, scale, bias, bias_dtype, y, ldy, M, N, K,
                                                nullptr, 0, stream);
  size_t need = (x_dtype == RA_F16 || x_dtype == RA_BF16) ? ra::auto_workspace_bytes(a) : 0;
  if (need > kScratchBytes) {  // only a tiled split plan can need more (split-K plans are capped)
    if (!ra::auto_workspace_optional(a)) return RA_ERR_WORKSPACE;
    need = 0;  // the tiled kernel runs its tile over all of K instead
  }
  void *ws = nullptr;
  size_t ws_bytes = 0;
  if (need > 0) {
    const int st = scratch_address(&ws, static_cast<hipStream_t>(stream));
    if (st != RA_OK) return st;
    ws_bytes = kScratchBytes;
  }
  return ra_w8a16_gemm_ws(x, ldx, x_dtype, w, ldw, scale, bias, bias_dtype, y, ldy, M, N, K, ws, ws_bytes, stream);
}
