// tvq_w8a8_linear_noalloc: the fused W8A8 linear (act-quant + GEMM) for
// callers that cannot allocate device memory (code under HIP-graph capture
// that must not call hipMalloc, tight serving loops, harnesses that forbid
// allocation). Its scratch memory -- the int8 activation codes, the
// per-token scales and the split-K workspace -- lives in one file-scope
// device array instead of caller buffers.
//
// `scratch` below is a device symbol: its host-side name is only a stand-in,
// so host code never passes it to a kernel or a copy. Each device's address
// comes from hipGetSymbolAddress on the first call with that device current,
// and is kept per device; every device holds its own copy of the array.
//
// Calls on one device share that device's array: calls that overlap on one
// GPU (several streams, or several host threads without ordering) race.
#include <mutex>

#include "../../include/tvq.h"
#include "tvq_internal.h"

namespace {

// Layout of the scratch array (every region 256-byte aligned):
//   [0, kWsBytes)                      split-K workspace: counters, partial tiles
//   [kWsBytes, +kXqMaxBytes)           int8 activation codes, M*K bytes
//   [kWsBytes + kXqMaxBytes, +4*M)     fp32 per-token scales
constexpr int64_t kWsBytes = (16 << 20) + (64 << 10);
constexpr int64_t kXqMaxBytes = TVQ_NOALLOC_MAX_XQ_BYTES;
constexpr int64_t kMaxRows = TVQ_NOALLOC_MAX_ROWS;
constexpr int64_t kScratchBytes = kWsBytes + kXqMaxBytes + kMaxRows * 4;
static_assert(kWsBytes % 256 == 0 && kXqMaxBytes % 256 == 0, "regions stay 256-byte aligned");

__device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
char* g_scratch[kMaxDevices] = {};

// Address of the current device's scratch array (looked up once per device).
// Nothing is cleared: a file-scope __device__ array is zero when the code
// object loads, and the split-K fixup's last arriver resets each tile counter
// it used, so the counter block is zero again after every completed call
// (the codes and scales are fully rewritten by each call's act-quant).
int device_scratch(char** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return tvq::report_error(TVQ_E_HIP, "tvq_w8a8_linear_noalloc: no current HIP device");
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return tvq::report_error(TVQ_E_HIP, "tvq_w8a8_linear_noalloc: hipGetSymbolAddress(scratch) failed");
    g_scratch[dev] = static_cast<char*>(p);
  }
  *out = g_scratch[dev];
  return TVQ_OK;
}

}  // namespace

extern "C" int tvq_w8a8_linear_noalloc(const void* x, int dtype, const int8_t* qweight, const float* w_scales,
                                       const void* bias, void* y, int64_t M, int64_t N, int64_t K, void* stream) {
  if (M < 0 || K <= 0 || N <= 0)
    return tvq::report_error(TVQ_E_INVALID, "tvq_w8a8_linear_noalloc: invalid shape");
  if (M > kMaxRows || M * K > kXqMaxBytes)
    return tvq::report_error(TVQ_E_UNSUPPORTED,
                             "tvq_w8a8_linear_noalloc: M*K exceeds the scratch maximum "
                             "(M <= TVQ_NOALLOC_MAX_ROWS, M*K <= TVQ_NOALLOC_MAX_XQ_BYTES)");
  if (M == 0) return tvq_w8a8_linear(x, dtype, qweight, w_scales, bias, y, M, N, K, nullptr, nullptr, nullptr, 0,
                                     stream);
  char* base = nullptr;
  if (int rc = device_scratch(&base)) return rc;
  int8_t* xq = reinterpret_cast<int8_t*>(base + kWsBytes);
  float* a_scales = reinterpret_cast<float*>(base + kWsBytes + kXqMaxBytes);
  return tvq_w8a8_linear(x, dtype, qweight, w_scales, bias, y, M, N, K, xq, a_scales, base, kWsBytes, stream);
}
