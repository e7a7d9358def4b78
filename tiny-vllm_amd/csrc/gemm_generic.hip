// Generic scalar W8A16 / W8A8 kernel: any K, any pointer alignment.
//
// Serves the shapes the vector paths cannot (K % 16 != 0, unaligned views),
// the role the reference's SIMT fallback kernels play
// (int8_weight_only_gemm.cu:178-297, w8a8_gemm.cu:89-205). One thread per
// output element, k ascending; the same epilogues as the MFMA paths.
#include "tvq_common.h"
#include "tvq_internal.h"

namespace tvq {
namespace {

template <typename T, bool kW8A8, bool kRaw, bool kDq = false>
__global__ __launch_bounds__(256) void generic_kernel(const void* __restrict__ xv, const float* __restrict__ a_scales,
                                                      const int8_t* __restrict__ qw, const float* __restrict__ ws,
                                                      const uint16_t* __restrict__ bias, void* __restrict__ yv,
                                                      int64_t M, int64_t N, int64_t K) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= M * N) return;
  const int64_t m = idx / N;
  const int64_t n = idx % N;
  const int8_t* w = qw + n * K;
  if constexpr (kW8A8) {
    const int8_t* x = static_cast<const int8_t*>(xv) + m * K;
    int32_t acc = 0;
    for (int64_t k = 0; k < K; ++k) acc += (int32_t)x[k] * (int32_t)w[k];
    if constexpr (kRaw) {
      static_cast<int32_t*>(yv)[idx] = acc;
    } else {
      const float b = bias ? to_float<T>(bias[n]) : 0.0f;
      static_cast<uint16_t*>(yv)[idx] = from_float<T>(epi_w8a8(acc, a_scales[m], ws[n], b));
    }
  } else {
    const uint16_t* x = static_cast<const uint16_t*>(xv) + m * K;
    float acc = 0.0f;
    if constexpr (kDq) {
      // T(T(q) * T(s)) per weight (int8_weight_only_gemm.cu:401-411)
      const float sr = round_to<T>(ws[n]);
      for (int64_t k = 0; k < K; ++k) acc = __builtin_fmaf(to_float<T>(x[k]), round_to<T>((float)w[k] * sr), acc);
    } else {
      for (int64_t k = 0; k < K; ++k) acc = __builtin_fmaf(to_float<T>(x[k]), (float)w[k], acc);
    }
    const float b = bias ? to_float<T>(bias[n]) : 0.0f;
    static_cast<uint16_t*>(yv)[idx] = from_float<T>(epi_w8a16(acc, kDq ? 1.0f : ws[n], b));
  }
}

template <typename T, bool kW8A8, bool kRaw, bool kDq = false>
hipError_t launch_t(const GemmArgs& a, hipStream_t stream) {
  const int64_t total = a.M * a.N;
  const dim3 grid((unsigned)((total + 255) / 256));
  generic_kernel<T, kW8A8, kRaw, kDq><<<grid, dim3(256), 0, stream>>>(
      a.x, a.a_scales, a.qweight, a.scales, static_cast<const uint16_t*>(a.bias), a.y, a.M, a.N, a.K);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_generic(const GemmArgs& a, hipStream_t stream) {
  if (a.w8a8) {
    if (a.raw_i32) return launch_t<BF16, true, true>(a, stream);
    return a.bf16 ? launch_t<BF16, true, false>(a, stream) : launch_t<F16, true, false>(a, stream);
  }
  return a.bf16 ? launch_t<BF16, false, false>(a, stream) : launch_t<F16, false, false>(a, stream);
}

hipError_t launch_generic_dq(const GemmArgs& a, hipStream_t stream) {
  return a.bf16 ? launch_t<BF16, false, false, true>(a, stream) : launch_t<F16, false, false, true>(a, stream);
}

}  // namespace tvq
