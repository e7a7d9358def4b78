// Per-token dynamic int8 activation quantization for gfx950.
//
// Restates quantize_int8_per_row_dynamic (nanovllm/quantization/utils.py:28-32)
// bit for bit, as one kernel instead of the reference's chain of ~9 torch
// elementwise/reduction launches with fp32 temporaries:
//   amax   = max_k |float(x[m,k])|                (exact, order-free)
//   s      = max(amax / 127.0f, eps)               (IEEE RN divide)
//   xq     = clamp(rint(float(x) / s), -127, 127)  (IEEE RN divide, ties-to-even;
//            computed as a multiply by RN(1/s) with an exact-divide fallback
//            near half-integers, see quant_code)
//
// One wave (64 lanes) owns one row; a 256-thread workgroup handles 4 rows.
// HBM traffic is the algorithmic minimum for rows that fit the register
// cache (K <= 64 * 8 * kCacheIters): 2 B read + 1 B written per element and
// 4 B per row. Longer rows are read a second time for the quantize pass
// (that second read is served by L2).
#include "tvq_common.h"
#include "tvq_internal.h"

namespace tvq {
namespace {

constexpr int kRowsPerBlock = 4;
constexpr int kCacheIters = 8;  // 8 x 512 elements -> K <= 4096 stays in VGPRs

__device__ __forceinline__ float wave_max(float v) {
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

template <typename T>
__device__ __forceinline__ float absmax8(u32x4 v) {
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m = fmaxf(m, fabsf(to_float<T>((uint16_t)(v[i] & 0xffffu))));
    m = fmaxf(m, fabsf(to_float<T>((uint16_t)(v[i] >> 16))));
  }
  return m;
}

__device__ __forceinline__ uint32_t q1(float x, float s, float rs) {
  return (uint32_t)((int32_t)quant_code(x, s, rs) & 0xff);
}

template <typename T>
__device__ __forceinline__ u32x2 quant8(u32x4 v, float s, float rs) {
  u32x2 r;
  r.x = q1(to_float<T>((uint16_t)(v[0] & 0xffffu)), s, rs) | (q1(to_float<T>((uint16_t)(v[0] >> 16)), s, rs) << 8) |
        (q1(to_float<T>((uint16_t)(v[1] & 0xffffu)), s, rs) << 16) | (q1(to_float<T>((uint16_t)(v[1] >> 16)), s, rs) << 24);
  r.y = q1(to_float<T>((uint16_t)(v[2] & 0xffffu)), s, rs) | (q1(to_float<T>((uint16_t)(v[2] >> 16)), s, rs) << 8) |
        (q1(to_float<T>((uint16_t)(v[3] & 0xffffu)), s, rs) << 16) | (q1(to_float<T>((uint16_t)(v[3] >> 16)), s, rs) << 24);
  return r;
}

// Vector path: K % 8 == 0 and 16-byte aligned x, 8-byte aligned xq.
template <typename T>
__global__ __launch_bounds__(256) void act_quant_vec_kernel(const uint16_t* __restrict__ x, int64_t M, int64_t K,
                                                            float eps, int8_t* __restrict__ xq,
                                                            float* __restrict__ a_scales) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= M) return;
  const uint16_t* xr = x + row * K;
  int8_t* qr = xq + row * K;
  const int64_t nvec = K >> 3;  // 8 elements per 16-byte vector

  u32x4 cache[kCacheIters];
  float amax = 0.0f;
#pragma unroll
  for (int it = 0; it < kCacheIters; ++it) {
    const int64_t v = (int64_t)it * kWave + lane;
    if (v < nvec) {
      cache[it] = ldg128_stream(xr + v * 8);
      amax = fmaxf(amax, absmax8<T>(cache[it]));
    }
  }
  for (int64_t v = (int64_t)kCacheIters * kWave + lane; v < nvec; v += kWave) {
    amax = fmaxf(amax, absmax8<T>(ldg128_stream(xr + v * 8)));
  }
  amax = wave_max(amax);
  const float s = fmaxf(__fdiv_rn(amax, 127.0f), eps);
  if (lane == 0) a_scales[row] = s;
  const float rs = __fdiv_rn(1.0f, s);

#pragma unroll
  for (int it = 0; it < kCacheIters; ++it) {
    const int64_t v = (int64_t)it * kWave + lane;
    if (v < nvec) *reinterpret_cast<u32x2*>(qr + v * 8) = quant8<T>(cache[it], s, rs);
  }
  for (int64_t v = (int64_t)kCacheIters * kWave + lane; v < nvec; v += kWave) {
    *reinterpret_cast<u32x2*>(qr + v * 8) = quant8<T>(ldg128(xr + v * 8), s, rs);
  }
}

// Scalar path for any K / alignment.
template <typename T>
__global__ __launch_bounds__(256) void act_quant_scalar_kernel(const uint16_t* __restrict__ x, int64_t M, int64_t K,
                                                               float eps, int8_t* __restrict__ xq,
                                                               float* __restrict__ a_scales) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= M) return;
  const uint16_t* xr = x + row * K;
  float amax = 0.0f;
  for (int64_t k = lane; k < K; k += kWave) amax = fmaxf(amax, fabsf(to_float<T>(xr[k])));
  amax = wave_max(amax);
  const float s = fmaxf(__fdiv_rn(amax, 127.0f), eps);
  if (lane == 0) a_scales[row] = s;
  const float rs = __fdiv_rn(1.0f, s);
  for (int64_t k = lane; k < K; k += kWave) xq[row * K + k] = (int8_t)q1(to_float<T>(xr[k]), s, rs);
}

}  // namespace

bool act_quant_vec_ok(const void* x, const void* xq, int64_t K) {
  return (K % 8 == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)xq % 8 == 0);
}

hipError_t launch_act_quant(const void* x, bool bf16, int64_t M, int64_t K, float eps, int8_t* xq, float* a_scales,
                            hipStream_t stream) {
  const dim3 grid((unsigned)((M + kRowsPerBlock - 1) / kRowsPerBlock));
  const dim3 block(256);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  if (act_quant_vec_ok(x, xq, K)) {
    if (bf16)
      act_quant_vec_kernel<BF16><<<grid, block, 0, stream>>>(xp, M, K, eps, xq, a_scales);
    else
      act_quant_vec_kernel<F16><<<grid, block, 0, stream>>>(xp, M, K, eps, xq, a_scales);
  } else {
    if (bf16)
      act_quant_scalar_kernel<BF16><<<grid, block, 0, stream>>>(xp, M, K, eps, xq, a_scales);
    else
      act_quant_scalar_kernel<F16><<<grid, block, 0, stream>>>(xp, M, K, eps, xq, a_scales);
  }
  return hipGetLastError();
}

}  // namespace tvq
