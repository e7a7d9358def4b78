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
// cache (K <= 64 * 8 * NI, NI = 1, 2, 4, 6 or 8 by K, so short rows keep few
// VGPRs and many waves in flight): 2 B read + 1 B written per element and
// 4 B per row. Longer rows are read a second time for the quantize pass
// (that second read is served by L2). Codes take quant_code_fast; a vector
// step in which any lane met a near-tie is redone with the exact quant_code
// (a few percent of steps), which keeps the common path branch-free.
#include "tvq_common.h"
#include "tvq_internal.h"

namespace tvq {
namespace {

constexpr int kRowsPerBlock = 4;
constexpr int kMaxIters = 8;  // 8 x 512 elements -> K <= 4096 stays in VGPRs

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
__device__ __forceinline__ uint32_t q1f(const u32x4& v, int i, float rs, bool& near) {
  const uint32_t w = v[i >> 1];
  const float x = to_float<T>((uint16_t)((i & 1) ? (w >> 16) : (w & 0xffffu)));
  return (uint32_t)((int32_t)quant_code_fast(x, rs, near) & 0xff);
}

// 8 codes, exact: fast codes unless some lane of the wave met a near-tie.
template <typename T>
__device__ __forceinline__ u32x2 quant8(u32x4 v, float s, float rs);
template <typename T>
__device__ __forceinline__ u32x2 quant8_wave(u32x4 v, float s, float rs) {
  bool near = false;
  u32x2 r;
  r.x = q1f<T>(v, 0, rs, near) | (q1f<T>(v, 1, rs, near) << 8) | (q1f<T>(v, 2, rs, near) << 16) |
        (q1f<T>(v, 3, rs, near) << 24);
  r.y = q1f<T>(v, 4, rs, near) | (q1f<T>(v, 5, rs, near) << 8) | (q1f<T>(v, 6, rs, near) << 16) |
        (q1f<T>(v, 7, rs, near) << 24);
  if (__builtin_amdgcn_ballot_w64(near) != 0) r = quant8<T>(v, s, rs);  // wave-uniform
  return r;
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
// NI >= 6: the compiler, left alone, took 129 (NI = 6) and 241 (NI = 8)
// VGPRs for what fits in ~60; asking for 6 waves per SIMD keeps them at
// 57 / 67 without spills (NI = 6 at 16384 x 3072: ~1.3 % of a W8A8 prefill).
template <typename T, int NI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NI >= 6 ? 6 : 1))) void act_quant_vec_kernel(const uint16_t* __restrict__ x, int64_t M, int64_t K,
                                                            float eps, int8_t* __restrict__ xq,
                                                            float* __restrict__ a_scales) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= M) return;
  const uint16_t* xr = x + row * K;
  int8_t* qr = xq + row * K;
  const int64_t nvec = K >> 3;  // 8 elements per 16-byte vector

  u32x4 cache[NI];
  float amax = 0.0f;
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int64_t v = (int64_t)it * kWave + lane;
    cache[it] = u32x4{0, 0, 0, 0};  // lanes past the row quantize zeros (no near-tie)
    if (v < nvec) {
      cache[it] = ldg128_stream(xr + v * 8);
      amax = fmaxf(amax, absmax8<T>(cache[it]));
    }
  }
  for (int64_t v = (int64_t)NI * kWave + lane; v < nvec; v += kWave) {
    amax = fmaxf(amax, absmax8<T>(ldg128_stream(xr + v * 8)));
  }
  amax = wave_max(amax);
  const float s = fmaxf(__fdiv_rn(amax, 127.0f), eps);
  if (lane == 0) a_scales[row] = s;
  const float rs = __fdiv_rn(1.0f, s);

#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int64_t v = (int64_t)it * kWave + lane;
    if (it * kWave < nvec) {  // wave-uniform: the ballot needs every active lane
      const u32x2 c = quant8_wave<T>(cache[it], s, rs);
      if (v < nvec) *reinterpret_cast<u32x2*>(qr + v * 8) = c;
    }
  }
  for (int64_t v0 = (int64_t)NI * kWave; v0 < nvec; v0 += kWave) {
    const int64_t v = v0 + lane;
    const u32x2 c = quant8_wave<T>(v < nvec ? ldg128(xr + v * 8) : u32x4{0, 0, 0, 0}, s, rs);
    if (v < nvec) *reinterpret_cast<u32x2*>(qr + v * 8) = c;
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
    // register cache sized to the row: 512 elements per iteration
#define TVQ_AQ(NI)                                                                    \
  (bf16 ? act_quant_vec_kernel<BF16, NI><<<grid, block, 0, stream>>>(xp, M, K, eps, xq, a_scales) \
        : act_quant_vec_kernel<F16, NI><<<grid, block, 0, stream>>>(xp, M, K, eps, xq, a_scales))
    if (K <= 512) TVQ_AQ(1);
    else if (K <= 1024) TVQ_AQ(2);
    else if (K <= 2048) TVQ_AQ(4);
    else if (K <= 3072) TVQ_AQ(6);
    else TVQ_AQ(kMaxIters);
#undef TVQ_AQ
  } else {
    if (bf16)
      act_quant_scalar_kernel<BF16><<<grid, block, 0, stream>>>(xp, M, K, eps, xq, a_scales);
    else
      act_quant_scalar_kernel<F16><<<grid, block, 0, stream>>>(xp, M, K, eps, xq, a_scales);
  }
  return hipGetLastError();
}

}  // namespace tvq
