// Per-token dynamic int8 activation quantization for gfx950.
//
// Restates quantize_int8_per_row_dynamic (nanovllm/quantization/utils.py:28-32)
// bit for bit, as one kernel instead of the reference's chain of ~9 torch
// elementwise/reduction launches with fp32 temporaries:
//   amax   = max_k |float(x[m,k])|                (exact, order-free)
//   s      = max(amax / 127.0f, eps)               (IEEE RN divide)
//   xq     = clamp(rint(float(x) / s), -127, 127)  (IEEE RN divide, ties-to-even;
//            computed as a multiply by RN(1/s) plus one exact fma correction,
//            see quant_code)
//
// A row is owned by TPR threads (one to four waves) of a 256-thread
// workgroup: 64 when there are enough rows to fill the GPU (4 rows per
// workgroup), up to 256 for small M, so that a decode-size call (M = 1..512)
// still spreads each row's loads over many lanes and the GPU has up to one
// workgroup per row. With TPR > 64 the row maximum is combined across the
// row's waves through LDS. HBM traffic is the algorithmic minimum for rows
// that fit the register cache (K <= TPR * 8 * NI, NI = 1, 2, 4, 6 or 8 by K,
// so short rows keep few VGPRs and many waves in flight): 2 B read + 1 B
// written per element and 4 B per row. Longer rows are read a second time
// for the quantize pass (that second read is served by L2). The codes are
// branch-free (quant_code: one multiply, two fma, rint, clamp per element).
#include "tvq_common.h"
#include "tvq_internal.h"

namespace tvq {
namespace {

constexpr int kBlock = 256;
constexpr int kRowsPerBlock = 4;  // scalar path
constexpr int kMaxIters = 8;      // 8 x 8 x TPR elements stay in VGPRs

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

// Vector path: K % 8 == 0 and 16-byte aligned x, 8-byte aligned xq.
// NI >= 6: the compiler, left alone, took 129 (NI = 6) and 241 (NI = 8)
// VGPRs for what fits in ~60; asking for 6 waves per SIMD keeps them at
// 57 / 67 without spills (NI = 6 at 16384 x 3072: ~1.3 % of a W8A8 prefill).
template <typename T, int TPR, int NI>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(NI >= 6 ? 6 : 1))) void act_quant_vec_kernel(
    const uint16_t* __restrict__ x, int64_t M, int64_t K, float eps, int8_t* __restrict__ xq,
    float* __restrict__ a_scales) {
  static_assert(TPR == 64 || TPR == 128 || TPR == 256, "a row is one, two or four waves");
  constexpr int kWavesPerRow = TPR / kWave;
  const int t = threadIdx.x % TPR;  // lane within the row
  const int64_t row = (int64_t)blockIdx.x * (kBlock / TPR) + threadIdx.x / TPR;
  if constexpr (kWavesPerRow == 1) {
    if (row >= M) return;  // no barrier below
  }
  const bool live = row < M;  // rows past M (TPR > 64) still reach the barrier
  const uint16_t* xr = x + (live ? row : 0) * K;
  int8_t* qr = xq + row * K;
  const int64_t nvec = live ? (K >> 3) : 0;  // 8 elements per 16-byte vector

  // All NI loads go out before any is used: the index is clamped into the
  // row instead of branching around the load, so no wait sits between them
  // (a load under a per-iteration branch with its use inside the branch
  // costs one memory round trip per iteration).
  u32x4 cache[NI];
  float amax = 0.0f;
  const int64_t vmax = nvec > 0 ? nvec - 1 : 0;
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int64_t v = (int64_t)it * TPR + t;
    cache[it] = ldg128_stream(xr + (v < vmax ? v : vmax) * 8);
  }
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int64_t v = (int64_t)it * TPR + t;
    if (v >= nvec) cache[it] = u32x4{0, 0, 0, 0};  // lanes past the row quantize zeros (no near-tie)
    amax = fmaxf(amax, absmax8<T>(cache[it]));
  }
  for (int64_t v = (int64_t)NI * TPR + t; v < nvec; v += TPR) {
    amax = fmaxf(amax, absmax8<T>(ldg128_stream(xr + v * 8)));
  }
  amax = wave_max(amax);
  if constexpr (kWavesPerRow > 1) {
    __shared__ float red[kBlock / kWave];
    const int w = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) red[w] = amax;
    __syncthreads();
    const int w0 = (threadIdx.x / TPR) * kWavesPerRow;
#pragma unroll
    for (int i = 0; i < kWavesPerRow; ++i) amax = fmaxf(amax, red[w0 + i]);
    if (!live) return;
  }
  const float s = fmaxf(__fdiv_rn(amax, 127.0f), eps);
  if (t == 0) a_scales[row] = s;
  const float rs = __fdiv_rn(1.0f, s);

#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int64_t v = (int64_t)it * TPR + t;
    if (v < nvec) *reinterpret_cast<u32x2*>(qr + v * 8) = quant_codes8<T>(cache[it], s, rs);
  }
  for (int64_t v0 = (int64_t)NI * TPR; v0 < nvec; v0 += TPR) {
    const int64_t v = v0 + t;
    if (v < nvec) *reinterpret_cast<u32x2*>(qr + v * 8) = quant_codes8<T>(ldg128(xr + v * 8), s, rs);
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

// Threads per row: 64 once M / 4 workgroups fill the GPU, more for fewer
// rows (up to one 256-thread workgroup per row), and always enough for the
// row to fit the register cache (8 vectors of 8 per thread), so long rows
// are never read twice.
int act_quant_tpr(int64_t M, int64_t K) {
  int tpr = M >= 1024 ? 64 : (M >= 512 ? 128 : 256);
  while (tpr < 256 && K > (int64_t)tpr * 8 * kMaxIters) tpr *= 2;
  return tpr;
}

namespace {

template <typename T, int TPR>
hipError_t launch_vec(const uint16_t* xp, int64_t M, int64_t K, float eps, int8_t* xq, float* a_scales,
                      hipStream_t stream) {
  const dim3 grid((unsigned)((M + kBlock / TPR - 1) / (kBlock / TPR)));
  const int64_t per = (K / 8 + TPR - 1) / TPR;  // 16-byte vectors per thread
  // register cache sized to the row
  if (per <= 1) act_quant_vec_kernel<T, TPR, 1><<<grid, kBlock, 0, stream>>>(xp, M, K, eps, xq, a_scales);
  else if (per <= 2) act_quant_vec_kernel<T, TPR, 2><<<grid, kBlock, 0, stream>>>(xp, M, K, eps, xq, a_scales);
  else if (per <= 4) act_quant_vec_kernel<T, TPR, 4><<<grid, kBlock, 0, stream>>>(xp, M, K, eps, xq, a_scales);
  else if (per <= 6) act_quant_vec_kernel<T, TPR, 6><<<grid, kBlock, 0, stream>>>(xp, M, K, eps, xq, a_scales);
  else act_quant_vec_kernel<T, TPR, kMaxIters><<<grid, kBlock, 0, stream>>>(xp, M, K, eps, xq, a_scales);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_vec_t(const uint16_t* xp, int64_t M, int64_t K, float eps, int8_t* xq, float* a_scales,
                        hipStream_t stream) {
  switch (act_quant_tpr(M, K)) {
    case 64: return launch_vec<T, 64>(xp, M, K, eps, xq, a_scales, stream);
    case 128: return launch_vec<T, 128>(xp, M, K, eps, xq, a_scales, stream);
    default: return launch_vec<T, 256>(xp, M, K, eps, xq, a_scales, stream);
  }
}

}  // namespace

hipError_t launch_act_quant(const void* x, bool bf16, int64_t M, int64_t K, float eps, int8_t* xq, float* a_scales,
                            hipStream_t stream) {
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  if (act_quant_vec_ok(x, xq, K)) {
    return bf16 ? launch_vec_t<BF16>(xp, M, K, eps, xq, a_scales, stream)
                : launch_vec_t<F16>(xp, M, K, eps, xq, a_scales, stream);
  }
  const dim3 grid((unsigned)((M + kRowsPerBlock - 1) / kRowsPerBlock));
  if (bf16)
    act_quant_scalar_kernel<BF16><<<grid, kBlock, 0, stream>>>(xp, M, K, eps, xq, a_scales);
  else
    act_quant_scalar_kernel<F16><<<grid, kBlock, 0, stream>>>(xp, M, K, eps, xq, a_scales);
  return hipGetLastError();
}

}  // namespace tvq
