// Producers of the quantized projections' inputs, with the per-token int8
// activation quantization fused in (gfx950).
//
// rmsnorm  (reference nanovllm/layers/layernorm.py:16-40, rms_forward and
//           add_rms_forward), per row of K elements:
//     h      = float(x) [+ float(residual)]          (fp32 add)
//     residual <- round(h)                            (when a residual is given)
//     r      = 1 / sqrt(mean(h*h) + eps)              (fp32, IEEE sqrt and divide)
//     y      = round(float(round(h * r)) * float(w))  (two roundings, as torch)
// silu_mul (reference nanovllm/layers/activation.py:11-14), per row of 2*I:
//     y      = round(silu(g) * u),  silu(g) = g / (1 + exp(-g)) in fp32,
//     g = row[0:I], u = row[I:2I]                     (one rounding, as the
//                                                      compiled reference)
// Either kernel may emit, instead of or beside y, the per-token int8 codes
// and scale of y exactly as quantize_int8_per_row_dynamic
// (nanovllm/quantization/utils.py:28-32) computes them from the rounded y:
//     s = max(amax|y| / 127, eps);  q = clamp(rint(y / s), -127, 127).
// So the W8A8 projections that consume them skip one bf16 write + read of
// the activations and one launch; the codes are bit-identical to running
// act-quant on this kernel's own y.
//
// One wave owns one row, 4 rows per 256-thread workgroup (like act-quant).
// Rows of up to 4096 elements (8 x 512) stay in registers, so HBM traffic is
// the algorithmic minimum: read x (+ residual, + w from L2), write residual
// and y (2 B/elem) and/or the codes (1 B/elem) + 4 B per row. Longer rows or
// K % 8 != 0 or unaligned pointers take a scalar path that re-reads the row
// (from L2).
#include <type_traits>

#include "tvq_common.h"
#include "tvq_internal.h"

namespace tvq {
namespace {

constexpr int kRows = 4;
constexpr int kIters = 8;  // at most 8 x 64 lanes x 8 elements = 4096 per row in registers

__device__ __forceinline__ float wsum(float v) {
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}
__device__ __forceinline__ float wmax(float v) {
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

__device__ __forceinline__ int8_t qcode(float y, float s, float rs) { return (int8_t)(int)quant_code(y, s, rs); }

template <typename T>
__device__ __forceinline__ float elt(const u32x4& v, int i) {
  const uint32_t w = v[i >> 1];
  return to_float<T>((uint16_t)((i & 1) ? (w >> 16) : (w & 0xffffu)));
}

template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return (uint32_t)from_float<T>(a) | ((uint32_t)from_float<T>(b) << 16);
}

// Quantize the 8-element bf16/fp16 vectors cached in y[] (already rounded)
// and store codes + scale. Codes take quant_code_fast; a vector step where
// any lane met a near-tie is redone with the exact quant_code.
template <typename T, int NI>
__device__ __forceinline__ void quant_store(const u32x4 (&y)[NI], int nvec, int lane, float eps, int8_t* qr,
                                            float* srow) {
  float amax = 0.0f;
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    if (it * kWave + lane < nvec) {
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(elt<T>(y[it], i)));
    }
  }
  amax = wmax(amax);
  const float s = fmaxf(__fdiv_rn(amax, 127.0f), eps);
  if (lane == 0) *srow = s;
  const float rs = __fdiv_rn(1.0f, s);
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int v = it * kWave + lane;
    if (it * kWave < nvec) {  // wave-uniform: the ballot needs every active lane
      const u32x4 yv = v < nvec ? y[it] : u32x4{0, 0, 0, 0};
      bool near = false;
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lo |= ((uint32_t)(int32_t)quant_code_fast(elt<T>(yv, i), rs, near) & 0xffu) << (8 * i);
        hi |= ((uint32_t)(int32_t)quant_code_fast(elt<T>(yv, i + 4), rs, near) & 0xffu) << (8 * i);
      }
      if (__builtin_amdgcn_ballot_w64(near) != 0) {
        lo = hi = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lo |= (uint32_t)(uint8_t)qcode(elt<T>(yv, i), s, rs) << (8 * i);
          hi |= (uint32_t)(uint8_t)qcode(elt<T>(yv, i + 4), s, rs) << (8 * i);
        }
      }
      if (v < nvec) *reinterpret_cast<u32x2*>(qr + (int64_t)v * 8) = u32x2{lo, hi};
    }
  }
}

template <typename T, bool kRes, bool kY, bool kQ, int NI>
__global__ __launch_bounds__(256) void rmsnorm_vec_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ res,
                                                          const uint16_t* __restrict__ w, float eps,
                                                          uint16_t* __restrict__ y, int8_t* __restrict__ xq,
                                                          float* __restrict__ a_scales, int64_t M, int K) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRows + (threadIdx.x >> 6);
  if (row >= M) return;
  const int nvec = K >> 3;
  const uint16_t* xr = x + row * K;
  float h[NI][8];
  float ss = 0.0f;
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int v = it * kWave + lane;
    if (v < nvec) {
      const u32x4 xv = ldg128_stream(xr + (int64_t)v * 8);
      u32x4 rv = {0, 0, 0, 0};
      if constexpr (kRes) rv = ldg128_stream(res + row * K + (int64_t)v * 8);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float t = elt<T>(xv, i);
        if constexpr (kRes) t += elt<T>(rv, i);
        h[it][i] = t;
        ss += t * t;
      }
      if constexpr (kRes) {
        u32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = pack2<T>(h[it][2 * i], h[it][2 * i + 1]);
        *reinterpret_cast<u32x4*>(res + row * K + (int64_t)v * 8) = o;
      }
    }
  }
  ss = wsum(ss);
  const float r = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, (float)K) + eps));
  u32x4 yv[NI];
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int v = it * kWave + lane;
    if (v < nvec) {
      const u32x4 wv = ldg128(w + (int64_t)v * 8);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = to_float<T>(from_float<T>(h[it][2 * i] * r)) * elt<T>(wv, 2 * i);
        const float b = to_float<T>(from_float<T>(h[it][2 * i + 1] * r)) * elt<T>(wv, 2 * i + 1);
        yv[it][i] = pack2<T>(a, b);
      }
      if constexpr (kY) *reinterpret_cast<u32x4*>(y + row * K + (int64_t)v * 8) = yv[it];
    }
  }
  if constexpr (kQ) quant_store<T, NI>(yv, nvec, lane, 1e-8f, xq + row * K, a_scales + row);
}

template <typename T, bool kY, bool kQ, int NI>
__global__ __launch_bounds__(256) void silu_mul_vec_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ y,
                                                           int8_t* __restrict__ xq, float* __restrict__ a_scales,
                                                           int64_t M, int I) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRows + (threadIdx.x >> 6);
  if (row >= M) return;
  const int nvec = I >> 3;
  const uint16_t* g = gu + row * 2 * I;
  const uint16_t* u = g + I;
  u32x4 yv[NI];
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int v = it * kWave + lane;
    if (v < nvec) {
      const u32x4 gv = ldg128_stream(g + (int64_t)v * 8);
      const u32x4 uv = ldg128_stream(u + (int64_t)v * 8);
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float a = elt<T>(gv, i);
        o[i] = silu_f(a) * elt<T>(uv, i);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) yv[it][i] = pack2<T>(o[2 * i], o[2 * i + 1]);
      if constexpr (kY) *reinterpret_cast<u32x4*>(y + row * I + (int64_t)v * 8) = yv[it];
    }
  }
  if constexpr (kQ) quant_store<T, NI>(yv, nvec, lane, 1e-8f, xq + row * I, a_scales + row);
}

// ---------------------------------------------------------------- scalar paths
// Any K, any alignment. Every pass recomputes h from x (+ residual) and each
// lane revisits only its own elements, so the residual is overwritten in the
// last pass; passes after the first hit L2.
template <typename T>
__device__ __forceinline__ float rms_y(const uint16_t* xr, const uint16_t* rr, const uint16_t* w, int k, float r,
                                       float* h_out) {
  float h = to_float<T>(xr[k]);
  if (rr) h += to_float<T>(rr[k]);
  *h_out = h;
  return to_float<T>(from_float<T>(to_float<T>(from_float<T>(h * r)) * to_float<T>(w[k])));
}

template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_scalar_kernel(const uint16_t* __restrict__ x, uint16_t* res,
                                                             const uint16_t* __restrict__ w, float eps, uint16_t* y,
                                                             int8_t* __restrict__ xq, float* __restrict__ a_scales,
                                                             int64_t M, int K) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRows + (threadIdx.x >> 6);
  if (row >= M) return;
  const uint16_t* xr = x + row * K;
  uint16_t* rr = res ? res + row * K : nullptr;
  float ss = 0.0f;
  for (int k = lane; k < K; k += kWave) {
    float t = to_float<T>(xr[k]);
    if (rr) t += to_float<T>(rr[k]);
    ss += t * t;
  }
  ss = wsum(ss);
  const float r = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, (float)K) + eps));
  float amax = 0.0f;
  for (int k = lane; k < K; k += kWave) {
    float h;
    const float v = rms_y<T>(xr, rr, w, k, r, &h);
    if (y) y[row * K + k] = from_float<T>(v);
    amax = fmaxf(amax, fabsf(v));
    if (rr && !xq) rr[k] = from_float<T>(h);
  }
  if (!xq) return;
  amax = wmax(amax);
  const float s = fmaxf(__fdiv_rn(amax, 127.0f), 1e-8f);
  if (lane == 0) a_scales[row] = s;
  const float rs = __fdiv_rn(1.0f, s);
  for (int k = lane; k < K; k += kWave) {
    float h;
    xq[row * K + k] = qcode(rms_y<T>(xr, rr, w, k, r, &h), s, rs);
    if (rr) rr[k] = from_float<T>(h);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void silu_mul_scalar_kernel(const uint16_t* __restrict__ gu, uint16_t* y,
                                                              int8_t* __restrict__ xq, float* __restrict__ a_scales,
                                                              int64_t M, int I) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRows + (threadIdx.x >> 6);
  if (row >= M) return;
  const uint16_t* g = gu + row * 2 * I;
  auto val = [&](int k) {
    const float a = to_float<T>(g[k]);
    return to_float<T>(from_float<T>(silu_f(a) * to_float<T>(g[I + k])));
  };
  float amax = 0.0f;
  for (int k = lane; k < I; k += kWave) {
    const float v = val(k);
    if (y) y[row * I + k] = from_float<T>(v);
    amax = fmaxf(amax, fabsf(v));
  }
  if (!xq) return;
  amax = wmax(amax);
  const float s = fmaxf(__fdiv_rn(amax, 127.0f), 1e-8f);
  if (lane == 0) a_scales[row] = s;
  const float rs = __fdiv_rn(1.0f, s);
  for (int k = lane; k < I; k += kWave) xq[row * I + k] = qcode(val(k), s, rs);
}

}  // namespace

bool producer_vec_ok(const void* a, const void* b, const void* c, const void* d, int64_t K) {
  auto al = [](const void* p, uintptr_t n) { return p == nullptr || ((uintptr_t)p % n) == 0; };
  return K % 8 == 0 && K <= kIters * kWave * 8 && al(a, 16) && al(b, 16) && al(c, 16) && al(d, 8);
}

template <typename T>
static hipError_t rms_t(const void* x, void* res, const void* w, float eps, void* y, int8_t* xq, float* as,
                        int64_t M, int64_t K, hipStream_t st) {
  const dim3 grid((unsigned)((M + kRows - 1) / kRows)), block(256);
  auto X = static_cast<const uint16_t*>(x);
  auto R = static_cast<uint16_t*>(res);
  auto W = static_cast<const uint16_t*>(w);
  auto Y = static_cast<uint16_t*>(y);
  const int k = (int)K;
  if (!producer_vec_ok(x, res, y, xq, K)) {
    rmsnorm_scalar_kernel<T><<<grid, block, 0, st>>>(X, R, W, eps, Y, xq, as, M, k);
    return hipGetLastError();
  }
  const bool hy = y != nullptr, hq = xq != nullptr;
  // row held in registers: NI iterations of 512 elements, sized to K
  auto go = [&](auto ni) {
    constexpr int NI = decltype(ni)::value;
#define TVQ_RMS(RES, YY, QQ) \
  rmsnorm_vec_kernel<T, RES, YY, QQ, NI><<<grid, block, 0, st>>>(X, R, W, eps, Y, xq, as, M, k)
    if (res) {
      if (hy && hq) TVQ_RMS(true, true, true);
      else if (hy) TVQ_RMS(true, true, false);
      else TVQ_RMS(true, false, true);
    } else {
      if (hy && hq) TVQ_RMS(false, true, true);
      else if (hy) TVQ_RMS(false, true, false);
      else TVQ_RMS(false, false, true);
    }
#undef TVQ_RMS
  };
  if (K <= 1024) go(std::integral_constant<int, 2>{});
  else if (K <= 2048) go(std::integral_constant<int, 4>{});
  else go(std::integral_constant<int, kIters>{});
  return hipGetLastError();
}

hipError_t launch_rmsnorm(const void* x, void* residual, const void* weight, float eps, void* y, int8_t* xq,
                          float* a_scales, bool bf16, int64_t M, int64_t K, hipStream_t stream) {
  return bf16 ? rms_t<BF16>(x, residual, weight, eps, y, xq, a_scales, M, K, stream)
              : rms_t<F16>(x, residual, weight, eps, y, xq, a_scales, M, K, stream);
}

template <typename T>
static hipError_t silu_t(const void* gu, void* y, int8_t* xq, float* as, int64_t M, int64_t I, hipStream_t st) {
  const dim3 grid((unsigned)((M + kRows - 1) / kRows)), block(256);
  auto G = static_cast<const uint16_t*>(gu);
  auto Y = static_cast<uint16_t*>(y);
  const int i = (int)I;
  if (!producer_vec_ok(gu, y, nullptr, xq, I) || ((uintptr_t)(G + I) % 16) != 0) {
    silu_mul_scalar_kernel<T><<<grid, block, 0, st>>>(G, Y, xq, as, M, i);
    return hipGetLastError();
  }
  auto go = [&](auto ni) {
    constexpr int NI = decltype(ni)::value;
    if (y && xq) silu_mul_vec_kernel<T, true, true, NI><<<grid, block, 0, st>>>(G, Y, xq, as, M, i);
    else if (y) silu_mul_vec_kernel<T, true, false, NI><<<grid, block, 0, st>>>(G, Y, xq, as, M, i);
    else silu_mul_vec_kernel<T, false, true, NI><<<grid, block, 0, st>>>(G, Y, xq, as, M, i);
  };
  if (I <= 1024) go(std::integral_constant<int, 2>{});
  else if (I <= 2048) go(std::integral_constant<int, 4>{});
  else if (I <= 3072) go(std::integral_constant<int, 6>{});
  else go(std::integral_constant<int, kIters>{});
  return hipGetLastError();
}

hipError_t launch_silu_mul(const void* gate_up, void* y, int8_t* xq, float* a_scales, bool bf16, int64_t M,
                           int64_t I, hipStream_t stream) {
  return bf16 ? silu_t<BF16>(gate_up, y, xq, a_scales, M, I, stream)
              : silu_t<F16>(gate_up, y, xq, a_scales, M, I, stream);
}

}  // namespace tvq
