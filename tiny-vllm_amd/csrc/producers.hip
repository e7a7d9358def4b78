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
// A row is owned by TPR threads of a 256-thread workgroup (like act-quant):
// one wave (4 rows per workgroup) when there are enough rows to fill the
// GPU, two or four waves for decode-size M, whose row sums and maxima are then
// combined through LDS. Rows of up to 8 x TPR x 8 elements stay in registers,
// so HBM traffic is the algorithmic minimum: read x (+ residual, + w from L2), write residual
// and y (2 B/elem) and/or the codes (1 B/elem) + 4 B per row. Longer rows or
// K % 8 != 0 or unaligned pointers take a scalar path that re-reads the row
// (from L2).
#include <type_traits>

#include "tvq_common.h"
#include "tvq_internal.h"

namespace tvq {
namespace {

constexpr int kRows = 4;   // scalar path: one wave per row
constexpr int kBlock = 256;
constexpr int kIters = 8;  // at most 8 x TPR lanes x 8 elements per row in registers

__device__ __forceinline__ float wsum(float v) {
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}
__device__ __forceinline__ float wmax(float v) {
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Sum / maximum over the TPR threads of a row. With TPR > 64 the row's
// waves meet in LDS (`lds` holds one slot per wave of the block; each call
// site passes its own array), so every thread of the block must call it.
template <int TPR, bool kMax>
__device__ __forceinline__ float row_reduce(float v, float* lds) {
  v = kMax ? wmax(v) : wsum(v);
  if constexpr (TPR > kWave) {
    if ((threadIdx.x & (kWave - 1)) == 0) lds[threadIdx.x / kWave] = v;
    __syncthreads();
    const int w0 = (threadIdx.x / TPR) * (TPR / kWave);
    v = lds[w0];
#pragma unroll
    for (int i = 1; i < TPR / kWave; ++i) v = kMax ? fmaxf(v, lds[w0 + i]) : v + lds[w0 + i];
  }
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
template <typename T, int TPR, int NI>
__device__ __forceinline__ void quant_store(const u32x4 (&y)[NI], int nvec, int t, bool live, float eps, int8_t* qr,
                                            float* srow, float* lds) {
  float amax = 0.0f;
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    if (it * TPR + t < nvec) {
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(elt<T>(y[it], i)));
    }
  }
  amax = row_reduce<TPR, true>(amax, lds);
  if (!live) return;
  const float s = fmaxf(__fdiv_rn(amax, 127.0f), eps);
  if (t == 0) *srow = s;
  const float rs = __fdiv_rn(1.0f, s);
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int v = it * TPR + t;
    if (v < nvec) *reinterpret_cast<u32x2*>(qr + (int64_t)v * 8) = quant_codes8<T>(y[it], s, rs);
  }
}

template <int TPR>
struct RowLane {
  int t;
  int64_t row;
  bool live;
  __device__ RowLane(int64_t M)
      : t((int)(threadIdx.x % TPR)), row((int64_t)blockIdx.x * (kBlock / TPR) + threadIdx.x / TPR), live(row < M) {}
};

template <typename T, bool kRes, bool kY, bool kQ, int TPR, int NI>
__global__ __launch_bounds__(kBlock) void rmsnorm_vec_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ res,
                                                             const uint16_t* __restrict__ w, float eps,
                                                             uint16_t* __restrict__ y, int8_t* __restrict__ xq,
                                                             float* __restrict__ a_scales, int64_t M, int K) {
  const RowLane<TPR> rl(M);
  if (TPR == kWave && !rl.live) return;  // one wave per row: no barriers
  __shared__ float lds_ss[kBlock / kWave], lds_max[kBlock / kWave];
  const int t = rl.t;
  const int64_t row = rl.live ? rl.row : 0;
  const int nvec = rl.live ? (K >> 3) : 0;
  const uint16_t* xr = x + row * K;
  float h[NI][8];
  float ss = 0.0f;
  // every load of the row is issued before the first use (clamped index, no
  // branch around the loads), so they are all in flight together
  const int vmax = nvec > 0 ? nvec - 1 : 0;
  // The norm weights are loaded with them: issued after the row reduction,
  // they added an L2 round trip to every row.
  // The residual is rewritten in place by the lane that owns each vector, so
  // a lane never loads a vector of res it does not own: rows past M (the
  // tail of the last workgroup) load nothing, and the clamped loads past the
  // row's end read x instead (their values are never used).
  u32x4 xin[NI] = {}, rin[NI] = {}, win[NI] = {};
  if (rl.live) {
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const int v = min(it * TPR + t, vmax);
      xin[it] = ldg128_stream(xr + (int64_t)v * 8);
      if constexpr (kRes) rin[it] = ldg128_stream((it * TPR + t < nvec ? res + row * K : xr) + (int64_t)v * 8);
      win[it] = ldg128(w + (int64_t)v * 8);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the first use
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int v = it * TPR + t;
    if (v < nvec) {
      const u32x4 xv = xin[it];
      u32x4 rv = {0, 0, 0, 0};
      if constexpr (kRes) rv = rin[it];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float tt = elt<T>(xv, i);
        if constexpr (kRes) tt += elt<T>(rv, i);
        h[it][i] = tt;
        ss += tt * tt;
      }
      if constexpr (kRes) {
        u32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = pack2<T>(h[it][2 * i], h[it][2 * i + 1]);
        *reinterpret_cast<u32x4*>(res + row * K + (int64_t)v * 8) = o;
      }
    }
  }
  ss = row_reduce<TPR, false>(ss, lds_ss);
  const float r = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, (float)K) + eps));
  u32x4 yv[NI];
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int v = it * TPR + t;
    if (v < nvec) {
      const u32x4 wv = win[it];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = to_float<T>(from_float<T>(h[it][2 * i] * r)) * elt<T>(wv, 2 * i);
        const float b = to_float<T>(from_float<T>(h[it][2 * i + 1] * r)) * elt<T>(wv, 2 * i + 1);
        yv[it][i] = pack2<T>(a, b);
      }
      if constexpr (kY) *reinterpret_cast<u32x4*>(y + row * K + (int64_t)v * 8) = yv[it];
    }
  }
  if constexpr (kQ) quant_store<T, TPR, NI>(yv, nvec, t, rl.live, 1e-8f, xq + row * K, a_scales + row, lds_max);
}

template <typename T, bool kY, bool kQ, int TPR, int NI>
__global__ __launch_bounds__(kBlock) void silu_mul_vec_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ y,
                                                              int8_t* __restrict__ xq, float* __restrict__ a_scales,
                                                              int64_t M, int I) {
  const RowLane<TPR> rl(M);
  if (TPR == kWave && !rl.live) return;  // one wave per row: no barriers
  __shared__ float lds_max[kBlock / kWave];
  const int t = rl.t;
  const int64_t row = rl.live ? rl.row : 0;
  const int nvec = rl.live ? (I >> 3) : 0;
  const uint16_t* g = gu + row * 2 * I;
  const uint16_t* u = g + I;
  u32x4 yv[NI], gin[NI], uin[NI];
  const int vmax = nvec > 0 ? nvec - 1 : 0;
#pragma unroll
  for (int it = 0; it < NI; ++it) {  // all loads in flight before the first use
    const int v = min(it * TPR + t, vmax);
    gin[it] = ldg128_stream(g + (int64_t)v * 8);
    uin[it] = ldg128_stream(u + (int64_t)v * 8);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the first use
  // Every lane computes (its loads were clamped into the row), then the
  // stores follow, guarded. Computing inside the guarded stores let the
  // compiler sink the last loads past the first stores.
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const u32x4 gv = gin[it];
    const u32x4 uv = uin[it];
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float a = elt<T>(gv, i);
      o[i] = silu_f(a) * elt<T>(uv, i);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) yv[it][i] = pack2<T>(o[2 * i], o[2 * i + 1]);
  }
  if constexpr (kY) {
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const int v = it * TPR + t;
      if (v < nvec) *reinterpret_cast<u32x4*>(y + row * I + (int64_t)v * 8) = yv[it];
    }
  }
  if constexpr (kQ) quant_store<T, TPR, NI>(yv, nvec, t, rl.live, 1e-8f, xq + row * I, a_scales + row, lds_max);
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

// Threads per row by M (as act-quant): one wave once M / 4 workgroups fill
// the GPU, up to four waves (one row per workgroup) for small M.
static int producer_tpr(int64_t M) { return M >= 1024 ? 64 : (M >= 512 ? 128 : 256); }

// Calls go(TPR, NI) with the register-cache depth sized to the row (8-element
// vectors per thread), for the TPR this M takes.
template <typename Go>
static void with_shape(int64_t M, int64_t K, Go&& go) {
  auto depth = [&](auto tpr) {
    constexpr int TPR = decltype(tpr)::value;
    const int64_t per = (K / 8 + TPR - 1) / TPR;
    if (per <= 2) go(tpr, std::integral_constant<int, 2>{});
    else if (per <= 4) go(tpr, std::integral_constant<int, 4>{});
    else if (per <= 6) go(tpr, std::integral_constant<int, 6>{});
    else go(tpr, std::integral_constant<int, kIters>{});
  };
  switch (producer_tpr(M)) {
    case 64: depth(std::integral_constant<int, 64>{}); break;
    case 128: depth(std::integral_constant<int, 128>{}); break;
    default: depth(std::integral_constant<int, 256>{}); break;
  }
}

static dim3 producer_grid(int64_t M) {
  const int64_t rows = kBlock / producer_tpr(M);
  return dim3((unsigned)((M + rows - 1) / rows));
}

template <typename T>
static hipError_t rms_t(const void* x, void* res, const void* w, float eps, void* y, int8_t* xq, float* as,
                        int64_t M, int64_t K, hipStream_t st) {
  auto X = static_cast<const uint16_t*>(x);
  auto R = static_cast<uint16_t*>(res);
  auto W = static_cast<const uint16_t*>(w);
  auto Y = static_cast<uint16_t*>(y);
  const int k = (int)K;
  if (!producer_vec_ok(x, res, y, xq, K)) {
    const dim3 grid((unsigned)((M + kRows - 1) / kRows));
    rmsnorm_scalar_kernel<T><<<grid, kBlock, 0, st>>>(X, R, W, eps, Y, xq, as, M, k);
    return hipGetLastError();
  }
  const bool hy = y != nullptr, hq = xq != nullptr;
  const dim3 grid = producer_grid(M);
  with_shape(M, K, [&](auto tpr, auto ni) {
    constexpr int TPR = decltype(tpr)::value, NI = decltype(ni)::value;
#define TVQ_RMS(RES, YY, QQ) \
  rmsnorm_vec_kernel<T, RES, YY, QQ, TPR, NI><<<grid, kBlock, 0, st>>>(X, R, W, eps, Y, xq, as, M, k)
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
  });
  return hipGetLastError();
}

hipError_t launch_rmsnorm(const void* x, void* residual, const void* weight, float eps, void* y, int8_t* xq,
                          float* a_scales, bool bf16, int64_t M, int64_t K, hipStream_t stream) {
  return bf16 ? rms_t<BF16>(x, residual, weight, eps, y, xq, a_scales, M, K, stream)
              : rms_t<F16>(x, residual, weight, eps, y, xq, a_scales, M, K, stream);
}

template <typename T>
static hipError_t silu_t(const void* gu, void* y, int8_t* xq, float* as, int64_t M, int64_t I, hipStream_t st) {
  auto G = static_cast<const uint16_t*>(gu);
  auto Y = static_cast<uint16_t*>(y);
  const int i = (int)I;
  if (!producer_vec_ok(gu, y, nullptr, xq, I) || ((uintptr_t)(G + I) % 16) != 0) {
    const dim3 grid((unsigned)((M + kRows - 1) / kRows));
    silu_mul_scalar_kernel<T><<<grid, kBlock, 0, st>>>(G, Y, xq, as, M, i);
    return hipGetLastError();
  }
  const dim3 grid = producer_grid(M);
  with_shape(M, I, [&](auto tpr, auto ni) {
    constexpr int TPR = decltype(tpr)::value, NI = decltype(ni)::value;
    if (y && xq) silu_mul_vec_kernel<T, true, true, TPR, NI><<<grid, kBlock, 0, st>>>(G, Y, xq, as, M, i);
    else if (y) silu_mul_vec_kernel<T, true, false, TPR, NI><<<grid, kBlock, 0, st>>>(G, Y, xq, as, M, i);
    else silu_mul_vec_kernel<T, false, true, TPR, NI><<<grid, kBlock, 0, st>>>(G, Y, xq, as, M, i);
  });
  return hipGetLastError();
}

hipError_t launch_silu_mul(const void* gate_up, void* y, int8_t* xq, float* a_scales, bool bf16, int64_t M,
                           int64_t I, hipStream_t stream) {
  return bf16 ? silu_t<BF16>(gate_up, y, xq, a_scales, M, I, stream)
              : silu_t<F16>(gate_up, y, xq, a_scales, M, I, stream);
}

}  // namespace tvq
