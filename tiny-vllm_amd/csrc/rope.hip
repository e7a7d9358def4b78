// Per-head q/k RMSNorm + rotary embedding, fused (gfx950).
//
// Replaces, for the attention input of one layer, the reference's
//   q = q_norm(q); k = k_norm(k)            (RMSNorm.rms_forward over head_dim,
//                                            nanovllm/layers/layernorm.py:16-26)
//   q, k = rotary_emb(positions, q, k)      (apply_rotary_emb, rotate-half,
//                                            nanovllm/layers/rotary_embedding.py:6-14)
// which is ~15 torch launches (casts, pow/mean/rsqrt, chunk/cat, mul/add)
// with fp32 temporaries, by one launch that reads q and k once from the packed
// qkv projection output and writes them once.
//
// Eight lanes per (token, head), head_dim D = 128: lane j of the group
// holds x[8j..8j+7] and x[64+8j..64+8j+7], exactly the pairs the rotate-half
// rotation mixes, so the rotation is lane-local, every access is 16 bytes
// per lane (32 for the fp32 cos/sin rows) and the RMS statistic is an
// 8-lane reduction. Eight heads per wave.
// Rounding follows the reference step by step:
//   n  = round(x * rsqrt(mean(x^2) + eps))     (fp32, IEEE sqrt and divide)
//   n  = round(n * w)                           (bf16 x bf16 -> one rounding)
//   y1 = round(n1 * cos - n2 * sin),  y2 = round(n2 * cos + n1 * sin)   (fp32)
// With no norm weights (models with q/k bias instead of q/k norm) only the
// rotation is applied.
//
// Optionally (prefill) the kernel also stores each token's rotated key and its
// value into the per-sequence KV cache [slots, Hkv, max_len, D] at (the
// token's slot, its position), replacing the reference's store_kvcache
// (attention.py:10-40) for the prompt tokens; v heads are then extra work
// items that only copy.
#include "tvq_common.h"
#include "tvq_internal.h"

namespace tvq {
namespace {

constexpr int kD = 128;
constexpr int kGroup = 8;                   // lanes per head
constexpr int kItemsPerBlock = 256 / kGroup;

__device__ __forceinline__ float group_sum(float v) {
  for (int off = kGroup / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, kGroup);
  return v;
}

// Eight 16-bit values <-> floats.
template <typename T>
__device__ __forceinline__ void unpack8(u32x4 w, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = to_float<T>((uint16_t)w[i]);
    f[2 * i + 1] = to_float<T>((uint16_t)(w[i] >> 16));
  }
}
template <typename T>
__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
  u32x4 w;
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = (uint32_t)from_float<T>(f[2 * i]) | ((uint32_t)from_float<T>(f[2 * i + 1]) << 16);
  return w;
}

template <typename T, bool kNorm>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(const uint16_t* __restrict__ qkv, int64_t row_stride,
                                                           const int64_t* __restrict__ positions,
                                                           const float* __restrict__ cos_t,
                                                           const float* __restrict__ sin_t,
                                                           const uint16_t* __restrict__ qw,
                                                           const uint16_t* __restrict__ kw, float eps, int T_, int Hq,
                                                           int Hkv, int max_pos, uint16_t* __restrict__ q_out,
                                                           uint16_t* __restrict__ k_out, uint16_t* __restrict__ k_cache,
                                                           uint16_t* __restrict__ v_cache,
                                                           const int64_t* __restrict__ slots, int num_slots,
                                                           int max_len) {
  const int j = threadIdx.x & (kGroup - 1);
  const int64_t item = (int64_t)blockIdx.x * kItemsPerBlock + (threadIdx.x / kGroup);
  const bool store = k_cache != nullptr;
  const int heads = Hq + Hkv + (store ? Hkv : 0);
  if (item >= (int64_t)T_ * heads) return;  // whole 8-lane groups leave together
  const int64_t t = item / heads;
  const int h = (int)(item % heads);
  const bool is_q = h < Hq;
  const uint16_t* src = qkv + t * row_stride + (int64_t)h * kD;
  // cache destination of this token (only for the k and v heads of a store)
  uint16_t* cache_row = nullptr;
  if (store && !is_q) {
    const int64_t slot = slots[t];
    const int64_t pos = positions[t];
    const int kvh = h < Hq + Hkv ? h - Hq : h - Hq - Hkv;
    if (slot >= 0 && slot < num_slots && pos >= 0 && pos < max_len)
      cache_row = (h < Hq + Hkv ? k_cache : v_cache) + ((slot * Hkv + kvh) * (int64_t)max_len + pos) * kD;
  }
  // read once: non-temporal
  const u32x4 lo = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + 8 * j));
  const u32x4 hi = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + 64 + 8 * j));
  if (h >= Hq + Hkv) {  // value head: copy to the cache only
    if (cache_row) {
      *reinterpret_cast<u32x4*>(cache_row + 8 * j) = lo;
      *reinterpret_cast<u32x4*>(cache_row + 64 + 8 * j) = hi;
    }
    return;
  }
  float x1[8], x2[8];
  unpack8<T>(lo, x1);
  unpack8<T>(hi, x2);
  if constexpr (kNorm) {
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += x1[e] * x1[e] + x2[e] * x2[e];
    ss = group_sum(ss);
    const float r = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, (float)kD) + eps));
    const uint16_t* w = is_q ? qw : kw;
    float w1[8], w2[8];
    unpack8<T>(*reinterpret_cast<const u32x4*>(w + 8 * j), w1);
    unpack8<T>(*reinterpret_cast<const u32x4*>(w + 64 + 8 * j), w2);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x1[e] = to_float<T>(from_float<T>(to_float<T>(from_float<T>(x1[e] * r)) * w1[e]));
      x2[e] = to_float<T>(from_float<T>(to_float<T>(from_float<T>(x2[e] * r)) * w2[e]));
    }
  }
  int64_t p = positions[t];
  p = p < 0 ? 0 : (p >= max_pos ? max_pos - 1 : p);
  const f32x4 c0 = *reinterpret_cast<const f32x4*>(cos_t + p * (kD / 2) + 8 * j);
  const f32x4 c1 = *reinterpret_cast<const f32x4*>(cos_t + p * (kD / 2) + 8 * j + 4);
  const f32x4 s0 = *reinterpret_cast<const f32x4*>(sin_t + p * (kD / 2) + 8 * j);
  const f32x4 s1 = *reinterpret_cast<const f32x4*>(sin_t + p * (kD / 2) + 8 * j + 4);
  float y1[8], y2[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float c = e < 4 ? c0[e] : c1[e - 4];
    const float sn = e < 4 ? s0[e] : s1[e - 4];
    y1[e] = x1[e] * c - x2[e] * sn;
    y2[e] = x2[e] * c + x1[e] * sn;
  }
  uint16_t* dst = is_q ? q_out + (t * Hq + h) * kD : k_out + (t * Hkv + (h - Hq)) * kD;
  const u32x4 o1 = pack8<T>(y1), o2 = pack8<T>(y2);
  *reinterpret_cast<u32x4*>(dst + 8 * j) = o1;
  *reinterpret_cast<u32x4*>(dst + 64 + 8 * j) = o2;
  if (cache_row) {
    *reinterpret_cast<u32x4*>(cache_row + 8 * j) = o1;
    *reinterpret_cast<u32x4*>(cache_row + 64 + 8 * j) = o2;
  }
}

}  // namespace

hipError_t launch_qk_norm_rope(const void* qkv, int64_t row_stride, const int64_t* positions, const float* cos_t,
                               const float* sin_t, const void* q_weight, const void* k_weight, float eps, int64_t T_,
                               int Hq, int Hkv, int max_pos, void* q_out, void* k_out, void* k_cache, void* v_cache,
                               const int64_t* slots, int num_slots, int max_len, bool bf16, hipStream_t stream) {
  const int64_t items = T_ * (Hq + Hkv + (k_cache ? Hkv : 0));
  const dim3 grid((unsigned)((items + kItemsPerBlock - 1) / kItemsPerBlock)), block(256);
  auto X = static_cast<const uint16_t*>(qkv);
  auto QW = static_cast<const uint16_t*>(q_weight);
  auto KW = static_cast<const uint16_t*>(k_weight);
  auto QO = static_cast<uint16_t*>(q_out);
  auto KO = static_cast<uint16_t*>(k_out);
  auto KC = static_cast<uint16_t*>(k_cache);
  auto VC = static_cast<uint16_t*>(v_cache);
  const bool norm = q_weight != nullptr;
#define TVQ_ROPE(TT, NN)                                                                                       \
  qk_norm_rope_kernel<TT, NN><<<grid, block, 0, stream>>>(X, row_stride, positions, cos_t, sin_t, QW, KW, eps, \
                                                          (int)T_, Hq, Hkv, max_pos, QO, KO, KC, VC, slots, num_slots, \
                                                          max_len)
  if (bf16) {
    if (norm) TVQ_ROPE(BF16, true); else TVQ_ROPE(BF16, false);
  } else {
    if (norm) TVQ_ROPE(F16, true); else TVQ_ROPE(F16, false);
  }
#undef TVQ_ROPE
  return hipGetLastError();
}

}  // namespace tvq
