// Decode attention over the engine's per-sequence KV cache (gfx950).
//
// Replaces the decode branch of the reference's Attention.forward
// (nanovllm/layers/attention.py:59-88): store_kvcache of the new token's
// key/value followed by flash_attn_with_kvcache(q, k_cache, v_cache,
// cache_seqlens, causal=True) for one query token per sequence.
//
// Cache layout: k_cache / v_cache [slots, kv_heads, max_len, D] (D = 128),
// one slot per running sequence. For sequence b (slot slots[b], length
// lens[b] including the new token) the kernel
//   1. writes k_new[b], v_new[b] to position lens[b]-1 of its slot, and
//   2. computes, for every query head h of kv head g = h / (Hq/Hkv),
//        o[b,h] = softmax(scale * q[b,h] . K[0:len]) V[0:len]
//      in fp32 (online softmax), the new token's K/V taken from k_new/v_new.
// Sequence lengths and slots are read from device memory, so one launch
// serves any mix of lengths and is safe to capture in a HIP graph.
//
// Work split: one 256-thread workgroup per (sequence, kv head). Each wave
// splits into 4 groups of 16 lanes; a group handles one position per step
// (lane li holds dims 8*li .. 8*li+7, so a 256-byte K or V row is one
// coalesced 16-byte load per lane) with its own online-softmax state for the
// G query heads that share the kv head. The 16 groups of the workgroup walk
// positions with stride 16; their states are merged through LDS at the end.
// HBM traffic is the algorithmic minimum: each K/V row of the sequence is
// read once (2 * len * D * 2 bytes per kv head).
#include "tvq_common.h"
#include "tvq_internal.h"

namespace tvq {
namespace {

constexpr int kD = 128;
constexpr int kGroups = 16;  // 16-lane groups per workgroup

template <typename T>
__device__ __forceinline__ void unpack8(const u32x4& v, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = to_float<T>((uint16_t)(v[i] & 0xffffu));
    f[2 * i + 1] = to_float<T>((uint16_t)(v[i] >> 16));
  }
}

template <typename T, int G>
__global__ __launch_bounds__(256) void decode_attn_kernel(const uint16_t* __restrict__ q, int64_t q_stride,
                                                          const uint16_t* __restrict__ k_new, int64_t k_stride,
                                                          const uint16_t* __restrict__ v_new, int64_t v_stride,
                                                          uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
                                                          const int32_t* __restrict__ slots,
                                                          const int32_t* __restrict__ lens, int Hkv, int max_len,
                                                          int num_slots, float scale, uint16_t* __restrict__ out) {
  const int b = blockIdx.x;
  const int g = blockIdx.y;
  const int tid = threadIdx.x;
  const int grp = tid >> 4;  // 0..15
  const int li = tid & 15;
  const int len = lens[b];
  const int64_t slot = slots[b];
  if (len < 1 || len > max_len || slot < 0 || slot >= num_slots) {
    // Invalid metadata: touch no cache memory, emit zeros (uniform per workgroup).
    for (int e = tid; e < G * kD; e += 256) out[((int64_t)b * Hkv * G + g * G) * kD + e] = 0;
    return;
  }
  const int64_t head_off = (slot * Hkv + g) * (int64_t)max_len * kD;
  const uint16_t* kc = k_cache + head_off;
  const uint16_t* vc = v_cache + head_off;
  const uint16_t* kn = k_new + (int64_t)b * k_stride + g * kD;
  const uint16_t* vn = v_new + (int64_t)b * v_stride + g * kD;

  // 1. append the new token to the cache (never read back by this launch)
  if (tid < 16) {
    *reinterpret_cast<u32x4*>(k_cache + head_off + (int64_t)(len - 1) * kD + 8 * tid) =
        *reinterpret_cast<const u32x4*>(kn + 8 * tid);
  } else if (tid < 32) {
    *reinterpret_cast<u32x4*>(v_cache + head_off + (int64_t)(len - 1) * kD + 8 * (tid - 16)) =
        *reinterpret_cast<const u32x4*>(vn + 8 * (tid - 16));
  }

  // 2. per-group online softmax over positions grp, grp+16, ...
  float qf[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float t[8];
    unpack8<T>(*reinterpret_cast<const u32x4*>(q + (int64_t)b * q_stride + (g * G + h) * kD + 8 * li), t);
#pragma unroll
    for (int i = 0; i < 8; ++i) qf[h][i] = t[i] * scale;
  }
  float m[G], l[G], o[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[h][i] = 0.0f;
  }

  const int steps = (len + kGroups - 1) / kGroups;
  for (int st = 0; st < steps; ++st) {
    const int p = st * kGroups + grp;
    const bool valid = p < len;
    const bool last = p == len - 1;
    const int pc = valid ? p : 0;
    const uint16_t* kp = last ? kn : kc + (int64_t)pc * kD;
    const uint16_t* vp = last ? vn : vc + (int64_t)pc * kD;
    float kf[8], vf[8];
    unpack8<T>(*reinterpret_cast<const u32x4*>(kp + 8 * li), kf);
    unpack8<T>(*reinterpret_cast<const u32x4*>(vp + 8 * li), vf);
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) s = fmaf(qf[h][i], kf[i], s);
      // reduce over the 16 lanes of the group
      s += __shfl_xor(s, 8, 16);
      s += __shfl_xor(s, 4, 16);
      s += __shfl_xor(s, 2, 16);
      s += __shfl_xor(s, 1, 16);
      if (valid) {
        const float mn = fmaxf(m[h], s);
        const float corr = expf(m[h] - mn);  // 0 on the first valid position (m = -inf)
        const float e = expf(s - mn);
        l[h] = l[h] * corr + e;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[h][i] = fmaf(o[h][i], corr, e * vf[i]);
        m[h] = mn;
      }
    }
  }

  // 3. merge the 16 group states: LDS [group][head] of (m, l, o[128])
  __shared__ float sm[kGroups][G][2];
  __shared__ float so[kGroups][G][kD];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    if (li == 0) {
      sm[grp][h][0] = m[h];
      sm[grp][h][1] = l[h];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) so[grp][h][8 * li + i] = o[h][i];
  }
  __syncthreads();
  for (int e = tid; e < G * kD; e += 256) {
    const int h = e / kD;
    const int d = e % kD;
    float M = -INFINITY;
#pragma unroll
    for (int x = 0; x < kGroups; ++x) M = fmaxf(M, sm[x][h][0]);
    float L = 0.0f, acc = 0.0f;
#pragma unroll
    for (int x = 0; x < kGroups; ++x) {
      const float w = sm[x][h][1] > 0.0f ? expf(sm[x][h][0] - M) : 0.0f;
      L = fmaf(sm[x][h][1], w, L);
      acc = fmaf(so[x][h][d], w, acc);
    }
    out[((int64_t)b * Hkv * G + g * G + h) * kD + d] = from_float<T>(acc / L);
  }
}

template <typename T>
hipError_t launch_t(const void* q, int64_t qs, const void* kn, int64_t ks, const void* vn, int64_t vs, void* kc,
                    void* vc, const int32_t* slots, const int32_t* lens, int B, int Hq, int Hkv, int max_len,
                    int num_slots, float scale, void* out, hipStream_t st) {
  const dim3 grid((unsigned)B, (unsigned)Hkv), block(256);
  auto Q = static_cast<const uint16_t*>(q);
  auto KN = static_cast<const uint16_t*>(kn);
  auto VN = static_cast<const uint16_t*>(vn);
  auto KC = static_cast<uint16_t*>(kc);
  auto VC = static_cast<uint16_t*>(vc);
  auto O = static_cast<uint16_t*>(out);
  switch (Hq / Hkv) {
    case 1: decode_attn_kernel<T, 1><<<grid, block, 0, st>>>(Q, qs, KN, ks, VN, vs, KC, VC, slots, lens, Hkv, max_len, num_slots, scale, O); break;
    case 2: decode_attn_kernel<T, 2><<<grid, block, 0, st>>>(Q, qs, KN, ks, VN, vs, KC, VC, slots, lens, Hkv, max_len, num_slots, scale, O); break;
    case 4: decode_attn_kernel<T, 4><<<grid, block, 0, st>>>(Q, qs, KN, ks, VN, vs, KC, VC, slots, lens, Hkv, max_len, num_slots, scale, O); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_decode_attention(const void* q, int64_t q_stride, const void* k_new, int64_t k_stride,
                                   const void* v_new, int64_t v_stride, void* k_cache, void* v_cache,
                                   const int32_t* slots, const int32_t* lens, int B, int Hq, int Hkv, int max_len,
                                   int num_slots, float scale, void* out, bool bf16, hipStream_t stream) {
  return bf16 ? launch_t<BF16>(q, q_stride, k_new, k_stride, v_new, v_stride, k_cache, v_cache, slots, lens, B, Hq,
                               Hkv, max_len, num_slots, scale, out, stream)
              : launch_t<F16>(q, q_stride, k_new, k_stride, v_new, v_stride, k_cache, v_cache, slots, lens, B, Hq, Hkv,
                              max_len, num_slots, scale, out, stream);
}

}  // namespace tvq
