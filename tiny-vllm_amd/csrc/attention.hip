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
// positions with stride 16, four positions per step; their states are merged
// through LDS at the end.
// HBM traffic is the algorithmic minimum: each K/V row of the sequence is
// read once (2 * len * D * 2 bytes per kv head).
#include "tvq_common.h"
#include "tvq_internal.h"
#include "../../include/tvq.h"

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

// ---- o_proj's per-token quantization, fused (W8A8) ----------------------
// A token's attention output row [Hq * 128] is produced by several
// workgroups (one per kv head or head group). In the quantizing variants
// every workgroup stores its slice with agent-scope stores, which go through
// the XCD's L2 to the device-coherent level, waits for them, and counts
// itself in its row block's counter with an agent-scope atomic; the last of
// the block's workgroups reads the rows back with agent-scope loads (past
// any stale L2 line) and writes their int8 codes and scales exactly as
// tvq_act_quant does (s = max(RN(amax / 127), eps), the divide-free code),
// then zeroes the counter. No workgroup waits on another, and the codes are
// bit-identical to quantizing the stored output with tvq_act_quant.

// Agent-scope 8-byte store of four 16-bit outputs.
__device__ __forceinline__ void store8_agent(uint16_t* p, u32x2 v) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), __builtin_bit_cast(uint64_t, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T>
__device__ __forceinline__ float absmax4(uint64_t w) {
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) m = fmaxf(m, fabsf(to_float<T>((uint16_t)(w >> (16 * i)))));
  return m;
}

template <typename T>
__device__ __forceinline__ uint32_t codes4(uint64_t w, float s, float rs) {
  uint32_t c = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) c |= ((uint32_t)(int32_t)quant_code(to_float<T>((uint16_t)(w >> (16 * i))), s, rs) & 0xffu)
                                   << (8 * i);
  return c;
}

// The handoff and, in the last arriving workgroup, the quantization of rows
// [r0, r1) of the [*, W] output (W % 4 == 0). Called by every thread of the
// workgroup after its output stores.
template <typename T, int kThreads>
__device__ __forceinline__ void quantize_rows_last(const uint16_t* out, int64_t r0, int64_t r1, int W, int32_t* cnt, int arrivals,
                                   int8_t* xq, float* xs, float eps) {
  __shared__ int last;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's output stores have completed
  __syncthreads();
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == arrivals - 1;
  __syncthreads();
  if (!last) return;
  constexpr int kWaves = kThreads / 64;
  constexpr int kCache = 8;  // 8-byte vectors per lane kept in registers: rows up to 2048 wide are read once
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int nv = W / 4;
  for (int64_t row = r0 + wave; row < r1; row += kWaves) {
    const uint64_t* src = reinterpret_cast<const uint64_t*>(out + row * W);
    uint64_t c[kCache];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < kCache; ++i) {
      const int v = lane + 64 * i;
      c[i] = v < nv ? __hip_atomic_load(src + v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
      amax = fmaxf(amax, absmax4<T>(c[i]));
    }
    for (int v = lane + 64 * kCache; v < nv; v += 64)
      amax = fmaxf(amax, absmax4<T>(__hip_atomic_load(src + v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)));
    for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
    const float s = fmaxf(__fdiv_rn(amax, 127.0f), eps);
    const float rs = __fdiv_rn(1.0f, s);
    if (lane == 0) xs[row] = s;
    uint32_t* dst = reinterpret_cast<uint32_t*>(xq + row * W);
#pragma unroll
    for (int i = 0; i < kCache; ++i) {
      const int v = lane + 64 * i;
      if (v < nv) dst[v] = codes4<T>(c[i], s, rs);
    }
    for (int v = lane + 64 * kCache; v < nv; v += 64)
      dst[v] = codes4<T>(__hip_atomic_load(src + v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), s, rs);
  }
  if (threadIdx.x == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T, int G, bool kQ = false>
__global__ __launch_bounds__(256) void decode_attn_kernel(const uint16_t* __restrict__ q, int64_t q_stride,
                                                          const uint16_t* __restrict__ k_new, int64_t k_stride,
                                                          const uint16_t* __restrict__ v_new, int64_t v_stride,
                                                          uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
                                                          const int32_t* __restrict__ slots,
                                                          const int32_t* __restrict__ lens, int Hkv, int max_len,
                                                          int num_slots, float scale, uint16_t* __restrict__ out,
                                                          AttnQuant qo) {
  const int b = blockIdx.x;
  const int g = blockIdx.y;
  const int tid = threadIdx.x;
  const int grp = tid >> 4;  // 0..15
  const int li = tid & 15;
  const int len = lens[b];
  const int64_t slot = slots[b];
  if (len < 1 || len > max_len || slot < 0 || slot >= num_slots) {
    // Invalid metadata: touch no cache memory, emit zeros (uniform per workgroup).
    if constexpr (kQ) {
      for (int e = 4 * tid; e < G * kD; e += 4 * 256) store8_agent(out + ((int64_t)b * Hkv * G + g * G) * kD + e, u32x2{0, 0});
      quantize_rows_last<T, 256>(out, b, b + 1, Hkv * G * kD, qo.counters + b, Hkv, qo.xq, qo.a_scales, qo.eps);
    } else {
      for (int e = tid; e < G * kD; e += 256) out[((int64_t)b * Hkv * G + g * G) * kD + e] = 0;
    }
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

  // 2. per-group online softmax over positions grp, grp+16, ..., four per
  //    step (their K/V loads in flight together). Logits are kept in the
  //    log2 domain (scale * log2(e) folded into q) so each exponential is one
  //    v_exp_f32.
  constexpr float kLog2e = 1.4426950408889634f;
  float qf[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float t[8];
    unpack8<T>(*reinterpret_cast<const u32x4*>(q + (int64_t)b * q_stride + (g * G + h) * kD + 8 * li), t);
#pragma unroll
    for (int i = 0; i < 8; ++i) qf[h][i] = t[i] * (scale * kLog2e);
  }
  float m[G], l[G], o[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[h][i] = 0.0f;
  }

  constexpr int kPP = 4;  // positions per group per step
  const int steps = (len + kPP * kGroups - 1) / (kPP * kGroups);
  for (int st = 0; st < steps; ++st) {
    const int p0 = st * kPP * kGroups + grp;
    if (p0 >= len) continue;  // nothing valid this step (whole groups agree)
    float kf[kPP][8], vf[kPP][8];
    bool ok[kPP];
#pragma unroll
    for (int u = 0; u < kPP; ++u) {
      const int pu = p0 + u * kGroups;
      ok[u] = pu < len;
      const int pc = ok[u] ? pu : p0;
      const uint16_t* kp = pc == len - 1 ? kn : kc + (int64_t)pc * kD;
      const uint16_t* vp = pc == len - 1 ? vn : vc + (int64_t)pc * kD;
      // non-temporal: every cache line is read exactly once per step (was
      // 5.35 -> 6.0 TB/s at 256 sequences x 800 positions)
      unpack8<T>(__builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kp + 8 * li)), kf[u]);
      unpack8<T>(__builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vp + 8 * li)), vf[u]);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float sc[kPP];
#pragma unroll
      for (int u = 0; u < kPP; ++u) {
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) a = fmaf(qf[h][i], kf[u][i], a);
        sc[u] = a;
      }
      // reduce over the 16 lanes of the group
#pragma unroll
      for (int off = 8; off >= 1; off >>= 1)
#pragma unroll
        for (int u = 0; u < kPP; ++u) sc[u] += __shfl_xor(sc[u], off, 16);
      float mn = m[h];
#pragma unroll
      for (int u = 0; u < kPP; ++u) {
        if (!ok[u]) sc[u] = -INFINITY;
        mn = fmaxf(mn, sc[u]);
      }
      const float corr = __builtin_amdgcn_exp2f(m[h] - mn);  // 0 on the first step (m = -inf)
      float e[kPP], es = 0.0f;
#pragma unroll
      for (int u = 0; u < kPP; ++u) {
        e[u] = __builtin_amdgcn_exp2f(sc[u] - mn);          // 0 past the end
        es += e[u];
      }
      l[h] = fmaf(l[h], corr, es);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float acc = o[h][i] * corr;
#pragma unroll
        for (int u = 0; u < kPP; ++u) acc = fmaf(e[u], vf[u][i], acc);
        o[h][i] = acc;
      }
      m[h] = mn;
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
  if constexpr (kQ) {
    // four consecutive dims per thread, one agent-scope 8-byte store
    for (int e = 4 * tid; e < G * kD; e += 4 * 256) {
      const int h = e / kD;
      float M = -INFINITY;
#pragma unroll
      for (int x = 0; x < kGroups; ++x) M = fmaxf(M, sm[x][h][0]);
      float L = 0.0f, acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int x = 0; x < kGroups; ++x) {
        const float w = sm[x][h][1] > 0.0f ? __builtin_amdgcn_exp2f(sm[x][h][0] - M) : 0.0f;
        L = fmaf(sm[x][h][1], w, L);
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = fmaf(so[x][h][e % kD + t], w, acc[t]);
      }
      u32x2 pk;
      pk.x = (uint32_t)from_float<T>(acc[0] / L) | ((uint32_t)from_float<T>(acc[1] / L) << 16);
      pk.y = (uint32_t)from_float<T>(acc[2] / L) | ((uint32_t)from_float<T>(acc[3] / L) << 16);
      store8_agent(out + ((int64_t)b * Hkv * G + g * G) * kD + e, pk);
    }
    quantize_rows_last<T, 256>(out, b, b + 1, Hkv * G * kD, qo.counters + b, Hkv, qo.xq, qo.a_scales, qo.eps);
  } else {
    for (int e = tid; e < G * kD; e += 256) {
      const int h = e / kD;
      const int d = e % kD;
      float M = -INFINITY;
#pragma unroll
      for (int x = 0; x < kGroups; ++x) M = fmaxf(M, sm[x][h][0]);
      float L = 0.0f, acc = 0.0f;
#pragma unroll
      for (int x = 0; x < kGroups; ++x) {
        const float w = sm[x][h][1] > 0.0f ? __builtin_amdgcn_exp2f(sm[x][h][0] - M) : 0.0f;
        L = fmaf(sm[x][h][1], w, L);
        acc = fmaf(so[x][h][d], w, acc);
      }
      out[((int64_t)b * Hkv * G + g * G + h) * kD + d] = from_float<T>(acc / L);
    }
  }
}

template <typename T, bool kQ>
hipError_t launch_t(const void* q, int64_t qs, const void* kn, int64_t ks, const void* vn, int64_t vs, void* kc,
                    void* vc, const int32_t* slots, const int32_t* lens, int B, int Hq, int Hkv, int max_len,
                    int num_slots, float scale, void* out, AttnQuant qo, hipStream_t st) {
  const dim3 grid((unsigned)B, (unsigned)Hkv), block(256);
  auto Q = static_cast<const uint16_t*>(q);
  auto KN = static_cast<const uint16_t*>(kn);
  auto VN = static_cast<const uint16_t*>(vn);
  auto KC = static_cast<uint16_t*>(kc);
  auto VC = static_cast<uint16_t*>(vc);
  auto O = static_cast<uint16_t*>(out);
  switch (Hq / Hkv) {
    case 1: decode_attn_kernel<T, 1, kQ><<<grid, block, 0, st>>>(Q, qs, KN, ks, VN, vs, KC, VC, slots, lens, Hkv, max_len, num_slots, scale, O, qo); break;
    case 2: decode_attn_kernel<T, 2, kQ><<<grid, block, 0, st>>>(Q, qs, KN, ks, VN, vs, KC, VC, slots, lens, Hkv, max_len, num_slots, scale, O, qo); break;
    case 4: decode_attn_kernel<T, 4, kQ><<<grid, block, 0, st>>>(Q, qs, KN, ks, VN, vs, KC, VC, slots, lens, Hkv, max_len, num_slots, scale, O, qo); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_decode_attention(const void* q, int64_t q_stride, const void* k_new, int64_t k_stride,
                                   const void* v_new, int64_t v_stride, void* k_cache, void* v_cache,
                                   const int32_t* slots, const int32_t* lens, int B, int Hq, int Hkv, int max_len,
                                   int num_slots, float scale, void* out, bool bf16, hipStream_t stream,
                                   const AttnQuant* quant) {
  const AttnQuant qo = quant ? *quant : AttnQuant{nullptr, nullptr, nullptr, 0.0f};
#define TVQ_DEC(TT, QQ)                                                                                              \
  launch_t<TT, QQ>(q, q_stride, k_new, k_stride, v_new, v_stride, k_cache, v_cache, slots, lens, B, Hq, Hkv, max_len, \
                   num_slots, scale, out, qo, stream)
  if (quant) return bf16 ? TVQ_DEC(BF16, true) : TVQ_DEC(F16, true);
  return bf16 ? TVQ_DEC(BF16, false) : TVQ_DEC(F16, false);
#undef TVQ_DEC
}


// ---------------------------------------------------------------------------
// Prefill (varlen, causal) attention.
//
// Replaces the prefill branch of Attention.forward
// (nanovllm/layers/attention.py:75-84: flash_attn_varlen_func(q, k, v,
// cu_seqlens, causal=True)) for prompts without a cached prefix. q, k, v are
// the packed new tokens of all sequences; a host-built block table lists the
// 64-query blocks (token offset of the sequence, its length, first query of
// the block), longest work first.
//
// Two kernels share the block table: prefill_attn32_kernel (below) for even
// GQA ratios, and prefill_attn_kernel for odd ones (G = 1 query head per
// workgroup). prefill_attn_kernel: one workgroup per (query block, group of
// G query heads sharing a kv head), 4 waves per head, each wave owning 16
// queries of one head; 64-key blocks of K and V are staged once for all G
// heads in LDS, both row-major, the next block's loads in flight (registers)
// while the current one is multiplied. Both products run on
// v_mfma_f32_16x16x32_bf16 in transposed form so no data moves between them:
//   S^T[key][q] = K[key][:] . Q[q][:]          (A = K rows, B = Q rows)
//   O^T[d][q]  += V^T[d][keys] . P^T[keys][q]  (B = P^T straight from the
//                                               S^T accumulators)
// The MFMA k-dimension may be permuted as long as A and B agree, so lane
// group g feeds keys {4g..4g+3, 16+4g..16+4g+3} of each 32-key chunk: exactly
// the keys its S^T accumulators hold. Softmax statistics are per query = per
// lane column; the online rescale is lane-local. fp32 accumulation, exp2 with
// the scale folded into log2(e), P rounded to the input dtype for the second
// product (as flash attention does).
namespace {

typedef short v4i16 __attribute__((ext_vector_type(4)));
#define TVQ_LDS_V4I16(p) ((__attribute__((address_space(3))) v4i16*)(p))
#define TVQ_AGPTR(p) ((__attribute__((address_space(1))) void*)(p))
#define TVQ_ALPTR(p) ((__attribute__((address_space(3))) void*)(p))

constexpr int kBlkQ = TVQ_PREFILL_BLOCK_Q;  // queries per block (16 per wave, or 32 in the 32x32 kernel)
constexpr int kBlkK = 64;
constexpr int kKStride = kD + 8;      // K tile row stride (elements): 16-row fragment reads hit distinct banks
constexpr int kVStride = kD + 16;     // V tile row stride (elements): the 4 rows of a transposing read hit distinct banks

template <typename T, int G, bool kQ = false>
__global__ __launch_bounds__(256 * G) void prefill_attn_kernel(const uint16_t* __restrict__ q,
                                                               const uint16_t* __restrict__ k,
                                                               const uint16_t* __restrict__ v, int64_t v_stride,
                                                               const int32_t* __restrict__ blocks, int Hq, int Hkv,
                                                               float scale_log2, uint16_t* __restrict__ out,
                                                               AttnQuant qo) {
  constexpr int kThreads = 256 * G;
  constexpr int kVec = kBlkK * kD / 8;                 // 16-byte vectors per K (or V) tile
  constexpr int kPer = kVec / kThreads;                // per thread
  static_assert(kVec % kThreads == 0, "tile vectors split evenly");
  __shared__ __attribute__((aligned(16))) uint16_t ks[2][kBlkK * kKStride];
  __shared__ __attribute__((aligned(16))) uint16_t vs[2][kBlkK * kVStride];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int r = lane & 15;
  const int h = blockIdx.y * G + (wave >> 2);        // this wave's query head
  const int hk = h / (Hq / Hkv);                      // the G heads of the workgroup share this kv head
  const int64_t seq0 = blocks[3 * blockIdx.x];      // token offset of the sequence
  const int len = blocks[3 * blockIdx.x + 1];
  const int q0 = blocks[3 * blockIdx.x + 2];         // first query of the block (within the sequence)

  // this lane's query (B operand rows of S^T, C columns of both products)
  const int qi = q0 + (wave & 3) * 16 + r;
  const int qc = min(qi, len - 1);
  u32x4 qf[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    qf[c] = *reinterpret_cast<const u32x4*>(q + ((seq0 + qc) * Hq + h) * kD + 32 * c + 8 * g);

  f32x4 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.0f;

  // K/V tile vectors of one key block, held in registers one block ahead.
  // Vector i -> key i / 16, dims 8 * (i % 16) .. +8 (16 lanes read one
  // 256-byte row), for K and V alike; both tiles stay row-major in LDS.
  u32x4 kreg[kPer], vreg[kPer];
  auto load_tiles = [&](int kv0) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = tid + j * kThreads;
      const int key = min(kv0 + (i >> 4), len - 1);
      kreg[j] = *reinterpret_cast<const u32x4*>(k + ((seq0 + key) * Hkv + hk) * kD + 8 * (i & 15));
      vreg[j] = *reinterpret_cast<const u32x4*>(v + (seq0 + key) * v_stride + hk * kD + 8 * (i & 15));
    }
  };
  auto store_tiles = [&](int buf) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = tid + j * kThreads;
      *reinterpret_cast<u32x4*>(&ks[buf][(i >> 4) * kKStride + 8 * (i & 15)]) = kreg[j];
      *reinterpret_cast<u32x4*>(&vs[buf][(i >> 4) * kVStride + 8 * (i & 15)]) = vreg[j];
    }
  };

  // Pipeline: block b is multiplied from LDS buffer b % 2 while block b+1 is
  // stored into the other buffer (its global loads were issued one block
  // earlier) and block b+2 is loaded into registers; one barrier per block.
  const int kv_end = min(len, q0 + kBlkQ);           // causal: keys < last query of the block + 1
  load_tiles(0);
  store_tiles(0);
  if (kBlkK < kv_end) load_tiles(kBlkK);
  __syncthreads();
  for (int kv0 = 0, cur = 0; kv0 < kv_end; kv0 += kBlkK, cur ^= 1) {
    if (kv0 + kBlkK < kv_end) {
      store_tiles(cur ^ 1);                               // block + 1 (buffer last read two blocks ago)
      if (kv0 + 2 * kBlkK < kv_end) load_tiles(kv0 + 2 * kBlkK);
    }
    const uint16_t* ksb = ks[cur];
    const uint16_t* vsb = vs[cur];

    // S^T tiles: 4 x (16 keys x 16 queries), k = head dim in 4 chunks of 32
    f32x4 s[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(&ksb[(kt * 16 + r) * kKStride + 32 * c + 8 * g]);
        acc = mfma16x16x32<T>(a, qf[c], acc);
      }
      s[kt] = acc;
    }
    // scale, causal + length mask, block max per query (lane column r)
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int key = kv0 + kt * 16 + 4 * g + t;
        const float sv = (key <= qi && key < len) ? s[kt][t] * scale_log2 : -INFINITY;
        s[kt][t] = sv;
        mx = fmaxf(mx, sv);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float mn = fmaxf(m, mx);  // finite: key 0 is valid for every query
    const float corr = __builtin_amdgcn_exp2f(m - mn);
    float ps = 0.0f;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float p = __builtin_amdgcn_exp2f(s[kt][t] - mn);
        s[kt][t] = p;
        ps += p;
      }
    ps += __shfl_xor(ps, 16, kWave);
    ps += __shfl_xor(ps, 32, kWave);
    l = l * corr + ps;
    m = mn;
    // P^T as the B operand: chunk c holds keys {4g..4g+3} of tiles 2c and 2c+1
    u32x4 pb[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      pb[c][0] = (uint32_t)from_float<T>(s[2 * c][0]) | ((uint32_t)from_float<T>(s[2 * c][1]) << 16);
      pb[c][1] = (uint32_t)from_float<T>(s[2 * c][2]) | ((uint32_t)from_float<T>(s[2 * c][3]) << 16);
      pb[c][2] = (uint32_t)from_float<T>(s[2 * c + 1][0]) | ((uint32_t)from_float<T>(s[2 * c + 1][1]) << 16);
      pb[c][3] = (uint32_t)from_float<T>(s[2 * c + 1][2]) | ((uint32_t)from_float<T>(s[2 * c + 1][3]) << 16);
    }
    // O^T tiles: 8 x (16 dims x 16 queries), k = 64 keys in 2 chunks. The
    // A operand V^T[d][keys] comes from the row-major V tile through the
    // LDS transposing read (ds_read_b64_tr_b16): within each 16-lane group,
    // result element e of lane i is element i % 4 of the 4-element row
    // addressed by lane 4e + i / 4. Lane (g, r) therefore addresses key
    // 4g + r / 4 (+ 32c, + 16 for the high half), dims 16dt + 4(r % 4) .. +4,
    // and receives V[32c + 4g + e][16dt + r], e = 0..3: row d = 16dt + r of
    // V^T at the keys its P^T chunk holds.
    const uint16_t* vrow = vsb + (4 * g + (r >> 2)) * kVStride + 4 * (r & 3);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      f32x4 acc = o[dt] * corr;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const uint16_t* p0 = vrow + 32 * c * kVStride + 16 * dt;
        const u32x2 lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(TVQ_LDS_V4I16(p0)));
        const u32x2 hi =
            __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(TVQ_LDS_V4I16(p0 + 16 * kVStride)));
        acc = mfma16x16x32<T>(u32x4{lo.x, lo.y, hi.x, hi.y}, pb[c], acc);
      }
      o[dt] = acc;
    }
    __syncthreads();  // buffer cur is free and buffer cur ^ 1 is complete
  }

  if (qi < len) {
    const float inv = 1.0f / l;
    uint16_t* dst = out + ((seq0 + qi) * Hq + h) * kD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      u32x2 pk;
      pk.x = (uint32_t)from_float<T>(o[dt][0] * inv) | ((uint32_t)from_float<T>(o[dt][1] * inv) << 16);
      pk.y = (uint32_t)from_float<T>(o[dt][2] * inv) | ((uint32_t)from_float<T>(o[dt][3] * inv) << 16);
      if constexpr (kQ)
        store8_agent(dst + 16 * dt + 4 * g, pk);
      else
        *reinterpret_cast<u32x2*>(dst + 16 * dt + 4 * g) = pk;
    }
  }
  if constexpr (kQ)
    quantize_rows_last<T, 256 * G>(out, seq0 + q0, seq0 + min(q0 + kBlkQ, len), Hq * kD, qo.counters + blockIdx.x,
                                   gridDim.y, qo.xq, qo.a_scales, qo.eps);
}

// Two values rounded to the 16-bit type, packed low | high << 16 (bf16:
// one v_cvt_pk_bf16_f32, round to nearest even like the scalar conversion).
template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b);
template <>
__device__ __forceinline__ uint32_t pack2<BF16>(float a, float b) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}
template <>
__device__ __forceinline__ uint32_t pack2<F16>(float a, float b) {
  return (uint32_t)from_float<F16>(a) | ((uint32_t)from_float<F16>(b) << 16);
}

// Variant for G = 2 and 4 (GQA ratios divisible by 2): two waves per head,
// each owning 32 queries, on v_mfma_f32_32x32x16_{bf16,f16}. A 32x32x16
// MFMA does twice the work of a 16x16x32 one for the same 1 KB A-fragment
// read, so every K and V fragment read from LDS feeds 32 queries instead of
// 16: the 16-query kernel is bound by those LDS reads (4 waves x 32 KB per
// 64-key block and head).
//   S^T[key][q] (2 tiles of 32 keys): A = K rows (lane 32hf + r: key r, dims
//     16c + 8hf .. +8), B = Q rows (lane 32hf + r: query r, same dims).
//   Accumulator lane 32hf + q, register v: key 8(v/4) + 4hf + v%4.
//   O^T[d][q] (4 tiles of 32 dims) += V^T . P^T in 4 steps of 16 keys: step
//     j = (tile kt, half u) feeds registers 8u .. 8u+7 of S^T tile kt as the
//     B operand, i.e. keys key0 + 0..3 and key0 + 8..11, key0 = 32kt + 16u +
//     4hf; the A operand (lane 32hf + r: dim r of the tile) is the same 8
//     keys of V^T, two transposing LDS reads of 4 keys each.
// K/V tiles arrive by LDS DMA (global_load_lds_dwordx4), one block ahead
// into the other half of a double buffer, so no register staging is needed
// (measured 131 -> 125 us per layer at 16 x 1024 tokens against register
// staging; 157 us for the 16-query kernel). The running max is taken on raw
// scores and the scale applied inside each exponent's fma. A wave skips the
// MFMAs of key blocks that lie wholly after its last query (the block's
// other wave may still need them) and the mask arithmetic of blocks that lie
// wholly before its first query.
template <typename T, int G, bool kQ = false>
__global__ __launch_bounds__(2 * kBlkQ * G) __attribute__((amdgpu_waves_per_eu(2))) void prefill_attn32_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int64_t v_stride,
    const int32_t* __restrict__ blocks, int Hq, int Hkv, float scale_log2, uint16_t* __restrict__ out,
    AttnQuant qo) {
  constexpr int kWph = kBlkQ / 32;                     // waves per head
  constexpr int kThreads = 64 * kWph * G;
  constexpr int kVec = kBlkK * kD / 8;                 // 16-byte vectors per K (or V) tile
  static_assert(kBlkQ % 32 == 0 && kVec % kThreads == 0, "tile vectors split evenly");
  // unpadded 256-byte rows, 16-byte chunks XOR-swizzled per row (K: chunk ^
  // row % 16, V: chunk ^ 2 (row % 8)) so the fragment and transposing reads
  // are bank-conflict free; filled by LDS DMA, 1 KB (4 rows) per op
  __shared__ __attribute__((aligned(1024))) uint16_t ks[2][kBlkK * kD];
  __shared__ __attribute__((aligned(1024))) uint16_t vs[2][kBlkK * kD];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int hf = lane >> 5;
  const int r = lane & 31;
  const int h = blockIdx.y * G + wave / kWph;        // this wave's query head
  const int hk = h / (Hq / Hkv);
  const int64_t seq0 = blocks[3 * blockIdx.x];
  const int len = blocks[3 * blockIdx.x + 1];
  const int q0 = blocks[3 * blockIdx.x + 2];
  const int qw0 = q0 + (wave % kWph) * 32;           // this wave's first query
  const int qi = qw0 + r;
  const int qc = min(qi, len - 1);
  // last key any query of the wave needs (-1: the wave has no queries)
  const int wave_last = qw0 < len ? min(qw0 + 31, len - 1) : -1;

  u32x4 qf[8];
#pragma unroll
  for (int c = 0; c < 8; ++c)
    qf[c] = *reinterpret_cast<const u32x4*>(q + ((seq0 + qc) * Hq + h) * kD + 16 * c + 8 * hf);

  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{};
  float m = -INFINITY, l = 0.0f;

  // DMA op t of a tile writes rows 4t .. 4t+3; lane l fills row 4t + l / 16,
  // physical chunk l % 16, with the row's logical chunk (l % 16) ^ swizzle.
  constexpr int kOpsPerWave = kBlkK / 4 / (kThreads / 64);
  static_assert(kOpsPerWave * (kThreads / 64) * 4 == kBlkK, "tile DMA ops split evenly over the waves");
  const int64_t kstride = (int64_t)Hkv * kD;         // elements per token, K
  // Whole blocks: a uniform base per block plus loop-invariant 32-bit lane
  // byte offsets (row * stride + chunk). The block that runs past the
  // sequence end clamps every key instead.
  uint32_t koff[kOpsPerWave], voff[kOpsPerWave];
#pragma unroll
  for (int j = 0; j < kOpsPerWave; ++j) {
    const int row = 4 * (wave + j * (kThreads / 64)) + (lane >> 4);
    koff[j] = (uint32_t)(row * kstride + 8 * ((lane & 15) ^ (row & 15))) * 2u;
    voff[j] = (uint32_t)(row * v_stride + 8 * ((lane & 15) ^ (2 * (row & 7)))) * 2u;
  }
  const char* kbase = reinterpret_cast<const char*>(k + seq0 * kstride + hk * kD);
  const char* vbase = reinterpret_cast<const char*>(v + seq0 * v_stride + hk * kD);
  auto dma_tiles = [&](int kv0, int buf) {
    if (kv0 + kBlkK <= len) {  // uniform
      const char* kb = kbase + (int64_t)kv0 * kstride * 2;
      const char* vb = vbase + (int64_t)kv0 * v_stride * 2;
#pragma unroll
      for (int j = 0; j < kOpsPerWave; ++j) {
        const int t = wave + j * (kThreads / 64);
        __builtin_amdgcn_global_load_lds(TVQ_AGPTR(kb + koff[j]), TVQ_ALPTR(&ks[buf][t * 512]), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(TVQ_AGPTR(vb + voff[j]), TVQ_ALPTR(&vs[buf][t * 512]), 16, 0, 0);
      }
    } else {
#pragma unroll
      for (int j = 0; j < kOpsPerWave; ++j) {
        const int t = wave + j * (kThreads / 64);
        const int row = 4 * t + (lane >> 4);
        const int key = min(kv0 + row, len - 1);
        const int kc = (lane & 15) ^ (row & 15);
        const int vc = (lane & 15) ^ (2 * (row & 7));
        __builtin_amdgcn_global_load_lds(TVQ_AGPTR(k + (seq0 + key) * kstride + hk * kD + 8 * kc),
                                         TVQ_ALPTR(&ks[buf][t * 512]), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(TVQ_AGPTR(v + (seq0 + key) * v_stride + hk * kD + 8 * vc),
                                         TVQ_ALPTR(&vs[buf][t * 512]), 16, 0, 0);
      }
    }
  };

  const int kv_end = min(len, q0 + kBlkQ);
  dma_tiles(0, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's DMA has landed in LDS
  __syncthreads();
  for (int kv0 = 0, cur = 0; kv0 < kv_end; kv0 += kBlkK, cur ^= 1) {
    // the other buffer was last read in the previous block, before its barrier
    if (kv0 + kBlkK < kv_end) dma_tiles(kv0 + kBlkK, cur ^ 1);
    if (kv0 <= wave_last) {  // wave-uniform
      const uint16_t* ksb = ks[cur];
      const uint16_t* vsb = vs[cur];
      f32x16 s[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        f32x16 acc = f32x16{};
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(&ksb[(32 * kt + r) * kD + 8 * ((2 * c + hf) ^ (r & 15))]);
          acc = mfma32x32x16<T>(a, qf[c], acc);
        }
        s[kt] = acc;
      }
      // the running max is kept on raw scores (scale > 0 preserves the order;
      // scale_log2 is applied inside the exponent's fma)
      float mx = -INFINITY;
      if (kv0 + kBlkK - 1 <= qw0 && kv0 + kBlkK <= len) {  // no key of the block is masked for this wave
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[kt][e]);
      } else {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int key = kv0 + 32 * kt + 8 * (e >> 2) + 4 * hf + (e & 3);
            const float sv = (key <= qi && key < len) ? s[kt][e] : -INFINITY;
            s[kt][e] = sv;
            mx = fmaxf(mx, sv);
          }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
      const float mn = fmaxf(m, mx * scale_log2);  // finite: key 0 is valid for every query
      const float corr = __builtin_amdgcn_exp2f(m - mn);
      float ps = 0.0f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float p = __builtin_amdgcn_exp2f(fmaf(s[kt][e], scale_log2, -mn));
          s[kt][e] = p;
          ps += p;
        }
      ps += __shfl_xor(ps, 32, kWave);
      l = l * corr + ps;
      m = mn;
      u32x4 pb[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) pb[j][i] = pack2<T>(s[j >> 1][8 * (j & 1) + 2 * i], s[j >> 1][8 * (j & 1) + 2 * i + 1]);
      // transposing read (see prefill_attn_kernel): lane i of a 16-lane group
      // addresses key key0 + i / 4, dims d0 + 4 (i % 4) .. +4 and receives
      // V[key0 + e][d0 + i], e = 0..3; d0 = 32dt + 16 (r / 16). Every key0
      // is 4hf modulo 8, so the row's swizzle 2 (row % 8) = 8hf + 2 (i / 4)
      // is the same for all j.
      const int vsw = 8 * hf + 2 * ((r & 15) >> 2);
      const uint16_t* vrow = vsb + (4 * hf + ((r & 15) >> 2)) * kD + 4 * (r & 1);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        f32x16 acc = o[dt] * corr;
        const int chunk = (4 * dt + 2 * (r >> 4) + ((r & 3) >> 1)) ^ vsw;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint16_t* p0 = vrow + (32 * (j >> 1) + 16 * (j & 1)) * kD + 8 * chunk;
          const u32x2 lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(TVQ_LDS_V4I16(p0)));
          const u32x2 hi =
              __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(TVQ_LDS_V4I16(p0 + 8 * kD)));
          acc = mfma32x32x16<T>(u32x4{lo.x, lo.y, hi.x, hi.y}, pb[j], acc);
        }
        o[dt] = acc;
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // next block's DMA has landed
    __syncthreads();
  }

  if (qi < len) {
    const float inv = 1.0f / l;
    uint16_t* dst = out + ((seq0 + qi) * Hq + h) * kD + 4 * hf;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u32x2 pk;
        pk.x = (uint32_t)from_float<T>(o[dt][4 * j] * inv) | ((uint32_t)from_float<T>(o[dt][4 * j + 1] * inv) << 16);
        pk.y = (uint32_t)from_float<T>(o[dt][4 * j + 2] * inv) | ((uint32_t)from_float<T>(o[dt][4 * j + 3] * inv) << 16);
        if constexpr (kQ)
          store8_agent(dst + 32 * dt + 8 * j, pk);
        else
          *reinterpret_cast<u32x2*>(dst + 32 * dt + 8 * j) = pk;
      }
  }
  if constexpr (kQ)
    quantize_rows_last<T, 2 * kBlkQ * G>(out, seq0 + q0, seq0 + min(q0 + kBlkQ, len), Hq * kD,
                                         qo.counters + blockIdx.x, gridDim.y, qo.xq, qo.a_scales, qo.eps);
}

template <typename T, bool kQ>
hipError_t launch_prefill_t(const uint16_t* Q, const uint16_t* K, const uint16_t* V, int64_t v_stride,
                            const int32_t* blocks, int nblocks, int Hq, int Hkv, float sl2, uint16_t* O, AttnQuant qo,
                            hipStream_t stream) {
  // G query heads per workgroup: the largest of 4, 2, 1 dividing the GQA
  // ratio Hq / Hkv, so the workgroup's heads share one kv head. G = 2 and 4
  // run the 32-query-per-wave kernel (2 waves per head), G = 1 the 16-query
  // one (4 waves per head).
  const int ratio = Hq / Hkv;
  const int G = ratio % 4 == 0 ? 4 : (ratio % 2 == 0 ? 2 : 1);
  const dim3 grid((unsigned)nblocks, (unsigned)(Hq / G));
  if (G == 4)
    prefill_attn32_kernel<T, 4, kQ><<<grid, 8 * kBlkQ, 0, stream>>>(Q, K, V, v_stride, blocks, Hq, Hkv, sl2, O, qo);
  else if (G == 2)
    prefill_attn32_kernel<T, 2, kQ><<<grid, 4 * kBlkQ, 0, stream>>>(Q, K, V, v_stride, blocks, Hq, Hkv, sl2, O, qo);
  else
    prefill_attn_kernel<T, 1, kQ><<<grid, 256, 0, stream>>>(Q, K, V, v_stride, blocks, Hq, Hkv, sl2, O, qo);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_prefill_attention(const void* q, const void* k, const void* v, int64_t v_stride,
                                    const int32_t* blocks, int nblocks, int Hq, int Hkv, float scale, void* out,
                                    bool bf16, hipStream_t stream, const AttnQuant* quant) {
  const float sl2 = scale * 1.4426950408889634f;  // log2(e)
  auto Q = static_cast<const uint16_t*>(q);
  auto Kp = static_cast<const uint16_t*>(k);
  auto V = static_cast<const uint16_t*>(v);
  auto O = static_cast<uint16_t*>(out);
  const AttnQuant qo = quant ? *quant : AttnQuant{nullptr, nullptr, nullptr, 0.0f};
  if (quant) {
    if (bf16) return launch_prefill_t<BF16, true>(Q, Kp, V, v_stride, blocks, nblocks, Hq, Hkv, sl2, O, qo, stream);
    return launch_prefill_t<F16, true>(Q, Kp, V, v_stride, blocks, nblocks, Hq, Hkv, sl2, O, qo, stream);
  }
  if (bf16) return launch_prefill_t<BF16, false>(Q, Kp, V, v_stride, blocks, nblocks, Hq, Hkv, sl2, O, qo, stream);
  return launch_prefill_t<F16, false>(Q, Kp, V, v_stride, blocks, nblocks, Hq, Hkv, sl2, O, qo, stream);
}

}  // namespace tvq
