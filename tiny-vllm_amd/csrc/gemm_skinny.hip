// Skinny (decode-size M <= 64) W8A16 / W8A8 GEMM for gfx950.
//
// Decode is weight-bandwidth bound: every int8 weight byte is read exactly
// once and the activations are tiny and L2-resident. The kernel therefore
// streams qweight [N,K] with 128-bit non-temporal loads and puts the weight
// rows on the MFMA "A" side (16 output channels per MFMA block) and the
// activation rows on the "B" side (16 tokens per block):
//
//   lane l = 16*g + r reads 16 consecutive int8 of weight row n0+r at
//   k = kc + 16*g, and the same k range of token row r of x.
//
// W8A8  : one v_mfma_i32_16x16x64_i8 consumes the 16 bytes directly (exact
//         int32 accumulation).
// W8A16 : the 16 bytes are converted in registers to two 8-element bf16/fp16
//         fragments (int8 is exact in both) and feed two
//         v_mfma_f32_16x16x32_{bf16,f16}. The fp32 per-channel scale is
//         applied once per output in the epilogue instead of per weight.
//
// Any consistent assignment of k to (lane group, register slot) yields the
// same dot products, so A and B only have to agree with each other.
//
// A workgroup of W waves owns 16*RG output channels; its waves split K into
// contiguous ranges of U-chunk runs (64 k per chunk) and are reduced through
// LDS at the end in a fixed order (deterministic output). W = 4 when there are
// enough workgroups to fill the chip (N >= 16384); otherwise 8 or 16 so that
// each wave needs about one run over K, which keeps more weight loads in
// flight per workgroup and the latency chains short.
#include <type_traits>

#include "tvq_common.h"
#include "tvq_internal.h"

namespace tvq {
namespace {

template <int MG, int RG>
struct SkinnyCfg {
  // Chunks in flight per wave: bounded so weight + activation registers stay
  // around 64 VGPRs.
  static constexpr int U = (8 / (RG * MG)) > 0 ? (8 / (RG * MG)) : 1;
};

template <typename T, bool kW8A8, bool kRaw, int MG, int RG, int kWaves, int U>
__global__ __launch_bounds__(64 * kWaves) void skinny_kernel(const void* __restrict__ xv, const float* __restrict__ a_scales,
                                                     const int8_t* __restrict__ qw, const float* __restrict__ ws,
                                                     const uint16_t* __restrict__ bias, void* __restrict__ yv,
                                                     int M, int N, int K) {
  using Acc = typename std::conditional<kW8A8, i32x4, f32x4>::type;
  constexpr int kXRegs = kW8A8 ? 1 : 2;  // 16-byte x vectors per (chunk, m-group)

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int n0 = blockIdx.x * (16 * RG);

  Acc acc[RG][MG];
#pragma unroll
  for (int i = 0; i < RG; ++i)
#pragma unroll
    for (int j = 0; j < MG; ++j) acc[i][j] = Acc{0, 0, 0, 0};

  // Per-lane row pointers. Rows past N (weights) or M (tokens) are clamped to
  // the last row: they are read but only feed accumulator entries whose
  // outputs are never stored, so the loads need no predicate.
  const int8_t* wrow[RG];
#pragma unroll
  for (int i = 0; i < RG; ++i) {
    const int n = n0 + 16 * i + r;
    wrow[i] = qw + (int64_t)(n < N ? n : N - 1) * K + 16 * g;
  }
  const char* xrow[MG];
#pragma unroll
  for (int j = 0; j < MG; ++j) {
    const int m = 16 * j + r;
    xrow[j] = static_cast<const char*>(xv) + ((int64_t)(m < M ? m : M - 1) * K + 16 * g) * (kW8A8 ? 1 : 2);
  }

  // Each wave owns one contiguous range of whole U-chunk runs, so its reads
  // of every weight row are contiguous.
  const int nchunks = (K + 63) >> 6;
  const int cpw = ((nchunks + kWaves * U - 1) / (kWaves * U)) * U;
  const int cend = min(nchunks, (wave + 1) * cpw);

  // One run of U chunks: loads (unpredicated when kGuard is false), then MFMAs.
  auto run = [&](int c0, auto guard) {
    constexpr bool kGuard = decltype(guard)::value;
    u32x4 wv[U][RG];
    u32x4 xvv[U][MG][kXRegs];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // kGuard: chunk inside this wave's range and the lane's 16 k inside K.
      const bool kok = !kGuard || ((c0 + u) < cend && (c0 + u) * 64 + 16 * g < K);
#pragma unroll
      for (int i = 0; i < RG; ++i) wv[u][i] = kok ? ldg128_stream(wrow[i] + (int64_t)(c0 + u) * 64) : u32x4{0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < MG; ++j) {
#pragma unroll
        for (int h = 0; h < kXRegs; ++h) {
          const int64_t off = (int64_t)(c0 + u) * 64 * (kW8A8 ? 1 : 2) + 16 * h;
          xvv[u][j][h] = kok ? ldg128(xrow[j] + off) : u32x4{0, 0, 0, 0};
        }
      }
    }
    // Every load of the run is issued before the first MFMA (left alone, the
    // scheduler sinks them among the MFMAs and keeps only ~10 in flight).
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int i = 0; i < RG; ++i) {
        if constexpr (kW8A8) {
#pragma unroll
          for (int j = 0; j < MG; ++j) acc[i][j] = mfma16x16x64_i8(wv[u][i], xvv[u][j][0], acc[i][j]);
        } else {
          const u32x2 a0 = i8x4_to_16x4<T>(wv[u][i][0]);
          const u32x2 a1 = i8x4_to_16x4<T>(wv[u][i][1]);
          const u32x2 a2 = i8x4_to_16x4<T>(wv[u][i][2]);
          const u32x2 a3 = i8x4_to_16x4<T>(wv[u][i][3]);
          const u32x4 alo = {a0.x, a0.y, a1.x, a1.y};
          const u32x4 ahi = {a2.x, a2.y, a3.x, a3.y};
#pragma unroll
          for (int j = 0; j < MG; ++j) {
            acc[i][j] = mfma16x16x32<T>(alo, xvv[u][j][0], acc[i][j]);
            acc[i][j] = mfma16x16x32<T>(ahi, xvv[u][j][1], acc[i][j]);
          }
        }
      }
    }
  };
  for (int c0 = wave * cpw; c0 < cend; c0 += U) {
    // The run is fully valid unless it reaches past the wave's range or K.
    if (c0 + U <= cend && (c0 + U) * 64 <= K)
      run(c0, std::false_type{});
    else
      run(c0, std::true_type{});
  }

  // Cross-wave reduction in a fixed order (wave 0 + 1 + 2 + 3).
  __shared__ Acc red[kWaves][RG * MG][64];
#pragma unroll
  for (int i = 0; i < RG; ++i)
#pragma unroll
    for (int j = 0; j < MG; ++j) red[wave][i * MG + j][lane] = acc[i][j];
  __syncthreads();

  constexpr int kItems = RG * MG * 64;
  for (int it = tid; it < kItems; it += 64 * kWaves) {
    const int ij = it >> 6;
    const int ln = it & 63;
    const int i = ij / MG;
    const int j = ij % MG;
    Acc v = red[0][ij][ln];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) v += red[w][ij][ln];
    const int m = 16 * j + (ln & 15);
    const int nb = n0 + 16 * i + 4 * (ln >> 4);
    if (m >= M) continue;
    if constexpr (kRaw) {
      int32_t* y = static_cast<int32_t*>(yv) + (int64_t)m * N;
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (nb + t < N) y[nb + t] = v[t];
    } else {
      uint16_t* y = static_cast<uint16_t*>(yv) + (int64_t)m * N;
      float o[4];
      float as = 0.0f;
      if constexpr (kW8A8) as = a_scales[m];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int n = nb + t < N ? nb + t : N - 1;
        const float b = bias ? to_float<T>(bias[n]) : 0.0f;
        if constexpr (kW8A8)
          o[t] = epi_w8a8(v[t], as, ws[n], b);
        else
          o[t] = epi_w8a16(v[t], ws[n], b);
      }
      if (nb + 3 < N && (N & 3) == 0) {
        u32x2 pk;
        pk.x = (uint32_t)from_float<T>(o[0]) | ((uint32_t)from_float<T>(o[1]) << 16);
        pk.y = (uint32_t)from_float<T>(o[2]) | ((uint32_t)from_float<T>(o[3]) << 16);
        *reinterpret_cast<u32x2*>(y + nb) = pk;
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if (nb + t < N) y[nb + t] = from_float<T>(o[t]);
      }
    }
  }
}

template <typename T, bool kW8A8, bool kRaw, int MG, int RG, int W, int U = SkinnyCfg<MG, RG>::U>
hipError_t launch_w(const GemmArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)((a.N + 16 * RG - 1) / (16 * RG)));
  const dim3 block(64 * W);
  skinny_kernel<T, kW8A8, kRaw, MG, RG, W, U><<<grid, block, 0, stream>>>(
      a.x, a.a_scales, a.qweight, a.scales, static_cast<const uint16_t*>(a.bias), a.y, (int)a.M, (int)a.N, (int)a.K);
  return hipGetLastError();
}

template <typename T, bool kW8A8, bool kRaw, int MG, int RG>
hipError_t launch_rg(const GemmArgs& a, hipStream_t stream) {
  // Waves per workgroup: enough that each wave needs about one run of U
  // chunks over K (at least 4; 16 or 8 only while the LDS reduction buffer,
  // W x RG x MG KB, stays within 32 KB).
  constexpr int U = SkinnyCfg<MG, RG>::U;
  const int64_t runs = (a.K + 64 * U - 1) / (64 * U);
  if constexpr (RG * MG <= 2) {
    if (runs > 8) return launch_w<T, kW8A8, kRaw, MG, RG, 16>(a, stream);
  }
  if (a.N >= 16384) return launch_w<T, kW8A8, kRaw, MG, RG, 4>(a, stream);
  // Short K (<= 1024) with one 16x16 block per wave: runs of 4 chunks keep all
  // 4 waves busy (measured 3-8 % faster at K = 1024 than 2 busy waves).
  if constexpr (RG * MG == 1) {
    if (a.K <= 1024) return launch_w<T, kW8A8, kRaw, MG, RG, 4, 4>(a, stream);
  }
  if constexpr (RG * MG <= 4) {
    if (runs > 4) return launch_w<T, kW8A8, kRaw, MG, RG, 8>(a, stream);
  }
  return launch_w<T, kW8A8, kRaw, MG, RG, 4>(a, stream);
}

template <typename T, bool kW8A8, bool kRaw, int MG>
hipError_t launch_mg(const GemmArgs& a, hipStream_t stream) {
  // Two row groups per wave only when that still leaves >= 4 workgroups per CU.
  if (a.N >= 16 * 2 * 1024) return launch_rg<T, kW8A8, kRaw, MG, 2>(a, stream);
  return launch_rg<T, kW8A8, kRaw, MG, 1>(a, stream);
}

template <typename T, bool kW8A8, bool kRaw>
hipError_t launch_t(const GemmArgs& a, hipStream_t stream) {
  const int mg = (int)((a.M + 15) / 16);
  switch (mg) {
    case 1: return launch_mg<T, kW8A8, kRaw, 1>(a, stream);
    case 2: return launch_mg<T, kW8A8, kRaw, 2>(a, stream);
    case 3: return launch_mg<T, kW8A8, kRaw, 3>(a, stream);
    default: return launch_mg<T, kW8A8, kRaw, 4>(a, stream);
  }
}

}  // namespace

hipError_t launch_skinny(const GemmArgs& a, hipStream_t stream) {
  if (a.w8a8) {
    if (a.raw_i32) return launch_t<BF16, true, true>(a, stream);
    return a.bf16 ? launch_t<BF16, true, false>(a, stream) : launch_t<F16, true, false>(a, stream);
  }
  return a.bf16 ? launch_t<BF16, false, false>(a, stream) : launch_t<F16, false, false>(a, stream);
}

}  // namespace tvq
