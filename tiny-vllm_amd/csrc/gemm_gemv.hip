// Row-contiguous GEMV for the smallest decode batches (M <= 2), gfx950.
//
// At M <= 2 the MFMA formulation of the skinny kernel wastes most of each
// 16x16 block and, more importantly, reads every weight row as 64-byte
// pieces of 16 different rows per instruction. Streaming whole 1 KB row
// chunks instead (each wave instruction = 64 lanes x 16 contiguous bytes of
// ONE row) measured 6.5 TB/s on the 8B gate_up weights against 5.85 TB/s for
// the 16-row pattern. So this kernel does the dot products on the vector
// ALUs:
//   W8A8 : v_dot4_i32_i8 on 4 int8 weights x 4 int8 codes (exact int32),
//   W8A16: int8 -> bf16/fp16 pairs (exact) and v_dot2_f32_{bf16,f16}.
// A lane owns k = 1024*c + 16*lane .. +16 of chunk c for every row it reads,
// so its activation slice (M tokens x 16 k per chunk) is loaded once into
// registers and reused for all R rows of its group.
//
// Work split: a group of R rows (8, or 4 / 2 for small short-K shapes) is
// handled by WPG waves (1, 2 or 4 of the workgroup's 4), wave i of the group
// taking chunks i, i+WPG, ... (at most CPW chunks). Each wave issues all its R x CPW weight loads before computing.
// Per (token, row) the 64 lanes are reduced with a butterfly, the WPG waves
// of a group through LDS in a fixed order (deterministic output), and the
// epilogue applies the fp32 per-channel scale once per output as the other
// kernels do. Rows past N and tokens past M are clamped (read, never stored).
// Requires K % 1024 == 0 and K <= 1024 * 4 * CPW; the dispatcher checks.
#include <type_traits>

#include "tvq_common.h"
#include "tvq_internal.h"

namespace tvq {
namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kMaxCpw = 3;  // chunks per wave: K <= 12288

template <typename T>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c);
template <>
__device__ __forceinline__ float dot2<BF16>(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}
template <>
__device__ __forceinline__ float dot2<F16>(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
}

// Sum of NV per-lane values over the 64 lanes of a wave, all NV at once: at
// each of the first log2(NV) steps (lane offsets 32, 16, ...) a lane keeps
// the half of its values selected by its lane bit, sends the other half to
// its partner across that bit and adds the partner's copy of the kept half,
// so the values in flight halve every step (NV - 1 exchanges instead of
// 6 * NV). The remaining offsets then sum within each group. Afterwards every
// lane of group j = lane / (64 / NV) holds the total of value j. The order of
// the additions is fixed, so the result is deterministic.
// One halving step over the first N values at lane offset OFF, then the
// next; every index is a compile-time constant (the values stay in VGPRs).
template <int N, int OFF, int NV, typename Acc>
__device__ __forceinline__ Acc fold_step(Acc (&c)[NV], int lane) {
  if constexpr (N > 1) {
    const bool hi = (lane & OFF) != 0;   // keep the upper half
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      const Acc send = hi ? c[i] : c[i + N / 2];
      const Acc keep = hi ? c[i + N / 2] : c[i];
      c[i] = keep + __shfl_xor(send, OFF, kWave);
    }
    return fold_step<N / 2, OFF / 2>(c, lane);
  } else {
    Acc v = c[0];
#pragma unroll
    for (int off = OFF; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
  }
}

template <int NV, typename Acc>
__device__ __forceinline__ Acc fold_sum(Acc (&c)[NV]) {
  static_assert(NV >= 1 && NV <= 64 && (NV & (NV - 1)) == 0, "a power of two up to 64 values");
  return fold_step<NV, 32>(c, (int)__lane_id());
}

template <typename T, bool kW8A8, bool kRaw, int MM, int R, int WPG, int CPW>
__global__ __launch_bounds__(256) void gemv_kernel(const void* __restrict__ xv, const float* __restrict__ a_scales,
                                                   const int8_t* __restrict__ qw, const float* __restrict__ ws,
                                                   const uint16_t* __restrict__ bias, void* __restrict__ yv, int M,
                                                   int N, int K) {
  using Acc = typename std::conditional<kW8A8, int32_t, float>::type;
  constexpr int kGroups = 4 / WPG;           // row groups per workgroup
  constexpr int kXRegs = kW8A8 ? 1 : 2;      // 16-byte x vectors per (chunk, token)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int grp = wave / WPG;
  const int wig = wave % WPG;
  const int nch = K >> 10;
  const int row0 = (blockIdx.x * kGroups + grp) * R;

  // ---- loads: weights (R rows x CPW chunks), then the activation slices ----
  u32x4 wv[CPW][R];
  u32x4 xq[CPW][MM][kXRegs];
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    const int c = wig + j * WPG;
    const bool ok = c < nch;  // wave-uniform
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int n = min(row0 + r, N - 1);
      wv[j][r] = ok ? ldg128_stream(qw + (int64_t)n * K + 1024 * c + 16 * lane) : u32x4{0, 0, 0, 0};
    }
  }
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    const int c = wig + j * WPG;
    const bool ok = c < nch;
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      const int mm = min(m, M - 1);
      const char* xr = static_cast<const char*>(xv) + ((int64_t)mm * K + 1024 * c + 16 * lane) * (kW8A8 ? 1 : 2);
#pragma unroll
      for (int h = 0; h < kXRegs; ++h) xq[j][m][h] = ok ? ldg128(xr + 16 * h) : u32x4{0, 0, 0, 0};
    }
  }

  // ---- dot products ----------------------------------------------------------
  Acc acc[MM][R];
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0;
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if constexpr (kW8A8) {
#pragma unroll
        for (int m = 0; m < MM; ++m)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            acc[m][r] = __builtin_amdgcn_sdot4((int)wv[j][r][e], (int)xq[j][m][0][e], acc[m][r], false);
      } else {
        // 16 int8 weights -> 8 pairs of 16-bit values, k order preserved
        uint32_t wp[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const u32x2 p = i8x4_to_16x4<T>(wv[j][r][e]);
          wp[2 * e] = p.x;
          wp[2 * e + 1] = p.y;
        }
#pragma unroll
        for (int m = 0; m < MM; ++m)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[m][r] = dot2<T>(wp[e], xq[j][m][e >> 2][e & 3], acc[m][r]);
      }
    }
  }

  // ---- reduction: 64 lanes, then the WPG waves of the group ------------------
  constexpr int kOut = MM * R;               // outputs per group, value j = m * R + r
  static_assert(kOut <= 64, "one lane per output");
  __shared__ Acc red[4][kOut];
  Acc v;
  if constexpr (CPW < 3) {
    constexpr int kGroup = 64 / kOut;        // lanes per value after fold_sum
    Acc flat[kOut];
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
      for (int r = 0; r < R; ++r) flat[m * R + r] = acc[m][r];
    const Acc total = fold_sum<kOut>(flat);  // total of value lane / kGroup
    if constexpr (WPG > 1) {
      if (lane % kGroup == 0) red[wave][lane / kGroup] = total;
      __syncthreads();
      if (wig != 0) return;
    }
    // one wave per group: lane j takes value j from the first lane of group j
    // (before any lane leaves: the source lanes may lie past kOut)
    Acc own{};
    if constexpr (WPG == 1) own = __shfl(total, (lane % kOut) * kGroup, kWave);
    if (lane >= kOut) return;
    if constexpr (WPG > 1) {
      v = red[grp * WPG][lane];
#pragma unroll
      for (int w = 1; w < WPG; ++w) v += red[grp * WPG + w][lane];
    } else {
      v = own;
    }
  } else {
    // three chunks per wave: one butterfly per value, reduced in place (the
    // fold's extra registers would cost a wave per SIMD: 128 -> 159 VGPRs)
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) acc[m][r] += __shfl_xor(acc[m][r], off, kWave);
    if constexpr (WPG > 1) {
      if (lane == 0) {
#pragma unroll
        for (int m = 0; m < MM; ++m)
#pragma unroll
          for (int r = 0; r < R; ++r) red[wave][m * R + r] = acc[m][r];
      }
      __syncthreads();
      if (wig != 0) return;
    }
    if (lane >= kOut) return;
    if constexpr (WPG > 1) {
      v = red[grp * WPG][lane];
#pragma unroll
      for (int w = 1; w < WPG; ++w) v += red[grp * WPG + w][lane];
    } else {
      v = acc[0][0];   // every lane holds every sum; pick this lane's one
#pragma unroll
      for (int mm = 0; mm < MM; ++mm)
#pragma unroll
        for (int rr = 0; rr < R; ++rr)
          if (mm * R + rr == lane) v = acc[mm][rr];
    }
  }
  const int m = lane / R;
  const int r = lane % R;
  const int n = row0 + r;
  if (m >= M || n >= N) return;
  if constexpr (kRaw) {
    static_cast<int32_t*>(yv)[(int64_t)m * N + n] = (int32_t)v;
  } else {
    const float b = bias ? to_float<T>(bias[n]) : 0.0f;
    float o;
    if constexpr (kW8A8)
      o = epi_w8a8(v, a_scales[m], ws[n], b);
    else
      o = epi_w8a16(v, ws[n], b);
    static_cast<uint16_t*>(yv)[(int64_t)m * N + n] = from_float<T>(o);
  }
}

template <typename T, bool kW8A8, bool kRaw, int MM, int R, int WPG, int CPW>
hipError_t launch_g(const GemmArgs& a, hipStream_t stream) {
  constexpr int kGroups = 4 / WPG;
  const int64_t groups = (a.N + R - 1) / R;
  const dim3 grid((unsigned)((groups + kGroups - 1) / kGroups)), block(256);
  gemv_kernel<T, kW8A8, kRaw, MM, R, WPG, CPW><<<grid, block, 0, stream>>>(
      a.x, a.a_scales, a.qweight, a.scales, static_cast<const uint16_t*>(a.bias), a.y, (int)a.M, (int)a.N, (int)a.K);
  return hipGetLastError();
}

// Short K (one to three 1 KB chunks per row): 8 rows per wave unless that
// leaves fewer than 2048 waves (8 per SIMD) to hide the load latency, then 4
// or 2.
template <typename T, bool kW8A8, bool kRaw, int MM, int WPG, int CPW>
hipError_t launch_r(const GemmArgs& a, hipStream_t stream) {
  constexpr int64_t kWantWaves = 2048;
  if ((a.N + 7) / 8 * WPG >= kWantWaves) return launch_g<T, kW8A8, kRaw, MM, 8, WPG, CPW>(a, stream);
  if ((a.N + 3) / 4 * WPG >= kWantWaves) return launch_g<T, kW8A8, kRaw, MM, 4, WPG, CPW>(a, stream);
  return launch_g<T, kW8A8, kRaw, MM, 2, WPG, CPW>(a, stream);
}

template <typename T, bool kW8A8, bool kRaw, int MM>
hipError_t launch_m(const GemmArgs& a, hipStream_t stream) {
  const int64_t nch = a.K / 1024;
  if (nch == 1) return launch_r<T, kW8A8, kRaw, MM, 1, 1>(a, stream);
  if (nch <= 3) return launch_r<T, kW8A8, kRaw, MM, 2, 2>(a, stream);
  if (nch <= 4) return launch_g<T, kW8A8, kRaw, MM, 8, 4, 1>(a, stream);
  if (nch <= 8) return launch_g<T, kW8A8, kRaw, MM, 8, 4, 2>(a, stream);
  return launch_g<T, kW8A8, kRaw, MM, 8, 4, kMaxCpw>(a, stream);
}

template <typename T, bool kW8A8, bool kRaw>
hipError_t launch_t(const GemmArgs& a, hipStream_t stream) {
  // Beyond M = 2 the vector-ALU work (one dot per 2 or 4 weights per token)
  // overtakes the load time and the MFMA skinny kernel is faster.
  if (a.M == 1) return launch_m<T, kW8A8, kRaw, 1>(a, stream);
  return launch_m<T, kW8A8, kRaw, 2>(a, stream);
}

}  // namespace

bool gemv_shape_ok(int64_t M, int64_t K) { return M >= 1 && M <= kGemvMaxM && K % 1024 == 0 && K <= 1024 * 4 * kMaxCpw; }

hipError_t launch_gemv(const GemmArgs& a, hipStream_t stream) {
  if (a.w8a8) {
    if (a.raw_i32) return launch_t<BF16, true, true>(a, stream);
    return a.bf16 ? launch_t<BF16, true, false>(a, stream) : launch_t<F16, true, false>(a, stream);
  }
  return a.bf16 ? launch_t<BF16, false, false>(a, stream) : launch_t<F16, false, false>(a, stream);
}

}  // namespace tvq
