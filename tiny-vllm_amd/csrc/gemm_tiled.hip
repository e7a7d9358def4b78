// Tiled (prefill-size M) W8A16 / W8A8 GEMM for gfx950.
//
// C^T tile = Wq_tile (BN x K, MFMA "A" side) x X_tile^T (BM x K, "B" side).
// Putting output channels on the A side makes each lane hold 4 consecutive
// output channels of one token in the accumulator, i.e. one 8-byte store of
// y[m, n..n+3].
//
// Workgroup: 256 threads = 4 waves in a 2 (n) x 2 (m) grid, each wave owning
// a (BN/2) x (BM/2) block of 16x16 MFMA tiles. Per K step the workgroup
// stages a BN x BK int8 weight tile and a BM x BK activation tile (int8 for
// W8A8, bf16/fp16 for W8A16) in LDS, double buffered: global loads for step
// t+1 are issued before the MFMAs of step t and written to the other buffer
// after them, so there is one barrier per K step. LDS rows are padded by 16
// bytes so the 16-lane fragment reads (16 rows, same column) hit distinct
// banks.
//
// W8A8  : v_mfma_i32_16x16x64_i8, exact int32 accumulation; epilogue
//         (float(acc)*a_s[m])*w_s[n] + b[n] -> bf16/fp16.
// W8A16 : int8 weight fragments are converted to bf16/fp16 in registers after
//         the LDS read (exact) and feed v_mfma_f32_16x16x32_{bf16,f16}; the
//         weight tile therefore occupies LDS as int8 (half the bytes of a
//         dequantized tile) and is never re-dequantized per M tile in memory.
//         Epilogue acc*s[n] + b[n].
//
// Tiles are assigned XCD-aware: hardware places workgroup b on XCD b % 8, so
// logical tile ids are remapped to give each XCD a contiguous run of tiles
// (n fastest), keeping the activation panel of those tiles in that XCD's L2.
#include <type_traits>

#include "tvq_common.h"
#include "tvq_internal.h"

namespace tvq {
namespace {

constexpr int kXcds = 8;

template <bool kW8A8, int BM, int BN, int BK>
struct TileCfg {
  static constexpr int kXBytes = kW8A8 ? 1 : 2;       // bytes per activation element
  static constexpr int kWRow = BK + 16;               // LDS row stride, weight tile (bytes)
  static constexpr int kXRow = BK * kXBytes + 16;     // LDS row stride, activation tile (bytes)
  static constexpr int kWStage = BN * kWRow;
  static constexpr int kXStage = BM * kXRow;
  static constexpr int kStage = kWStage + kXStage;
  static constexpr int kWChunks = BN * BK / 16;       // 16-byte chunks per stage
  static constexpr int kXChunks = BM * BK * kXBytes / 16;
  static constexpr int kWPerThr = kWChunks / 256;
  static constexpr int kXPerThr = kXChunks / 256;
  static constexpr int kWChunksPerRow = BK / 16;
  static constexpr int kXChunksPerRow = BK * kXBytes / 16;
  static constexpr int FN = BN / 2 / 16;  // 16-row MFMA tiles per wave along n
  static constexpr int FM = BM / 2 / 16;  // along m
  static_assert(kWChunks % 256 == 0 && kXChunks % 256 == 0, "tile must split evenly over 256 threads");
  static_assert(BK % 64 == 0, "BK must be a multiple of 64");
};

template <typename T, bool kW8A8, bool kRaw, int BM, int BN, int BK>
__global__ __launch_bounds__(256) void tiled_kernel(const void* __restrict__ xv, const float* __restrict__ a_scales,
                                                    const int8_t* __restrict__ qw, const float* __restrict__ ws,
                                                    const uint16_t* __restrict__ bias, void* __restrict__ yv, int M,
                                                    int N, int K) {
  using C = TileCfg<kW8A8, BM, BN, BK>;
  using Acc = typename std::conditional<kW8A8, i32x4, f32x4>::type;
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int wn = wave & 1;
  const int wm = wave >> 1;

  // XCD-aware tile order.
  const int tiles_n = (N + BN - 1) / BN;
  const int tiles_m = (M + BM - 1) / BM;
  const int total = tiles_n * tiles_m;
  int bid = blockIdx.x;
  if (total % kXcds == 0) bid = (bid % kXcds) * (total / kXcds) + bid / kXcds;
  const int tn = bid % tiles_n;
  const int tm = bid / tiles_n;
  const int n0 = tn * BN;
  const int m0 = tm * BM;

  const int64_t xrow_bytes = (int64_t)K * C::kXBytes;
  const char* xbase = static_cast<const char*>(xv);

  // Global->register staging, one 16-byte chunk per slot.
  u32x4 wreg[C::kWPerThr];
  u32x4 xreg[C::kXPerThr];

  auto gload = [&](int k0) {
#pragma unroll
    for (int s = 0; s < C::kWPerThr; ++s) {
      const int c = tid + 256 * s;
      const int row = c / C::kWChunksPerRow;
      const int col = c % C::kWChunksPerRow;
      const int n = n0 + row;
      const int k = k0 + col * 16;
      wreg[s] = (n < N && k < K) ? ldg128(qw + (int64_t)n * K + k) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int s = 0; s < C::kXPerThr; ++s) {
      const int c = tid + 256 * s;
      const int row = c / C::kXChunksPerRow;
      const int col = c % C::kXChunksPerRow;
      const int m = m0 + row;
      const int64_t kb = (int64_t)k0 * C::kXBytes + col * 16;
      xreg[s] = (m < M && kb < xrow_bytes) ? ldg128(xbase + (int64_t)m * xrow_bytes + kb) : u32x4{0, 0, 0, 0};
    }
  };
  auto lstore = [&](int stage) {
    char* wl = smem + stage * C::kStage;
    char* xl = wl + C::kWStage;
#pragma unroll
    for (int s = 0; s < C::kWPerThr; ++s) {
      const int c = tid + 256 * s;
      const int row = c / C::kWChunksPerRow;
      const int col = c % C::kWChunksPerRow;
      *reinterpret_cast<u32x4*>(wl + row * C::kWRow + col * 16) = wreg[s];
    }
#pragma unroll
    for (int s = 0; s < C::kXPerThr; ++s) {
      const int c = tid + 256 * s;
      const int row = c / C::kXChunksPerRow;
      const int col = c % C::kXChunksPerRow;
      *reinterpret_cast<u32x4*>(xl + row * C::kXRow + col * 16) = xreg[s];
    }
  };

  Acc acc[C::FN][C::FM];
#pragma unroll
  for (int i = 0; i < C::FN; ++i)
#pragma unroll
    for (int j = 0; j < C::FM; ++j) acc[i][j] = Acc{0, 0, 0, 0};

  const int nk = (K + BK - 1) / BK;
  gload(0);
  lstore(0);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) gload((kt + 1) * BK);

    const char* wl = smem + cur * C::kStage + (wn * (BN / 2) + r) * C::kWRow + 16 * g;
    const char* xl = smem + cur * C::kStage + C::kWStage + (wm * (BM / 2) + r) * C::kXRow;
#pragma unroll
    for (int ks = 0; ks < BK / 64; ++ks) {
      u32x4 a[C::FN];
#pragma unroll
      for (int i = 0; i < C::FN; ++i) a[i] = *reinterpret_cast<const u32x4*>(wl + i * 16 * C::kWRow + ks * 64);
      if constexpr (kW8A8) {
#pragma unroll
        for (int j = 0; j < C::FM; ++j) {
          const u32x4 b = *reinterpret_cast<const u32x4*>(xl + j * 16 * C::kXRow + ks * 64 + 16 * g);
#pragma unroll
          for (int i = 0; i < C::FN; ++i) acc[i][j] = mfma16x16x64_i8(a[i], b, acc[i][j]);
        }
      } else {
        u32x4 alo[C::FN], ahi[C::FN];
#pragma unroll
        for (int i = 0; i < C::FN; ++i) {
          const u32x2 c0 = i8x4_to_16x4<T>(a[i][0]);
          const u32x2 c1 = i8x4_to_16x4<T>(a[i][1]);
          const u32x2 c2 = i8x4_to_16x4<T>(a[i][2]);
          const u32x2 c3 = i8x4_to_16x4<T>(a[i][3]);
          alo[i] = u32x4{c0.x, c0.y, c1.x, c1.y};
          ahi[i] = u32x4{c2.x, c2.y, c3.x, c3.y};
        }
#pragma unroll
        for (int j = 0; j < C::FM; ++j) {
          const char* xp = xl + j * 16 * C::kXRow + ks * 128 + 32 * g;
          const u32x4 b0 = *reinterpret_cast<const u32x4*>(xp);
          const u32x4 b1 = *reinterpret_cast<const u32x4*>(xp + 16);
#pragma unroll
          for (int i = 0; i < C::FN; ++i) {
            acc[i][j] = mfma16x16x32<T>(alo[i], b0, acc[i][j]);
            acc[i][j] = mfma16x16x32<T>(ahi[i], b1, acc[i][j]);
          }
        }
      }
    }

    if (more) lstore(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds y[m, nb..nb+3] for each (i, j).
#pragma unroll
  for (int j = 0; j < C::FM; ++j) {
    const int m = m0 + wm * (BM / 2) + 16 * j + r;
    if (m >= M) continue;
    float as = 0.0f;
    if constexpr (kW8A8 && !kRaw) as = a_scales[m];
#pragma unroll
    for (int i = 0; i < C::FN; ++i) {
      const int nb = n0 + wn * (BN / 2) + 16 * i + 4 * g;
      const Acc v = acc[i][j];
      if constexpr (kRaw) {
        int32_t* y = static_cast<int32_t*>(yv) + (int64_t)m * N;
        if (nb + 3 < N && (N & 3) == 0) {
          *reinterpret_cast<i32x4*>(y + nb) = v;
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            if (nb + t < N) y[nb + t] = v[t];
        }
      } else {
        uint16_t* y = static_cast<uint16_t*>(yv) + (int64_t)m * N;
        float o[4];
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
}

template <typename T, bool kW8A8, bool kRaw, int BM, int BN, int BK>
hipError_t launch_cfg(const GemmArgs& a, hipStream_t stream) {
  using C = TileCfg<kW8A8, BM, BN, BK>;
  auto kern = tiled_kernel<T, kW8A8, kRaw, BM, BN, BK>;
  const size_t lds = 2 * (size_t)C::kStage;
  static bool attr_set = false;  // benign race: idempotent attribute set
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int64_t tiles = ((a.N + BN - 1) / BN) * ((a.M + BM - 1) / BM);
  kern<<<dim3((unsigned)tiles), dim3(256), lds, stream>>>(a.x, a.a_scales, a.qweight, a.scales,
                                                          static_cast<const uint16_t*>(a.bias), a.y, (int)a.M,
                                                          (int)a.N, (int)a.K);
  return hipGetLastError();
}

template <typename T, bool kW8A8, bool kRaw>
hipError_t launch_t(const GemmArgs& a, hipStream_t stream) {
  if constexpr (kW8A8)
    return launch_cfg<T, kW8A8, kRaw, 128, 128, 128>(a, stream);
  else
    return launch_cfg<T, kW8A8, kRaw, 128, 128, 64>(a, stream);
}

}  // namespace

hipError_t launch_tiled(const GemmArgs& a, hipStream_t stream) {
  if (a.w8a8) {
    if (a.raw_i32) return launch_t<BF16, true, true>(a, stream);
    return a.bf16 ? launch_t<BF16, true, false>(a, stream) : launch_t<F16, true, false>(a, stream);
  }
  return a.bf16 ? launch_t<BF16, false, false>(a, stream) : launch_t<F16, false, false>(a, stream);
}

}  // namespace tvq
