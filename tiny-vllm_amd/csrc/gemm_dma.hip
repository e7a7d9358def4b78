// Instantiations of the LDS-DMA pipelined GEMM and the M/N-bucketed choice
// among them (used when M > 16 and K % 128 == 0).
//
// Table (measured on MI355X over the BASELINE shapes; tile = BM x BN, waves,
// ring depth S, MFMA shape):
//   W8A8  >= 256 256x256 tiles          256x256, 8 waves (2x4), S=2, 32x32x32 i8
//         >= 200 256x128 tiles          256x128, 8 waves (4x2), S=2, 32x32x32 i8
//         M > 256                        64x64,   4 waves,       S=4, 16x16x64 i8
//         32 < M <= 64, N >= 16384       64x128,  8 waves (2x4), S=4, 16x16x64 i8
//         otherwise                      32x64,   4 waves,       S=4, 16x16x64 i8
//   W8A16 >= 200 128x256 tiles          128x256, 8 waves (2x4), S=2, 32x32x16 bf16
//         M > 256                        64x128,  4 waves,       S=4, 32x32x16
//         32 < M <= 64, N >= 16384       64x128,  4 waves,       S=4, 32x32x16
//         M <= 64                        32x64,   4 waves,       S=4, 16x16x32 bf16
//         otherwise                      64x64,   4 waves,       S=4, 32x32x16
// For 16 < M <= 64 these tiles beat the skinny kernel, whose 16-channel
// workgroups re-read all M activation rows per workgroup (8x the weight
// traffic at M = 64).
// Large tiles amortize the LDS traffic, which bounds this loop: per 128-k
// stage a 2x4-wave 256x256 tile reads 192 KB of fragments and takes 64 KB of
// DMA writes against 2048 MFMA cycles per SIMD, i.e. ~128 B/clk, the CU's
// LDS rate. (Fewer, larger wave tiles need 1 wave/SIMD and measured slower.)
// Small tiles keep >= 256 workgroups in flight at decode-batch M.
#include "gemm_dma_kernel.h"
#include "tvq_internal.h"

namespace tvq {
namespace {

using dma::launch_dma;

enum class DmaCfg {
  kI8_256x256, kI8_256x128, kI8_64x64, kI8_64x128, kI8_32x64, kH_128x256, kH_64x128, kH_64x64, kH_32x64
};

int64_t tiles(int64_t M, int64_t N, int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); }

DmaCfg choose(bool w8a8, int64_t M, int64_t N) {
  if (w8a8) {
    if (tiles(M, N, 256, 256) >= 256) return DmaCfg::kI8_256x256;
    if (tiles(M, N, 256, 128) >= 200) return DmaCfg::kI8_256x128;
    if (M > 256) return DmaCfg::kI8_64x64;
    if (M > 32 && M <= 64 && N >= 16384) return DmaCfg::kI8_64x128;
    return DmaCfg::kI8_32x64;
  }
  if (tiles(M, N, 128, 256) >= 200) return DmaCfg::kH_128x256;
  if (M > 256) return DmaCfg::kH_64x128;
  if (M <= 64) return (M > 32 && N >= 16384) ? DmaCfg::kH_64x128 : DmaCfg::kH_32x64;
  return DmaCfg::kH_64x64;
}

// Workgroups that run together should share operand panels in L2: walk m
// inside groups of 8 n-tiles when the weights are the bigger operand, else
// walk n inside groups of 8 m-tiles.
int m_major(const GemmArgs& a) {
  const int64_t xbytes = a.M * a.K * (a.w8a8 ? 1 : 2);
  return a.N * a.K > xbytes ? 1 : 0;
}

template <typename T, bool kW8A8, bool kRaw>
hipError_t run(const GemmArgs& a, hipStream_t s) {
  const int M = (int)a.M, N = (int)a.N, K = (int)a.K, mm = m_major(a);
  const int8_t* q = a.qweight;
  if constexpr (kW8A8) {
    const auto* x = a.x;
    const auto* as = a.a_scales;
    switch (choose(true, a.M, a.N)) {
      case DmaCfg::kI8_256x256:
        return launch_dma<T, true, kRaw, 256, 256, 2, 4, 2, 32>(x, as, q, a.scales, a.bias, a.y, M, N, K, 8, mm, s);
      case DmaCfg::kI8_256x128:
        return launch_dma<T, true, kRaw, 256, 128, 4, 2, 2, 32>(x, as, q, a.scales, a.bias, a.y, M, N, K, 8, mm, s);
      case DmaCfg::kI8_64x64:
        return launch_dma<T, true, kRaw, 64, 64, 2, 2, 4, 16>(x, as, q, a.scales, a.bias, a.y, M, N, K, 8, mm, s);
      case DmaCfg::kI8_64x128:
        return launch_dma<T, true, kRaw, 64, 128, 2, 4, 4, 16>(x, as, q, a.scales, a.bias, a.y, M, N, K, 8, mm, s);
      default:
        return launch_dma<T, true, kRaw, 32, 64, 2, 2, 4, 16>(x, as, q, a.scales, a.bias, a.y, M, N, K, 8, mm, s);
    }
  } else {
    switch (choose(false, a.M, a.N)) {
      case DmaCfg::kH_128x256:
        return launch_dma<T, false, false, 128, 256, 2, 4, 2, 32>(a.x, nullptr, q, a.scales, a.bias, a.y, M, N, K, 8,
                                                                  mm, s);
      case DmaCfg::kH_64x128:
        return launch_dma<T, false, false, 64, 128, 2, 2, 4, 32>(a.x, nullptr, q, a.scales, a.bias, a.y, M, N, K, 8,
                                                                 mm, s);
      case DmaCfg::kH_32x64:
        return launch_dma<T, false, false, 32, 64, 2, 2, 4, 16>(a.x, nullptr, q, a.scales, a.bias, a.y, M, N, K, 8,
                                                                mm, s);
      default:
        return launch_dma<T, false, false, 64, 64, 2, 2, 4, 32>(a.x, nullptr, q, a.scales, a.bias, a.y, M, N, K, 8, mm,
                                                                s);
    }
  }
}

}  // namespace

bool dma_shape_ok(int64_t K) { return K % 128 == 0; }

const char* dma_path_name(bool w8a8, int64_t M, int64_t N) {
  switch (choose(w8a8, M, N)) {
    case DmaCfg::kI8_256x256: return "dma_mfma_i8_256x256";
    case DmaCfg::kI8_256x128: return "dma_mfma_i8_256x128";
    case DmaCfg::kI8_64x64: return "dma_mfma_i8_64x64";
    case DmaCfg::kI8_64x128: return "dma_mfma_i8_64x128";
    case DmaCfg::kI8_32x64: return "dma_mfma_i8_32x64";
    case DmaCfg::kH_128x256: return "dma_mfma_f16x_128x256";
    case DmaCfg::kH_64x128: return "dma_mfma_f16x_64x128";
    case DmaCfg::kH_32x64: return "dma_mfma_f16x_32x64";
    default: return "dma_mfma_f16x_64x64";
  }
}

hipError_t launch_dma_gemm(const GemmArgs& a, hipStream_t stream) {
  if (a.w8a8) {
    if (a.raw_i32) return run<BF16, true, true>(a, stream);
    return a.bf16 ? run<BF16, true, false>(a, stream) : run<F16, true, false>(a, stream);
  }
  return a.bf16 ? run<BF16, false, false>(a, stream) : run<F16, false, false>(a, stream);
}

}  // namespace tvq
