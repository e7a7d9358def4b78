// Instantiations of the LDS-DMA pipelined GEMM and the M/N/K-bucketed choice
// among them (used when M > 16 and K % 128 == 0).
//
// Table (measured on MI355X over the BASELINE shapes; tile = BM x BN, waves,
// ring depth S, MFMA shape):
//   W8A8  >= 256 256x256 tiles          256x256, 8 waves (2x4), S=2, 32x32x32 i8
//         >= 200 256x128 tiles          256x128, 8 waves (4x2), S=3, 32x32x32 i8 (one tile per CU
//                                        at N = 1024: nothing else hides the stage latency)
//         M > 256, or split-K M > 32,    64x64,   4 waves,       S=4, 16x16x64 i8
//         or 64 < M with >= 256 such tiles
//         32 < M <= 64, N >= 16384       64x128,  8 waves (2x4), S=4, 16x16x64 i8
//         otherwise                      32x64,   4 waves,       S=4, 16x16x64 i8
//   W8A16 >= 200 128x256 tiles          128x256, 8 waves (2x4), S=2, 32x32x16 bf16
//         M > 256                        64x128,  4 waves,       S=4, 32x32x16
//         split-K M > 32                 64x64,   4 waves,       S=4, 32x32x16
//         32 < M <= 64, N >= 16384       64x128,  8 waves (2x4), S=4, 16x16x32 (30 % faster
//                                        than 4 waves of 32x32x16 at the 8B gate_up shape)
//         M <= 64                        32x64,   4 waves,       S=4, 16x16x32 bf16
//         otherwise                      64x64,   4 waves,       S=4, 32x32x16
// Stream-K (TVQ_STREAMK=1, M <= 64): W8A8 64x128 (M > 32) / 32x64; W8A16
// 64x256 (M > 32), 32x256 (M > 16), 16x128 (M <= 16).
// For 16 < M <= 64 these tiles beat the skinny kernel, whose 16-channel
// workgroups re-read all M activation rows per workgroup (8x the weight
// traffic at M = 64).
// Large tiles amortize the LDS traffic, which bounds this loop: per 128-k
// stage a 2x4-wave 256x256 tile reads 192 KB of fragments and takes 64 KB of
// DMA writes against 2048 MFMA cycles per SIMD, i.e. ~128 B/clk, the CU's
// LDS rate. (Fewer, larger wave tiles need 1 wave/SIMD and measured slower.)
// Split-K: decode-size shapes (M <= 64, N < 16384, K >= 2048) leave most CUs
// idle with whole-K tiles (e.g. 64 tiles of 64x64 for N = 4096), so with a
// caller workspace they split K into up to CUs/tiles ranges of >= 8 stages,
// one work unit per CU (e.g. 8B down_proj at M = 64: 49 -> 22 us W8A16).
#include <stdlib.h>

#include "gemm_dma_kernel.h"
#include "tvq_internal.h"

namespace tvq {
namespace {

using dma::launch_dma;

enum class DmaCfg {
  kI8_256x256, kI8_256x128, kI8_64x64, kI8_64x128, kI8_32x64, kH_128x256, kH_64x128, kH_64x64, kH_32x64, kH_64x128w8,
  kI8_256x256w4, kH_128x256w4, kH_16x128, kH_64x256, kH_32x256
};

// Tile BM x BN, waves WM x WN, ring depth S, MFMA tile MF, per DmaCfg.
struct CfgInfo {
  bool w8a8;
  int bm, bn, wm, wn, s, mf, ks;  // ks: k values per ring stage
  const char* name;
  const char* name_split;  // the same tiles with K split over several workgroups
  const char* name_streamk;  // the same tiles with stream-K (equal k-stage shares per CU)
};
constexpr CfgInfo kInfo[] = {
    {true, 256, 256, 2, 4, 2, 32, 128, "dma_mfma_i8_256x256", "dma_mfma_i8_256x256_splitk",
     "dma_mfma_i8_256x256_streamk"},
    {true, 256, 128, 4, 2, 3, 32, 128, "dma_mfma_i8_256x128", "dma_mfma_i8_256x128_splitk",
     "dma_mfma_i8_256x128_streamk"},
    {true, 64, 64, 2, 2, 4, 16, 128, "dma_mfma_i8_64x64", "dma_mfma_i8_64x64_splitk",
     "dma_mfma_i8_64x64_streamk"},
    {true, 64, 128, 2, 4, 4, 16, 128, "dma_mfma_i8_64x128", "dma_mfma_i8_64x128_splitk",
     "dma_mfma_i8_64x128_streamk"},
    {true, 32, 64, 2, 2, 4, 16, 128, "dma_mfma_i8_32x64", "dma_mfma_i8_32x64_splitk",
     "dma_mfma_i8_32x64_streamk"},
    {false, 128, 256, 2, 4, 2, 32, 128, "dma_mfma_f16x_128x256", "dma_mfma_f16x_128x256_splitk",
     "dma_mfma_f16x_128x256_streamk"},
    {false, 64, 128, 2, 2, 4, 32, 128, "dma_mfma_f16x_64x128", "dma_mfma_f16x_64x128_splitk",
     "dma_mfma_f16x_64x128_streamk"},
    {false, 64, 64, 2, 2, 4, 32, 128, "dma_mfma_f16x_64x64", "dma_mfma_f16x_64x64_splitk",
     "dma_mfma_f16x_64x64_streamk"},
    {false, 32, 64, 2, 2, 4, 16, 128, "dma_mfma_f16x_32x64", "dma_mfma_f16x_32x64_splitk",
     "dma_mfma_f16x_32x64_streamk"},
    {false, 64, 128, 2, 4, 4, 16, 128, "dma_mfma_f16x_64x128w8", "dma_mfma_f16x_64x128w8_splitk",
     "dma_mfma_f16x_64x128w8_streamk"},
    // Prefill tiles of 4 waves with 4x4 fragments of 32x32 each (TVQ_PREFILL_W4=1): fewer LDS fragment
    // reads per MFMA (8 per 16 instead of 6 per 8), one wave per SIMD, 64-k stages
    {true, 256, 256, 2, 2, 4, 32, 64, "dma_mfma_i8_256x256w4", "dma_mfma_i8_256x256w4_splitk",
     "dma_mfma_i8_256x256w4_streamk"},
    {false, 128, 256, 2, 2, 4, 32, 64, "dma_mfma_f16x_128x256w4", "dma_mfma_f16x_128x256w4_splitk",
     "dma_mfma_f16x_128x256w4_streamk"},
    // W8A16 at M <= 16 under stream-K: one 16-token row of MFMA blocks, so the
    // activation panel is a quarter of the weight bytes (2 * 16 / 128)
    {false, 16, 128, 1, 4, 4, 16, 128, "dma_mfma_f16x_16x128", "dma_mfma_f16x_16x128_splitk",
     "dma_mfma_f16x_16x128_streamk"},
    // W8A16 at 16 < M <= 64 under stream-K: 256 output channels per tile, so
    // the bf16 activation panel a tile re-reads is half (M = 64) or a quarter
    // (M = 32) of its weight bytes, where the 64x128 tile reads as many
    // activation bytes as weight bytes; 48 / 40 KB stages, 3-deep ring
    {false, 64, 256, 2, 4, 3, 16, 128, "dma_mfma_f16x_64x256", "dma_mfma_f16x_64x256_splitk",
     "dma_mfma_f16x_64x256_streamk"},
    {false, 32, 256, 2, 4, 3, 16, 128, "dma_mfma_f16x_32x256", "dma_mfma_f16x_32x256_splitk",
     "dma_mfma_f16x_32x256_streamk"},
};

static_assert(sizeof(kInfo) / sizeof(kInfo[0]) == (int)DmaCfg::kH_32x256 + 1, "one entry per DmaCfg");
static_assert(kInfo[(int)DmaCfg::kI8_32x64].bm == 32 && kInfo[(int)DmaCfg::kH_128x256].bn == 256 &&
                  !kInfo[(int)DmaCfg::kH_64x64].w8a8 && kInfo[(int)DmaCfg::kI8_64x128].bn == 128,
              "kInfo follows the DmaCfg order");

template <DmaCfg c>
constexpr CfgInfo info() {
  return kInfo[(int)c];
}

// Tiles with BM <= 64 (decode-size M) may split K.
template <DmaCfg c>
constexpr bool splittable() {
  return info<c>().bm <= 64;
}

int64_t tiles(int64_t M, int64_t N, int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); }

// Decode-size shapes whose tiles cannot fill the GPU split K (given a
// workspace): M <= 64, fewer than 16384 output channels, K >= 2048.
bool split_shape(int64_t M, int64_t N, int64_t K) { return M <= 64 && N < 16384 && K >= 2048; }

// Stream-K for decode-size M (TVQ_STREAMK=1): every CU takes an equal share
// of the tiles' k-stages (gemm_dma_kernel.h), so shapes whose tile count is
// not a multiple of the CU count (e.g. 192 tiles of 64x128 on 256 CUs at the
// 8B gate_up) keep every CU's weight stream busy. It needs a workspace of
// two accumulator images per workgroup.
bool streamk_shape(int64_t M) { return M <= 64 && switches().streamk; }

// TVQ_PREFILL_W4=1: the 4-wave prefill tiles in place of the 8-wave 256x256
// (W8A8) and 128x256 (W8A16) ones.
bool prefill_w4() { return switches().prefill_w4; }

#ifdef TVQ_TEST_HOOKS
// CPU-emulation builds of the tests only (never defined for the GPU library):
// a DmaCfg index that choose() returns for its own family, so that every tile
// configuration can be exercised at small shapes.
extern "C" int tvq_test_force_dma_cfg;
int tvq_test_force_dma_cfg = -1;
#endif

// opt_in: whether the opt-in switches (TVQ_STREAMK, TVQ_PREFILL_W4) may
// change the tile; the rounded-dequant mode keeps the default tiles.
DmaCfg choose(bool w8a8, int64_t M, int64_t N, int64_t K, bool opt_in = true) {
#ifdef TVQ_TEST_HOOKS
  if (tvq_test_force_dma_cfg >= 0 && kInfo[tvq_test_force_dma_cfg].w8a8 == w8a8)
    return (DmaCfg)tvq_test_force_dma_cfg;
#endif
  if (opt_in && streamk_shape(M)) {
    // the widest decode tiles: activation traffic per weight byte 2M/BN (W8A16), M/BN (W8A8)
    if (w8a8) return M > 32 ? DmaCfg::kI8_64x128 : DmaCfg::kI8_32x64;
    return M > 32 ? DmaCfg::kH_64x256 : (M > 16 ? DmaCfg::kH_32x256 : DmaCfg::kH_16x128);
  }
  const bool split = split_shape(M, N, K);
  if (w8a8) {
    if (tiles(M, N, 256, 256) >= 256) return opt_in && prefill_w4() ? DmaCfg::kI8_256x256w4 : DmaCfg::kI8_256x256;
    if (tiles(M, N, 256, 128) >= 200) return DmaCfg::kI8_256x128;
    if (M > 256 || (split && M > 32)) return DmaCfg::kI8_64x64;
    if (M > 32 && M <= 64 && N >= 16384) return DmaCfg::kI8_64x128;
    // 64 < M <= 256: 64x64 tiles once they alone fill the 256 CUs (each
    // weight panel then streams through L2 to M/64 tiles instead of M/32;
    // headline M = 256: 6.19 -> 6.04 us)
    if (M > 64 && tiles(M, N, 64, 64) >= 256) return DmaCfg::kI8_64x64;
    return DmaCfg::kI8_32x64;
  }
  if (tiles(M, N, 128, 256) >= 200) return opt_in && prefill_w4() ? DmaCfg::kH_128x256w4 : DmaCfg::kH_128x256;
  if (M > 256) return DmaCfg::kH_64x128;
  if (M <= 64) {
    if (split && M > 32) return DmaCfg::kH_64x64;
    return (M > 32 && N >= 16384) ? DmaCfg::kH_64x128w8 : DmaCfg::kH_32x64;
  }
  return DmaCfg::kH_64x64;
}

// Workgroups that run together should share operand panels in L2: walk m
// inside groups of 8 n-tiles when the weights are the bigger operand, else
// walk n inside groups of 8 m-tiles.
int m_major(const GemmArgs& a) {
  const int64_t xbytes = a.M * a.K * (a.w8a8 ? 1 : 2);
  return a.N * a.K > xbytes ? 1 : 0;
}

// Stream-K range length for configuration c (0: no stream-K launch).
template <DmaCfg c>
int streamk_len(int64_t M, int64_t N, int64_t K, const void* ws, int64_t ws_bytes) {
  if constexpr (!splittable<c>()) {
    return 0;
  } else {
    if (!streamk_shape(M)) return 0;
    constexpr CfgInfo i = info<c>();
    int grid = 0;
    return dma::choose_streamk((int)tiles(M, N, i.bm, i.bn), (int)(K / i.ks), dma::device_cus(), i.bm * i.bn * 4, ws,
                               ws_bytes, &grid);
  }
}

template <DmaCfg c>
int splits_of(int64_t M, int64_t N, int64_t K, const void* ws, int64_t ws_bytes) {
  if constexpr (!splittable<c>()) {
    return 1;
  } else {
    if (!split_shape(M, N, K)) return 1;
    constexpr CfgInfo i = info<c>();
    return dma::choose_splits((int)tiles(M, N, i.bm, i.bn), (int)(K / i.ks), dma::device_cus(), i.bm * i.bn * 4, ws,
                              ws_bytes);
  }
}

int splits_for(DmaCfg c, int64_t M, int64_t N, int64_t K, const void* ws, int64_t ws_bytes) {
  switch (c) {
#define TVQ_CASE(C) \
  case DmaCfg::C: return splits_of<DmaCfg::C>(M, N, K, ws, ws_bytes);
    TVQ_CASE(kI8_256x256) TVQ_CASE(kI8_256x128) TVQ_CASE(kI8_64x64) TVQ_CASE(kI8_64x128) TVQ_CASE(kI8_32x64)
    TVQ_CASE(kH_128x256) TVQ_CASE(kH_64x128) TVQ_CASE(kH_64x64) TVQ_CASE(kH_32x64) TVQ_CASE(kH_64x128w8)
    TVQ_CASE(kI8_256x256w4) TVQ_CASE(kH_128x256w4) TVQ_CASE(kH_16x128) TVQ_CASE(kH_64x256) TVQ_CASE(kH_32x256)
#undef TVQ_CASE
  }
  return 1;
}

int streamk_for(DmaCfg c, int64_t M, int64_t N, int64_t K, const void* ws, int64_t ws_bytes) {
  switch (c) {
#define TVQ_CASE(C) \
  case DmaCfg::C: return streamk_len<DmaCfg::C>(M, N, K, ws, ws_bytes);
    TVQ_CASE(kI8_256x256) TVQ_CASE(kI8_256x128) TVQ_CASE(kI8_64x64) TVQ_CASE(kI8_64x128) TVQ_CASE(kI8_32x64)
    TVQ_CASE(kH_128x256) TVQ_CASE(kH_64x128) TVQ_CASE(kH_64x64) TVQ_CASE(kH_32x64) TVQ_CASE(kH_64x128w8)
    TVQ_CASE(kI8_256x256w4) TVQ_CASE(kH_128x256w4) TVQ_CASE(kH_16x128) TVQ_CASE(kH_64x256) TVQ_CASE(kH_32x256)
#undef TVQ_CASE
  }
  return 0;
}

template <typename T, bool kRaw, DmaCfg c>
hipError_t go(const GemmArgs& a, hipStream_t s) {
  constexpr CfgInfo i = info<c>();
  const int splits = splits_for(c, a.M, a.N, a.K, a.workspace, a.workspace_bytes);
  // Unsplit launches use the instantiation without the split-K fixup (fewer
  // registers; measured ~4 % faster on the M=256 headline shape).
  if constexpr (splittable<c>()) {
    if (streamk_for(c, a.M, a.N, a.K, a.workspace, a.workspace_bytes) > 0)
      return launch_dma<T, i.w8a8, kRaw, i.bm, i.bn, i.wm, i.wn, i.s, i.mf, i.ks, true, i.w8a8, false, false, false,
                        false, true>(a.x, a.a_scales, a.qweight, a.scales, a.bias, a.y, (int)a.M, (int)a.N, (int)a.K,
                                     8, m_major(a), 1, a.workspace, a.workspace_bytes, s);
    // W8A8 at decode-size M (<= 64, one or two m-tiles): each weight byte is
    // read by at most two workgroups, so the weight stream takes the
    // non-temporal hint
    // (measured 2-5 % on the decode shapes; W8A16 gained nothing).
    constexpr bool kNt = i.w8a8;
    if (splits > 1)
      return launch_dma<T, i.w8a8, kRaw, i.bm, i.bn, i.wm, i.wn, i.s, i.mf, i.ks, true, kNt>(
          a.x, a.a_scales, a.qweight, a.scales, a.bias, a.y, (int)a.M, (int)a.N, (int)a.K, 8, m_major(a), splits,
          a.workspace, a.workspace_bytes, s);
    if (kNt && a.M <= 64)
      return launch_dma<T, i.w8a8, kRaw, i.bm, i.bn, i.wm, i.wn, i.s, i.mf, i.ks, false, kNt>(
          a.x, a.a_scales, a.qweight, a.scales, a.bias, a.y, (int)a.M, (int)a.N, (int)a.K, 8, m_major(a), 1, nullptr,
          0, s);
  }
  return launch_dma<T, i.w8a8, kRaw, i.bm, i.bn, i.wm, i.wn, i.s, i.mf, i.ks, false>(
      a.x, a.a_scales, a.qweight, a.scales, a.bias, a.y, (int)a.M, (int)a.N, (int)a.K, 8, m_major(a), 1, nullptr, 0,
      s);
}

template <typename T, bool kW8A8, bool kRaw>
hipError_t run(const GemmArgs& a, hipStream_t s) {
  if constexpr (kW8A8) {
    switch (choose(true, a.M, a.N, a.K)) {
      case DmaCfg::kI8_256x256: return go<T, kRaw, DmaCfg::kI8_256x256>(a, s);
      case DmaCfg::kI8_256x256w4: return go<T, kRaw, DmaCfg::kI8_256x256w4>(a, s);
      case DmaCfg::kI8_256x128: return go<T, kRaw, DmaCfg::kI8_256x128>(a, s);
      case DmaCfg::kI8_64x64: return go<T, kRaw, DmaCfg::kI8_64x64>(a, s);
      case DmaCfg::kI8_64x128: return go<T, kRaw, DmaCfg::kI8_64x128>(a, s);
      default: return go<T, kRaw, DmaCfg::kI8_32x64>(a, s);
    }
  } else {
    switch (choose(false, a.M, a.N, a.K)) {
      case DmaCfg::kH_128x256: return go<T, false, DmaCfg::kH_128x256>(a, s);
      case DmaCfg::kH_128x256w4: return go<T, false, DmaCfg::kH_128x256w4>(a, s);
      case DmaCfg::kH_16x128: return go<T, false, DmaCfg::kH_16x128>(a, s);
      case DmaCfg::kH_64x256: return go<T, false, DmaCfg::kH_64x256>(a, s);
      case DmaCfg::kH_32x256: return go<T, false, DmaCfg::kH_32x256>(a, s);
      case DmaCfg::kH_64x128: return go<T, false, DmaCfg::kH_64x128>(a, s);
      case DmaCfg::kH_32x64: return go<T, false, DmaCfg::kH_32x64>(a, s);
      case DmaCfg::kH_64x128w8: return go<T, false, DmaCfg::kH_64x128w8>(a, s);
      default: return go<T, false, DmaCfg::kH_64x64>(a, s);
    }
  }
}

}  // namespace

bool dma_streamk_on(int64_t M) { return streamk_shape(M); }

// K % 128 == 0 (whole stages), and K <= 2^22 so that every per-lane DMA
// source offset (tile row x row bytes + stage offset, at most 256 x 2K bytes)
// fits the unsigned 32-bit lane offset of the saddr-form loads.
bool dma_shape_ok(int64_t K) { return K % 128 == 0 && K <= (int64_t(1) << 22); }

int dma_splits(bool w8a8, int64_t M, int64_t N, int64_t K, int64_t workspace_bytes) {
  static char probe;  // any non-null address: only the size is consulted
  return splits_for(choose(w8a8, M, N, K), M, N, K, workspace_bytes > 0 ? &probe : nullptr, workspace_bytes);
}

const char* dma_path_name(bool w8a8, int64_t M, int64_t N, int64_t K, int64_t workspace_bytes) {
  static char probe;
  const DmaCfg c = choose(w8a8, M, N, K);
  const CfgInfo& i = kInfo[(int)c];
  if (streamk_for(c, M, N, K, workspace_bytes > 0 ? &probe : nullptr, workspace_bytes) > 0) return i.name_streamk;
  return dma_splits(w8a8, M, N, K, workspace_bytes) > 1 ? i.name_split : i.name;
}

// W8A8 gate_up with the SiLU-and-mul epilogue (gate/up rows interleaved in
// 32-row blocks; y is [M, N/2]): the 256x256 tiles, whose wave tiles hold
// one 32-column gate block and its up block.
hipError_t launch_dma_glu(const GemmArgs& a, hipStream_t stream) {
  constexpr CfgInfo i = info<DmaCfg::kI8_256x256>();
  if (a.bf16)
    return launch_dma<BF16, true, false, i.bm, i.bn, i.wm, i.wn, i.s, i.mf, i.ks, false, false, true>(
        a.x, a.a_scales, a.qweight, a.scales, nullptr, a.y, (int)a.M, (int)a.N, (int)a.K, 8, m_major(a), 1, nullptr, 0,
        stream);
  return launch_dma<F16, true, false, i.bm, i.bn, i.wm, i.wn, i.s, i.mf, i.ks, false, false, true>(
      a.x, a.a_scales, a.qweight, a.scales, nullptr, a.y, (int)a.M, (int)a.N, (int)a.K, 8, m_major(a), 1, nullptr, 0,
      stream);
}

namespace {

// The operand-delivery floor of configuration c: the kernel with kDmaOnly,
// unsplit, with the weight-stream hint the real launch uses.
template <DmaCfg c>
hipError_t floor_of(const GemmArgs& a, hipStream_t s) {
  constexpr CfgInfo i = info<c>();
  if (i.w8a8 && a.M <= 64)
    return launch_dma<BF16, i.w8a8, false, i.bm, i.bn, i.wm, i.wn, i.s, i.mf, i.ks, false, true, false, false, true>(
        a.x, nullptr, a.qweight, nullptr, nullptr, nullptr, (int)a.M, (int)a.N, (int)a.K, 8, m_major(a), 1, nullptr,
        0, s);
  return launch_dma<BF16, i.w8a8, false, i.bm, i.bn, i.wm, i.wn, i.s, i.mf, i.ks, false, false, false, false, true>(
      a.x, nullptr, a.qweight, nullptr, nullptr, nullptr, (int)a.M, (int)a.N, (int)a.K, 8, m_major(a), 1, nullptr, 0,
      s);
}

}  // namespace

// W8A16 with the reference's rounded dequantization (kDq), unsplit.
template <typename T, DmaCfg c>
hipError_t dq_of(const GemmArgs& a, hipStream_t s) {
  constexpr CfgInfo i = info<c>();
  return launch_dma<T, false, false, i.bm, i.bn, i.wm, i.wn, i.s, i.mf, i.ks, false, false, false, false, false, true>(
      a.x, nullptr, a.qweight, a.scales, a.bias, a.y, (int)a.M, (int)a.N, (int)a.K, 8, m_major(a), 1, nullptr, 0, s);
}

template <typename T>
hipError_t dq_t(const GemmArgs& a, hipStream_t s) {
  switch (choose(false, a.M, a.N, a.K, /*opt_in=*/false)) {
    case DmaCfg::kH_128x256: return dq_of<T, DmaCfg::kH_128x256>(a, s);
    case DmaCfg::kH_64x128: return dq_of<T, DmaCfg::kH_64x128>(a, s);
    case DmaCfg::kH_32x64: return dq_of<T, DmaCfg::kH_32x64>(a, s);
    case DmaCfg::kH_64x128w8: return dq_of<T, DmaCfg::kH_64x128w8>(a, s);
    default: return dq_of<T, DmaCfg::kH_64x64>(a, s);
  }
}

hipError_t launch_dma_dq(const GemmArgs& a, hipStream_t stream) {
  return a.bf16 ? dq_t<BF16>(a, stream) : dq_t<F16>(a, stream);
}

hipError_t launch_dma_floor(const GemmArgs& a, hipStream_t stream) {
  switch (choose(a.w8a8, a.M, a.N, a.K)) {
#define TVQ_CASE(C) \
  case DmaCfg::C: return floor_of<DmaCfg::C>(a, stream);
    TVQ_CASE(kI8_256x256) TVQ_CASE(kI8_256x128) TVQ_CASE(kI8_64x64) TVQ_CASE(kI8_64x128) TVQ_CASE(kI8_32x64)
    TVQ_CASE(kH_128x256) TVQ_CASE(kH_64x128) TVQ_CASE(kH_64x64) TVQ_CASE(kH_32x64) TVQ_CASE(kH_64x128w8)
    TVQ_CASE(kI8_256x256w4) TVQ_CASE(kH_128x256w4) TVQ_CASE(kH_16x128) TVQ_CASE(kH_64x256) TVQ_CASE(kH_32x256)
#undef TVQ_CASE
  }
  return hipErrorInvalidValue;
}

hipError_t launch_dma_gemm(const GemmArgs& a, hipStream_t stream) {
  if (a.w8a8) {
    if (a.raw_i32) return run<BF16, true, true>(a, stream);
    return a.bf16 ? run<BF16, true, false>(a, stream) : run<F16, true, false>(a, stream);
  }
  return a.bf16 ? run<BF16, false, false>(a, stream) : run<F16, false, false>(a, stream);
}

}  // namespace tvq
