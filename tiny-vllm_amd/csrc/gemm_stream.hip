// Decode-size (M <= 64), wide-N W8A16 / W8A8 GEMM for gfx950: weight
// streaming with the activations shared through LDS.
//
// Decode is weight-bandwidth bound: every int8 weight byte is read once, the
// activations (M x K, small) are read by every workgroup. So:
//
//  * a 256-thread workgroup owns 64 output channels (16 per wave, the MFMA A
//    side) over all of K; each wave streams its own 16 weight rows from HBM
//    straight into registers with 128-bit non-temporal loads, one group of
//    G = 4 64-k chunks ahead of the MFMAs;
//  * the activations of that K range are loaded cooperatively (each wave a
//    quarter, two groups ahead) and written to a 2-slot LDS ring, where the 4
//    waves share them as MFMA B fragments (16 tokens per block); their L2
//    traffic is M/64 (int8) or M/32 (bf16) of the weight traffic instead of
//    M/16 per wave. All loads are ordinary (compiler-tracked) vector loads, so
//    the waits the compiler inserts are exact;
//  * W8A8 feeds v_mfma_i32_16x16x64_i8 directly; W8A16 converts the 16 int8
//    of a lane to two bf16/fp16 halves (exact) for v_mfma_f32_16x16x32.
//
// It needs N/64 workgroups to fill the GPU, so the dispatcher uses it only
// for wide layers (N >= 16384) with M > 8, where sharing the activations pays;
// narrower decode GEMMs go to the skinny kernel (16 rows per workgroup, K
// split across its waves), which measured faster there.
//
// LDS block layout (16 rows x 64 bytes per 1 KB block, lane i = 16g + r owns
// bytes 16i..16i+15): int8 block <- x[m=r][k0 + 16g .. +16]; 16-bit block h
// <- x[m=r][k0 + 16g + 8h .. +8]; the matching weight lane holds
// qw[n][k0 + 16g .. +16] and uses bytes 8h..8h+7 against block h. A fragment
// read is one conflict-free ds_read_b128 at block + 16*lane.
#include <type_traits>

#include "gemm_dma_kernel.h"
#include "tvq_common.h"
#include "tvq_internal.h"

namespace tvq {
namespace {

constexpr int kG = 4;          // 64-k chunks per group
constexpr int kRowsPerWG = 64;

// Barrier that publishes this wave's LDS writes to the workgroup without the
// workgroup fence of __syncthreads(), which would also drain (vmcnt(0)) the
// weight loads prefetched for the next groups.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <bool kW8A8, int MG>
struct StreamCfg {
  static constexpr int kXH = kW8A8 ? 1 : 2;                  // blocks per (m-group, chunk)
  static constexpr int kXBlocks = MG * kG * kXH;             // per group
  static constexpr int kSlotBytes = kXBlocks * 1024;
  static constexpr int kXPerWave = kXBlocks / 4;             // activation loads per wave per group
  static_assert(kXBlocks % 4 == 0, "groups split evenly over the 4 waves");
};

template <typename T, bool kW8A8, bool kRaw, int MG>
__global__ __launch_bounds__(256) void stream_kernel(const void* __restrict__ xv, const float* __restrict__ a_scales,
                                                     const int8_t* __restrict__ qw, const float* __restrict__ ws,
                                                     const uint16_t* __restrict__ bias, void* __restrict__ yv, int M,
                                                     int N, int K) {
  using C = StreamCfg<kW8A8, MG>;
  using Acc = typename std::conditional<kW8A8, i32x4, f32x4>::type;
  __shared__ __attribute__((aligned(1024))) char xring[2][C::kSlotBytes];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int nblk = blockIdx.x;
  const int ngroups = K / (64 * kG);  // whole groups (K % 256 == 0)

  // weight row of this lane (clamped rows feed outputs that are never stored)
  const int n_lane = nblk * kRowsPerWG + wave * 16 + r;
  const int8_t* wrow = qw + (int64_t)min(n_lane, N - 1) * K + 16 * g;

  // activation sources: this wave's quarter of a group's blocks (chunk u of
  // the group folded into the pointer)
  const char* xsrc[C::kXPerWave];
  int xoff[C::kXPerWave];
#pragma unroll
  for (int j = 0; j < C::kXPerWave; ++j) {
    const int b = j * 4 + wave;  // block id within the group: ((mg * kG + u) * kXH + h)
    const int h = b % C::kXH;
    const int mg = b / (C::kXH * kG);
    const int m = min(16 * mg + r, M - 1);
    const int u = (b / C::kXH) % kG;
    xoff[j] = b * 1024 + lane * 16;
    if constexpr (kW8A8)
      xsrc[j] = static_cast<const char*>(xv) + (int64_t)m * K + 64 * u + 16 * g;
    else
      xsrc[j] = static_cast<const char*>(xv) + 2 * ((int64_t)m * K + 64 * u + 16 * g + 8 * h);
  }
  constexpr int kXStep = 64 * (kW8A8 ? 1 : 2);  // activation bytes per 64-k chunk

  // Two groups of weights and activations are in flight in registers; the
  // buffers are selected at compile time (the group loop is unrolled by 2).
  u32x4 wbuf0[kG], wbuf1[kG];
  u32x4 xbuf0[C::kXPerWave], xbuf1[C::kXPerWave];
  // K % 256 == 0, so every group is full: chunks
  // c0..c0+3 are read from one base with immediate offsets, branch-free (the
  // compiler's waits then stay exact across iterations).
  auto load = [&](int grp, u32x4* wb, u32x4* xb) {
    const int c0 = grp * kG;
    const int8_t* wp = wrow + (int64_t)c0 * 64;
#pragma unroll
    for (int j = 0; j < C::kXPerWave; ++j) xb[j] = ldg128(xsrc[j] + (int64_t)c0 * kXStep);
#pragma unroll
    for (int u = 0; u < kG; ++u) wb[u] = ldg128_stream(wp + 64 * u);
  };
  auto stage = [&](int grp, const u32x4* xb) {
    char* slot = xring[grp & 1];
#pragma unroll
    for (int j = 0; j < C::kXPerWave; ++j) *reinterpret_cast<u32x4*>(slot + xoff[j]) = xb[j];
  };

  Acc acc[MG];
#pragma unroll
  for (int j = 0; j < MG; ++j) acc[j] = Acc{};

  auto compute = [&](int grp, const u32x4* wb) {
    const char* slot = xring[grp & 1] + lane * 16;
#pragma unroll
    for (int u = 0; u < kG; ++u) {
      const u32x4 w = wb[u];
      if constexpr (kW8A8) {
#pragma unroll
        for (int mg = 0; mg < MG; ++mg) {
          const u32x4 b = *reinterpret_cast<const u32x4*>(slot + (mg * kG + u) * 1024);
          acc[mg] = mfma16x16x64_i8(w, b, acc[mg]);
        }
      } else {
        const u32x2 c0 = i8x4_to_16x4<T>(w[0]);
        const u32x2 c1 = i8x4_to_16x4<T>(w[1]);
        const u32x2 c2 = i8x4_to_16x4<T>(w[2]);
        const u32x2 c3 = i8x4_to_16x4<T>(w[3]);
        const u32x4 alo = {c0.x, c0.y, c1.x, c1.y};
        const u32x4 ahi = {c2.x, c2.y, c3.x, c3.y};
#pragma unroll
        for (int mg = 0; mg < MG; ++mg) {
          const char* bp = slot + ((mg * kG + u) * 2) * 1024;
          acc[mg] = mfma16x16x32<T>(alo, *reinterpret_cast<const u32x4*>(bp), acc[mg]);
          acc[mg] = mfma16x16x32<T>(ahi, *reinterpret_cast<const u32x4*>(bp + 1024), acc[mg]);
        }
      }
    }
  };

  // The loop body has no branches (the compiler's waits stay exact): loads
  // past the last group re-read the last group (an L2 hit) into buffers that
  // are never computed, and an odd last group is peeled after the loop.
  // K >= 256, so there is at least one group.
  const int last = ngroups - 1;
  load(0, wbuf0, xbuf0);
  stage(0, xbuf0);
  load(min(1, last), wbuf1, xbuf1);
  lds_barrier();
  // Group grp computes from slot grp&1 and its weight registers; meanwhile the
  // activations of grp+1 go to the other slot (last read in group grp-1,
  // which every wave finished before the previous barrier) and group grp+2 is
  // loaded into the registers grp just released.
  const int pairs = ngroups >> 1;
  for (int pr = 0; pr < pairs; ++pr) {
    const int grp = 2 * pr;
    compute(grp, wbuf0);
    stage(grp + 1, xbuf1);
    load(min(grp + 2, last), wbuf0, xbuf0);
    lds_barrier();
    compute(grp + 1, wbuf1);
    stage(grp + 2, xbuf0);
    load(min(grp + 3, last), wbuf1, xbuf1);
    lds_barrier();
  }
  if (ngroups & 1) compute(last, wbuf0);

  // Lane owns y[m, nb..nb+3], m = 16*mg + r, nb = row block + 16*wave + 4g.
  const int nb = nblk * kRowsPerWG + wave * 16 + 4 * g;
#pragma unroll
  for (int mg = 0; mg < MG; ++mg) {
    const int m = 16 * mg + r;
    if (m >= M) continue;
    const float as = (kW8A8 && !kRaw) ? a_scales[m] : 0.0f;
    dma::store4<T, kW8A8, kRaw>(yv, ws, bias, as, m, nb, N, acc[mg][0], acc[mg][1], acc[mg][2], acc[mg][3]);
  }
}

template <typename T, bool kW8A8, bool kRaw, int MG>
hipError_t launch_mg(const GemmArgs& a, hipStream_t stream) {
  const int nblocks = (int)((a.N + kRowsPerWG - 1) / kRowsPerWG);
  stream_kernel<T, kW8A8, kRaw, MG><<<dim3(nblocks), dim3(256), 0, stream>>>(
      a.x, a.a_scales, a.qweight, a.scales, static_cast<const uint16_t*>(a.bias), a.y, (int)a.M, (int)a.N, (int)a.K);
  return hipGetLastError();
}

template <typename T, bool kW8A8, bool kRaw>
hipError_t launch_t(const GemmArgs& a, hipStream_t stream) {
  switch ((a.M + 15) / 16) {
    case 1: return launch_mg<T, kW8A8, kRaw, 1>(a, stream);
    case 2: return launch_mg<T, kW8A8, kRaw, 2>(a, stream);
    case 3: return launch_mg<T, kW8A8, kRaw, 3>(a, stream);
    default: return launch_mg<T, kW8A8, kRaw, 4>(a, stream);
  }
}

}  // namespace

bool stream_shape_ok(int64_t M, int64_t N, int64_t K) { return K % (64 * kG) == 0 && N >= 16384 && M > 8; }

hipError_t launch_stream(const GemmArgs& a, hipStream_t stream) {
  if (a.w8a8) {
    if (a.raw_i32) return launch_t<BF16, true, true>(a, stream);
    return a.bf16 ? launch_t<BF16, true, false>(a, stream) : launch_t<F16, true, false>(a, stream);
  }
  return a.bf16 ? launch_t<BF16, false, false>(a, stream) : launch_t<F16, false, false>(a, stream);
}

}  // namespace tvq
