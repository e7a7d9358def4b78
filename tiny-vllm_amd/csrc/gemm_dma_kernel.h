// Multi-stage LDS-DMA pipelined W8A16 / W8A8 GEMM for gfx950 (kernel template).
//
// Operands are moved global -> LDS with global_load_lds_dwordx4 (no register
// staging) into an S-deep ring of stages; each stage covers KS = 128 (or 64)
// k values, so S-1 stages of loads are in flight while the MFMAs of the
// current one run. Each wave's DMA ops for a stage go out in two halves,
// one sub-step apart.
//
// One wave-level DMA fills one 1 KB block: 8 rows x 128 contiguous bytes of
// the operand (full cache lines). Lane i fetches row rho = i/8 of the block,
// 16-byte chunk c = (i%8) ^ swz(row), and the hardware writes it to
// block + 16*i; so chunk c of row rho sits in slot rho*8 + (c ^ swz(row)),
// with swz(row) = (row/2) % 8 over the row's index in the tile. The LDS
// serves a 128-bit read 16 lanes at a time over 256 bytes of banks: rows
// of equal parity land 256 bytes apart, and swz gives the 8 rows of each
// parity in a 16-row group 8 different chunk slots, so the 16 lanes of a
// fragment read (16 rows, one logical chunk) never share a bank, while every
// DMA still reads whole 128-byte lines. (With KS = 64 a block holds 16 rows
// x 64 bytes and the same reasoning gives swz(row) = (row/4) % 4.)
//
// Fragment reads (one ds_read_b128 per lane; 16x16 MFMA tiles, lane =
// 16*g + r):
//   weight / int8 activation, 64-k sub-step ks: row r, chunk 4*ks + g
//     (k = 64*ks + 16g .. +16)
//   16-bit activation (two blocks per 8 rows: k 0-63 and 64-127), sub-step
//     ks, half b: row r, chunk 2g + b of block ks (k = 64*ks + 16g + 8b .. +8)
// With 32x32 MFMA tiles (lane = 32*g + r) the sub-steps are 32 k wide and
// lane group g reads chunk 2*ks + g of row r in the same way.
// For W8A16 the 16 int8 weights of a lane (k = 16g..16g+15) are converted to
// two 8-element bf16/fp16 halves; half b pairs with activation half b, which
// holds the same 8 k values. Any consistent k assignment gives the same dot
// product.
//
// Output channels are the MFMA A side, so each lane owns y[m, n..n+3].
//
// Row indices past M or N are clamped to the last row: those rows only feed
// output rows/columns that are never stored. K must be a multiple of 128
// (checked by the dispatcher), so no K tail is read. A DMA source is a
// wave-uniform tile base in scalar registers plus an unsigned 32-bit lane
// offset (the saddr form, no 64-bit address per op in VGPRs); the
// dispatcher's K <= 2^22 keeps those offsets within 32 bits.
//
// Waits are explicit: the compiler does not track LDS-DMA completion, so each
// step waits on vmcnt for its own stage and then crosses an s_barrier (a bare
// barrier, without the workgroup fence that would force vmcnt(0)). The
// fragments of each sub-step are read from LDS one sub-step ahead into a
// second register set, and the crossing into the next stage happens before
// the MFMAs of a stage's last sub-step, so the matrix core always has queued
// work while a wave waits.
//
// The grid is persistent when there are more tiles than resident workgroups:
// each workgroup walks tiles blockIdx.x, +gridDim.x, ... After the last
// k-stage of a tile it issues the first S-1 stages of its next tile into ring
// slots 0..S-2 and only then runs the epilogue, so the operand fetch of tile
// i+1 overlaps the output stores of tile i. The epilogue needs no global
// loads (which would queue behind that DMA): the tile's per-token scales,
// per-channel scales and bias are loaded into registers at tile start and
// parked in LDS after the tile's last k-stage (where the wait for them is
// free; at tile start it would drain the ring).
// It stages each wave's MF-row slice of its output through a wave-private
// area of the idle ring slot S-1 and writes whole row segments of 16-byte
// stores.
//
// Split-K (decode-size M, when there are fewer tiles than resident
// workgroups): each tile's k-stages are cut into `splits` contiguous ranges
// and the grid walks (range, tile) work units. A unit writes its raw
// accumulators (int32 or fp32) to the caller's workspace as a register image
// with device-scope stores, waits for them to complete and bumps the tile's
// counter; the unit that arrives last sums all images in range order (so the
// result does not depend on arrival order; int32 sums are exact) and runs the
// normal epilogue, then returns the counter to zero. The counters must be
// zero when a call starts and are zero again when it ends.
//
// kDq (W8A16 only): each weight is dequantized to T(T(q) * T(s[n])) before
// the MFMA, as the reference's kernel does, and the epilogue adds only the
// bias (the scale is already inside the sum).
//
// kDmaOnly (measurement): the same grid, tile walk, DMA ops, waits and
// barriers with the fragment reads, MFMAs, scale/bias loads and epilogue
// compiled out: it reads only xv and qw (a_scales, ws, bias and yv may be
// null) and writes nothing to global memory. Its time is the operand-delivery
// floor of the tiling, against which the full kernel is judged.
#pragma once

#include <stdlib.h>

#include <type_traits>

#include "tvq_common.h"
#include "tvq_internal.h"

// Timeline hooks for instrumented builds (no code in the library).
#ifndef TVQ_TL_MARK
#define TVQ_TL_MARK(ev)
#endif

namespace tvq {
namespace dma {

#define TVQ_GPTR(p) ((__attribute__((address_space(1))) void*)(p))
#define TVQ_LPTR(p) ((__attribute__((address_space(3))) void*)(p))

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

// s_waitcnt immediate for lgkmcnt(0) with vmcnt and expcnt left at their
// maxima (gfx9 encoding: vmcnt 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int kWaitLgkm0 = 0xC07F;

// Wait until at most `ahead` later stages (each `LPW` DMA ops) are in flight
// (0 <= ahead <= S-2); vmcnt retires in issue order.
template <int LPW, int S, int A = S - 2>
__device__ __forceinline__ void wait_stage(int ahead) {
  static_assert(LPW * (S - 2) < 64, "too many DMA ops in flight for vmcnt");
  if constexpr (A <= 0) {
    wait_vm<0>();
  } else {
    if (ahead >= A) {
      wait_vm<LPW * A>();
      return;
    }
    wait_stage<LPW, S, A - 1>(ahead);
  }
}

// Split-K workspace layout: tile counters (int32) first, then the partial
// accumulator images, BM*BN 4-byte values per (tile, range).
constexpr int64_t kSplitCntBytes = 64 * 1024;
constexpr int kSplitMaxTiles = (int)(kSplitCntBytes / 4);

template <bool kW8A8, int BM, int BN, int WM, int WN, int S, int MF, int KS>
struct Cfg {
  static constexpr int kThreads = 64 * WM * WN;
  static constexpr int kWaves = WM * WN;
  static constexpr int kXRow = kW8A8 ? KS : 2 * KS;      // activation bytes per row per stage
  static constexpr int kXRb = kXRow < 128 ? kXRow : 128;  // activation block row width
  static constexpr int kXHalves = kXRow / kXRb;           // activation blocks per row group per stage
  static constexpr int kWBlk = BN * KS / 1024;            // weight blocks per stage
  static constexpr int kXBlk = BM * kXRow / 1024;         // activation blocks per stage
  static constexpr int kBlkStage = kWBlk + kXBlk;
  static constexpr int kStageBytes = kBlkStage * 1024;
  static constexpr int kRingBytes = kStageBytes * S;
  static constexpr int kLPW = kBlkStage / kWaves;         // DMA ops per wave per stage
  static constexpr int kKStage = KS;                      // k values per stage
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int FM = TM / MF, FN = TN / MF;        // MFMA tiles per wave
  static constexpr int kEpiBytes = MF * TN * 2;           // per-wave staging: MF rows x TN 16-bit outputs
  static constexpr int kScN = BM + 2 * BN;                // per-tile a_scales | w_scales | bias (fp32, in LDS)
  static constexpr int kLdsBytes = kRingBytes + kScN * 4 + 16;   // + the split-K "last unit" flag
  static_assert(MF == 16 || MF == 32, "MFMA tile is 16x16 or 32x32");
  static_assert(kBlkStage % kWaves == 0, "stage blocks must split evenly over waves");
  static_assert(TM % MF == 0 && TN % MF == 0, "wave tile must be a multiple of the MFMA tile");
  static_assert(S >= 2, "at least double buffering");
  static_assert(KS == 64 || KS == 128, "stage depth is 64 or 128 k");
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
  static_assert(kWaves * kEpiBytes <= kStageBytes, "epilogue staging must fit in one ring stage");
};

// Store four consecutive outputs y[m, nb..nb+3] with the path's epilogue.
template <typename T, bool kW8A8, bool kRaw, typename V>
__device__ __forceinline__ void store4(void* yv, const float* ws, const uint16_t* bias, float as, int m, int nb, int N,
                                       V v0, V v1, V v2, V v3) {
  if constexpr (kRaw) {
    int32_t* y = static_cast<int32_t*>(yv) + (int64_t)m * N;
    const int32_t v[4] = {(int32_t)v0, (int32_t)v1, (int32_t)v2, (int32_t)v3};
    if (nb + 3 < N && (N & 3) == 0) {
      *reinterpret_cast<i32x4*>(y + nb) = i32x4{v[0], v[1], v[2], v[3]};
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (nb + t < N) y[nb + t] = v[t];
    }
  } else {
    uint16_t* y = static_cast<uint16_t*>(yv) + (int64_t)m * N;
    const V v[4] = {v0, v1, v2, v3};
    float o[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int n = nb + t < N ? nb + t : N - 1;
      const float bb = bias ? to_float<T>(bias[n]) : 0.0f;
      if constexpr (kW8A8)
        o[t] = epi_w8a8(v[t], as, ws[n], bb);
      else
        o[t] = epi_w8a16(v[t], ws[n], bb);
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

// Offset (bytes) of 16-byte chunk `c` of row `row` inside a run of 8-row
// blocks laid out by the DMA (chunk c of row rho at slot rho*8 + (c ^ swz)).
// For 64-byte rows (16-row blocks, 4 chunks per row) the same rule reads: chunk c
// of row rho at slot rho*4 + (c ^ swz(row)), swz(row) = (row/4) % 4.
template <int RB>
__device__ __forceinline__ int swz(int row) {
  return RB == 128 ? (row >> 1) & 7 : (row >> 2) & 3;
}

template <int RB>
__device__ __forceinline__ int chunk_off(int row, int c) {
  constexpr int kR = 1024 / RB, kC = RB / 16;  // rows per block, chunks per row
  return (row / kR) * 1024 + 16 * ((row % kR) * kC + (c ^ swz<RB>(row)));
}

// Tile order: XCD chunking (workgroup i runs on XCD i % 8, so each XCD gets a
// contiguous range of logical tiles), then a grouped swizzle so that the
// tiles in flight on one XCD share operand panels in its L2.
__device__ __forceinline__ void tile_coords(int pid, int tiles_m, int tiles_n, int group, int m_major, int& tm,
                                            int& tn) {
  const int total = tiles_m * tiles_n;
  if (total % 8 == 0) pid = (pid % 8) * (total / 8) + pid / 8;
  if (m_major) {
    // consecutive tiles walk m inside groups of `group` n-tiles
    const int per_group = group * tiles_m;
    const int first = (pid / per_group) * group;
    const int gsz = min(tiles_n - first, group);
    const int in = pid % per_group;
    tn = first + in % gsz;
    tm = in / gsz;
  } else {
    // consecutive tiles walk n inside groups of `group` m-tiles
    const int per_group = group * tiles_n;
    const int first = (pid / per_group) * group;
    const int gsz = min(tiles_m - first, group);
    const int in = pid % per_group;
    tm = first + in % gsz;
    tn = in / gsz;
  }
}

template <typename T, bool kW8A8, bool kRaw, int BM, int BN, int WM, int WN, int S, int MF, int KS, bool kSplit,
          bool kNtW = false, bool kGlu = false, bool kRot = false, bool kDmaOnly = false, bool kDq = false,
          bool kSK = false>
__global__ __launch_bounds__(64 * WM * WN) void gemm_dma_kernel(const void* __restrict__ xv,
                                                                const float* __restrict__ a_scales,
                                                                const int8_t* __restrict__ qw,
                                                                const float* __restrict__ ws,
                                                                const uint16_t* __restrict__ bias,
                                                                void* __restrict__ yv, int M, int N, int K,
                                                                int group, int m_major, int splits,
                                                                char* __restrict__ wsp, int sk_len) {
  using C = Cfg<kW8A8, BM, BN, WM, WN, S, MF, KS>;
  using Acc = typename std::conditional<
      MF == 32, typename std::conditional<kW8A8, i32x16, f32x16>::type,
      typename std::conditional<kW8A8, i32x4, f32x4>::type>::type;
  constexpr int kAccN = MF == 32 ? 16 : 4;
  extern __shared__ __attribute__((aligned(1024))) char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar registers
  const int wn = wave % WN;
  const int wm = wave / WN;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  const int total = tiles_m * tiles_n;
  const int units = total * splits;
  const int nk_all = K / C::kKStage;
  const int nk_per = (nk_all + splits - 1) / splits;   // k-stages per split range
  // Work unit u -> tile u % total, k range u / total (range-major, so units
  // that run together share the range's activation panel).
  auto unit_coords = [&](int u, int& tm_, int& tn_, int& tl_, int& sk_, int& kb_, int& kn_) {
    tl_ = u % total;
    sk_ = u / total;
    tile_coords(tl_, tiles_m, tiles_n, group, m_major, tm_, tn_);
    kb_ = sk_ * nk_per;
    kn_ = max(0, min(nk_all, kb_ + nk_per) - kb_);
  };
  // Stream-K (sk_len > 0): the tiles' k-stages form one sequence, tile-major
  // (tile t owns positions t*nk_all .. t*nk_all + nk_all - 1), and workgroup w
  // owns positions [w*sk_len, (w+1)*sk_len). Its range cuts into segments at
  // tile boundaries; only its first and last segment can be part of a tile.
  static_assert(!kSK || kSplit, "stream-K uses the split-K fixup");
  constexpr bool streamk = kSK;
  int sk_pos = (int)blockIdx.x * sk_len;
  const int sk_end = streamk ? min(total * nk_all, sk_pos + sk_len) : 0;
  auto seg_coords = [&](int& tm_, int& tn_, int& tl_, int& kb_, int& kn_) {
    tl_ = sk_pos / nk_all;
    kb_ = sk_pos - tl_ * nk_all;
    kn_ = min(nk_all - kb_, sk_end - sk_pos);
    tile_coords(tl_, tiles_m, tiles_n, group, m_major, tm_, tn_);
  };
  if (streamk && sk_pos >= sk_end) return;  // (the host sizes the grid so that this never happens)

  // ---- per-lane DMA sources for this wave's blocks ----------------------
  // Each source is a wave-uniform tile base (scalar registers) plus a 32-bit
  // per-lane offset, which keeps the address state of the kLPW streams small.
  const char* wbase = reinterpret_cast<const char*>(qw);
  const char* xbase = static_cast<const char*>(xv);
  uint32_t soff[C::kLPW];
  constexpr int kWCh = KS / 16, kXCh = C::kXRb / 16;   // 16-byte chunks per block row
  // kRot: a tile walks its k-stages starting at stage (tm + tn) % nk and
  // wrapping around, so the tiles that share an operand panel do not all
  // request the same cache lines at the same time. Only the order of the
  // k-stages changes (exact for int32 sums; a fixed, per-tile order for fp32).
  int rot = 0, rot_nk = 1;
  auto set_sources = [&](int m0, int n0, int kb, int nk_tile, int rot_seed) {
    if constexpr (kRot) {
      rot_nk = nk_tile > 0 ? nk_tile : 1;
      rot = rot_seed % rot_nk;
    }
    wbase = reinterpret_cast<const char*>(qw) + (int64_t)n0 * K + (int64_t)kb * C::kKStage;
    xbase = static_cast<const char*>(xv) + ((int64_t)m0 * K + (int64_t)kb * C::kKStage) * (kW8A8 ? 1 : 2);
#pragma unroll
    for (int j = 0; j < C::kLPW; ++j) {
      const int b = j * C::kWaves + wave;
      if (b < C::kWBlk) {
        const int row = (1024 / KS) * b + lane / kWCh;      // row of the tile's weight panel
        const int n = min(n0 + row, N - 1) - n0;
        soff[j] = n * K + 16 * ((lane % kWCh) ^ swz<KS>(row));
      } else {
        const int xb = b - C::kWBlk;
        const int row = (1024 / C::kXRb) * (xb / C::kXHalves) + lane / kXCh;  // row of the activation panel
        const int m = min(m0 + row, M - 1) - m0;
        const int half = xb % C::kXHalves;
        soff[j] = m * K * (kW8A8 ? 1 : 2) + C::kXRb * half + 16 * ((lane % kXCh) ^ swz<C::kXRb>(row));
      }
    }
  };
  auto issue = [&](int kt, int j0 = 0, int j1 = C::kLPW) {
    char* stage = smem + (kt % S) * C::kStageBytes;
#pragma unroll
    for (int j = 0; j < C::kLPW; ++j) {
      if (j < j0 || j >= j1) continue;
      const int b = j * C::kWaves + wave;
      const bool wblk = b < C::kWBlk;
      const int step = wblk ? KS : C::kXRow;
      // uniform 64-bit base + unsigned 32-bit lane offset: the saddr form of
      // the DMA, so no 64-bit address per op stays live in VGPRs
      int kq = kt;
      if constexpr (kRot) {
        kq += rot;
        if (kq >= rot_nk) kq -= rot_nk;
      }
      const char* p = (wblk ? wbase : xbase) + (uint32_t)(soff[j] + (uint32_t)(kq * step));
      // kNtW: weight blocks that no other tile reads again (one m-tile)
      // stream with the non-temporal hint, so they do not evict the
      // activation panel every tile shares from L2
      if (kNtW && wblk)
        __builtin_amdgcn_global_load_lds(TVQ_GPTR(p), TVQ_LPTR(stage + b * 1024), 16, 0, 2);
      else
        __builtin_amdgcn_global_load_lds(TVQ_GPTR(p), TVQ_LPTR(stage + b * 1024), 16, 0, 0);
    }
  };

  // ---- lane-constant fragment offsets within a stage ---------------------
  // MF = 16: lane = 16*g + r, sub-steps of 64 k (KS / 64 per stage).
  // MF = 32: lane = 32*h + r, sub-steps of 32 k (KS / 32 per stage).
  constexpr int kSub = KS / (MF == 32 ? 32 : 64);
  constexpr int kRows = MF;                        // rows per fragment
  const int r = lane % MF;
  const int g = lane / MF;                         // lane group: 0..3 (MF 16) or 0..1 (MF 32)
  int woff[kSub];        // weight / int8 activation fragment
  int xoff[kSub][2];     // 16-bit activation fragment, halves b = 0, 1
#pragma unroll
  for (int ks = 0; ks < kSub; ++ks) {
    // 16 bytes per lane: k = ks*(KS/kSub) + 16*g .. +16
    const int c = ks * (kWCh / kSub) + g;
    woff[ks] = chunk_off<KS>(r, c);
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      // 16-bit activations: k = ks*(KS/kSub) + 16*g + 8*b .. +8, one 128-byte
      // block (64 k) per half of the row
      const int k = ks * (KS / kSub) + 16 * g + 8 * b;
      xoff[ks][b] = (r >> 3) * 1024 * C::kXHalves + (k >> 6) * 1024 + 16 * ((r & 7) * 8 + (((k & 63) >> 3) ^ swz<128>(r)));
    }
  }
  constexpr int kWFrag = kRows * KS;               // bytes per weight fragment (rows x KS bytes)
  constexpr int kXFrag = kRows * C::kXRow;
  constexpr int kReadsPerSub = C::FN + C::FM * (kW8A8 ? 1 : 2);   // ds_read_b128 per sub-step
  constexpr int kMfmaPerSub = C::FN * C::FM * (kW8A8 ? 1 : 2);    // MFMAs per sub-step
  static_assert(kSub % 2 == 0, "fragment buffers alternate per sub-step across stages");

  // ---- per-tile scales and bias, parked in LDS for the epilogue ----------
  // The values are loaded into registers with the tile's first stage DMAs
  // (as raw bits; the bias is converted only when stored) and written to LDS
  // after the tile's last k-stage, where every DMA op of the tile has
  // already been waited for: the compiler's wait for the loads (vmcnt(0): it
  // cannot count the ops in flight across the persistent loop) then costs
  // nothing. Written at tile start, that wait drained the whole ring there.
  // Every lane issues the same loads (addresses selected and clamped, no
  // per-lane branch): a load register that another branch writes makes the
  // compiler wait vmcnt(0) on it, which would drain the ring right after the
  // tile's stage DMAs. The bias goes to its own registers under a
  // wave-uniform branch.
  float* sc = reinterpret_cast<float*>(smem + C::kRingBytes);  // [a_s: BM | w_s: BN | bias: BN]
  constexpr int kScPer = (C::kScN + C::kThreads - 1) / C::kThreads;
  float scv[kScPer];
  uint16_t sbv[kScPer];
  auto load_scales = [&](int m0, int n0) {
#pragma unroll
    for (int u = 0; u < kScPer; ++u) {
      const int idx = (int)threadIdx.x + u * C::kThreads;
      // idx < BM: the token's scale (W8A8); otherwise channel idx - BM (the
      // slots past BM + BN load a valid channel and are not used)
      const float* p = ws + min(n0 + max(idx - BM, 0), N - 1);
      if constexpr (kW8A8) p = idx < BM ? a_scales + min(m0 + idx, M - 1) : p;
      scv[u] = *p;
    }
    if (bias != nullptr) {
#pragma unroll
      for (int u = 0; u < kScPer; ++u) {
        const int idx = (int)threadIdx.x + u * C::kThreads;
        sbv[u] = bias[min(n0 + max(idx - BM - BN, 0), N - 1)];
      }
    }
  };
  auto store_scales = [&]() {
#pragma unroll
    for (int u = 0; u < kScPer; ++u) {
      const int idx = (int)threadIdx.x + u * C::kThreads;
      if (idx < BM + BN)
        sc[idx] = scv[u];
      else if (idx < C::kScN)
        sc[idx] = bias != nullptr ? to_float<T>(sbv[u]) : 0.0f;
    }
  };

  TVQ_TL_MARK(0);
  int unit = blockIdx.x;
  int tm, tn, tl, sk, kb, nk;
  if (streamk) {
    sk = 0;  // stream-K: 0 while in the workgroup's first segment, 1 after it
    seg_coords(tm, tn, tl, kb, nk);
  } else {
    unit_coords(unit, tm, tn, tl, sk, kb, nk);
  }
  set_sources(tm * BM, tn * BN, kb, nk, tm + tn);
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < nk) issue(s);
  if constexpr (!kRaw && !kDmaOnly) load_scales(tm * BM, tn * BN);

  static_assert(!kDq || !kW8A8, "rounded dequantization is a W8A16 mode");
  while (true) {
    const int n0 = tn * BN;
    const int m0 = tm * BM;
    const int cur_tl = tl, cur_sk = sk, cur_nk = nk;
    // kDq: the rounded scale of the channel each weight fragment row holds
    float dqs[kDq ? C::FN : 1];
    if constexpr (kDq) {
#pragma unroll
      for (int i = 0; i < C::FN; ++i) dqs[i] = round_to<T>(ws[min(n0 + wn * C::TN + MF * i + (lane % MF), N - 1)]);
    }
    Acc acc[C::FN][C::FM];
#pragma unroll
    for (int i = 0; i < C::FN; ++i)
#pragma unroll
      for (int j = 0; j < C::FM; ++j) acc[i][j] = Acc{};

    // Fragments are double-buffered in registers: the LDS reads of sub-step
    // ks+1 are issued among the MFMAs of sub-step ks, so their latency hides
    // behind the matrix core instead of stalling the wave. The stage boundary
    // is crossed one sub-step early: before the MFMAs of a stage's last
    // sub-step the waves wait for the next stage's DMA, meet at the barrier,
    // refill the ring and read the next stage's first fragments, so the
    // pipeline never drains at a barrier.
    u32x4 fa[2][C::FN];
    u32x4 fb[2][C::FM][kW8A8 ? 1 : 2];
    auto load_frags = [&](int kt, int ks, int buf) {
      const char* wst = smem + (kt % S) * C::kStageBytes + wn * C::FN * kWFrag;
      const char* xst = smem + (kt % S) * C::kStageBytes + C::kWBlk * 1024 + wm * C::FM * kXFrag;
#pragma unroll
      for (int i = 0; i < C::FN; ++i) fa[buf][i] = *reinterpret_cast<const u32x4*>(wst + i * kWFrag + woff[ks]);
#pragma unroll
      for (int j = 0; j < C::FM; ++j) {
        if constexpr (kW8A8) {
          fb[buf][j][0] = *reinterpret_cast<const u32x4*>(xst + j * kXFrag + woff[ks]);
        } else {
          fb[buf][j][0] = *reinterpret_cast<const u32x4*>(xst + j * kXFrag + xoff[ks][0]);
          fb[buf][j][1] = *reinterpret_cast<const u32x4*>(xst + j * kXFrag + xoff[ks][1]);
        }
      }
    };

    wait_stage<C::kLPW, S>(min(S - 2, cur_nk - 1));
    barrier();
    TVQ_TL_MARK(1);
    if (S - 1 < cur_nk) issue(S - 1);
    if constexpr (!kDmaOnly) load_frags(0, 0, 0);

    for (int kt = 0; kt < cur_nk; ++kt) {
#pragma unroll
      for (int ks = 0; ks < kSub; ++ks) {
        const int cb = ks & 1;
        // This sub-step's fragments were requested one sub-step ago. The
        // wait is the s_waitcnt builtin (not inline asm) so the compiler
        // knows every earlier LDS read is complete and adds no wait of its
        // own after the reads issued next.
        __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
        __builtin_amdgcn_sched_barrier(0);
        // Second half of the DMA ops for stage kt - 1 + S (the first half
        // went out at the previous stage crossing): spreading a stage's
        // loads over two sub-steps keeps the waves from stalling behind a
        // burst of vector-memory issues while the matrix core idles.
        if (ks == 0 && kt > 0 && kt - 1 + S < cur_nk) issue(kt - 1 + S, C::kLPW / 2, C::kLPW);
        if (ks + 1 < kSub) {
          if constexpr (!kDmaOnly) load_frags(kt, ks + 1, cb ^ 1);
        } else if (kt + 1 < cur_nk) {
          // Every wave's reads of stage kt are complete (the wait above);
          // once all are past the barrier the slot of stage kt can take
          // stage kt + S.
          wait_stage<C::kLPW, S>(min(S - 2, cur_nk - 2 - kt));
          barrier();
          if (kt + S < cur_nk) issue(kt + S, 0, C::kLPW / 2);
          if constexpr (!kDmaOnly) load_frags(kt + 1, 0, cb ^ 1);
        }
        if constexpr (kDmaOnly) {
          // operand-delivery floor: the same DMA, waits and barriers, no arithmetic
        } else if constexpr (kW8A8) {
#pragma unroll
          for (int j = 0; j < C::FM; ++j) {
#pragma unroll
            for (int i = 0; i < C::FN; ++i) {
              if constexpr (MF == 32)
                acc[i][j] = mfma32x32x32_i8(fa[cb][i], fb[cb][j][0], acc[i][j]);
              else
                acc[i][j] = mfma16x16x64_i8(fa[cb][i], fb[cb][j][0], acc[i][j]);
            }
          }
        } else {
#pragma unroll
          for (int i = 0; i < C::FN; ++i) {
            u32x2 c0, c1, c2, c3;
            if constexpr (kDq) {
              c0 = i8x4_dq_to_16x4<T>(fa[cb][i][0], dqs[i]);
              c1 = i8x4_dq_to_16x4<T>(fa[cb][i][1], dqs[i]);
              c2 = i8x4_dq_to_16x4<T>(fa[cb][i][2], dqs[i]);
              c3 = i8x4_dq_to_16x4<T>(fa[cb][i][3], dqs[i]);
            } else {
              c0 = i8x4_to_16x4<T>(fa[cb][i][0]);
              c1 = i8x4_to_16x4<T>(fa[cb][i][1]);
              c2 = i8x4_to_16x4<T>(fa[cb][i][2]);
              c3 = i8x4_to_16x4<T>(fa[cb][i][3]);
            }
            const u32x4 alo = u32x4{c0.x, c0.y, c1.x, c1.y};
            const u32x4 ahi = u32x4{c2.x, c2.y, c3.x, c3.y};
#pragma unroll
            for (int j = 0; j < C::FM; ++j) {
              if constexpr (MF == 32) {
                acc[i][j] = mfma32x32x16<T>(alo, fb[cb][j][0], acc[i][j]);
                acc[i][j] = mfma32x32x16<T>(ahi, fb[cb][j][1], acc[i][j]);
              } else {
                acc[i][j] = mfma16x16x32<T>(alo, fb[cb][j][0], acc[i][j]);
                acc[i][j] = mfma16x16x32<T>(ahi, fb[cb][j][1], acc[i][j]);
              }
            }
          }
        }
        // All of the next fragments' reads go out ahead of this sub-step's
        // MFMAs (otherwise the scheduler sinks them below the MFMAs that
        // last read the registers it would reuse, exposing their latency).
        if (ks + 1 < kSub) {
          __builtin_amdgcn_sched_group_barrier(0x100, kReadsPerSub, 0);  // DS reads
          __builtin_amdgcn_sched_group_barrier(0x008, kMfmaPerSub, 0);   // MFMAs
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }

    // Every wave has consumed its last fragments: the ring is free. The
    // previous tile's epilogue finished before this tile's first barrier, so
    // the scale area is free too: park this tile's scales there (their loads
    // completed with the tile's DMA) and publish them before the epilogue.
    barrier();
    if constexpr (!kRaw && !kDmaOnly) {
      store_scales();
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      barrier();
    }
    TVQ_TL_MARK(2);
    // ---- next tile: start its operand stream before this tile's stores ----
    bool more;
    if (streamk) {
      sk_pos += cur_nk;
      more = sk_pos < sk_end;
    } else {
      more = unit + (int)gridDim.x < units;
    }
    if (more) {
      if (streamk) {
        sk = 1;
        seg_coords(tm, tn, tl, kb, nk);
      } else {
        unit += (int)gridDim.x;
        unit_coords(unit, tm, tn, tl, sk, kb, nk);
      }
      set_sources(tm * BM, tn * BN, kb, nk, tm + tn);
#pragma unroll
      for (int s = 0; s < S - 1; ++s)
        if (s < nk) issue(s);
      if constexpr (!kRaw && !kDmaOnly) load_scales(tm * BM, tn * BN);
    }

    // ---- split-K fixup ------------------------------------------------------
    // The images are written and read with device-scope (agent) atomic stores
    // and loads, which bypass the per-XCD L2 and meet at the coherent memory
    // side; so completing the stores (vmcnt 0) before the counter update is
    // the whole release, and no L2 write-back or invalidate is needed.
    // Stream-K: the workgroups w0..w1 whose ranges meet this tile contribute
    // to it, in k order. Contributor w's image is image 2w when the tile is
    // its first segment (every contributor after w0, and w0 when its range
    // starts inside the tile), else 2w + 1 (its last segment).
    int sk_w0 = 0, sk_parts = splits;
    if (streamk) {
      sk_w0 = cur_tl * nk_all / sk_len;
      sk_parts = ((cur_tl + 1) * nk_all - 1) / sk_len - sk_w0 + 1;
    }
    if (kSplit && sk_parts > 1) {
      using E = typename std::conditional<kW8A8, int32_t, float>::type;
      constexpr int kQ4 = kAccN / 4;
      E* part = reinterpret_cast<E*>(wsp + kSplitCntBytes);
      int* cnt = reinterpret_cast<int*>(wsp);
      int* last_flag = reinterpret_cast<int*>(smem + C::kRingBytes + C::kScN * 4);
      // Image index of contribution s (0 .. sk_parts-1, in k order) to this tile.
      auto img_index = [&](int s) -> int64_t {
        if (!streamk) return (int64_t)cur_tl * splits + s;
        const int w = sk_w0 + s;
        return 2 * (int64_t)w + ((int64_t)w * sk_len >= (int64_t)cur_tl * nk_all ? 0 : 1);
      };
      // Register image: value e of 4-value group q of fragment (i, j) of this
      // wave at (((wave * FN + i) * FM + j) * kQ4 + q) * 256 + 64 * e + lane,
      // so each store instruction of a wave covers 256 contiguous bytes.
      auto img = [&](int64_t idx, int i, int j, int q, int e) {
        return part + idx * (BM * BN) + (((wave * C::FN + i) * C::FM + j) * kQ4 + q) * 256 + 64 * e + lane;
      };
      const int64_t own = streamk ? 2 * (int64_t)blockIdx.x + cur_sk : img_index(cur_sk);
#pragma unroll
      for (int i = 0; i < C::FN; ++i)
#pragma unroll
        for (int j = 0; j < C::FM; ++j)
#pragma unroll
          for (int q = 0; q < kQ4; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              __hip_atomic_store(img(own, i, j, q, e), (E)acc[i][j][4 * q + e], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
      wait_vm<0>();
      __syncthreads();
      if (threadIdx.x == 0)
        *last_flag =
            __hip_atomic_fetch_add(cnt + cur_tl, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == sk_parts - 1;
      __syncthreads();
      if (!*last_flag) {
        if (!more) break;
        continue;
      }
      // Sum every range's image (this unit's own included, re-read so that the
      // order is the range order whichever unit finishes last).
#pragma unroll
      for (int i = 0; i < C::FN; ++i)
#pragma unroll
        for (int j = 0; j < C::FM; ++j) acc[i][j] = Acc{};
      for (int s = 0; s < sk_parts; ++s) {
        const int64_t idx = img_index(s);
#pragma unroll
        for (int i = 0; i < C::FN; ++i)
#pragma unroll
          for (int j = 0; j < C::FM; ++j)
#pragma unroll
            for (int q = 0; q < kQ4; ++q)
#pragma unroll
              for (int e = 0; e < 4; ++e)
                acc[i][j][4 * q + e] += __hip_atomic_load(img(idx, i, j, q, e), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      if (threadIdx.x == 0) __hip_atomic_exchange(cnt + cur_tl, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    if constexpr (!kDmaOnly) {
    // ---- epilogue -----------------------------------------------------------
    // MF 16: acc reg t -> n = 4g + t.  MF 32: reg v -> n = 8*(v/4) + 4g + v%4.
    // Either way a lane owns runs of 4 consecutive output channels of token r.
    constexpr int kQ = kAccN / 4;
    const int ncol0 = n0 + wn * C::TN;             // first output column of the wave tile
    if constexpr (kRaw) {
#pragma unroll
      for (int j = 0; j < C::FM; ++j) {
        const int m = m0 + wm * C::TM + MF * j + r;
        if (m >= M) continue;
#pragma unroll
        for (int i = 0; i < C::FN; ++i) {
          const Acc v = acc[i][j];
#pragma unroll
          for (int q = 0; q < kQ; ++q) {
            const int nb = ncol0 + MF * i + 8 * q + 4 * g;
            store4<T, kW8A8, kRaw>(yv, ws, bias, 0.0f, m, nb, N, v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
          }
        }
      }
    } else {
      // Per MF-row slice of the wave tile: scale and round, write to the
      // wave's staging area (row stride 2*TN bytes; 16-byte chunk index XORed
      // with (row / rows-per-256-bytes) so the column-aligned writes of 16
      // consecutive rows use different banks), then read it back
      // row-contiguous and store 16 bytes per lane: every row segment of the
      // slice leaves as whole 2*TN-byte runs.
      // kGlu: the weight rows come as 32-row blocks of gate and up channels
      // (block 2b = gate channels 32b.., block 2b+1 = the matching up
      // channels), so FN = 2 puts a gate column and its up column in the same
      // lane; the slice stores round(silu(round(g)) * round(u)) into an
      // output of N / 2 columns, exactly what the separate SiLU-and-mul
      // kernel computes from the rounded gate_up output.
      static_assert(!kGlu || (kW8A8 && MF == 32 && C::FN == 2), "GLU epilogue: W8A8, 32x32 tiles, FN = 2");
      constexpr int kOutTN = kGlu ? C::TN / 2 : C::TN;  // output columns of the wave tile
      const int n_out = kGlu ? N / 2 : N;
      const int ncol_out = kGlu ? ncol0 / 2 : ncol0;
      constexpr int kRowB = 2 * kOutTN;            // bytes per staged row
      constexpr int kCh = kRowB / 16;              // 16-byte chunks per row
      constexpr int kSwz = (kCh < 8 ? kCh : 8) - 1;
      constexpr int kRowsPer256 = kRowB >= 256 ? 1 : 256 / kRowB;
      auto sswz = [](int row) { return (row / kRowsPer256) & kSwz; };
      constexpr int kPass = MF * kCh / 64;         // read-back passes per slice
      static_assert((MF * kCh) % 64 == 0, "slice must split evenly over the wave");
      char* stg = smem + (S - 1) * C::kStageBytes + wave * C::kEpiBytes;
      const float* sc_w = sc + BM + wn * C::TN;
      const float* sc_b = sc + BM + BN + wn * C::TN;
      uint16_t* y = static_cast<uint16_t*>(yv);
      const bool vec = (n_out & 7) == 0;
      // Per-channel scales of this lane's columns, read once for all row
      // slices (LDS reads of the scales were a large share of the epilogue).
      // The W8A16 4-wave tile (4 x 2 fragments of 32 x 32) would cache 16
      // vectors, 64 VGPRs next to its 128 accumulator AGPRs, and spilled 2
      // VGPRs doing so: it reads each scale vector at its use instead and
      // spills none. (The W8A8 4-wave tile spills either way, fewer with the
      // cache.) The bias is always read per use.
      constexpr bool kCacheWs = kW8A8 || C::FN * kQ <= 8;
      f32x4 wsv[kCacheWs ? C::FN : 1][kCacheWs ? kQ : 1];
      if constexpr (kCacheWs) {
#pragma unroll
        for (int i = 0; i < C::FN; ++i)
#pragma unroll
          for (int q = 0; q < kQ; ++q)
            wsv[i][q] = kDq ? f32x4{1.0f, 1.0f, 1.0f, 1.0f}
                            : *reinterpret_cast<const f32x4*>(sc_w + MF * i + 8 * q + 4 * g);
      }
      auto wscale = [&](int i, int q) -> f32x4 {
        if constexpr (kCacheWs) return wsv[i][q];
        else if constexpr (kDq) return f32x4{1.0f, 1.0f, 1.0f, 1.0f};
        else return *reinterpret_cast<const f32x4*>(sc_w + MF * i + 8 * q + 4 * g);
      };
      const bool has_bias = bias != nullptr;
      TVQ_TL_MARK(4);
      auto epi_slices = [&](auto bias_c) {
        constexpr bool kBias = decltype(bias_c)::value;
#pragma unroll
        for (int j = 0; j < C::FM; ++j) {
          const int mrow0 = m0 + wm * C::TM + MF * j;  // first output row of this slice
          float as = 0.0f;
          if constexpr (kW8A8) as = sc[wm * C::TM + MF * j + r];
          if constexpr (kGlu) {
#pragma unroll
            for (int q = 0; q < kQ; ++q) {
              const int nl = 8 * q + 4 * g;  // output column within the wave tile
              float o[4];
              const f32x4 wg = wscale(0, q), wu = wscale(1, q);
#pragma unroll
              for (int t = 0; t < 4; ++t) {
                const float gt = to_float<T>(from_float<T>(epi_w8a8_nb(acc[0][j][4 * q + t], as, wg[t])));
                const float ut = to_float<T>(from_float<T>(epi_w8a8_nb(acc[1][j][4 * q + t], as, wu[t])));
                o[t] = silu_f(gt) * ut;
              }
              u32x2 pk;
              pk.x = (uint32_t)from_float<T>(o[0]) | ((uint32_t)from_float<T>(o[1]) << 16);
              pk.y = (uint32_t)from_float<T>(o[2]) | ((uint32_t)from_float<T>(o[3]) << 16);
              *reinterpret_cast<u32x2*>(stg + r * kRowB + 16 * ((nl >> 3) ^ sswz(r)) + 2 * (nl & 7)) = pk;
            }
          } else
#pragma unroll
          for (int i = 0; i < C::FN; ++i) {
#pragma unroll
            for (int q = 0; q < kQ; ++q) {
              const int nl = MF * i + 8 * q + 4 * g;   // column within the wave tile (multiple of 4)
              f32x4 bv = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
              if constexpr (kBias) bv = *reinterpret_cast<const f32x4*>(sc_b + nl);
              float o[4];
              const f32x4 wv = wscale(i, q);
#pragma unroll
              for (int t = 0; t < 4; ++t) {
                if constexpr (kW8A8)
                  o[t] = kBias ? epi_w8a8(acc[i][j][4 * q + t], as, wv[t], bv[t])
                               : epi_w8a8_nb(acc[i][j][4 * q + t], as, wv[t]);
                else
                  o[t] = kBias ? epi_w8a16(acc[i][j][4 * q + t], wv[t], bv[t])
                               : epi_w8a16_nb(acc[i][j][4 * q + t], wv[t]);
              }
              u32x2 pk;
              pk.x = (uint32_t)from_float<T>(o[0]) | ((uint32_t)from_float<T>(o[1]) << 16);
              pk.y = (uint32_t)from_float<T>(o[2]) | ((uint32_t)from_float<T>(o[3]) << 16);
              *reinterpret_cast<u32x2*>(stg + r * kRowB + 16 * ((nl >> 3) ^ sswz(r)) + 2 * (nl & 7)) = pk;
            }
          }
          // LDS operations of one wave complete in order; the wait and the
          // compiler barrier keep the read-back after the writes above.
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          TVQ_TL_MARK(5);
#pragma unroll
          for (int ps = 0; ps < kPass; ++ps) {
            const int e = ps * 64 + lane;
            const int row = e / kCh;
            const int ch = e % kCh;
            const u32x4 val = *reinterpret_cast<const u32x4*>(stg + row * kRowB + 16 * (ch ^ sswz(row)));
            const int mo = mrow0 + row;
            const int no = ncol_out + 8 * ch;
            if (mo < M && no < n_out) {
              uint16_t* dst = y + (int64_t)mo * n_out + no;
              if (vec && no + 8 <= n_out) {
                *reinterpret_cast<u32x4*>(dst) = val;
              } else {
#pragma unroll
                for (int t = 0; t < 8; ++t)
                  if (no + t < n_out) dst[t] = (uint16_t)(val[t >> 1] >> (16 * (t & 1)));
              }
            }
          }
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          TVQ_TL_MARK(6);
        }
      };
      if (has_bias)
        epi_slices(std::true_type{});
      else
        epi_slices(std::false_type{});
    }
    }
    if (!more) break;
  }
  TVQ_TL_MARK(3);
}

// CU count of the current device (cached per device; 0 without a device).
inline int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
#ifdef TVQ_TEST_HOOKS
  cus[dev] = 0;  // CPU-emulation builds of the tests: the CU count may change between calls
#endif
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
    cus[dev] = n;
  }
  return cus[dev];
}

// Workgroups one CU holds for a given LDS footprint, times the CU count: the
// persistent grid size.
inline int resident_workgroups(int lds_bytes) {
  const int per_cu = lds_bytes > 0 ? (160 * 1024) / lds_bytes : 1;
  return device_cus() * (per_cu > 0 ? per_cu : 1);
}

// Host-side launcher for one configuration.
// Number of split-K ranges for a launch: as many as keep the work units
// within one per CU (more units than CUs measured slower: a second round, or
// two units sharing a CU's load bandwidth), at least kMinStages k-stages per
// range, and a workspace that holds every range's accumulator image
// (1 = no split).
inline int choose_splits(int tiles, int nk, int cus, int tile_bytes, const void* wsp, int64_t ws_bytes) {
  constexpr int kMinStages = 8, kMaxSplits = 16;
  if (wsp == nullptr || cus <= 0 || tiles <= 0 || tiles > kSplitMaxTiles) return 1;
  int s = min(cus / tiles, min(nk / kMinStages, kMaxSplits));
  while (s > 1 && kSplitCntBytes + (int64_t)tiles * s * tile_bytes > ws_bytes) --s;
  if (s <= 1) return 1;
  const int per = (nk + s - 1) / s;  // every range non-empty
  return (nk + per - 1) / per;
}

// Stream-K range length (tile-stages per workgroup) for `tiles` tiles of `nk`
// k-stages on `cus` CUs: one workgroup per CU, each owning an equal share of
// the tiles' k-stages, but at least min_stages of them (TVQ_STREAMK_MIN,
// default 8); 0 when the workspace cannot hold two accumulator images per
// workgroup or the counters (then the launch does not use stream-K). *grid
// receives the workgroup count.
inline int streamk_min_stages() { return switches().streamk_min; }

inline int choose_streamk(int tiles, int nk, int cus, int tile_bytes, const void* wsp, int64_t ws_bytes, int* grid) {
  const int kMinStages = streamk_min_stages();
  if (wsp == nullptr || cus <= 0 || tiles <= 0 || nk <= 0 || tiles > kSplitMaxTiles) return 0;
  const int64_t total = (int64_t)tiles * nk;
  int64_t g = min((int64_t)cus, total / kMinStages);
  if (g < 1) g = 1;
  const int64_t len = (total + g - 1) / g;
  g = (total + len - 1) / len;  // every workgroup's range is non-empty
  if (kSplitCntBytes + 2 * g * (int64_t)tile_bytes > ws_bytes) return 0;
  *grid = (int)g;
  return (int)len;
}

// kSK: stream-K (one workgroup per CU, equal k-stage shares; falls back to an
// unsplit launch when the workspace cannot hold two images per workgroup).
template <typename T, bool kW8A8, bool kRaw, int BM, int BN, int WM, int WN, int S, int MF, int KS, bool kSplit,
          bool kNtW = false, bool kGlu = false, bool kRot = false, bool kDmaOnly = false, bool kDq = false,
          bool kSK = false>
hipError_t launch_dma(const void* x, const float* a_s, const int8_t* qw, const float* ws, const void* bias, void* y,
                      int M, int N, int K, int group, int m_major, int splits, void* wsp, int64_t ws_bytes,
                      hipStream_t stream) {
  using C = Cfg<kW8A8, BM, BN, WM, WN, S, MF, KS>;
  if constexpr (kSK) {
    int g = 0;
    const int len = choose_streamk(((M + BM - 1) / BM) * ((N + BN - 1) / BN), K / KS, device_cus(), BM * BN * 4, wsp,
                                   ws_bytes, &g);
    if (len <= 0)
      return launch_dma<T, kW8A8, kRaw, BM, BN, WM, WN, S, MF, KS, false, kNtW, kGlu, kRot, kDmaOnly, kDq>(
          x, a_s, qw, ws, bias, y, M, N, K, group, m_major, 1, nullptr, 0, stream);
    auto kern = gemm_dma_kernel<T, kW8A8, kRaw, BM, BN, WM, WN, S, MF, KS, true, kNtW, kGlu, kRot, kDmaOnly, kDq, true>;
    static bool sk_attr_set = false;
    if (!sk_attr_set) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, C::kLdsBytes);
      if (e != hipSuccess) return e;
      sk_attr_set = true;
    }
    kern<<<dim3(g), dim3(C::kThreads), C::kLdsBytes, stream>>>(x, a_s, qw, ws, static_cast<const uint16_t*>(bias), y,
                                                                M, N, K, group, m_major, 1, static_cast<char*>(wsp),
                                                                len);
    return hipGetLastError();
  }
  auto kern = gemm_dma_kernel<T, kW8A8, kRaw, BM, BN, WM, WN, S, MF, KS, kSplit, kNtW, kGlu, kRot, kDmaOnly, kDq>;
  static bool attr_set = false;  // idempotent; a benign race sets it twice
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, C::kLdsBytes);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  // The kernel writes tiles * splits images and `tiles` counters into the
  // workspace: anything that does not fit runs unsplit.
  if (!kSplit || wsp == nullptr || splits < 1 || tiles > kSplitMaxTiles ||
      kSplitCntBytes + (int64_t)tiles * splits * (BM * BN * 4) > ws_bytes)
    splits = 1;
  const int units = tiles * splits;
  const int resident = resident_workgroups(C::kLdsBytes);
  int grid = units;
  // keep whole XCD rounds (8 XCDs), but never round a small device's grid to zero
  if (resident > 0 && units > resident) grid = resident >= 8 ? resident - resident % 8 : resident;
  kern<<<dim3(grid), dim3(C::kThreads), C::kLdsBytes, stream>>>(x, a_s, qw, ws, static_cast<const uint16_t*>(bias),
                                                                 y, M, N, K, group, m_major, splits,
                                                                 static_cast<char*>(wsp), 0);
  return hipGetLastError();
}

}  // namespace dma
}  // namespace tvq
