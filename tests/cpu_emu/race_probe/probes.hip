// Kernels that pin the emulation's race checker (test infrastructure, built
// only for the CPU emulation by tests/test_cpu_emu_race.py; never for a GPU).
// Each racy probe has a correctly synchronised twin: the checker must report
// the first and stay silent on the second. Run with EMU_DMA=late.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__device__ __forceinline__ void wait_vm0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// one wave writes LDS, the others read it: with and without a barrier between
template <bool kBarrier>
__global__ void lds_cross_wave(int* out) {
  __shared__ int s[4];
  if (threadIdx.x % 64 == 0) s[threadIdx.x / 64] = threadIdx.x;
  if (kBarrier) __syncthreads();
  out[threadIdx.x] = s[(threadIdx.x / 64 + 1) % 4];
}

// lanes of one wave exchange values through LDS (lockstep: no barrier needed)
__global__ void lds_within_wave(int* out) {
  __shared__ int s[64];
  s[threadIdx.x] = threadIdx.x;
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  out[threadIdx.x] = s[63 - threadIdx.x];
}

// two workgroups update one word: plainly, or both atomically
template <bool kAtomic>
__global__ void two_groups_one_word(int* p) {
  if (threadIdx.x != 0) return;
  if (kAtomic)
    __hip_atomic_fetch_add(p, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    p[0] += 1;
}

// one workgroup writes a word plainly, another reads it atomically
__global__ void plain_write_atomic_read(int* p) {
  if (threadIdx.x != 0) return;
  if (blockIdx.x == 0)
    p[0] = 5;
  else
    p[1] = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// workgroups write disjoint words
__global__ void disjoint_groups(int* p) { p[blockIdx.x * 64 + threadIdx.x] = threadIdx.x; }

// wave 0 copies 64 words into LDS by DMA and reads them back (its own copy):
// without waiting for it, or after vmcnt(0)
template <bool kWait>
__global__ void dma_own_read(int* p) {
  __shared__ int s[64];
  if (threadIdx.x < 64) {
    __builtin_amdgcn_global_load_lds(p + 64 + threadIdx.x, s, 4, 0, 0);
    if (kWait) wait_vm0();
    p[threadIdx.x] = s[63 - threadIdx.x];
  }
}

// wave 0 copies into LDS and waits; wave 1 reads the copy, with or without a
// barrier after the wait
template <bool kBarrier>
__global__ void dma_other_wave_read(int* p) {
  __shared__ int s[64];
  if (threadIdx.x < 64) {
    __builtin_amdgcn_global_load_lds(p + 64 + threadIdx.x, s, 4, 0, 0);
    wait_vm0();
  }
  if (kBarrier) __syncthreads();
  if (threadIdx.x >= 64) p[threadIdx.x] = s[threadIdx.x - 64];
}

// wave 1 reads an LDS buffer that wave 0 then refills by DMA: in the same
// barrier interval, or after a barrier (the refill waits before the end)
template <bool kBarrier>
__global__ void dma_overwrites_read(int* p) {
  __shared__ int s[64];
  if (threadIdx.x < 64) s[threadIdx.x] = 1;
  __syncthreads();
  if (threadIdx.x >= 64) p[threadIdx.x] = s[threadIdx.x - 64];
  if (kBarrier) __syncthreads();
  if (threadIdx.x < 64) {
    __builtin_amdgcn_global_load_lds(p + 256 + threadIdx.x, s, 4, 0, 0);
    wait_vm0();
  }
}

}  // namespace

// Probe `which` on p (1024 ints); returns -1 for an unknown probe.
extern "C" int race_probe(int which, int* p) {
  switch (which) {
    case 0: lds_cross_wave<false><<<1, 256, 0, nullptr>>>(p); break;
    case 1: lds_cross_wave<true><<<1, 256, 0, nullptr>>>(p); break;
    case 2: lds_within_wave<<<1, 64, 0, nullptr>>>(p); break;
    case 3: two_groups_one_word<false><<<2, 64, 0, nullptr>>>(p); break;
    case 4: two_groups_one_word<true><<<2, 64, 0, nullptr>>>(p); break;
    case 5: plain_write_atomic_read<<<2, 64, 0, nullptr>>>(p); break;
    case 6: disjoint_groups<<<4, 64, 0, nullptr>>>(p); break;
    case 7: dma_own_read<false><<<1, 64, 0, nullptr>>>(p); break;
    case 8: dma_own_read<true><<<1, 64, 0, nullptr>>>(p); break;
    case 9: dma_other_wave_read<false><<<1, 128, 0, nullptr>>>(p); break;
    case 10: dma_other_wave_read<true><<<1, 128, 0, nullptr>>>(p); break;
    case 11: dma_overwrites_read<false><<<1, 128, 0, nullptr>>>(p); break;
    case 12: dma_overwrites_read<true><<<1, 128, 0, nullptr>>>(p); break;
    default: return -1;
  }
  return 0;
}
