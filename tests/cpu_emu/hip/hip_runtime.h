// CPU emulation of the HIP runtime and of the gfx950 builtins that the
// kernels in tiny-vllm_amd/csrc use. TEST INFRASTRUCTURE ONLY: it lets the
// unchanged kernel sources be compiled for the host (tests/cpu_emu/build.py)
// and run on the CPU, under AddressSanitizer, against the oracle. The
// product library is never built with it, and nothing in the package loads it.
//
// Execution model. A launch runs its workgroups one after another, or
// EMU_CONCURRENT=n of them interleaved. Every work-item is a cooperative
// fiber (ucontext) on one OS thread; a fiber runs until it reaches a workgroup barrier, a wave-level
// operation or its end. Wave-level operations (cross-lane shuffles,
// readfirstlane, MFMA, the transposing LDS read, LDS DMA) are executed by the
// scheduler for all lanes of the wave that wait on it, once no fiber can run:
// lanes that have exited or sit elsewhere are the inactive lanes. Every
// resident workgroup has its own LDS, static and dynamic, fresh and poisoned
// (0xff) when the workgroup starts; EMU_CONCURRENT=n interleaves n workgroups.
//
// Arithmetic. MFMA results are computed in double and rounded once to fp32
// (exact for the int8 forms); v_dot2 likewise. exp2 and rcp are the libm
// results, so those differ from the hardware's by about an ulp. LDS DMA
// completes when issued (the earliest time the hardware may complete it).
// With EMU_DMA=late it lands only at the wave's vmcnt wait (the latest).
// An LDS wait (s_waitcnt lgkmcnt) is a rendezvous of the wave's lanes, which
// stands in for the hardware's lockstep execution of a wave. EMU_SHUFFLE=seed
// runs the fibers in a seeded random order instead of round-robin, and lets
// interleaved workgroups sit out steps at random.
#pragma once

#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <functional>
#include <tuple>
#include <type_traits>
#include <utility>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __constant__
#define __align__(n) __attribute__((aligned(n)))

#ifndef __HIP_MEMORY_SCOPE_AGENT
#define __HIP_MEMORY_SCOPE_AGENT 3
#endif
#ifndef __HIP_MEMORY_SCOPE_WORKGROUP
#define __HIP_MEMORY_SCOPE_WORKGROUP 2
#endif

struct dim3 {
  unsigned x, y, z;
  constexpr dim3(unsigned x_ = 1, unsigned y_ = 1, unsigned z_ = 1) : x(x_), y(y_), z(z_) {}
};

typedef struct emu_stream* hipStream_t;
enum hipError_t { hipSuccess = 0, hipErrorInvalidValue = 1, hipErrorOutOfMemory = 2, hipErrorLaunchFailure = 719,
                  hipErrorInvalidConfiguration = 9 };
enum hipFuncAttribute { hipFuncAttributeMaxDynamicSharedMemorySize = 8 };
enum hipDeviceAttribute_t { hipDeviceAttributeMultiprocessorCount = 63 };

namespace emu {

// ---- fibers ---------------------------------------------------------------
struct Lane;
typedef void (*WaveFn)(Lane** lanes);  // lanes[0..63]: waiting lanes of one wave, nullptr = inactive

struct Lane {
  dim3 tid;
  int wave, lane;
  int state;
  WaveFn fn;
  alignas(64) unsigned char in[4][64];
  alignas(64) unsigned char out[64];
  void* priv;  // scheduler-private
};

Lane* cur();
const dim3& block_idx();
const dim3& block_dim();
const dim3& grid_dim();
void barrier();
void wave_sync(WaveFn fn);  // post this lane's inputs (in[]) and wait for the wave's result (out)
void* dyn_smem();
void* lds_slot(const void* key, size_t bytes);  // this workgroup's storage for one static __shared__ array

// A static __shared__ declaration becomes a reference to per-workgroup
// storage (tests/cpu_emu/build.py rewrites it); `key` is unique per
// declaration and template instantiation.
template <typename T>
inline T& lds(const void* key) {
  return *static_cast<T*>(lds_slot(key, sizeof(T)));
}
int cu_count();
void set_last_error(hipError_t e);
hipError_t take_last_error();
void run_grid(dim3 grid, dim3 block, size_t shmem, const std::function<void()>& body, const void* kernel);

template <typename... P, typename... A>
void launch(void (*k)(P...), dim3 grid, dim3 block, size_t shmem, hipStream_t, A&&... args) {
  static_assert(sizeof...(P) == sizeof...(A), "kernel argument count");
  std::tuple<std::decay_t<P>...> t(((std::decay_t<P>)(args))...);
  run_grid(grid, block, shmem, [&]() { std::apply(k, t); }, (const void*)k);
}

// `kern<<<...>>>` where kern is itself a function-pointer variable
template <typename... P, typename... A>
void launch(void (**k)(P...), dim3 grid, dim3 block, size_t shmem, hipStream_t st, A&&... args) {
  launch(*k, grid, block, shmem, st, std::forward<A>(args)...);
}

// A wave-level operation's operands pass through the lane's in[] / out[]
// slots, which the scheduler reads and writes between the lanes' turns: not
// memory of the kernel, so the race-checking build leaves these copies
// uninstrumented (the operation's own memory accesses are checked through
// lane_access).
#define EMU_UNCHECKED __attribute__((no_sanitize("thread")))
template <typename T>
EMU_UNCHECKED inline void put(Lane* l, int slot, const T& v) {
  static_assert(sizeof(T) <= 64, "wave-op operand");
  __builtin_memcpy_inline(l->in[slot], &v, sizeof(T));
}
template <typename T>
EMU_UNCHECKED inline T get_in(const Lane* l, int slot) {
  T v;
  __builtin_memcpy_inline(&v, l->in[slot], sizeof(T));
  return v;
}
template <typename T>
EMU_UNCHECKED inline T get_out(const Lane* l) {
  T v;
  __builtin_memcpy_inline(&v, l->out, sizeof(T));
  return v;
}

// The memory access of one lane within a wave-level operation (the scheduler
// performs the operation for the wave): checked as that lane's access in the
// race-checking build, a no-op otherwise.
void lane_access(Lane* l, const void* p, size_t n, bool write);

// ---- cross-lane ---------------------------------------------------------
void wait_vm(int n);
template <int B>
void shfl_fn(Lane** L) {  // in[0]: value (B bytes), in[1]: source lane
  unsigned char tmp[64][B];
  for (int i = 0; i < 64; ++i)
    if (L[i]) {
      const int src = get_in<int>(L[i], 1);
      if (src < 0 || src >= 64 || !L[src]) {
        memset(tmp[i], 0, B);  // inactive source lane: no defined value
      } else {
        memcpy(tmp[i], L[src]->in[0], B);
      }
    }
  for (int i = 0; i < 64; ++i)
    if (L[i]) memcpy(L[i]->out, tmp[i], B);
}

template <typename T>
T shfl_from(T v, int src) {
  Lane* l = cur();
  put(l, 0, v);
  put(l, 1, src);
  wave_sync(&shfl_fn<sizeof(T)>);
  return get_out<T>(l);
}

inline void rfl_fn(Lane** L) {
  int first = -1;
  for (int i = 0; i < 64; ++i)
    if (L[i]) { first = i; break; }
  for (int i = 0; i < 64; ++i)
    if (L[i]) memcpy(L[i]->out, L[first]->in[0], 4);
}

inline void ballot_fn(Lane** L) {
  uint64_t m = 0;
  for (int i = 0; i < 64; ++i)
    if (L[i] && get_in<int>(L[i], 0)) m |= uint64_t(1) << i;
  for (int i = 0; i < 64; ++i)
    if (L[i]) memcpy(L[i]->out, &m, 8);
}

inline void nop_fn(Lane**) {}

// A wave's lanes run in lockstep on the hardware, so LDS written by one lane
// is visible to the others once the writing instruction has completed (the
// kernels wait for it with s_waitcnt lgkmcnt). The emulation makes such a
// wait a rendezvous of the wave's active lanes.
inline void wave_barrier() { wave_sync(&nop_fn); }

}  // namespace emu

#define threadIdx (::emu::cur()->tid)
#define blockIdx (::emu::block_idx())
#define blockDim (::emu::block_dim())
#define gridDim (::emu::grid_dim())
#define hipLaunchKernelGGL(k, g, b, s, st, ...) ::emu::launch(k, dim3(g), dim3(b), s, st, __VA_ARGS__)
#define HIP_SYMBOL(x) ((const void*)&(x))

inline void __syncthreads() { ::emu::barrier(); }
inline unsigned __lane_id() { return (unsigned)::emu::cur()->lane; }

template <typename T>
inline T __shfl_xor(T v, int mask, int width = 64) {
  const int lane = ::emu::cur()->lane;
  const int base = lane & ~(width - 1);
  int src = lane ^ mask;
  if (src >= base + width) src = lane;
  return ::emu::shfl_from(v, src);
}
template <typename T>
inline T __shfl(T v, int src, int width = 64) {
  const int lane = ::emu::cur()->lane;
  return ::emu::shfl_from(v, (lane & ~(width - 1)) + (src & (width - 1)));
}

inline int __builtin_amdgcn_readfirstlane(int v) {
  ::emu::Lane* l = ::emu::cur();
  ::emu::put(l, 0, v);
  ::emu::wave_sync(&::emu::rfl_fn);
  return ::emu::get_out<int>(l);
}

inline uint64_t __builtin_amdgcn_ballot_w64(bool p) {
  ::emu::Lane* l = ::emu::cur();
  ::emu::put(l, 0, (int)p);
  ::emu::wave_sync(&::emu::ballot_fn);
  return ::emu::get_out<uint64_t>(l);
}

// ---- scalar helpers ---------------------------------------------------------
// HIP's integer min / max (device overloads; mixed types take the common type)
template <typename A, typename B, typename = std::enable_if_t<std::is_integral<A>::value && std::is_integral<B>::value>>
inline std::common_type_t<A, B> min(A a, B b) { return a < b ? a : b; }
template <typename A, typename B, typename = std::enable_if_t<std::is_integral<A>::value && std::is_integral<B>::value>>
inline std::common_type_t<A, B> max(A a, B b) { return a < b ? b : a; }

inline float __fdiv_rn(float a, float b) { return a / b; }
inline float __fsqrt_rn(float a) { return sqrtf(a); }
inline float __builtin_amdgcn_exp2f(float a) { return exp2f(a); }
inline float __builtin_amdgcn_rcpf(float a) { return 1.0f / a; }
// s_waitcnt immediate (gfx9): lgkmcnt in bits 11:8; any wait with lgkmcnt < 15
// orders this wave's LDS accesses: a wave rendezvous in the emulation
// and the vmcnt field (bits 3:0 and 15:14) completes this wave's queued DMA.
inline void __builtin_amdgcn_s_waitcnt(int imm) {
  const int vm = (imm & 15) | (((imm >> 14) & 3) << 4);
  if (vm < 63) ::emu::wait_vm(vm);
  if (((imm >> 8) & 15) != 15) ::emu::wave_barrier();
}
inline void __builtin_amdgcn_sched_barrier(int) {}
inline void __builtin_amdgcn_sched_group_barrier(int, int, int) {}

// v_perm_b32: byte i of the result is selected by byte i of sel from the
// 8 bytes {src1 (bytes 0-3), src0 (bytes 4-7)}; 12 gives 0x00, 13-15 0xff,
// 8-11 the sign of byte 1, 3, 5, 7 replicated.
inline uint32_t __builtin_amdgcn_perm(uint32_t src0, uint32_t src1, uint32_t sel) {
  const uint64_t v = ((uint64_t)src0 << 32) | src1;
  uint32_t r = 0;
  for (int i = 0; i < 4; ++i) {
    const uint32_t s = (sel >> (8 * i)) & 0xff;
    uint32_t b;
    if (s < 8) b = (uint32_t)(v >> (8 * s)) & 0xff;
    else if (s < 12) b = ((v >> (8 * (2 * (s - 8) + 1) + 7)) & 1) ? 0xff : 0x00;
    else if (s == 12) b = 0;
    else b = 0xff;
    r |= b << (8 * i);
  }
  return r;
}

inline int __builtin_amdgcn_sdot4(int a, int b, int c, bool) {
  int64_t s = c;
  for (int i = 0; i < 4; ++i) s += (int64_t)(int8_t)(a >> (8 * i)) * (int8_t)(b >> (8 * i));
  return (int)s;  // the kernels never reach the clamp range
}

typedef __bf16 emu_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 emu_f16x2 __attribute__((ext_vector_type(2)));
inline float __builtin_amdgcn_fdot2_f32_bf16(emu_bf16x2 a, emu_bf16x2 b, float c, bool) {
  return (float)((double)(float)a[0] * (double)(float)b[0] + (double)(float)a[1] * (double)(float)b[1] + (double)c);
}
inline float __builtin_amdgcn_fdot2(emu_f16x2 a, emu_f16x2 b, float c, bool) {
  return (float)((double)(float)a[0] * (double)(float)b[0] + (double)(float)a[1] * (double)(float)b[1] + (double)c);
}

// ---- atomics: clang's __hip_atomic_* builtins also exist for the host target.

// ---- MFMA -----------------------------------------------------------------
// 16x16xK: lane l holds A row l%16 and B column l%16 for k group l/16 (the
// k order inside the dot product is irrelevant to the result as long as A and
// B agree, which the instruction guarantees); D element v of lane l is row
// 4*(l/16) + v, column l%16.
// 32x32xK: A row / B column l%32, k group l/32; D element v of lane l is row
// 8*(v/4) + 4*(l/32) + v%4, column l%32.
namespace emu {
template <typename E, int NE, bool kInt, int MN>
void mfma_fn(Lane** L) {  // in[0]: A (NE elements), in[1]: B, in[2]: C (MN*MN/64 values)
  constexpr int G = 64 / MN;        // k groups
  constexpr int NV = MN * MN / 64;  // accumulators per lane
  double a[MN][G][NE], b[MN][G][NE];
  for (int l = 0; l < 64; ++l) {
    if (!L[l]) {
      for (int e = 0; e < NE; ++e) a[l % MN][l / MN][e] = b[l % MN][l / MN][e] = 0.0;
      continue;
    }
    E av[NE], bv[NE];
    memcpy(av, L[l]->in[0], sizeof(av));
    memcpy(bv, L[l]->in[1], sizeof(bv));
    for (int e = 0; e < NE; ++e) {
      a[l % MN][l / MN][e] = (double)av[e];
      b[l % MN][l / MN][e] = (double)bv[e];
    }
  }
  for (int l = 0; l < 64; ++l) {
    if (!L[l]) continue;
    const int j = l % MN;
    for (int v = 0; v < NV; ++v) {
      const int i = MN == 16 ? 4 * (l / 16) + v : 8 * (v / 4) + 4 * (l / 32) + v % 4;
      double s = 0.0;
      for (int g = 0; g < G; ++g)
        for (int e = 0; e < NE; ++e) s += a[i][g][e] * b[j][g][e];
      if (kInt) {
        int32_t c;
        memcpy(&c, L[l]->in[2] + 4 * v, 4);
        const int32_t r = (int32_t)((int64_t)c + (int64_t)s);
        memcpy(L[l]->out + 4 * v, &r, 4);
      } else {
        float c;
        memcpy(&c, L[l]->in[2] + 4 * v, 4);
        const float r = (float)((double)c + s);
        memcpy(L[l]->out + 4 * v, &r, 4);
      }
    }
  }
}

template <typename R, typename E, int NE, bool kInt, int MN, typename VA, typename VC>
inline R mfma(const VA& a, const VA& b, const VC& c) {
  Lane* l = cur();
  put(l, 0, a);
  put(l, 1, b);
  put(l, 2, c);
  wave_sync(&mfma_fn<E, NE, kInt, MN>);
  return get_out<R>(l);
}
}  // namespace emu

typedef __bf16 emu_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 emu_f16x8 __attribute__((ext_vector_type(8)));
typedef float emu_f32x4 __attribute__((ext_vector_type(4)));
typedef float emu_f32x16 __attribute__((ext_vector_type(16)));
typedef int32_t emu_i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t emu_i32x16 __attribute__((ext_vector_type(16)));

inline emu_f32x4 __builtin_amdgcn_mfma_f32_16x16x32_bf16(emu_bf16x8 a, emu_bf16x8 b, emu_f32x4 c, int, int, int) {
  return ::emu::mfma<emu_f32x4, __bf16, 8, false, 16>(a, b, c);
}
inline emu_f32x4 __builtin_amdgcn_mfma_f32_16x16x32_f16(emu_f16x8 a, emu_f16x8 b, emu_f32x4 c, int, int, int) {
  return ::emu::mfma<emu_f32x4, _Float16, 8, false, 16>(a, b, c);
}
inline emu_f32x16 __builtin_amdgcn_mfma_f32_32x32x16_bf16(emu_bf16x8 a, emu_bf16x8 b, emu_f32x16 c, int, int, int) {
  return ::emu::mfma<emu_f32x16, __bf16, 8, false, 32>(a, b, c);
}
inline emu_f32x16 __builtin_amdgcn_mfma_f32_32x32x16_f16(emu_f16x8 a, emu_f16x8 b, emu_f32x16 c, int, int, int) {
  return ::emu::mfma<emu_f32x16, _Float16, 8, false, 32>(a, b, c);
}
inline emu_i32x4 __builtin_amdgcn_mfma_i32_16x16x64_i8(emu_i32x4 a, emu_i32x4 b, emu_i32x4 c, int, int, int) {
  return ::emu::mfma<emu_i32x4, int8_t, 16, true, 16>(a, b, c);
}
inline emu_i32x16 __builtin_amdgcn_mfma_i32_32x32x32_i8(emu_i32x4 a, emu_i32x4 b, emu_i32x16 c, int, int, int) {
  return ::emu::mfma<emu_i32x16, int8_t, 16, true, 32>(a, b, c);
}

// ---- LDS ------------------------------------------------------------------
// ds_read_b64_tr_b16: within each 16-lane group, element e of lane i is
// 16-bit element i%4 of the 8-byte row addressed by lane 4e + i/4.
typedef short emu_v4i16 __attribute__((ext_vector_type(4)));
namespace emu {
inline void tr16_fn(Lane** L) {
  for (int i = 0; i < 64; ++i) {
    if (!L[i]) continue;
    const int g = i & ~15, li = i & 15;
    short r[4];
    for (int e = 0; e < 4; ++e) {
      Lane* src = L[g + 4 * e + li / 4];
      if (!src) { r[e] = 0; continue; }
      const short* row = get_in<const short*>(src, 0);
      r[e] = row[li % 4];
    }
    memcpy(L[i]->out, r, 8);
  }
  for (int i = 0; i < 64; ++i)
    if (L[i]) lane_access(L[i], get_in<const short*>(L[i], 0), 8, false);  // each lane's address: 8 bytes
}

// global_load_lds: lane l copies `size` bytes from its global address to
// LDS at (the first active lane's LDS pointer) + offset + l * size. In the
// default mode the copy happens at issue; with EMU_DMA=late it is queued on
// the wave and lands only when the wave waits for it (s_waitcnt vmcnt), the
// latest time the hardware may complete it.
bool dma_late();
void dma_enqueue(Lane* issuer, char* dst, const char* src, int size);
void wait_vm(int n);  // this wave: complete queued DMA until at most n remain

inline void dma_fn(Lane** L) {
  int first = -1;
  for (int i = 0; i < 64; ++i)
    if (L[i]) { first = i; break; }
  char* base = get_in<char*>(L[first], 1);
  const int size = get_in<int>(L[first], 2);
  const int off = get_in<int>(L[first], 3);
  const bool late = dma_late();
  if (late) dma_enqueue(L[first], nullptr, nullptr, -1);  // one vm op per instruction
  for (int i = 0; i < 64; ++i) {
    if (!L[i]) continue;
    const char* src = get_in<const char*>(L[i], 0);
    if (late) {
      dma_enqueue(L[i], base + off + i * size, src, size);  // checked where it lands
    } else {
      lane_access(L[i], src, size, false);
      lane_access(L[i], base + off + i * size, size, true);
      memcpy(base + off + i * size, src, size);
    }
  }
}
}  // namespace emu

inline emu_v4i16 __builtin_amdgcn_ds_read_tr16_b64_v4i16(emu_v4i16* p) {
  ::emu::Lane* l = ::emu::cur();
  ::emu::put(l, 0, (const short*)p);
  ::emu::wave_sync(&::emu::tr16_fn);
  return ::emu::get_out<emu_v4i16>(l);
}

inline void __builtin_amdgcn_global_load_lds(const void* g, void* lds, int size, int offset, int) {
  ::emu::Lane* l = ::emu::cur();
  ::emu::put(l, 0, (const char*)g);
  ::emu::put(l, 1, (char*)lds);
  ::emu::put(l, 2, size);
  ::emu::put(l, 3, offset);
  ::emu::wave_sync(&::emu::dma_fn);
}

// ---- host API -------------------------------------------------------------
inline hipError_t hipGetLastError() { return ::emu::take_last_error(); }
inline hipError_t hipPeekAtLastError() { return hipSuccess; }
inline const char* hipGetErrorString(hipError_t e) {
  switch (e) {
    case hipSuccess: return "no error";
    case hipErrorInvalidValue: return "invalid argument";
    case hipErrorInvalidConfiguration: return "invalid configuration argument";
    default: return "emulated HIP error";
  }
}
inline hipError_t hipGetDevice(int* d) { *d = 0; return hipSuccess; }
inline hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t a, int) {
  *v = a == hipDeviceAttributeMultiprocessorCount ? ::emu::cu_count() : 0;
  return hipSuccess;
}
template <typename K>
inline hipError_t hipFuncSetAttribute(K, hipFuncAttribute, int) { return hipSuccess; }
inline hipError_t hipMalloc(void** p, size_t n) { *p = calloc(1, n ? n : 1); return *p ? hipSuccess : hipErrorOutOfMemory; }
inline hipError_t hipFree(void* p) { free(p); return hipSuccess; }
inline hipError_t hipGetSymbolAddress(void** p, const void* sym) { *p = const_cast<void*>(sym); return hipSuccess; }
