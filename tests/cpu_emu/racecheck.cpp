// Race checker of the emulated kernels (test infrastructure): the rules are
// in racecheck.h. Shadow state per 4-byte granule: two writes and two reads
// (the latest of two different waves), each with the bytes it touched, its
// workgroup, wave, barrier intervals, position in the launch and code
// address; two accesses conflict only where their bytes overlap (rows of
// 2-byte or 1-byte elements may meet inside a granule).
// Launches run on one OS thread in this build, so nothing here is shared
// between threads.
#include "racecheck.h"

#include <cxxabi.h>
#include <dlfcn.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <set>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace emu {
namespace race {
namespace {

enum : uint8_t { kValid = 1, kWrite = 2, kAtomic = 4, kDma = 8 };

struct Acc {
  const void* pc;
  uint32_t blk, lo, hi, seq;
  uint16_t wave;
  uint8_t flags, mask;  // mask: bytes of the granule
};

struct Ent {
  Acc w[2], r[2];
};

constexpr int kPageShift = 12;                         // 4 KiB of memory per shadow page
constexpr int kGranules = (1 << kPageShift) / 4;       // 4-byte granules

std::unordered_map<uint64_t, Ent*> g_pages;
std::vector<Ent*> g_free;
uint64_t g_last_key = ~0ull;
Ent* g_last = nullptr;
uint32_t g_seq = 1;
const void* g_kernel = nullptr;
std::set<std::pair<const void*, const void*>> g_seen;
int g_reports = 0;

Ent* page(uint64_t key, bool create) {
  if (key == g_last_key) return g_last;
  auto it = g_pages.find(key);
  Ent* p = nullptr;
  if (it != g_pages.end()) {
    p = it->second;
  } else {
    if (!create) return nullptr;
    if (!g_free.empty()) {
      p = g_free.back();
      g_free.pop_back();
    } else {
      p = static_cast<Ent*>(malloc(sizeof(Ent) * kGranules));
      if (!p) abort();
    }
    memset(p, 0, sizeof(Ent) * kGranules);
    g_pages.emplace(key, p);
  }
  g_last_key = key;
  g_last = p;
  return p;
}

std::string symbol(const void* pc) {
  Dl_info info;
  if (pc == nullptr || !dladdr(pc, &info)) return "?";
  std::string name = "?";
  if (info.dli_sname) {
    int st = 0;
    char* d = abi::__cxa_demangle(info.dli_sname, nullptr, nullptr, &st);
    name = st == 0 && d ? d : info.dli_sname;
    free(d);
    if (name.size() > 160) name = name.substr(0, 160) + "...";
  }
  char off[64];
  snprintf(off, sizeof off, " (%s+0x%lx)", info.dli_fname ? strrchr(info.dli_fname, '/') + 1 : "?",
           (unsigned long)((const char*)pc - (const char*)info.dli_fbase));
  return name + off;
}

void describe(const char* role, const Acc& a) {
  fprintf(stderr, "  %s %s%s%s by workgroup %u wave %u, barrier interval %u", role,
          a.flags & kAtomic ? "atomic " : "", a.flags & kDma ? "LDS DMA " : "", a.flags & kWrite ? "write" : "read",
          a.blk, a.wave, a.lo);
  if (a.hi != a.lo) fprintf(stderr, "-%u", a.hi);
  fprintf(stderr, "\n    at %s\n", symbol(a.pc).c_str());
}

void report(const void* addr, const Acc& prev, const Acc& cur) {
  if (!g_seen.insert({prev.pc, cur.pc}).second) return;  // one report per pair of code addresses
  ++g_reports;
  fprintf(stderr, "emu race: kernel %s, address %p\n", symbol(g_kernel).c_str(), addr);
  describe("this", cur);
  describe("previous", prev);
}

// Whether accesses a (earlier) and b (now) are unordered on the GPU.
bool unordered(const Acc& a, const Acc& b, uint32_t dma_seq) {
  if (a.blk != b.blk) return true;
  if (a.wave == b.wave) return dma_seq != 0 && a.seq >= dma_seq;  // the wave's own access between issue and wait
  return a.lo <= b.hi && b.lo <= a.hi;
}

void check(const void* addr, const Acc& prev, const Acc& cur, uint32_t dma_seq) {
  if (!(prev.flags & kValid) || !(prev.mask & cur.mask)) return;
  if (!((prev.flags | cur.flags) & kWrite)) return;
  if (prev.flags & cur.flags & kAtomic) return;
  if (unordered(prev, cur, dma_seq)) report(addr, prev, cur);
}

bool same_actor(const Acc& a, const Acc& b) { return a.blk == b.blk && a.wave == b.wave; }

// Record cur in one of two slots: the same wave's (bytes merged), a free one,
// one whose bytes cur covers, or else in place of the older one.
void record(Acc (&slot)[2], const Acc& cur) {
  for (Acc& a : slot)
    if ((a.flags & kValid) && same_actor(a, cur)) {
      const uint8_t m = a.mask | cur.mask;
      a = cur;
      a.mask = m;
      return;
    }
  for (Acc& a : slot)
    if (!(a.flags & kValid) || (a.mask & ~cur.mask) == 0) {
      a = cur;
      return;
    }
  slot[1] = slot[0];
  slot[0] = cur;
}

}  // namespace

void launch_begin(const void* kernel) {
  for (auto& kv : g_pages) g_free.push_back(kv.second);
  g_pages.clear();
  g_last_key = ~0ull;
  g_last = nullptr;
  g_seq = 1;
  g_kernel = kernel;
}

uint32_t seq() { return g_seq; }

void reset(const void* p, size_t n) {
  const uintptr_t a = (uintptr_t)p & ~(uintptr_t)3, end = (uintptr_t)p + n;
  for (uintptr_t g = a; g < end; g += 4) {
    Ent* pg = page(g >> kPageShift, false);
    if (pg) memset(&pg[(g >> 2) & (kGranules - 1)], 0, sizeof(Ent));
  }
}

void access(const void* p, size_t n, bool write, bool atomic, const Who& w, const void* pc, uint32_t dma_seq) {
  if (n == 0) return;
  Acc cur{pc, w.blk, w.lo, w.hi, g_seq++, w.wave,
          (uint8_t)(kValid | (write ? kWrite : 0) | (atomic ? kAtomic : 0) | (dma_seq ? kDma : 0)), 0};
  const uintptr_t lo = (uintptr_t)p, hi = lo + n;
  for (uintptr_t g = lo & ~(uintptr_t)3; g < hi; g += 4) {
    const uintptr_t b0 = lo > g ? lo - g : 0, b1 = hi < g + 4 ? hi - g : 4;
    cur.mask = (uint8_t)(((1u << b1) - 1) & ~((1u << b0) - 1));
    Ent& e = page(g >> kPageShift, true)[(g >> 2) & (kGranules - 1)];
    for (const Acc& a : e.w) check((const void*)g, a, cur, dma_seq);
    if (write) {
      for (const Acc& a : e.r) check((const void*)g, a, cur, dma_seq);
      record(e.w, cur);
    } else {
      record(e.r, cur);
    }
  }
}

}  // namespace race
}  // namespace emu

// ---- the instrumentation's entry points --------------------------------------
using emu::race::Who;

namespace {
inline void rc(const void* p, size_t n, bool write, bool atomic, const void* pc) {
  Who w;
  if (emu::race::current(&w, p)) emu::race::access(p, n, write, atomic, w, pc);
}
}  // namespace

#define RC_PC __builtin_extract_return_addr(__builtin_return_address(0))

extern "C" {
int tvq_emu_race_reports(void) { return emu::race::g_reports; }

void __tsan_init(void) {}
void __tsan_func_entry(void*) {}
void __tsan_func_exit(void) {}
void __tsan_vptr_update(void**, void*) {}
void __tsan_vptr_read(void**) {}

#define RC_RW(N)                                                                         \
  void __tsan_read##N(void* p) { rc(p, N, false, false, RC_PC); }                        \
  void __tsan_write##N(void* p) { rc(p, N, true, false, RC_PC); }                        \
  void __tsan_unaligned_read##N(void* p) { rc(p, N, false, false, RC_PC); }              \
  void __tsan_unaligned_write##N(void* p) { rc(p, N, true, false, RC_PC); }              \
  void __tsan_volatile_read##N(void* p) { rc(p, N, false, false, RC_PC); }               \
  void __tsan_volatile_write##N(void* p) { rc(p, N, true, false, RC_PC); }
RC_RW(1)
RC_RW(2)
RC_RW(4)
RC_RW(8)
RC_RW(16)
#undef RC_RW

void __tsan_read_range(void* p, unsigned long n) { rc(p, n, false, false, RC_PC); }
void __tsan_write_range(void* p, unsigned long n) { rc(p, n, true, false, RC_PC); }
void* __tsan_memcpy(void* d, const void* s, unsigned long n) {
  rc(s, n, false, false, RC_PC);
  rc(d, n, true, false, RC_PC);
  return memcpy(d, s, n);
}
void* __tsan_memmove(void* d, const void* s, unsigned long n) {
  rc(s, n, false, false, RC_PC);
  rc(d, n, true, false, RC_PC);
  return memmove(d, s, n);
}
void* __tsan_memset(void* d, int c, unsigned long n) {
  rc(d, n, true, false, RC_PC);
  return memset(d, c, n);
}

void __tsan_atomic_thread_fence(int) { __atomic_thread_fence(__ATOMIC_SEQ_CST); }
void __tsan_atomic_signal_fence(int) {}

// Atomics: the instrumentation replaces the operation with the call, so
// these perform it (sequentially consistent: one OS thread runs a launch).
#define RC_ATOMIC(N, T)                                                                            \
  T __tsan_atomic##N##_load(const volatile T* a, int) {                                            \
    rc((const void*)a, sizeof(T), false, true, RC_PC);                                             \
    return __atomic_load_n(a, __ATOMIC_SEQ_CST);                                                   \
  }                                                                                                \
  void __tsan_atomic##N##_store(volatile T* a, T v, int) {                                         \
    rc((const void*)a, sizeof(T), true, true, RC_PC);                                              \
    __atomic_store_n(a, v, __ATOMIC_SEQ_CST);                                                      \
  }                                                                                                \
  T __tsan_atomic##N##_exchange(volatile T* a, T v, int) {                                         \
    rc((const void*)a, sizeof(T), true, true, RC_PC);                                              \
    return __atomic_exchange_n(a, v, __ATOMIC_SEQ_CST);                                            \
  }                                                                                                \
  T __tsan_atomic##N##_fetch_add(volatile T* a, T v, int) {                                        \
    rc((const void*)a, sizeof(T), true, true, RC_PC);                                              \
    return __atomic_fetch_add(a, v, __ATOMIC_SEQ_CST);                                             \
  }                                                                                                \
  T __tsan_atomic##N##_fetch_sub(volatile T* a, T v, int) {                                        \
    rc((const void*)a, sizeof(T), true, true, RC_PC);                                              \
    return __atomic_fetch_sub(a, v, __ATOMIC_SEQ_CST);                                             \
  }                                                                                                \
  T __tsan_atomic##N##_fetch_and(volatile T* a, T v, int) {                                        \
    rc((const void*)a, sizeof(T), true, true, RC_PC);                                              \
    return __atomic_fetch_and(a, v, __ATOMIC_SEQ_CST);                                             \
  }                                                                                                \
  T __tsan_atomic##N##_fetch_or(volatile T* a, T v, int) {                                         \
    rc((const void*)a, sizeof(T), true, true, RC_PC);                                              \
    return __atomic_fetch_or(a, v, __ATOMIC_SEQ_CST);                                              \
  }                                                                                                \
  T __tsan_atomic##N##_fetch_xor(volatile T* a, T v, int) {                                        \
    rc((const void*)a, sizeof(T), true, true, RC_PC);                                              \
    return __atomic_fetch_xor(a, v, __ATOMIC_SEQ_CST);                                             \
  }                                                                                                \
  T __tsan_atomic##N##_fetch_nand(volatile T* a, T v, int) {                                       \
    rc((const void*)a, sizeof(T), true, true, RC_PC);                                              \
    return __atomic_fetch_nand(a, v, __ATOMIC_SEQ_CST);                                            \
  }                                                                                                \
  int __tsan_atomic##N##_compare_exchange_strong(volatile T* a, T* c, T v, int, int) {             \
    rc((const void*)a, sizeof(T), true, true, RC_PC);                                              \
    return __atomic_compare_exchange_n(a, c, v, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST);        \
  }                                                                                                \
  int __tsan_atomic##N##_compare_exchange_weak(volatile T* a, T* c, T v, int, int) {               \
    rc((const void*)a, sizeof(T), true, true, RC_PC);                                              \
    return __atomic_compare_exchange_n(a, c, v, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST);        \
  }                                                                                                \
  T __tsan_atomic##N##_compare_exchange_val(volatile T* a, T c, T v, int, int) {                   \
    rc((const void*)a, sizeof(T), true, true, RC_PC);                                              \
    __atomic_compare_exchange_n(a, &c, v, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST);              \
    return c;                                                                                      \
  }
RC_ATOMIC(8, int8_t)
RC_ATOMIC(16, int16_t)
RC_ATOMIC(32, int32_t)
RC_ATOMIC(64, int64_t)
#undef RC_ATOMIC
}
