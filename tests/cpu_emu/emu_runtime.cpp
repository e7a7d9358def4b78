// Fiber scheduler of the CPU emulation of HIP kernels (test infrastructure;
// see hip/hip_runtime.h for the execution model).
//
// A launch runs its workgroups EMU_CONCURRENT at a time (default 1): the
// fibers of all resident workgroups share one scheduler, so workgroups that
// hand work to each other through global memory (split-K and stream-K
// fixups, the attention kernels' fused quantization) meet in whatever order
// the interleaving produces. Each resident workgroup has its own LDS: the
// dynamic allocation and every static __shared__ array (see lds_slot).
// With one resident workgroup (the default), the workgroups of a launch are
// independent of each other's timing and are spread over EMU_THREADS OS
// threads (default: the host's CPUs, at most 8), each with its own scheduler.
#include <setjmp.h>
#include <stdio.h>
#include <sys/mman.h>
#include <ucontext.h>

#include <algorithm>
#include <deque>
#include <random>
#include <thread>
#include <unordered_map>
#include <vector>

#include "hip/hip_runtime.h"
#ifdef EMU_RACE
#include "racecheck.h"
#endif

#if defined(__has_feature)
#if __has_feature(address_sanitizer)
#define EMU_ASAN 1
#endif
#endif
#ifdef EMU_ASAN
extern "C" {
void __sanitizer_start_switch_fiber(void** fake_stack_save, const void* bottom, size_t size);
void __sanitizer_finish_switch_fiber(void* fake_stack_save, const void** bottom_old, size_t* size_old);
}
#endif

namespace emu {
namespace {

enum { kRun = 0, kWave = 1, kBar = 2, kDone = 3 };
constexpr size_t kStack = 256 << 10;

struct Block;

// Switches: a fiber starts on its own stack through ucontext (once); after
// that, scheduler and fiber switch with _setjmp / _longjmp, which unlike
// swapcontext make no signal-mask system call. The AddressSanitizer build
// keeps swapcontext throughout (its fiber annotations assume it).
struct Fiber {
  Lane lane;
  ucontext_t ctx;
  jmp_buf jb;
  bool started = false;
  char* stack = nullptr;
  Block* blk = nullptr;
};

struct DmaOp {
  char* dst;
  const char* src;
  int size;  // -1: the start of one wave instruction (one vm op)
  Lane* issuer;
  uint32_t iv, seq;  // race checking: barrier interval and access position at issue
};

struct Block {
  dim3 bid, bdim, gdim;
  int n = 0;
  Fiber* fibers = nullptr;
  void* smem = nullptr;
  std::unordered_map<const void*, void*> lds;  // static __shared__ arrays of this workgroup
  std::vector<std::deque<DmaOp>> dma;          // per wave
  bool active = false;
  uint32_t serial = 0;    // position in the launch (race checking)
  uint32_t interval = 0;  // workgroup barriers passed
};

thread_local ucontext_t g_sched;
thread_local jmp_buf g_sched_jb;
thread_local const void* g_sched_stack_bottom = nullptr;
thread_local size_t g_sched_stack_size = 0;
thread_local Block* g_blk = nullptr;
thread_local Fiber* g_cur = nullptr;
thread_local uint32_t g_serial = 0;  // workgroups started in this launch
const std::function<void()>* g_body = nullptr;  // the running launch's kernel call (read-only while it runs)
hipError_t g_err = hipSuccess;

// Land the queued DMA of wave w until at most keep_ops instructions remain
// (`check`: the race-checking build checks each copy where it lands).
void dma_flush_wave(Block& b, int w, int keep_ops, bool check) {
  std::deque<DmaOp>& q = b.dma[w];
  int ops = 0;
  for (const DmaOp& d : q) ops += d.size < 0;
  while (ops > keep_ops && !q.empty()) {
    q.pop_front();  // instruction marker
    --ops;
    while (!q.empty() && q.front().size >= 0) {
      const DmaOp& d = q.front();
#ifdef EMU_RACE
      if (check) {
        race::Who who{b.serial, d.iv, b.interval, (uint16_t)w};
        race::access(d.src, d.size, false, false, who, nullptr, d.seq);
        race::access(d.dst, d.size, true, false, who, nullptr, d.seq);
      }
#else
      (void)check;
#endif
      memcpy(d.dst, d.src, d.size);
      q.pop_front();
    }
  }
}

void to_sched() {
#ifdef EMU_ASAN
  __sanitizer_start_switch_fiber(nullptr, g_sched_stack_bottom, g_sched_stack_size);
  swapcontext(&g_cur->ctx, &g_sched);
  __sanitizer_finish_switch_fiber(nullptr, nullptr, nullptr);
#else
  if (!_setjmp(g_cur->jb)) _longjmp(g_sched_jb, 1);
#endif
}

// Scheduler side: run fiber f until it blocks or ends.
void switch_to(Fiber* f) {
#ifdef EMU_ASAN
  __sanitizer_start_switch_fiber(nullptr, f->stack, kStack);
  swapcontext(&g_sched, &f->ctx);
  __sanitizer_finish_switch_fiber(nullptr, nullptr, nullptr);
#else
  if (!_setjmp(g_sched_jb)) {
    if (!f->started) {
      f->started = true;
      setcontext(&f->ctx);
    }
    _longjmp(f->jb, 1);
  }
#endif
}

void fiber_entry() {
#ifdef EMU_ASAN
  __sanitizer_finish_switch_fiber(nullptr, &g_sched_stack_bottom, &g_sched_stack_size);
#endif
  (*g_body)();
  g_cur->lane.state = kDone;
#ifdef EMU_ASAN
  __sanitizer_start_switch_fiber(nullptr, g_sched_stack_bottom, g_sched_stack_size);
  setcontext(&g_sched);
#else
  _longjmp(g_sched_jb, 1);
#endif
}

void start_block(Block& b, Fiber* fibers, dim3 bid, size_t shmem) {
  b.bid = bid;
  b.fibers = fibers;
  b.active = true;
  // dynamic shared memory: a fresh allocation of exactly the launch's size,
  // filled with a NaN pattern (uninitialised LDS)
  b.smem = shmem ? malloc(shmem) : nullptr;
  if (shmem) memset(b.smem, 0xff, shmem);
#ifdef EMU_RACE
  b.serial = g_serial++;
  b.interval = 0;
  if (shmem) race::reset(b.smem, shmem);
#endif
  b.dma.assign((b.n + 63) / 64, {});
  for (int i = 0; i < b.n; ++i) {
    Fiber& f = fibers[i];
    const unsigned t = (unsigned)i;
    f.blk = &b;
    f.lane.tid = dim3(t % b.bdim.x, (t / b.bdim.x) % b.bdim.y, t / (b.bdim.x * b.bdim.y));
    f.lane.wave = i / 64;
    f.lane.lane = i % 64;
    f.lane.state = kRun;
    f.lane.fn = nullptr;
    f.started = false;
    getcontext(&f.ctx);
    f.ctx.uc_stack.ss_sp = f.stack;
    f.ctx.uc_stack.ss_size = kStack;
    f.ctx.uc_link = nullptr;
    makecontext(&f.ctx, fiber_entry, 0);
  }
}

void finish_block(Block& b) {
  // copies never waited for land at the end (their wave may have read the
  // destination before)
  for (size_t w = 0; w < b.dma.size(); ++w) dma_flush_wave(b, (int)w, 0, true);
  free(b.smem);
  b.smem = nullptr;
  for (auto& kv : b.lds) free(kv.second);
  b.lds.clear();
  b.active = false;
}

// Resolve the wave-level operations of every wave of `b` whose waiting lanes
// all wait on the same one; returns whether any ran.
bool resolve_waves(Block& b) {
  bool resolved = false;
  const int nwaves = (b.n + 63) / 64;
  for (int w = 0; w < nwaves; ++w) {
    Lane* L[64] = {};
    WaveFn fn = nullptr;
    bool any = false;
    for (int l = 0; l < 64 && w * 64 + l < b.n; ++l) {
      Lane& ln = b.fibers[w * 64 + l].lane;
      if (ln.state != kWave) continue;
      if (fn == nullptr) fn = ln.fn;
      if (ln.fn != fn) {
        fprintf(stderr, "emu: wave %d of block (%u,%u,%u): lanes wait on different wave operations\n", w, b.bid.x,
                b.bid.y, b.bid.z);
        abort();
      }
      L[l] = &ln;
      any = true;
    }
    if (!any) continue;
    Block* saved = g_blk;
    g_blk = &b;
    fn(L);
    g_blk = saved;
    for (int l = 0; l < 64; ++l)
      if (L[l]) L[l]->state = kRun;
    resolved = true;
  }
  return resolved;
}

}  // namespace

Lane* cur() { return &g_cur->lane; }
const dim3& block_idx() { return g_blk->bid; }
const dim3& block_dim() { return g_blk->bdim; }
const dim3& grid_dim() { return g_blk->gdim; }
void* dyn_smem() { return g_blk->smem; }

void* lds_slot(const void* key, size_t bytes) {
  void*& p = g_blk->lds[key];
  if (p == nullptr) {
    p = aligned_alloc(1024, (bytes + 1023) / 1024 * 1024);
    memset(p, 0xff, bytes);
#ifdef EMU_RACE
    race::reset(p, bytes);
#endif
  }
  return p;
}

void lane_access(Lane* l, const void* p, size_t n, bool write) {
#ifdef EMU_RACE
  race::Who w;
  race::who_of(l, &w);
  race::access(p, n, write, false, w, nullptr);
#else
  (void)l, (void)p, (void)n, (void)write;
#endif
}

#ifdef EMU_RACE
namespace race {
bool current(Who* w, const void* addr) {
  if (g_cur == nullptr) return false;  // host code, or the scheduler
  if ((const char*)addr >= g_cur->stack && (const char*)addr < g_cur->stack + kStack) return false;
  who_of(&g_cur->lane, w);
  return true;
}
void who_of(Lane* l, Who* w) {
  const Block* b = reinterpret_cast<Fiber*>(l)->blk;  // the lane is the fiber's first member
  *w = Who{b->serial, b->interval, b->interval, (uint16_t)l->wave};
}
}  // namespace race
#endif

int cu_count() {
  const char* e = getenv("EMU_CUS");
  return e ? atoi(e) : 256;
}

void barrier() {
  g_cur->lane.state = kBar;
  to_sched();
}

void wave_sync(WaveFn fn) {
  g_cur->lane.fn = fn;
  g_cur->lane.state = kWave;
  to_sched();
}

bool dma_late() {
  static const char* e = getenv("EMU_DMA");
  return e != nullptr && strcmp(e, "late") == 0;
}

void dma_enqueue(Lane* issuer, char* dst, const char* src, int size) {
  uint32_t seq = 0;
#ifdef EMU_RACE
  seq = race::seq();
#endif
  g_blk->dma[issuer->wave].push_back(DmaOp{dst, src, size, issuer, g_blk->interval, seq});
}

void wait_vm(int n) {
  if (g_cur != nullptr && !g_blk->dma.empty()) dma_flush_wave(*g_blk, g_cur->lane.wave, n, true);
}

void set_last_error(hipError_t e) { g_err = e; }
hipError_t take_last_error() {
  const hipError_t e = g_err;
  g_err = hipSuccess;
  return e;
}

namespace {

// Run workgroups first, first + stride, ... of the launch, `conc` resident
// at a time, on this thread.
void run_range(dim3 grid, dim3 block, size_t shmem, long first, long stride, int conc_req) {
  const long n = (long)block.x * block.y * block.z;
  const long nblocks = (long)grid.x * grid.y * grid.z;
  const long mine = first < nblocks ? (nblocks - first + stride - 1) / stride : 0;
  if (mine == 0) return;
  const int conc = (int)std::max(1L, std::min(mine, (long)conc_req));
  std::vector<Fiber> pool(n * conc);
  for (Fiber& f : pool) {
    void* st = mmap(nullptr, kStack, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
    if (st == MAP_FAILED) abort();
    f.stack = static_cast<char*>(st);
  }
  static const char* shuffle = getenv("EMU_SHUFFLE");
  static std::mt19937 rng(shuffle ? (unsigned)atoi(shuffle) : 0u);
  std::vector<Block> slots(conc);
  long next = 0;  // index into this thread's workgroups
  auto bid_of = [&](long j) {
    const long i = first + j * stride;
    return dim3((unsigned)(i % grid.x), (unsigned)((i / grid.x) % grid.y), (unsigned)(i / ((long)grid.x * grid.y)));
  };
  for (int s = 0; s < conc; ++s) {
    slots[s].bdim = block;
    slots[s].gdim = grid;
    slots[s].n = (int)n;
    start_block(slots[s], &pool[s * n], bid_of(next++), shmem);
  }
  // One step of a resident workgroup: run its runnable fibers (each until it
  // blocks); else resolve its waves' pending wave-level operations; else
  // release its barrier, or retire it and start the next workgroup in its
  // slot. Returns whether it progressed.
  std::vector<Fiber*> order;
  auto step = [&](int s) -> bool {
    Block& b = slots[s];
    order.clear();
    for (int i = 0; i < b.n; ++i)
      if (b.fibers[i].lane.state == kRun) order.push_back(&b.fibers[i]);
    if (shuffle) std::shuffle(order.begin(), order.end(), rng);
    for (Fiber* f : order) {
      g_cur = f;
      g_blk = f->blk;
      switch_to(f);
      g_cur = nullptr;
    }
    if (!order.empty()) return true;
    if (resolve_waves(b)) return true;
    int live = 0, at_bar = 0;
    for (int i = 0; i < b.n; ++i) {
      if (b.fibers[i].lane.state != kDone) ++live;
      if (b.fibers[i].lane.state == kBar) ++at_bar;
    }
    if (live == 0) {
      finish_block(b);
      if (next < mine) start_block(b, &pool[s * n], bid_of(next++), shmem);
      return true;
    }
    if (at_bar == live) {
      ++b.interval;
      for (int i = 0; i < b.n; ++i)
        if (b.fibers[i].lane.state == kBar) b.fibers[i].lane.state = kRun;
      return true;
    }
    return false;
  };
  std::vector<int> perm(conc);
  for (int s = 0; s < conc; ++s) perm[s] = s;
  for (;;) {
    bool any_active = false, progress = false;
    if (shuffle) std::shuffle(perm.begin(), perm.end(), rng);
    for (int s : perm) {
      if (!slots[s].active) continue;
      any_active = true;
      // shuffled mode: a resident workgroup sits out a step at random, so
      // workgroups drift apart instead of moving in lockstep
      if (shuffle && conc > 1 && (rng() & 1)) continue;
      progress |= step(s);
    }
    if (!any_active) break;
    if (progress) continue;
    for (int s : perm)  // a step with nothing stalled
      if (slots[s].active) progress |= step(s);
    if (!progress) {
      fprintf(stderr, "emu: deadlock (no workgroup can progress)\n");
      abort();
    }
  }
  for (Fiber& f : pool) munmap(f.stack, kStack);
  g_blk = nullptr;
}

}  // namespace

void run_grid(dim3 grid, dim3 block, size_t shmem, const std::function<void()>& body, const void* kernel) {
  const long n = (long)block.x * block.y * block.z;
  if (n <= 0 || n > 1024 || grid.x == 0 || grid.y == 0 || grid.z == 0 || shmem > (160u << 10)) {
    set_last_error(hipErrorInvalidConfiguration);
    return;
  }
  const long nblocks = (long)grid.x * grid.y * grid.z;
  static const char* conc_env = getenv("EMU_CONCURRENT");
  static const char* thr_env = getenv("EMU_THREADS");
  const int conc = conc_env ? std::max(1, atoi(conc_env)) : 1;
  int threads = thr_env ? std::max(1, atoi(thr_env))
                        : (int)std::min(8u, std::max(1u, std::thread::hardware_concurrency()));
  if (conc > 1 || nblocks < 2) threads = 1;  // interleaved workgroups share one scheduler
#ifdef EMU_RACE
  threads = 1;  // the checker's shadow state is not shared between threads
  g_serial = 0;
  race::launch_begin(kernel);
#else
  (void)kernel;
#endif
  threads = (int)std::min<long>(threads, nblocks);
  const std::function<void()>* saved_body = g_body;
  g_body = &body;
  if (threads == 1) {
    run_range(grid, block, shmem, 0, 1, conc);
  } else {
    std::vector<std::thread> ts;
    for (int t = 0; t < threads; ++t) ts.emplace_back(run_range, grid, block, shmem, (long)t, (long)threads, 1);
    for (auto& t : ts) t.join();
  }
  g_body = saved_body;
}

}  // namespace emu
