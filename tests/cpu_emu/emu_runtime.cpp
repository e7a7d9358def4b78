// Fiber scheduler of the CPU emulation of HIP kernels (test infrastructure;
// see hip/hip_runtime.h for the execution model).
#include <stdio.h>
#include <sys/mman.h>
#include <ucontext.h>

#include <deque>
#include <random>
#include <vector>

#include "hip/hip_runtime.h"

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

struct Fiber {
  Lane lane;
  ucontext_t ctx;
  char* stack = nullptr;
};

struct Block {
  dim3 bid, bdim, gdim;
  int n = 0;
  std::vector<Fiber>* fibers = nullptr;
  const std::function<void()>* body = nullptr;
  void* smem = nullptr;
  ucontext_t sched;
  const void* sched_stack_bottom = nullptr;
  size_t sched_stack_size = 0;
};

struct DmaOp {
  char* dst;
  const char* src;
  int size;  // -1: the start of one wave instruction (one vm op)
};
std::vector<std::deque<DmaOp>> g_dma;  // per wave of the running workgroup

void dma_flush_wave(int w, int keep_ops) {
  std::deque<DmaOp>& q = g_dma[w];
  int ops = 0;
  for (const DmaOp& d : q) ops += d.size < 0;
  while (ops > keep_ops && !q.empty()) {
    q.pop_front();  // instruction marker
    --ops;
    while (!q.empty() && q.front().size >= 0) {
      memcpy(q.front().dst, q.front().src, q.front().size);
      q.pop_front();
    }
  }
}

Block* g_blk = nullptr;
Fiber* g_cur = nullptr;
hipError_t g_err = hipSuccess;
std::vector<Fiber> g_pool;

void to_sched() {
#ifdef EMU_ASAN
  __sanitizer_start_switch_fiber(nullptr, g_blk->sched_stack_bottom, g_blk->sched_stack_size);
#endif
  swapcontext(&g_cur->ctx, &g_blk->sched);
#ifdef EMU_ASAN
  __sanitizer_finish_switch_fiber(nullptr, nullptr, nullptr);
#endif
}

void fiber_entry() {
#ifdef EMU_ASAN
  __sanitizer_finish_switch_fiber(nullptr, &g_blk->sched_stack_bottom, &g_blk->sched_stack_size);
#endif
  (*g_blk->body)();
  g_cur->lane.state = kDone;
#ifdef EMU_ASAN
  __sanitizer_start_switch_fiber(nullptr, g_blk->sched_stack_bottom, g_blk->sched_stack_size);
#endif
  setcontext(&g_blk->sched);
}

void run_block(Block& b) {
  std::vector<Fiber>& F = *b.fibers;
  for (int i = 0; i < b.n; ++i) {
    Fiber& f = F[i];
    const unsigned t = (unsigned)i;
    f.lane.tid = dim3(t % b.bdim.x, (t / b.bdim.x) % b.bdim.y, t / (b.bdim.x * b.bdim.y));
    f.lane.wave = i / 64;
    f.lane.lane = i % 64;
    f.lane.state = kRun;
    f.lane.fn = nullptr;
    getcontext(&f.ctx);
    f.ctx.uc_stack.ss_sp = f.stack;
    f.ctx.uc_stack.ss_size = kStack;
    f.ctx.uc_link = nullptr;
    makecontext(&f.ctx, fiber_entry, 0);
  }
  const int nwaves = (b.n + 63) / 64;
  g_dma.assign(nwaves, {});
  static const char* shuffle = getenv("EMU_SHUFFLE");
  static std::mt19937 rng(shuffle ? (unsigned)atoi(shuffle) : 0u);
  std::vector<int> order(b.n);
  for (int i = 0; i < b.n; ++i) order[i] = i;
  for (;;) {
    bool ran = false;
    if (shuffle) std::shuffle(order.begin(), order.end(), rng);
    for (int oi = 0; oi < b.n; ++oi) {
      const int i = order[oi];
      if (F[i].lane.state != kRun) continue;
      g_cur = &F[i];
#ifdef EMU_ASAN
      __sanitizer_start_switch_fiber(nullptr, F[i].stack, kStack);
#endif
      swapcontext(&b.sched, &F[i].ctx);
#ifdef EMU_ASAN
      __sanitizer_finish_switch_fiber(nullptr, nullptr, nullptr);
#endif
      g_cur = nullptr;
      ran = true;
    }
    if (ran) continue;
    // nothing runnable: resolve the wave-level operations first
    bool resolved = false;
    for (int w = 0; w < nwaves; ++w) {
      Lane* L[64] = {};
      WaveFn fn = nullptr;
      bool any = false;
      for (int l = 0; l < 64 && w * 64 + l < b.n; ++l) {
        Lane& ln = F[w * 64 + l].lane;
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
      fn(L);
      for (int l = 0; l < 64; ++l)
        if (L[l]) L[l]->state = kRun;
      resolved = true;
    }
    if (resolved) continue;
    int live = 0, at_bar = 0;
    for (int i = 0; i < b.n; ++i) {
      if (F[i].lane.state != kDone) ++live;
      if (F[i].lane.state == kBar) ++at_bar;
    }
    if (live == 0) {
      for (int w = 0; w < nwaves; ++w) dma_flush_wave(w, 0);
      break;
    }
    if (at_bar == live) {
      for (int i = 0; i < b.n; ++i)
        if (F[i].lane.state == kBar) F[i].lane.state = kRun;
      continue;
    }
    fprintf(stderr, "emu: deadlock in block (%u,%u,%u)\n", b.bid.x, b.bid.y, b.bid.z);
    abort();
  }
}

}  // namespace

Lane* cur() { return &g_cur->lane; }
const dim3& block_idx() { return g_blk->bid; }
const dim3& block_dim() { return g_blk->bdim; }
const dim3& grid_dim() { return g_blk->gdim; }
void* dyn_smem() { return g_blk->smem; }

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

void dma_enqueue(int wave, char* dst, const char* src, int size) { g_dma[wave].push_back(DmaOp{dst, src, size}); }

void wait_vm(int n) {
  if (g_cur != nullptr && !g_dma.empty()) dma_flush_wave(g_cur->lane.wave, n);
}

void set_last_error(hipError_t e) { g_err = e; }
hipError_t take_last_error() {
  const hipError_t e = g_err;
  g_err = hipSuccess;
  return e;
}

void run_grid(dim3 grid, dim3 block, size_t shmem, const std::function<void()>& body) {
  const long n = (long)block.x * block.y * block.z;
  if (n <= 0 || n > 1024 || grid.x == 0 || grid.y == 0 || grid.z == 0 || shmem > (160u << 10)) {
    set_last_error(hipErrorInvalidConfiguration);
    return;
  }
  if ((long)g_pool.size() < n) {
    const size_t old = g_pool.size();
    g_pool.resize(n);
    for (size_t i = old; i < g_pool.size(); ++i) {
      void* s = mmap(nullptr, kStack, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
      if (s == MAP_FAILED) abort();
      g_pool[i].stack = static_cast<char*>(s);
    }
  }
  Block b;
  b.gdim = grid;
  b.bdim = block;
  b.n = (int)n;
  b.fibers = &g_pool;
  b.body = &body;
  Block* saved = g_blk;
  g_blk = &b;
  for (unsigned z = 0; z < grid.z; ++z)
    for (unsigned y = 0; y < grid.y; ++y)
      for (unsigned x = 0; x < grid.x; ++x) {
        b.bid = dim3(x, y, z);
        // dynamic shared memory: a fresh allocation of exactly the launch's
        // size per workgroup, filled with a NaN pattern (uninitialised LDS)
        b.smem = shmem ? malloc(shmem) : nullptr;
        if (shmem) memset(b.smem, 0xff, shmem);
        run_block(b);
        free(b.smem);
        b.smem = nullptr;
      }
  g_blk = saved;
}

}  // namespace emu
