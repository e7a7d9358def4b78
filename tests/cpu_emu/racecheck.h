// Race checking of the emulated kernels (test infrastructure; the _race
// build of tests/cpu_emu/build.py). The kernel sources are compiled with the
// host compiler's ThreadSanitizer instrumentation, which turns every memory
// access into a call; racecheck.cpp supplies those calls (no ThreadSanitizer
// runtime is involved) and checks each access against the GPU's rules, using
// what the emulator knows of the accessing work-item:
//   * two work-items of one workgroup conflict when they are in different
//     waves and in the same barrier interval (between two workgroup
//     barriers); the lanes of one wave run in lockstep and never conflict;
//   * two workgroups of one launch always conflict (nothing orders them);
//   * a conflict needs a write and at least one non-atomic access;
//   * an LDS DMA copy that lands late (EMU_DMA=late) spans the barrier
//     intervals from its issue to its wave's vmcnt wait, and also conflicts
//     with its own wave's accesses between issue and wait;
//   * launches are ordered (a new launch forgets the previous one's
//     accesses); host code, the lanes' own stacks and the scheduler are not
//     checked.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace emu {
struct Lane;
namespace race {

struct Who {
  uint32_t blk;     // workgroup serial within the launch
  uint32_t lo, hi;  // barrier intervals the access spans
  uint16_t wave;
};

// Implemented by the scheduler (emu_runtime.cpp).
bool current(Who* w, const void* addr);  // the running work-item; false: not checked here
void who_of(Lane* l, Who* w);            // a lane's, during a wave-level operation

// Implemented by racecheck.cpp.
void launch_begin(const void* kernel);
uint32_t seq();  // position of the next access in the launch's order
void reset(const void* p, size_t n);  // fresh memory (a workgroup's LDS)
// dma_seq != 0: a late DMA copy's landing; dma_seq is seq() when it was issued
void access(const void* p, size_t n, bool write, bool atomic, const Who& w, const void* pc, uint32_t dma_seq = 0);

}  // namespace race
}  // namespace emu
