// phases.h - ordering of the phases of a one-launch operation.
//
// A plan operation runs as one AOT launch (one entry point per (profile,
// operation), kernels/launch_contract/types.mbt:16-27). Where its work has
// steps that depend on each other row band by row band (quantize the
// activation rows, then the GEMM that reads them; gate/up, then the hidden
// quantizer, then down), the grid holds the steps' blocks in step order,
// and a block of a later step waits, with a bounded poll, for a counter
// that the blocks of the earlier step add to once their stores are
// complete. All counters live in the operation's workspace (the sync area,
// at its start), each in a 128-byte line of its own:
//   byte 0                     error word: 0, or 1 once a wait ran out (sticky)
//   byte 128                   done counter of the last step's blocks
//   byte 256 + 128 (s bands + b)  band counter of step s, row band b
// sized sync_bytes(steps, bands). (Counters sharing a line with the ones
// hundreds of blocks poll reached those blocks ~8 us late: the W8A16
// one-launch GatedMlp's four slice counts in one line, polled by 256 blocks,
// became visible 4-8 us after their last add; one line each, ~1 us.) The
// binding zero-fills the area once; the last
// block of the last step to finish puts every counter back to zero, so every
// launch starts from zeros.
//
// Why the waits end. Workgroups are dispatched in index order on each XCD,
// and a block only waits for blocks of lower index. Take the lowest block
// that has not finished: every block it waits for has finished, and every
// block before it on its XCD has finished and freed its CU, so it is
// dispatched and runs to its end. The polls are bounded all the same (about
// 2^20 polls, ~30 ms): a poll that runs out sets the error word, and the
// block stores nothing and returns.
// After an error: the last block does not reset the counters, and every
// wait of a later launch reads the error word with its first poll and fails,
// so no block that depends on a wait stores an output (blocks of a first
// step, which wait for nothing, may still rewrite their part of the
// workspace); the host reads the word after a synchronous launch,
// zero-fills the workspace and reports the failure.
//
// Visibility. The stores a later step reads go through the XCD's L2 to
// memory (agent-scope atomic stores and write-through stores: the sc1
// cache policy), and a block counts itself done only after every wave's
// stores have completed (s_waitcnt vmcnt(0), then the block barrier). A
// reader loads the rows of a band only after the band's counter reached its
// target, and no block of the launch touches those lines before that (the
// writer's own XCD keeps its write-through copy current; a launch starts
// with the L2 invalidated), so the reader's L2 misses and fetches the
// written values. This keeps L2-wide write-back and invalidate fences off
// the path (they cost the W8A16 one-launch GatedMlp 2-3x its time).
#pragma once

#include "device_common.h"

namespace phase {

constexpr int kSpinLimit = 1 << 20;

LF_DEVICE int load_agent(const int *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
LF_DEVICE void store_agent(int *p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Ints per 128-byte line: counters polled by many blocks get a line each.
constexpr int kLineInts = 32;

struct Sync {
  int *base;
  int bands;
  LF_DEVICE int *error() const { return base; }
  LF_DEVICE int *done() const { return base + kLineInts; }
  LF_DEVICE int *band(int step, int b) const { return base + kLineInts * (2 + step * bands + b); }
};

LF_DEVICE uint64_t sync_bytes(int steps, int bands) {
  return 256 + 128ull * static_cast<uint64_t>(steps) * static_cast<uint64_t>(bands);
}

// The flag word every block keeps in LDS to broadcast thread 0's decisions.
struct Flag {
  int value;
};

// Counts this block into `counter` once the stores of all its waves have
// completed.
LF_DEVICE void signal(int *counter) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits until *counter >= target. False if the poll ran out (the error word
// is then set) or another block's had: the caller loads nothing that
// depends on the wait and stores nothing.
// Each poll is one device-scope round trip (the counter); the error word is
// read every 32nd poll only (measured: a second, dependent load per poll
// put the wait's end 2.5-5 us after the last count).
// The first poll also reads the error word (both loads in flight at once),
// so a launch on a failed workspace stores nothing without a separate check.
LF_DEVICE bool wait_for(const int *counter, int target, int *error, Flag &flag) {
  if (threadIdx.x == 0) {
    int ok = 1, spins = 0;
    const int first = load_agent(counter);
    if (load_agent(error) != 0) ok = 0;
    for (int c = first; ok && c < target; c = load_agent(counter)) {
      if ((++spins & 31) == 0) {
        if (load_agent(error) != 0) {
          ok = 0;
          break;
        }
        if (spins > kSpinLimit) {
          store_agent(error, 1);
          ok = 0;
          break;
        }
      }
      __builtin_amdgcn_s_sleep(1);
    }
    flag.value = ok;
  }
  __syncthreads();
  const bool ok = flag.value != 0;
  __syncthreads();
  return ok;
}
LF_DEVICE bool wait_for(const Sync &s, const int *counter, int target, Flag &flag) {
  return wait_for(counter, target, s.error(), flag);
}

// Called by every block of the last step once it is done (its waits are
// over): the last of `total` such blocks resets the `steps` x bands band
// counters and the done counter, unless the error word is set.
LF_DEVICE void finish(const Sync &s, int total, int steps, Flag &flag) {
  __syncthreads();
  if (threadIdx.x == 0) {
    const int before = __hip_atomic_fetch_add(s.done(), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    flag.value = before == total - 1 && load_agent(s.error()) == 0;
  }
  __syncthreads();
  if (flag.value != 0) {
    for (int i = threadIdx.x; i < steps * s.bands; i += blockDim.x) store_agent(s.band(0, 0) + kLineInts * i, 0);
    if (threadIdx.x == 0) store_agent(s.done(), 0);
  }
}

// 16 bytes stored through the XCD's L2 (the cache policy of an agent-scope
// atomic store), for outputs that blocks on other XCDs read in this launch.
LF_DEVICE void store16_through(void *p, u32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}

}  // namespace phase
