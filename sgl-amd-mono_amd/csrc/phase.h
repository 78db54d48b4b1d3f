// What a phase of the layer needs from the launch that runs it: the guard, the launch
// tag and the CTA's shared flags, whether it runs as its own launch or as one phase of
// the whole-layer launch.
//
// Standalone, a launch's kernel reads the guard head, runs one phase and advances the
// epoch on its way out. In the layer launch the four phases run back to back in every
// CTA; between two phases sits a grid barrier (every CTA's stores of phase k drained
// before it arrives, the last arrival raises the barrier's flag to the launch tag), and
// each phase waits for it only after issuing the loads that do not depend on the phase
// before it (weights, cache pages). Every hand-off from one phase to the next is stored
// device coherent (sc1, write-through) and drained before its CTA arrives. The next phase
// reads it through L2: no cache line survives a kernel boundary, and within the launch no
// CU reads a hand-off buffer before its barrier, so no L2 can hold a stale copy of it. The
// one exception is a row's own cache entry, which the attention phase prefetches (its
// page) before the barrier: that one is read again device coherent after it.
#pragma once

#include "mono_device.h"

namespace mono {

// CTA-shared words of a launch: the guard head as read once, and the CTA's ok flag
struct LaunchShared {
  uint32_t head[4];
  int ok;
};

// Read the guard head (one coherent load, shared in LDS) and set up the guard; returns
// the launch tag (epoch + 1). Every thread calls it.
__device__ __attribute__((always_inline)) inline uint32_t launch_begin(LaunchShared& sh, Guard& guard, int32_t* gw,
                                        uint32_t* host_err, int fault_site, int fault_after) {
  if (threadIdx.x == 0) {
    const v4i hd = ld16<CP_DEV>(rsrc(gw, 16), 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) sh.head[i] = (uint32_t)hd[i];
    sh.ok = 1;
  }
  __syncthreads();
  guard.init(gw, host_err, fault_site, sh.head, (uint32_t)fault_after);
  return sh.head[MONO_GUARD_EPOCH] + 1u;
}

// The CTA leaves the launch: the last one out resets the exit counter, runs `last`
// (state the next launch expects zero) and advances the epoch to this launch's tag.
template <class Last>
__device__ __attribute__((always_inline)) inline void launch_end(int32_t* gw, uint32_t tag, Last last) {
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t* w = reinterpret_cast<uint32_t*>(gw);
    drain();
    const uint32_t old = add_dev(w + MONO_GUARD_EXIT, 1u);
    if (old == gridDim.x - 1u) {
      last();
      st_dev(w + MONO_GUARD_EXIT, 0u);
      st_dev(w + MONO_GUARD_EPOCH, tag);
    }
  }
}

// the phase needs nothing from a phase before it (a launch of its own)
struct NoWait {
  __device__ bool operator()() const { return true; }
};

// A grid barrier between two phases of the layer launch: `count` (zero between launches)
// and `flag` words in scratch. Arriving: every wave drains its stores, then one thread
// adds to the count; the last arrival resets the count and raises the flag to the tag.
struct PhaseBarrier {
  uint32_t* count;
  uint32_t* flag;

  // always inlined: a call would take the address of the kernel argument holding the
  // barrier, which keeps the whole argument block in scratch memory
  __device__ __attribute__((always_inline)) void arrive(uint32_t tag) const {
    drain();
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t old = add_dev(count, 1u);
      if (old == gridDim.x - 1u) {
        st_dev(count, 0u);
        drain();  // the reset lands before the flag lets anyone on
        st_dev(flag, tag);
      }
    }
  }
};

// Waiting for a barrier: wave 0 polls the flag under the guard's deadline, then the CTA
// agrees on the result (false: the launch is failing, the phase skips its work).
struct BarrierWait {
  const PhaseBarrier* bar;
  Guard* guard;
  uint32_t tag;
  int site;
  int* ok_s;

  __device__ __attribute__((always_inline)) bool operator()() const {
    bool ok = true;
    if ((threadIdx.x >> 6) == 0)
      ok = wait_until<4>(*guard, site, [&]() { return __all(ld_dev(bar->flag) == tag); });
    return cta_all(ok, *ok_s);
  }
};

}  // namespace mono
