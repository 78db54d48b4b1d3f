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

// CTA-shared words of a launch: the guard head as read once, the CTA's ok flag and its
// part in the launch's end (0: not the last CTA out, 1: last, 2: last of a failed launch)
struct LaunchShared {
  uint32_t head[4];
  int ok;
  int role;
};

// A kernel's LDS: ONE arena of BYTES (the phases' carving) with the launch's shared words
// after it. As the kernel's only LDS variable the arena starts at LDS address 0, so an
// offset into it is the LDS address a buffer -> LDS copy writes (see LDS_DMA_END).
template <int BYTES>
struct LdsArena {
  static constexpr int BODY = (BYTES + 15) & ~15;
  static constexpr int TOTAL = BODY + (int)sizeof(LaunchShared);
  static_assert(TOTAL <= 160 * 1024, "gfx950 LDS");
};

// The launch tag after `epoch`. Tags run 1 .. 0xFFFFFFFE and then start again at 1:
// never 0 (the tag of a pair nobody wrote or the scrub cleared), and the cycle is even,
// so the buffers indexed by the tag's parity keep alternating across the wrap.
__device__ inline uint32_t tag_after(uint32_t epoch) {
  return epoch >= 0xFFFFFFFEu ? 1u : epoch + 1u;
}

// bytes of the launch's scratch the last CTA out zeroes per launch, in turn: a pair
// left unwritten is cleared within (scratch bytes / SCRUB_CHUNK) launches, long before
// its tag could come round again
constexpr uint32_t SCRUB_CHUNK = 16384;
constexpr uint32_t NAN_BF16X2 = 0x7FC07FC0u;  // two bf16 quiet NaNs
constexpr uint32_t NAN_F32 = 0x7FC00000u;

// An output a failed launch overwrites with NaN: `bytes` (a multiple of 16) of the
// 32-bit pattern `fill`; p == nullptr: none
struct Poison {
  void* p;
  uint32_t bytes;
  uint32_t fill;
};

// The guard head's one coherent load (thread 0; zeros elsewhere). A launch issues it
// first, ahead of its first weight loads, so that the wait for it in launch_begin_from
// does not queue behind them.
__device__ inline v4i launch_head_issue(int32_t* gw) {
  return threadIdx.x == 0 ? ld16<CP_DEV>(rsrc(gw, 16), 0) : v4i{0, 0, 0, 0};
}

// Share the guard head `hd` (launch_head_issue) in LDS and set up the guard; returns the
// launch tag (epoch + 1). Every thread calls it.
__device__ __attribute__((always_inline)) inline uint32_t launch_begin_from(
    LaunchShared& sh, Guard& guard, v4i hd, int32_t* gw, uint32_t* host_err, int fault_site,
    int fault_after) {
  if (threadIdx.x == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) sh.head[i] = (uint32_t)hd[i];
    sh.ok = 1;
  }
  __syncthreads();
  guard.init(gw, host_err, fault_site, sh.head, (uint32_t)fault_after);
  return tag_after(sh.head[MONO_GUARD_EPOCH]);
}

// Read the guard head and set up the guard; returns the launch tag. Every thread calls it.
__device__ __attribute__((always_inline)) inline uint32_t launch_begin(LaunchShared& sh, Guard& guard, int32_t* gw,
                                        uint32_t* host_err, int fault_site, int fault_after) {
  return launch_begin_from(sh, guard, launch_head_issue(gw), gw, host_err, fault_site,
                           fault_after);
}

// The CTA leaves the launch. The last CTA out (every other CTA has drained its stores
// and left) zeroes one SCRUB_CHUNK of the launch's scratch, and, if the launch failed
// (the guard's abort word is set: a wait timed out in this launch or in an earlier one
// of the same guard block, which stays set until the host resets the block), fills the
// outputs `o0` and `o1` with NaN, so no step that failed can hand on numbers that look
// valid, also where no host code runs between launches (a replayed graph). Every output
// store of the launch is device coherent (sc1, write-through), so no L2 of another XCD
// holds a dirty line that could overwrite the NaN when the kernel ends. Then thread 0
// runs `last` (state the next launch expects zero), resets the exit counter and
// advances the epoch to this launch's tag, without waiting for the scrub or the NaN
// fill: the end of the launch orders them all before any later reader. Every thread
// calls it.
template <class Last>
__device__ __attribute__((always_inline)) inline void launch_end(LaunchShared& sh, int32_t* gw,
                                                                uint32_t tag, uint8_t* scratch,
                                                                uint32_t scratch_bytes, Poison o0,
                                                                Poison o1, Last last) {
  uint32_t* w = reinterpret_cast<uint32_t*>(gw);
  __syncthreads();
  if (threadIdx.x == 0) {
    drain();
    const uint32_t old = add_dev(w + MONO_GUARD_EXIT, 1u);
    sh.role = old != gridDim.x - 1u ? 0 : (ld_dev(w + MONO_GUARD_ABORT) ? 2 : 1);
  }
  __syncthreads();
  const int role = sh.role;
  if (role == 0) return;
  const uint32_t nchunk = (scratch_bytes + SCRUB_CHUNK - 1) / SCRUB_CHUNK;
  if (nchunk) {
    // past the end of the scratch the buffer resource drops the store
    const __amdgpu_buffer_rsrc_t r = rsrc(scratch, scratch_bytes);
    const uint32_t base = (tag % nchunk) * SCRUB_CHUNK;
    for (uint32_t o = threadIdx.x * 16u; o < SCRUB_CHUNK; o += blockDim.x * 16u)
      st16<CP_DEV>(r, base + o, v4i{0, 0, 0, 0});
  }
  if (role == 2) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const Poison& o = k ? o1 : o0;
      if (!o.p) continue;
      const __amdgpu_buffer_rsrc_t r = rsrc(o.p, o.bytes);
      const int32_t f = (int32_t)o.fill;
      for (uint32_t off = threadIdx.x * 16u; off < o.bytes; off += blockDim.x * 16u)
        st16<CP_DEV>(r, off, v4i{f, f, f, f});
    }
  }
  // no drain or barrier ahead of the final stores: nothing in this launch reads these
  // words again, and the launch's end makes every store visible before the next launch
  // (or the host) reads the guard words, the scratch or the outputs, so the scrub, the
  // resets and the epoch complete in one round trip
  if (threadIdx.x == 0) {
    last();
    st_dev(w + MONO_GUARD_EXIT, 0u);
    st_dev(w + MONO_GUARD_EPOCH, tag);
  }
}

// the phase needs nothing from a phase before it (a launch of its own)
struct NoWait {
  __device__ bool operator()() const { return true; }
};

// A grid barrier between two phases of the layer launch: `count` and `flag` words in
// scratch, a line apart (the arrivals' adds do not queue behind the polls). The count is
// zero at launch entry; the last CTA out of a launch zeroes it again. Arriving: every
// wave drains its stores (write-through, so they are acknowledged device-wide), then one
// thread adds to the count; the last arrival raises the flag to the launch tag at once
// (the count needs no reset on the way). Waiting: wave 0 polls the flag.
struct PhaseBarrier {
  uint32_t* count;
  uint32_t* flag;

  // always inlined: a call would take the address of the kernel argument holding the
  // barrier, which keeps the whole argument block in scratch memory
  __device__ __attribute__((always_inline)) void arrive(uint32_t tag) const {
    drain();
    __syncthreads();
    if (threadIdx.x == 0 && add_dev(count, 1u) == gridDim.x - 1u) st_dev(flag, tag);
  }
  // for the last CTA out, once every CTA has arrived
  __device__ __attribute__((always_inline)) void reset() const { st_dev(count, 0u); }
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
