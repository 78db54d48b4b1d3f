// Host-side helpers of the C ABI: error strings, launch checks, the co-resident grid.
#pragma once

#include <hip/hip_runtime.h>

#include "mono_amd.h"

namespace mono {

// record `msg` as this thread's last error and return `code`
int set_error(int code, const char* msg);
// MONO_E_LAUNCH if the last launch failed to enqueue
int check_launch(const char* where);
// CTAs of a monokernel launch on the current device (one per CU) after checking the
// device is gfx950; MONO_E_DEVICE otherwise
int monokernel_grid(int* grid);

// the launch must fit one CTA of `threads` per CU with `lds` dynamic bytes: every CTA of
// a persistent launch has to be resident at once or a wait never completes
template <class K>
int check_coresident(K kernel, int threads, size_t lds, const char* where) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, lds) != hipSuccess ||
      n < 1)
    return set_error(MONO_E_DEVICE, where);
  return MONO_OK;
}

}  // namespace mono
