// The library-wide entry points of the C ABI: version, errors, device facts, the
// guard block's deadline and the reset after a failed launch.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "mono_abi.h"
#include "mono_device.h"

namespace mono {

static thread_local char g_err[512] = "";

int set_error(int code, const char* msg) {
  snprintf(g_err, sizeof g_err, "%s", msg);
  return code;
}

int check_launch(const char* where) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char buf[400];
    snprintf(buf, sizeof buf, "%s: %s", where, hipGetErrorString(e));
    return set_error(MONO_E_LAUNCH, buf);
  }
  return MONO_OK;
}

namespace {
constexpr int MAX_DEV = 64;
std::mutex g_mu;
MonoDeviceInfo g_info[MAX_DEV];
bool g_have[MAX_DEV];

int query(int dev, MonoDeviceInfo* out) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (dev < 0 || dev >= MAX_DEV) return set_error(MONO_E_ARG, "device index out of range");
  if (!g_have[dev]) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess)
      return set_error(MONO_E_DEVICE, "hipGetDeviceProperties failed");
    MonoDeviceInfo info;
    info.cus = prop.multiProcessorCount;
    info.lds_bytes = (int32_t)prop.maxSharedMemoryPerMultiProcessor;
    info.is_gfx950 = strncmp(prop.gcnArchName, "gfx950", 6) == 0;
    info.grid = info.cus;
    g_info[dev] = info;
    g_have[dev] = true;
  }
  *out = g_info[dev];
  return MONO_OK;
}
}  // namespace

int monokernel_grid(int* grid) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(MONO_E_DEVICE, "no current HIP device");
  MonoDeviceInfo info;
  int rc = query(dev, &info);
  if (rc) return rc;
  if (!info.is_gfx950) return set_error(MONO_E_DEVICE, "the monokernels need a gfx950 device");
  *grid = info.grid;
  return MONO_OK;
}

__global__ void set_deadline_kernel(int32_t* guard, uint32_t lo, uint32_t hi) {
  st_dev(reinterpret_cast<uint32_t*>(guard) + MONO_GUARD_DEADLINE_LO, lo);
  st_dev(reinterpret_cast<uint32_t*>(guard) + MONO_GUARD_DEADLINE_HI, hi);
}

// zero `n` bytes (n a multiple of 4) and the guard block's words other than the deadline
__global__ void reset_kernel(uint32_t* scratch, size_t words, int32_t* guard) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += stride)
    scratch[i] = 0u;
  if (guard && blockIdx.x == 0 && threadIdx.x < MONO_GUARD_WORDS &&
      threadIdx.x != MONO_GUARD_DEADLINE_LO && threadIdx.x != MONO_GUARD_DEADLINE_HI)
    guard[threadIdx.x] = 0;
}

}  // namespace mono

using namespace mono;

extern "C" int mono_version(void) { return 1; }

extern "C" const char* mono_last_error(void) { return g_err; }

extern "C" int mono_device_info(int32_t device, MonoDeviceInfo* out) {
  if (!out) return set_error(MONO_E_ARG, "mono_device_info: null out");
  return query(device, out);
}

extern "C" int mono_set_deadline(int32_t* guard, double seconds, mono_stream_t stream) {
  if (!guard) return set_error(MONO_E_ARG, "mono_set_deadline: null guard");
  // waits compare 64-bit tick differences; an hour bounds any sane deadline
  if (!(seconds > 0.0) || seconds > 3600.0)
    return set_error(MONO_E_ARG, "mono_set_deadline: deadline must be in (0, 3600] s");
  const uint64_t ticks = (uint64_t)(seconds * MONO_CLOCK_HZ);
  hipLaunchKernelGGL(set_deadline_kernel, dim3(1), dim3(1), 0, (hipStream_t)stream, guard,
                     (uint32_t)ticks, (uint32_t)(ticks >> 32));
  return check_launch("mono_set_deadline");
}

extern "C" int mono_reset(void* scratch, size_t scratch_bytes, int32_t* guard,
                          mono_stream_t stream) {
  if ((scratch_bytes && !scratch) || (scratch_bytes & 3))
    return set_error(MONO_E_ARG, "mono_reset: scratch must be non-null, bytes a multiple of 4");
  hipLaunchKernelGGL(reset_kernel, dim3(256), dim3(256), 0, (hipStream_t)stream,
                     static_cast<uint32_t*>(scratch), scratch_bytes / 4, guard);
  return check_launch("mono_reset");
}
