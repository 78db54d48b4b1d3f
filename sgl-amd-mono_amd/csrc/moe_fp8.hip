// The FP8 MoE launch (its phase: moe_fp8_phase.h), its C entry points and the allocation-free variant.
#include "moe_fp8_phase.h"

namespace mono {

template <int H, int I, bool SHUF>
__global__ void __launch_bounds__(1024, 1) moe_fp8_kernel(MoeFp8Params p) {
  using Arena = LdsArena<MoeLds<H, I>::BYTES>;
  __shared__ __attribute__((aligned(16))) uint8_t lds[Arena::TOTAL];
  LaunchShared& sh = *reinterpret_cast<LaunchShared*>(lds + Arena::BODY);
  stamp(p.timeline, MONO_TL_START);
  Guard guard;
  uint32_t tag = 0;
  moe_phase<H, I, SHUF, false>(p, lds, guard, tag, sh.ok, NoWait());
  stamp(p.timeline, MONO_TL_DOWN);
  // every other CTA is past its last queue grab once the last one leaves: the counters
  // restart at zero
  launch_end(sh, p.guard, tag, p.scratch, (uint32_t)MoeFp8Geom<H, I>::BYTES,
             Poison{p.out, (uint32_t)p.rows * H * 2u, NAN_BF16X2},
             Poison{p.y, (uint32_t)p.rows * H * 4u, NAN_F32},
             [&]() { moe_reset_queues<H, I>(p); });
  stamp(p.timeline, MONO_TL_END);
}

}  // namespace mono

using namespace mono;

extern "C" size_t mono_moe_fp8_scratch_bytes(int32_t hidden, int32_t inter, int32_t experts) {
  if (experts != MOE_NEXP) return 0;
  if (hidden == 7168 && inter == 512) return MoeFp8Geom<7168, 512>::BYTES;
  return 0;
}

// the launch over the given scratch and guard block (the caller's, or the static one)
static int moe_fp8_launch_on(const MonoMoeFp8Args* a, mono_stream_t stream, void* scratch_ptr,
                             int32_t* guard_ptr, const char* who) {
  char msg[160];
  auto fail = [&](int code, const char* what) {
    snprintf(msg, sizeof msg, "%s: %s", who, what);
    return set_error(code, msg);
  };
  if (a->rows < 1 || a->rows > MOE_MAXR) return fail(MONO_E_ARG, "rows must be 1..16");
  if (a->experts != MOE_NEXP) return fail(MONO_E_ARG, "experts must be 256");
  if (!a->a || !a->out || !a->g_post || !a->w_r || !a->bias || !a->w13 || !a->s13 || !a->w2 ||
      !a->s2 || !scratch_ptr || !guard_ptr)
    return fail(MONO_E_ARG, "null tensor");
  if (!route_groups_ok(a->n_group, a->topk_group))
    return fail(MONO_E_ARG, "n_group / topk_group: 2..16 groups dividing 256, keeping >= 8 experts");
  MoeFp8Params p;
  p.rows = a->rows;
  p.eps = a->eps;
  p.route_scale = a->route_scale;
  p.n_group = a->n_group;
  p.topk_group = a->topk_group;
  p.a = static_cast<const uint16_t*>(a->a);
  p.ssq = nullptr;
  p.out = static_cast<uint16_t*>(a->out);
  p.g_post = static_cast<const uint16_t*>(a->g_post);
  p.w_r = static_cast<const uint16_t*>(a->w_r);
  p.bias = a->bias;
  p.w13 = a->w13;
  p.s13 = a->s13;
  p.w2 = a->w2;
  p.s2 = a->s2;
  p.y = a->y;
  p.scores = a->scores;
  p.ids = a->ids;
  p.weights = a->weights;
  p.scratch = static_cast<uint8_t*>(scratch_ptr);
  p.guard = guard_ptr;
  p.host_err = nullptr;
  if (a->host_error) {
    void* dptr = nullptr;
    if (hipHostGetDevicePointer(&dptr, a->host_error, 0) != hipSuccess || !dptr)
      return fail(MONO_E_ARG, "host_error is not pinned host memory");
    p.host_err = static_cast<uint32_t*>(dptr);
  }
  p.fault_site = a->fault_site;
  p.fault_after = a->fault_after;
  p.timeline = a->timeline;
  int grid = 0;
  int rc = monokernel_grid(&grid);
  if (rc) return rc;
  if (a->layout != MONO_LAYOUT_ROWMAJOR && a->layout != MONO_LAYOUT_AITER16)
    return fail(MONO_E_ARG, "unknown weight layout");
  if (a->hidden != 7168 || a->inter != 512) return fail(MONO_E_ARG, "unsupported hidden/inter");
  auto k = a->layout == MONO_LAYOUT_AITER16 ? moe_fp8_kernel<7168, 512, true>
                                            : moe_fp8_kernel<7168, 512, false>;
  rc = check_coresident(k, 1024, 0, "mono_moe_fp8: one 1024-thread CTA per CU does not fit");
  if (rc) return rc;
  hipLaunchKernelGGL(k, dim3(grid), dim3(1024), 0, (hipStream_t)stream, p);
  return check_launch(who);
}

extern "C" int mono_moe_fp8_launch(const MonoMoeFp8Args* a, mono_stream_t stream) {
  if (!a) return set_error(MONO_E_ARG, "mono_moe_fp8_launch: null args");
  return moe_fp8_launch_on(a, stream, a->scratch, a->guard, "mono_moe_fp8_launch");
}

// ------------------------------------------------------------------ allocation-free launch
// The guard block (256 B, its 16 words first) and the launch's scratch in one static
// device array: every GPU the library runs on holds its own copy until the process ends,
// zeroed when the code object loads. Host code never uses the array's name as an address:
// its per-device address comes from hipGetSymbolAddress on the first call on a device.
constexpr size_t MOE_STATIC_GUARD = 256;
constexpr size_t MOE_STATIC_BYTES = MOE_STATIC_GUARD + MoeFp8Geom<7168, 512>::BYTES;
static_assert(MONO_GUARD_WORDS * 4 <= MOE_STATIC_GUARD, "the guard block fits its slot");

static __device__ __align__(256) uint8_t scratch[MOE_STATIC_BYTES];

namespace {
constexpr int STATIC_MAX_DEV = 64;
std::mutex g_static_mu;
void* g_static_ptr[STATIC_MAX_DEV];

// this device's address of the static block, looked up once per device (device current)
int static_block(int dev, uint8_t** out) {
  std::lock_guard<std::mutex> lk(g_static_mu);
  if (dev < 0 || dev >= STATIC_MAX_DEV)
    return set_error(MONO_E_DEVICE, "mono_moe_fp8_launch_static: device index out of range");
  if (!g_static_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      char msg[200];
      snprintf(msg, sizeof msg, "mono_moe_fp8_launch_static: hipGetSymbolAddress: %s",
               hipGetErrorString(e));
      return set_error(MONO_E_DEVICE, msg);
    }
    g_static_ptr[dev] = ptr;
  }
  *out = static_cast<uint8_t*>(g_static_ptr[dev]);
  return MONO_OK;
}
}  // namespace

extern "C" int mono_moe_fp8_launch_static(const MonoMoeFp8Args* a, mono_stream_t stream) {
  if (!a) return set_error(MONO_E_ARG, "mono_moe_fp8_launch_static: null args");
  if (a->scratch || a->guard)
    return set_error(MONO_E_ARG, "mono_moe_fp8_launch_static: scratch and guard must be null "
                                 "(they live in the library's static block)");
  if (a->rows < 1 || a->rows > MOE_MAXR)
    return set_error(MONO_E_ARG, "mono_moe_fp8_launch_static: rows must be 1..16 (the static "
                                 "block holds the hand-offs of at most 16 rows)");
  if (a->hidden != 7168 || a->inter != 512 || a->experts != MOE_NEXP)
    return set_error(MONO_E_ARG, "mono_moe_fp8_launch_static: the static block is sized for "
                                 "hidden 7168, inter 512, 256 experts");
  if (a->host_error && *a->host_error != 0u)
    return set_error(MONO_E_FAILED, "mono_moe_fp8_launch_static: an earlier call timed out "
                                    "(host_error set): the static block cannot be reset");
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess)
    return set_error(MONO_E_DEVICE, "mono_moe_fp8_launch_static: no current HIP device");
  uint8_t* base = nullptr;
  const int rc = static_block(dev, &base);
  if (rc) return rc;
  return moe_fp8_launch_on(a, stream, base + MOE_STATIC_GUARD, reinterpret_cast<int32_t*>(base),
                           "mono_moe_fp8_launch_static");
}
