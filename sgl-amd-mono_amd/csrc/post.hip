// The output-block launch of the layer (its phase: post_phase.h) and its C entry points.
#include "post_phase.h"

namespace mono {

__global__ void __launch_bounds__(1024, 1) post_kernel(PostParams p) {
  using Arena = LdsArena<PO_LDS_BYTES>;
  __shared__ __attribute__((aligned(16))) uint8_t lds[Arena::TOTAL];
  LaunchShared& sh = *reinterpret_cast<LaunchShared*>(lds + Arena::BODY);
  stamp(p.timeline, MONO_TL_START);
  Guard guard;
  const uint32_t tag = launch_begin(sh, guard, p.guard, p.host_err, p.fault_site, p.fault_after);
  post_phase<false>(p, lds, guard, tag, sh.ok, NoWait());
  stamp(p.timeline, MONO_TL_ROUTED);
  launch_end(sh, p.guard, tag, p.scratch, (uint32_t)PostScratch::BYTES,
             Poison{p.out, (uint32_t)p.rows * PO_HID * 2u, NAN_BF16X2}, Poison{nullptr, 0, 0},
             []() {});
  stamp(p.timeline, MONO_TL_END);
}

}  // namespace mono

using namespace mono;

extern "C" size_t mono_post_scratch_bytes(void) { return PostScratch::BYTES; }

extern "C" int mono_post_launch(const MonoPostArgs* a, mono_stream_t stream) {
  if (!a) return set_error(MONO_E_ARG, "mono_post_launch: null args");
  if (a->rows < 1 || a->rows > PO_MAXR)
    return set_error(MONO_E_ARG, "mono_post_launch: rows must be 1..16");
  if (a->heads != PO_HEADS || a->hidden != PO_HID)
    return set_error(MONO_E_ARG, "mono_post_launch: built for 32 heads and hidden 7168");
  if (a->layout != MONO_LAYOUT_ROWMAJOR && a->layout != MONO_LAYOUT_AITER16)
    return set_error(MONO_E_ARG, "mono_post_launch: unknown weight layout");
  if (!a->o_lat || !a->h || !a->w_uv || !a->s_uv || !a->w_o || !a->s_o || !a->out ||
      !a->scratch || !a->guard)
    return set_error(MONO_E_ARG, "mono_post_launch: null tensor");
  PostParams p;
  p.rows = a->rows;
  p.shuf = a->layout == MONO_LAYOUT_AITER16;
  p.o_lat = static_cast<const uint16_t*>(a->o_lat);
  p.h = static_cast<const uint16_t*>(a->h);
  p.w_uv = a->w_uv;
  p.s_uv = a->s_uv;
  p.w_o = a->w_o;
  p.s_o = a->s_o;
  p.out = static_cast<uint16_t*>(a->out);
  p.scratch = static_cast<uint8_t*>(a->scratch);
  p.o = static_cast<uint16_t*>(a->o);
  p.ssq = nullptr;
  p.guard = a->guard;
  p.host_err = nullptr;
  if (a->host_error) {
    void* dptr = nullptr;
    if (hipHostGetDevicePointer(&dptr, a->host_error, 0) != hipSuccess || !dptr)
      return set_error(MONO_E_ARG, "mono_post_launch: host_error is not pinned host memory");
    p.host_err = static_cast<uint32_t*>(dptr);
  }
  p.fault_site = a->fault_site;
  p.fault_after = a->fault_after;
  p.timeline = a->timeline;
  int grid = 0;
  int rc = monokernel_grid(&grid);
  if (rc) return rc;
  if (grid > PO_MAX_GRID) return set_error(MONO_E_DEVICE, "mono_post_launch: grid too large");
  rc = check_coresident(post_kernel, 1024, 0,
                        "mono_post_launch: one 1024-thread CTA per CU does not fit");
  if (rc) return rc;
  hipLaunchKernelGGL(post_kernel, dim3(grid), dim3(1024), 0, (hipStream_t)stream, p);
  return check_launch("mono_post_launch");
}
