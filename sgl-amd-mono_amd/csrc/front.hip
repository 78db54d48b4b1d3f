// The front launch of the layer (its phase: front_phase.h) and its C entry points.
#include "front_phase.h"

namespace mono {

__global__ void __launch_bounds__(1024, 1) front_kernel(FrontParams p) {
  using Arena = LdsArena<FR_LDS_BYTES>;
  __shared__ __attribute__((aligned(16))) uint8_t lds[Arena::TOTAL];
  LaunchShared& sh = *reinterpret_cast<LaunchShared*>(lds + Arena::BODY);
  stamp(p.timeline, MONO_TL_START);
  Guard guard;
  const v4i hd = launch_head_issue(p.guard);
  const uint32_t tag = front_phase(p, lds, guard, sh.ok, [&]() {
    return launch_begin_from(sh, guard, hd, p.guard, p.host_err, p.fault_site, p.fault_after);
  });
  stamp(p.timeline, MONO_TL_MIDQ);
  launch_end(sh, p.guard, tag, p.scratch, (uint32_t)FrontScratch::BYTES,
             Poison{p.q, (uint32_t)p.rows * FR_HEADS * FR_Q * 2u, NAN_BF16X2},
             Poison{p.iw, (uint32_t)p.rows * FR_IH * 4u, NAN_F32}, []() {});
  stamp(p.timeline, MONO_TL_END);
}

}  // namespace mono

using namespace mono;

extern "C" size_t mono_front_scratch_bytes(void) { return FrontScratch::BYTES; }

extern "C" int mono_front_launch(const MonoFrontArgs* a, mono_stream_t stream) {
  if (!a) return set_error(MONO_E_ARG, "mono_front_launch: null args");
  if (a->rows < 1 || a->rows > FR_MAXR)
    return set_error(MONO_E_ARG, "mono_front_launch: rows must be 1..8");
  if (a->hidden != FR_H || a->heads != FR_HEADS)
    return set_error(MONO_E_ARG, "mono_front_launch: built for hidden 7168 and 32 heads");
  if (a->layout != MONO_LAYOUT_ROWMAJOR && a->layout != MONO_LAYOUT_AITER16)
    return set_error(MONO_E_ARG, "mono_front_launch: unknown weight layout");
  if (a->index_format < MONO_INDEX_FP4_PLANE || a->index_format > MONO_INDEX_FP8_ROWS)
    return set_error(MONO_E_ARG, "mono_front_launch: unknown index_format");
  const bool fp4 = a->index_format == MONO_INDEX_FP4_PLANE;
  if (a->rope_rows < 1 || a->kv_slots < 1 || a->plane_pages < 1 || a->plane_pages > (1u << 19) ||
      (uint64_t)a->kv_slots * FR_KVA > 0x7FFFFFFFull || (uint64_t)a->rope_rows * 64 > 0x7FFFFFFFull)
    return set_error(MONO_E_ARG, "mono_front_launch: cache or table sizes out of range");
  if (!a->h || !a->g_in || !a->g_q || !a->g_kv || !a->w_qkv_a || !a->s_qkv_a || !a->w_k ||
      !a->s_k || !a->w_w || !a->g_k || !a->b_k || !a->w_qb || !a->s_qb || !a->w_iq || !a->s_iq ||
      !a->w_uk || !a->s_uk || !a->cos || !a->sin || !a->positions || !a->slots || !a->kv ||
      !a->plane || (fp4 && (!a->plane_scale || !a->iqs)) || !a->q || !a->iq || !a->iw ||
      !a->scratch || !a->guard)
    return set_error(MONO_E_ARG, "mono_front_launch: null tensor");
  FrontParams p;
  p.rows = a->rows;
  p.shuf = a->layout == MONO_LAYOUT_AITER16;
  p.rope_rows = a->rope_rows;
  p.kv_slots = a->kv_slots;
  p.plane_pages = a->plane_pages;
  p.index_fmt = a->index_format;
  p.eps = a->eps;
  p.h = static_cast<const uint16_t*>(a->h);
  p.g_in = static_cast<const uint16_t*>(a->g_in);
  p.g_q = static_cast<const uint16_t*>(a->g_q);
  p.g_kv = static_cast<const uint16_t*>(a->g_kv);
  p.w_qkv_a = a->w_qkv_a;
  p.s_qkv_a = a->s_qkv_a;
  p.w_k = a->w_k;
  p.s_k = a->s_k;
  p.w_w = static_cast<const uint16_t*>(a->w_w);
  p.g_k = a->g_k;
  p.b_k = a->b_k;
  p.w_qb = a->w_qb;
  p.s_qb = a->s_qb;
  p.w_iq = a->w_iq;
  p.s_iq = a->s_iq;
  p.w_uk = a->w_uk;
  p.s_uk = a->s_uk;
  p.cos = static_cast<const uint16_t*>(a->cos);
  p.sin = static_cast<const uint16_t*>(a->sin);
  p.positions = a->positions;
  p.slots = a->slots;
  p.kv = a->kv;
  p.kv_scale = a->kv_scale;
  p.plane = a->plane;
  p.plane_scale = a->plane_scale;
  p.q = static_cast<uint16_t*>(a->q);
  p.iq = a->iq;
  p.iqs = a->iqs;
  p.iw = a->iw;
  p.scratch = static_cast<uint8_t*>(a->scratch);
  p.guard = a->guard;
  p.host_err = nullptr;
  if (a->host_error) {
    void* dptr = nullptr;
    if (hipHostGetDevicePointer(&dptr, a->host_error, 0) != hipSuccess || !dptr)
      return set_error(MONO_E_ARG, "mono_front_launch: host_error is not pinned host memory");
    p.host_err = static_cast<uint32_t*>(dptr);
  }
  p.fault_site = a->fault_site;
  p.fault_after = a->fault_after;
  p.timeline = a->timeline;
  p.ik_raw = a->ik_raw;
  p.iq_raw = static_cast<uint16_t*>(a->iq_raw);
  int grid = 0;
  int rc = monokernel_grid(&grid);
  if (rc) return rc;
  // every stage-A task, every row task and every W_UK tile on a CTA of its own, and at
  // most two B tiles a CTA
  if (grid > FR_MAX_GRID || grid < FR_ATASKS + 4 * a->rows || grid < FR_CT || 2 * grid < FR_BT)
    return set_error(MONO_E_DEVICE, "mono_front_launch: needs 224..1024 CUs (and 168 + 4 rows)");
  rc = check_coresident(front_kernel, 1024, 0,
                        "mono_front_launch: one 1024-thread CTA per CU does not fit");
  if (rc) return rc;
  hipLaunchKernelGGL(front_kernel, dim3(grid), dim3(1024), 0, (hipStream_t)stream, p);
  return check_launch("mono_front_launch");
}
