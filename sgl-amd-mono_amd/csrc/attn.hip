// The attention launch of the layer (its phase: attn_phase.h) and its C entry points.
#include "attn_phase.h"

namespace mono {

template <int SPLIT, bool LONG, bool DSA>
__global__ void __launch_bounds__(AT_THREADS, 1) attn_kernel(AttnParams p) {
  using Arena = LdsArena<AT_LDS_BYTES>;
  __shared__ __attribute__((aligned(16))) uint8_t lds[Arena::TOTAL];
  LaunchShared& sh = *reinterpret_cast<LaunchShared*>(lds + Arena::BODY);
  stamp(p.timeline, MONO_TL_START);
  Guard guard;
  const uint32_t tag = launch_begin(sh, guard, p.guard, p.host_err, p.fault_site, p.fault_after);
  attn_phase<SPLIT, false, LONG, DSA>(p, lds, guard, tag, sh.ok, NoWait());
  stamp(p.timeline, MONO_TL_DOWN);
  launch_end(sh, p.guard, tag, p.scratch, (uint32_t)AttnScratch(p.rows_max).bytes,
             Poison{p.out, (uint32_t)p.rows * AT_HEADS * AT_LAT * 2u, NAN_BF16X2},
             Poison{nullptr, 0, 0}, []() {});
  stamp(p.timeline, MONO_TL_END);
}

}  // namespace mono

using namespace mono;

extern "C" size_t mono_attn_scratch_bytes(int32_t rows_max) {
  return (rows_max >= 1 && rows_max <= AT_MAXR) ? AttnScratch(rows_max).bytes : 0;
}

extern "C" int mono_attn_launch(const MonoAttnArgs* a, mono_stream_t stream) {
  if (!a) return set_error(MONO_E_ARG, "mono_attn_launch: null args");
  if (a->rows_max < 1 || a->rows_max > AT_MAXR || a->rows < 1 || a->rows > a->rows_max)
    return set_error(MONO_E_ARG, "mono_attn_launch: rows must be 1..rows_max, rows_max 1..48");
  if (a->heads != AT_HEADS || a->index_heads != AT_IHEADS || a->topk != AT_TOPK ||
      a->page != AT_PAGE)
    return set_error(MONO_E_ARG, "mono_attn_launch: built for 32 heads, 64 index heads, "
                                 "top-2048 and 64-token pages");
  if (a->ctx_max < 1 || a->ctx_max > AT_MAXCTX)
    return set_error(MONO_E_ARG, "mono_attn_launch: ctx_max must be 1..163840");
  if (a->pt_stride < (a->ctx_max + AT_PAGE - 1) / AT_PAGE || a->pt_rows < 1 ||
      (uint64_t)a->pt_rows * a->pt_stride * 4 > 0x7FFFFFFFull)
    return set_error(MONO_E_ARG, "mono_attn_launch: page table rows shorter than ctx_max");
  if (a->plane_pages == 0 || a->plane_pages > (1u << 19) || a->kv_slots == 0 ||
      (uint64_t)a->kv_slots * AT_KV > 0x7FFFFFFFull)
    return set_error(MONO_E_ARG, "mono_attn_launch: plane_pages / kv_slots out of range");
  if (a->index_format < MONO_INDEX_FP4_PLANE || a->index_format > MONO_INDEX_FP8_ROWS)
    return set_error(MONO_E_ARG, "mono_attn_launch: unknown index_format");
  const bool fp4 = a->index_format == MONO_INDEX_FP4_PLANE;
  if (!a->positions || !a->req_ids || !a->page_table || !a->q || !a->iq || !a->iw ||
      (fp4 && (!a->iqs || !a->plane_scale)) || !a->plane || !a->kv || !a->out || !a->scratch ||
      !a->guard)
    return set_error(MONO_E_ARG, "mono_attn_launch: null tensor");
  AttnParams p;
  p.rows = a->rows;
  p.rows_max = a->rows_max;
  p.ctx_max = a->ctx_max;
  p.pt_stride = a->pt_stride;
  p.pt_rows = a->pt_rows;
  p.sm_scale = a->sm_scale;
  p.plane_pages = a->plane_pages;
  p.index_fmt = a->index_format;
  p.kv_slots = a->kv_slots;
  p.positions = a->positions;
  p.req_ids = a->req_ids;
  p.page_table = a->page_table;
  p.q = static_cast<const uint16_t*>(a->q);
  p.iq = a->iq;
  p.iqs = a->iqs;
  p.iw = a->iw;
  p.plane = a->plane;
  p.plane_scale = a->plane_scale;
  p.kv = a->kv;
  p.kv_scale = a->kv_scale;
  p.out = static_cast<uint16_t*>(a->out);
  p.scores_out = a->scores;
  p.topk_out = a->topk_pos;
  p.scratch = static_cast<uint8_t*>(a->scratch);
  p.guard = a->guard;
  p.host_err = nullptr;
  if (a->host_error) {
    void* dptr = nullptr;
    if (hipHostGetDevicePointer(&dptr, a->host_error, 0) != hipSuccess || !dptr)
      return set_error(MONO_E_ARG, "mono_attn_launch: host_error is not pinned host memory");
    p.host_err = static_cast<uint32_t*>(dptr);
  }
  p.fault_site = a->fault_site;
  p.fault_after = a->fault_after;
  p.timeline = a->timeline;
  p.uv_w = nullptr;  // W_UV runs in the output block's own launch
  p.uv_s = nullptr;
  p.uv_shuf = 0;
  p.uv_obuf[0] = p.uv_obuf[1] = nullptr;
  int grid = 0;
  int rc = monokernel_grid(&grid);
  if (rc) return rc;
  // 64-key splits when the rows' 32 splits each take one CTA, else 128-key splits
  // rows that may span more than one top-k block take the multi-block variant
  const bool s64 = p.rows * (AT_TOPK / 64) <= grid, lng = p.ctx_max > AT_TKBLOCK;
  // DSA (FP8) index pages take their own instances (their score code holds more registers)
  using K = void (*)(AttnParams);
  const K kerns[2][2][2] = {{{attn_kernel<128, false, false>, attn_kernel<128, false, true>},
                             {attn_kernel<128, true, false>, attn_kernel<128, true, true>}},
                            {{attn_kernel<64, false, false>, attn_kernel<64, false, true>},
                             {attn_kernel<64, true, false>, attn_kernel<64, true, true>}}};
  const K kern = kerns[s64][lng][!fp4];
  rc = check_coresident(kern, AT_THREADS, 0,
                        "mono_attn_launch: one 1024-thread CTA per CU does not fit");
  if (rc) return rc;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(AT_THREADS), 0, (hipStream_t)stream, p);
  return check_launch("mono_attn_launch");
}
