// The C ABI of the one-launch decoder layer (the kernel: layer_kernel.h): argument
// checks, the phases' parameters, instance choice and the launch.
#include "layer_kernel.h"
using namespace mono;

extern "C" size_t mono_layer_scratch_bytes(int32_t rows_max) {
  return (rows_max >= 1 && rows_max <= LY_MAXR) ? LayerScratch(rows_max).bytes : 0;
}

extern "C" int mono_layer_launch(const MonoLayerArgs* a, mono_stream_t stream) {
  if (!a) return set_error(MONO_E_ARG, "mono_layer_launch: null args");
  if (a->rows_max < 1 || a->rows_max > LY_MAXR || a->rows < 1 || a->rows > a->rows_max)
    return set_error(MONO_E_ARG, "mono_layer_launch: rows must be 1..rows_max, rows_max 1..8");
  if (a->hidden != LY_H || a->heads != FR_HEADS || a->inter != LY_I || a->experts != MOE_NEXP)
    return set_error(MONO_E_ARG, "mono_layer_launch: built for hidden 7168, 32 heads, "
                                 "expert intermediate 512 and 256 experts");
  if (a->layout != MONO_LAYOUT_ROWMAJOR && a->layout != MONO_LAYOUT_AITER16)
    return set_error(MONO_E_ARG, "mono_layer_launch: unknown weight layout");
  if (!route_groups_ok(a->n_group, a->topk_group))
    return set_error(MONO_E_ARG, "mono_layer_launch: n_group / topk_group: 2..16 groups "
                                 "dividing 256, keeping >= 8 experts");
  if (a->ctx_max < 1 || a->ctx_max > AT_MAXCTX)
    return set_error(MONO_E_ARG, "mono_layer_launch: ctx_max must be 1..163840");
  if (a->pt_stride < (a->ctx_max + AT_PAGE - 1) / AT_PAGE || a->pt_rows < 1 ||
      (uint64_t)a->pt_rows * a->pt_stride * 4 > 0x7FFFFFFFull)
    return set_error(MONO_E_ARG, "mono_layer_launch: page table rows shorter than ctx_max");
  if (a->rope_rows < 1 || (uint64_t)a->rope_rows * 64 > 0x7FFFFFFFull || a->kv_slots == 0 ||
      (uint64_t)a->kv_slots * AT_KV > 0x7FFFFFFFull || a->plane_pages == 0 ||
      a->plane_pages > (1u << 19))
    return set_error(MONO_E_ARG, "mono_layer_launch: cache or table sizes out of range");
  if (a->index_format < MONO_INDEX_FP4_PLANE || a->index_format > MONO_INDEX_FP8_ROWS)
    return set_error(MONO_E_ARG, "mono_layer_launch: unknown index_format");
  const bool fp4 = a->index_format == MONO_INDEX_FP4_PLANE;
  if (a->expert_format != MONO_EXPERTS_FP8 && a->expert_format != MONO_EXPERTS_MXFP4)
    return set_error(MONO_E_ARG, "mono_layer_launch: unknown expert_format");
  const bool mx = a->expert_format == MONO_EXPERTS_MXFP4;
  if (!a->h || !a->out || !a->positions || !a->slots || !a->req_ids || !a->page_table ||
      !a->kv || !a->plane || (fp4 && !a->plane_scale) || !a->g_in || !a->g_q || !a->g_kv ||
      !a->w_qkv_a || !a->s_qkv_a || !a->w_k || !a->s_k || !a->w_w || !a->g_k || !a->b_k ||
      !a->w_qb || !a->s_qb || !a->w_iq || !a->s_iq || !a->w_uk || !a->s_uk || !a->cos ||
      !a->sin || !a->w_uv || !a->s_uv || !a->w_o || !a->s_o || !a->g_post || !a->w_r ||
      !a->bias || !a->w13 || !a->w2 || (!mx && (!a->s13 || !a->s2)) ||
      (mx && (!a->e13 || !a->e2)) || !a->scratch || !a->guard)
    return set_error(MONO_E_ARG, "mono_layer_launch: null tensor");
  uint32_t* host_err = nullptr;
  if (a->host_error) {
    void* dptr = nullptr;
    if (hipHostGetDevicePointer(&dptr, a->host_error, 0) != hipSuccess || !dptr)
      return set_error(MONO_E_ARG, "mono_layer_launch: host_error is not pinned host memory");
    host_err = static_cast<uint32_t*>(dptr);
  }
  const LayerScratch S(a->rows_max);
  uint8_t* sc = static_cast<uint8_t*>(a->scratch);
  const int R = a->rows;
  const int shuf = a->layout == MONO_LAYOUT_AITER16;
  // the hand-offs between phases: the caller's buffer when given, else scratch
  uint16_t* q = a->q ? static_cast<uint16_t*>(a->q) : reinterpret_cast<uint16_t*>(sc + S.q);
  uint8_t* iq = a->iq ? a->iq : sc + S.iq;
  uint8_t* iqs = a->iqs ? a->iqs : sc + S.iqs;
  float* iw = a->iw ? a->iw : reinterpret_cast<float*>(sc + S.iw);
  uint16_t* o_lat = a->o_lat ? static_cast<uint16_t*>(a->o_lat)
                             : reinterpret_cast<uint16_t*>(sc + S.o_lat);
  uint16_t* st = a->a ? static_cast<uint16_t*>(a->a) : reinterpret_cast<uint16_t*>(sc + S.a);

  LayerParams p;
  FrontParams& f = p.f;
  f.rows = R;
  f.shuf = shuf;
  f.rope_rows = a->rope_rows;
  f.kv_slots = a->kv_slots;
  f.plane_pages = a->plane_pages;
  f.index_fmt = a->index_format;
  f.eps = a->eps;
  f.h = static_cast<const uint16_t*>(a->h);
  f.g_in = static_cast<const uint16_t*>(a->g_in);
  f.g_q = static_cast<const uint16_t*>(a->g_q);
  f.g_kv = static_cast<const uint16_t*>(a->g_kv);
  f.w_qkv_a = a->w_qkv_a;
  f.s_qkv_a = a->s_qkv_a;
  f.w_k = a->w_k;
  f.s_k = a->s_k;
  f.w_w = static_cast<const uint16_t*>(a->w_w);
  f.g_k = a->g_k;
  f.b_k = a->b_k;
  f.w_qb = a->w_qb;
  f.s_qb = a->s_qb;
  f.w_iq = a->w_iq;
  f.s_iq = a->s_iq;
  f.w_uk = a->w_uk;
  f.s_uk = a->s_uk;
  f.cos = static_cast<const uint16_t*>(a->cos);
  f.sin = static_cast<const uint16_t*>(a->sin);
  f.positions = a->positions;
  f.slots = a->slots;
  f.kv = a->kv;
  f.kv_scale = a->kv_scale;
  f.plane = a->plane;
  f.plane_scale = a->plane_scale;
  f.q = q;
  f.iq = iq;
  f.iqs = iqs;
  f.iw = iw;
  f.ik_raw = nullptr;
  f.iq_raw = nullptr;
  f.scratch = sc + S.front;
  f.guard = a->guard;
  f.host_err = host_err;
  f.fault_site = a->fault_site;
  f.fault_after = a->fault_after;
  f.timeline = nullptr;

  AttnParams& at = p.at;
  at.rows = R;
  at.rows_max = a->rows_max;
  at.ctx_max = a->ctx_max;
  at.pt_stride = a->pt_stride;
  at.pt_rows = a->pt_rows;
  at.sm_scale = a->sm_scale;
  at.plane_pages = a->plane_pages;
  at.index_fmt = a->index_format;
  at.kv_slots = a->kv_slots;
  at.positions = a->positions;
  at.req_ids = a->req_ids;
  at.page_table = a->page_table;
  at.q = q;
  at.iq = iq;
  at.iqs = iqs;
  at.iw = iw;
  at.plane = a->plane;
  at.plane_scale = a->plane_scale;
  at.kv = a->kv;
  at.kv_scale = a->kv_scale;
  at.out = o_lat;
  at.scores_out = a->scores;
  at.topk_out = a->topk_pos;
  at.scratch = sc + S.attn;
  at.guard = a->guard;
  at.host_err = host_err;
  at.fault_site = a->fault_site;
  at.fault_after = a->fault_after;
  at.timeline = nullptr;
  at.uv_w = a->w_uv;  // W_UV in the attention's merge
  at.uv_s = a->s_uv;
  at.uv_shuf = shuf;
  for (int k = 0; k < 2; ++k)
    at.uv_obuf[k] = reinterpret_cast<uint16_t*>(sc + S.post + k * PostScratch::OBUF);

  PostParams& po = p.po;
  po.rows = R;
  po.shuf = shuf;
  po.o_lat = o_lat;
  po.h = static_cast<const uint16_t*>(a->h);
  po.w_uv = a->w_uv;
  po.s_uv = a->s_uv;
  po.w_o = a->w_o;
  po.s_o = a->s_o;
  po.out = st;
  po.o = nullptr;
  po.ssq = reinterpret_cast<float*>(sc + S.ssq);
  po.scratch = sc + S.post;
  po.guard = a->guard;
  po.host_err = host_err;
  po.fault_site = a->fault_site;
  po.fault_after = a->fault_after;
  po.timeline = nullptr;

  MoeFp8Params& m = p.m;
  m.rows = R;
  m.eps = a->eps;
  m.route_scale = a->route_scale;
  m.n_group = a->n_group;
  m.topk_group = a->topk_group;
  m.a = st;
  m.ssq = reinterpret_cast<const float*>(sc + S.ssq);
  m.out = static_cast<uint16_t*>(a->out);
  m.g_post = static_cast<const uint16_t*>(a->g_post);
  m.w_r = static_cast<const uint16_t*>(a->w_r);
  m.bias = a->bias;
  m.w13 = a->w13;
  m.s13 = a->s13;
  m.w2 = a->w2;
  m.s2 = a->s2;
  m.e13 = mx ? a->e13 : nullptr;
  m.e2 = mx ? a->e2 : nullptr;
  m.y = a->y;
  m.scores = a->moe_scores;
  m.ids = a->ids;
  m.weights = a->weights;
  m.scratch = sc + S.moe;
  m.guard = a->guard;
  m.host_err = host_err;
  m.fault_site = a->fault_site;
  m.fault_after = a->fault_after;
  m.timeline = nullptr;

  for (int k = 0; k < 2; ++k) {
    p.bar[k].count = reinterpret_cast<uint32_t*>(sc + LayerScratch::BARRIERS + 256 * k);
    p.bar[k].flag = reinterpret_cast<uint32_t*>(sc + LayerScratch::BARRIERS + 256 * k + 128);
  }
  p.scratch = sc;
  p.guard = a->guard;
  p.host_err = host_err;
  p.fault_site = a->fault_site;
  p.fault_after = a->fault_after;
  p.timeline = a->timeline;

  int grid = 0;
  int rc = monokernel_grid(&grid);
  if (rc) return rc;
  if (a->phase_timeline) {
    const size_t per = (size_t)grid * MONO_TL_COLS;
    f.timeline = a->phase_timeline;
    at.timeline = a->phase_timeline + per;
    po.timeline = a->phase_timeline + 2 * per;
    m.timeline = a->phase_timeline + 3 * per;
  }
  // the front's placement: every stage-A task, every row task and every W_UK tile on a
  // CTA of its own, at most two B tiles a CTA
  if (grid > FR_MAX_GRID || grid < FR_ATASKS + 4 * R || grid < FR_CT || 2 * grid < FR_BT)
    return set_error(MONO_E_DEVICE, "mono_layer_launch: needs 224..1024 CUs (and 168 + 4 rows)");
  // 64-key splits, the rows' 32 splits each on a CTA of its own (8 rows: 256 CTAs)
  if (R * (AT_TOPK / 64) > grid)
    return set_error(MONO_E_DEVICE, "mono_layer_launch: needs a CTA for each of the rows' "
                                    "32 attention splits (32 x rows CUs)");
  // rows that may span more than one top-k block take the multi-block variant
  const bool lng = a->ctx_max > AT_TKBLOCK;
  // DSA (FP8) index pages take their own instances (their score code holds more registers)
  // MXFP4 experts: instances of their own (layer_mx.hip)
  using K = LayerKernel;
  const K kerns[2][2][2] = {
      {{layer_kernel<false, 64, false, false, false>, layer_kernel<false, 64, false, true, false>},
       {layer_kernel<false, 64, true, false, false>, layer_kernel<false, 64, true, true, false>}},
      {{layer_kernel<true, 64, false, false, false>, layer_kernel<true, 64, false, true, false>},
       {layer_kernel<true, 64, true, false, false>, layer_kernel<true, 64, true, true, false>}}};
  const K kern = mx ? layer_kernel_mx(shuf, lng, !fp4) : kerns[shuf][lng][!fp4];
  rc = check_coresident(kern, 1024, 0, "mono_layer_launch: one 1024-thread CTA per CU does not fit");
  if (rc) return rc;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(1024), 0, (hipStream_t)stream, p);
  return check_launch("mono_layer_launch");
}
