// The whole decoder layer as one persistent gfx950 launch: the front, the attention phase,
// the output block and the FP8 MoE run back to back in every CTA of one 256-CTA launch.
//
// Before the attention and before the MoE sits a grid barrier (phase.h): a phase's stores
// are device coherent and drained before its CTA arrives, the last arrival raises the
// barrier's flag to the launch tag, and the next phase waits for the flag only after
// issuing the loads that do not depend on the phase before it:
//   attention  the index pages of its first score task (the rows' own keys, written by the
//              front in this launch, are read again device coherent after the wait);
//   MoE        the norm weight and its router tile's weights.
// The output block needs none: the attention's merge runs W_UV on the latents it merges
// and stores o as complemented words, which o_proj's loads poll (zero: not written yet).
// Every wait is deadline guarded; a failing wait lets every CTA run to the end of the
// launch. The launch tag is the guard's epoch + 1, shared by the four phases (each keeps
// its own scratch region), and the last CTA out zeroes the barrier counts and advances the
// epoch.
//
// Replaces the reference's one-launch layer kernel, sgl_amd_mono/glm53/gfx950/kernel.py:
// 171-5282 (launch arguments :5191-5234), driven per layer by Glm53LayerOp.launch
// (sgl_amd_mono/glm53/gfx950/runner.py:240-321).
#include "attn_phase.h"
#include "front_phase.h"
#include "moe_fp8_phase.h"
#include "post_phase.h"

namespace mono {

constexpr int LY_H = 7168, LY_I = 512;
constexpr int LY_MAXR = FR_MAXR;  // the front builds x of at most 8 rows in LDS

constexpr int cmax(int a, int b) { return a > b ? a : b; }
constexpr int LY_LDS_BYTES =
    cmax(cmax(FR_LDS_BYTES, AT_LDS_BYTES), cmax(PO_LDS_BYTES, MoeLds<LY_H, LY_I>::BYTES));

// scratch of the layer launch for `rm` rows: the barriers, each phase's scratch, and the
// hand-offs between phases that the caller does not ask to see
struct LayerScratch {
  static constexpr size_t BARRIERS = 0;  // count k at 256 k, flag k at 256 k + 128
  size_t front, attn, post, moe, q, iq, iqs, iw, o_lat, a, bytes;
  __host__ __device__ explicit LayerScratch(int rm) {
    front = 1024;
    attn = at_align(front + FrontScratch::BYTES);
    post = at_align(attn + AttnScratch(rm).bytes);
    moe = at_align(post + PostScratch::BYTES);
    q = at_align(moe + MoeFp8Geom<LY_H, LY_I>::BYTES);
    iq = at_align(q + (size_t)rm * AT_HEADS * AT_KV * 2);
    iqs = at_align(iq + (size_t)rm * AT_IHEADS * 256);  // FP4 codes, or a DSA page's bf16 query
    iw = at_align(iqs + (size_t)rm * 256);
    o_lat = at_align(iw + (size_t)rm * AT_IHEADS * 4);
    a = at_align(o_lat + (size_t)rm * AT_HEADS * AT_LAT * 2);
    bytes = at_align(a + (size_t)rm * LY_H * 2);
  }
};

struct LayerParams {
  FrontParams f;
  AttnParams at;
  PostParams po;
  MoeFp8Params m;
  PhaseBarrier bar[2];  // front -> attention, output block -> MoE
  uint8_t* scratch;
  int32_t* guard;
  uint32_t* host_err;
  int fault_site, fault_after;
  uint64_t* timeline;
};

// layer timeline marks: start, each phase's end, exit
constexpr int LY_TL_FRONT = 1, LY_TL_ATTN = 2, LY_TL_POST = 3, LY_TL_MOE = 4, LY_TL_END = 5;

template <bool SHUF, int SPLIT, bool LONG, bool DSA>
__global__ void __launch_bounds__(1024, 1) layer_kernel(LayerParams p) {
  using Arena = LdsArena<LY_LDS_BYTES>;
  __shared__ __attribute__((aligned(16))) uint8_t lds[Arena::TOTAL];
  LaunchShared& sh = *reinterpret_cast<LaunchShared*>(lds + Arena::BODY);
  stamp(p.timeline, MONO_TL_START);
  Guard guard;
  uint32_t tag = launch_begin(sh, guard, p.guard, p.host_err, p.fault_site, p.fault_after);
  front_phase(p.f, lds, guard, tag, sh.ok);
  p.bar[0].arrive(tag);
  stamp(p.timeline, LY_TL_FRONT);
  attn_phase<SPLIT, true, LONG, DSA>(p.at, lds, guard, tag, sh.ok,
                          BarrierWait{&p.bar[0], &guard, tag, MONO_SITE_PHASE, &sh.ok});
  stamp(p.timeline, LY_TL_ATTN);
  // no barrier: the merge ran W_UV, and o's complemented words are their own hand-off
  post_phase<true>(p.po, lds, guard, tag, sh.ok, NoWait{});
  p.bar[1].arrive(tag);
  stamp(p.timeline, LY_TL_POST);
  moe_phase<LY_H, LY_I, SHUF, true>(p.m, lds, guard, tag, sh.ok,
                                    BarrierWait{&p.bar[1], &guard, tag, MONO_SITE_PHASE, &sh.ok});
  stamp(p.timeline, LY_TL_MOE);
  launch_end(sh, p.guard, tag, p.scratch,
             (uint32_t)LayerScratch(p.at.rows_max).bytes,
             Poison{p.m.out, (uint32_t)p.m.rows * LY_H * 2u, NAN_BF16X2},
             Poison{p.m.y, (uint32_t)p.m.rows * LY_H * 4u, NAN_F32},
             [&]() {
               moe_reset_queues<LY_H, LY_I>(p.m);
#pragma unroll
               for (int k = 0; k < 2; ++k) p.bar[k].reset();
             });
  stamp(p.timeline, LY_TL_END);
}

}  // namespace mono

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
  if (!a->h || !a->out || !a->positions || !a->slots || !a->req_ids || !a->page_table ||
      !a->kv || !a->plane || (fp4 && !a->plane_scale) || !a->g_in || !a->g_q || !a->g_kv ||
      !a->w_qkv_a || !a->s_qkv_a || !a->w_k || !a->s_k || !a->w_w || !a->g_k || !a->b_k ||
      !a->w_qb || !a->s_qb || !a->w_iq || !a->s_iq || !a->w_uk || !a->s_uk || !a->cos ||
      !a->sin || !a->w_uv || !a->s_uv || !a->w_o || !a->s_o || !a->g_post || !a->w_r ||
      !a->bias || !a->w13 || !a->s13 || !a->w2 || !a->s2 || !a->scratch || !a->guard)
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
  m.out = static_cast<uint16_t*>(a->out);
  m.g_post = static_cast<const uint16_t*>(a->g_post);
  m.w_r = static_cast<const uint16_t*>(a->w_r);
  m.bias = a->bias;
  m.w13 = a->w13;
  m.s13 = a->s13;
  m.w2 = a->w2;
  m.s2 = a->s2;
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
  using K = void (*)(LayerParams);
  const K kerns[2][2][2] = {
      {{layer_kernel<false, 64, false, false>, layer_kernel<false, 64, false, true>},
       {layer_kernel<false, 64, true, false>, layer_kernel<false, 64, true, true>}},
      {{layer_kernel<true, 64, false, false>, layer_kernel<true, 64, false, true>},
       {layer_kernel<true, 64, true, false>, layer_kernel<true, 64, true, true>}}};
  const K kern = kerns[shuf][lng][!fp4];
  rc = check_coresident(kern, 1024, 0, "mono_layer_launch: one 1024-thread CTA per CU does not fit");
  if (rc) return rc;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(1024), 0, (hipStream_t)stream, p);
  return check_launch("mono_layer_launch");
}
