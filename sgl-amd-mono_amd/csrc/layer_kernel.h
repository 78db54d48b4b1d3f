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
// (sgl_amd_mono/glm53/gfx950/runner.py:240-321); its MoE phase takes FP8 W8A8 experts or
// MXFP4 A16W4 ones (the reference's expert_mxfp4, kernel.py:179, :906-995, :4475-4490).
#pragma once

#include "attn_phase.h"
#include "front_phase.h"
#include "moe_fp8_phase.h"
#include "post_phase.h"

namespace mono {

constexpr int LY_H = 7168, LY_I = 512;
constexpr int LY_MAXR = FR_MAXR;  // the front builds x of at most 8 rows in LDS

constexpr int cmax(int a, int b) { return a > b ? a : b; }
constexpr int LY_LDS_BYTES =
    cmax(cmax(FR_LDS_BYTES, AT_LDS_BYTES),
         cmax(PO_LDS_BYTES, cmax(MoeLds<LY_H, LY_I>::BYTES, MoeLds<LY_H, LY_I, true>::BYTES)));
static_assert(PO_HID == LY_H, "the output block's 16-column tiles cover the MoE's rows");
static_assert(MoeFp8Geom<LY_H, LY_I>::BYTES == MoeFp8Geom<LY_H, LY_I, true>::BYTES,
              "FP8 and MXFP4 layers share one scratch layout");

// scratch of the layer launch for `rm` rows: the barriers, each phase's scratch, and the
// hand-offs between phases that the caller does not ask to see
struct LayerScratch {
  static constexpr size_t BARRIERS = 0;  // count k at 256 k, flag k at 256 k + 128
  size_t front, attn, post, moe, q, iq, iqs, iw, o_lat, a, ssq, bytes;
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
    ssq = at_align(a + (size_t)rm * LY_H * 2);            // f32 [LY_H / 16][16]
    bytes = at_align(ssq + (size_t)(LY_H / 16) * 16 * 4);
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

// MX: MXFP4 (A16W4) experts, else FP8
template <bool SHUF, int SPLIT, bool LONG, bool DSA, bool MX>
__global__ void __launch_bounds__(1024, 1) layer_kernel(LayerParams p) {
  using Arena = LdsArena<LY_LDS_BYTES>;
  __shared__ __attribute__((aligned(16))) uint8_t lds[Arena::TOTAL];
  LaunchShared& sh = *reinterpret_cast<LaunchShared*>(lds + Arena::BODY);
  stamp(p.timeline, MONO_TL_START);
  Guard guard;
  const v4i hd = launch_head_issue(p.guard);
  uint32_t tag = front_phase(p.f, lds, guard, sh.ok, [&]() {
    return launch_begin_from(sh, guard, hd, p.guard, p.host_err, p.fault_site, p.fault_after);
  });
  p.bar[0].arrive(tag);
  stamp(p.timeline, LY_TL_FRONT);
  attn_phase<SPLIT, true, LONG, DSA>(p.at, lds, guard, tag, sh.ok,
                          BarrierWait{&p.bar[0], &guard, tag, MONO_SITE_PHASE, &sh.ok});
  stamp(p.timeline, LY_TL_ATTN);
  // no barrier: the merge ran W_UV, and o's complemented words are their own hand-off
  post_phase<true>(p.po, lds, guard, tag, sh.ok, NoWait{});
  p.bar[1].arrive(tag);
  stamp(p.timeline, LY_TL_POST);
  moe_phase<LY_H, LY_I, SHUF, true, MX>(p.m, lds, guard, tag, sh.ok,
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

using LayerKernel = void (*)(LayerParams);
// the MXFP4-expert instances (their own translation unit): [shuf][long][dsa]
LayerKernel layer_kernel_mx(bool shuf, bool lng, bool dsa);

}  // namespace mono
