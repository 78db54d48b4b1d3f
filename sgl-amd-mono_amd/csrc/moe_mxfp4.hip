// MXFP4 (A16W4) routed MoE as one persistent gfx950 launch.
//
// Stages, every CTA in order:
//   0  the CTA's MFMA B operands (each wave's K slice of the bf16 rows) load into
//      registers while waves 0..R-1 route one row each from the given logits: sigmoid,
//      + bias, top-8 with lowest-id ties, weights raw / sum * scale. Every CTA routes
//      for itself (the logits are inputs), so nothing is handed off before up/gate.
//   1  up/gate: task (u, c) = 32 gate + 32 up rows of distinct expert u over all of K;
//      task t runs on CTA t mod grid. Waves 0-7 take the gate rows, 8-15 the up rows,
//      each wave a quarter of K of one 16-row group. A lane's 16 code bytes are one
//      row's 32-group, which shares one E8M0 scale (in the AITER layout one scale dword
//      serves two 128-K steps): v_cvt_scalef32_pk_bf16_fp4 dequantises them exactly to
//      32 bf16 for four 16x16x32 bf16 MFMAs; the B operands (the rows) wait in LDS. Each
//      wave keeps two tasks of weights in flight. Waves 0 and 1 reduce each task and
//      store mid = bf16(silu(g) * u) by slot (row, pick); only after the CTA's last task
//      do they wait for those stores, then the CTA's done word gets the launch tag.
//   2  down: task f = 16 output rows over every distinct expert, run by CTA grid - 1 - f
//      (the CTAs with the fewest up/gate tasks), wave w < 15 taking the experts
//      u = w (mod 15). Its first four experts' weights are in flight before wave 15,
//      which has no loads of its own, polls every CTA's done word and copies the R x 9
//      mid slot rows into LDS; each expert is computed as soon as its weights are in.
//      Each expert's partial is scaled by the row's route weight; a fixed-order
//      reduction over the waves and out = bf16(res + y).
// The tag of a launch is the guard block's epoch + 1; the last CTA out advances it.
//
// Reference: A16W4 operands sgl_amd_mono/minimax_m31/a16w4.py:26-92 (lane = one row's
// 32-group, scale folded into the fp4 -> bf16 convert); MXFP4 units
// sgl_amd_mono/glm53/gfx950/kernel.py:906-995; route as
// test/kernels/test_minimax_m31_ffn.py:146-151; the e8m0 shuffle index
// sgl_amd_mono/common/mx.py:40-44.
#include <hip/hip_runtime.h>

#include "moe_common.h"
#include "mono_abi.h"
#include "mx_common.h"
#include "phase.h"

namespace mono {

template <int H, int I>
struct MoeMxGeom {
  static constexpr int WAVES = 16;
  static constexpr int THREADS = WAVES * WAVE;
  static constexpr int QK = 4;          // waves splitting K for one 16-row group (up/gate)
  static constexpr int NKS = H / 128;   // 128-K steps of the hidden dim
  static constexpr int KSW = NKS / QK;  // steps of a wave's K slice
  static constexpr int NUG = I / 32;    // up/gate tasks per expert (32 gate + 32 up rows)
  static constexpr int NDS = I / 128;   // 128-K steps of the intermediate
  static constexpr int NDN = H / 16;    // down tasks (one a CTA: the grid must hold them)
  static constexpr int DW = WAVES - 1;  // down: waves that stream weights (the last one waits)
  static constexpr int RING = 4;        // experts of down weights a wave keeps in flight
  static_assert(NKS % QK == 0, "hidden must split into 4 slices of 128-steps");
  static_assert(I % 128 == 0, "intermediate must be whole 128-steps");

  // scratch layout (bytes)
  static constexpr size_t OFF_MID = 0;  // bf16 [R x 9 slots][I]
  static constexpr size_t SZ_MID = (size_t)MOE_MAXR * MOE_SLOTS * I * 2;
  static constexpr int MAX_GRID = 1024;
  static constexpr size_t OFF_DONE = (OFF_MID + SZ_MID + 255) & ~(size_t)255;  // u32 per CTA
  static constexpr size_t BYTES = (OFF_DONE + MAX_GRID * 4 + 255) & ~(size_t)255;
};

struct MoeMxParams {
  int rows;
  float route_scale;
  int n_group, topk_group;  // group-limited routing (n_group <= 1: none)
  const uint16_t* x;
  const uint16_t* res;
  uint16_t* out;
  const float* logits;
  const float* bias;
  const uint8_t* w13;
  const uint8_t* s13;
  const uint8_t* w2;
  const uint8_t* s2;
  float* y;
  float* scores;
  int32_t* ids;
  float* weights;
  uint8_t* scratch;
  int32_t* guard;
  uint32_t* host_err;
  int fault_site, fault_after;
  uint64_t* timeline;
};

template <int H, int I, bool SHUF>
__global__ void __launch_bounds__(1024, 1) moe_mxfp4_kernel(MoeMxParams p) {
  using G = MoeMxGeom<H, I>;
  using W13 = MxOperand<SHUF, H>;  // [2 I, H]
  using W2 = MxOperand<SHUF, I>;   // [H, I]
  using S13 = MxScales<SHUF, H>;
  using S2 = MxScales<SHUF, I>;
  constexpr int KSW = G::KSW, NUG = G::NUG, NDS = G::NDS, QK = G::QK, RING = G::RING;
  constexpr int THREADS = G::THREADS, DW = G::DW;
  const int tid = threadIdx.x, l = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = l & 15, grp = l >> 4;  // MFMA column (row of the batch) and K group
  // up/gate roles: gate or up half, 16-row group of the task's pair, K slice
  const int half = w >> 3, rsub = (w >> 2) & 1, kq = w & 3;
  const int R = p.rows;
  const int nblk = gridDim.x, b = blockIdx.x;

  // One arena (the kernel's only LDS variable, at LDS address 0), carved here:
  //   MID   up/gate: the rows as MFMA B operands, [step][d][lane] (16 B: 8 bf16 of row
  //         lane % 16 at K 128 step + 32 (lane / 16) + 8 d); down: the mid slot rows,
  //         bf16 [R x 9][I], copied by buffer -> LDS copies, so first and below 128 KB
  //   RL    RouteLds;  RED  v4f [2][16][64] (up/gate: by task parity; down: [0])
  //   WS    f32 [R x 9]: route weight of each (expert, row) slot;  HEAD  u32 [4];  OK  int
  constexpr int MID = 0, MID_BYTES = MOE_MAXR * MOE_SLOTS * I * 2;
  constexpr int RL = (MID + MID_BYTES + 15) & ~15;
  constexpr int RED = (RL + (int)sizeof(RouteLds) + 15) & ~15;
  constexpr int WS = RED + 2 * G::WAVES * 64 * 16;
  constexpr int HEAD = (WS + MOE_MAXR * MOE_SLOTS * 4 + 15) & ~15;
  constexpr int OK = HEAD + 16;
  using Arena = LdsArena<OK + 4>;
  static_assert(MID + MID_BYTES <= LDS_DMA_END, "the mid copies below 128 KB");
  static_assert(G::NKS * 4 * 64 * 16 <= MID_BYTES, "B operand staging");
  __shared__ __attribute__((aligned(16))) uint8_t lds[Arena::TOTAL];
  uint8_t* const mid_lds = lds + MID;
  RouteLds& rl = *reinterpret_cast<RouteLds*>(lds + RL);
  v4f (*red)[G::WAVES][64] = reinterpret_cast<v4f (*)[G::WAVES][64]>(lds + RED);
  float* const wslot = reinterpret_cast<float*>(lds + WS);
  uint32_t* const head_s = reinterpret_cast<uint32_t*>(lds + HEAD);
  int& ok_s = *reinterpret_cast<int*>(lds + OK);
  LaunchShared& sh = *reinterpret_cast<LaunchShared*>(lds + Arena::BODY);

  uint16_t* mid = reinterpret_cast<uint16_t*>(p.scratch + G::OFF_MID);
  uint32_t* done = reinterpret_cast<uint32_t*>(p.scratch + G::OFF_DONE);
  v4i* x_lds = reinterpret_cast<v4i*>(mid_lds);

  stamp(p.timeline, MONO_TL_START);
  // the loads everything else waits on, in the order they are needed: the routing
  // waves' logits and biases, the guard words, the rows
  float lg[4] = {0.f, 0.f, 0.f, 0.f}, bs[4] = {0.f, 0.f, 0.f, 0.f};
  if (w < R) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lg[i] = p.logits[w * MOE_NEXP + l + 64 * i];
      bs[i] = p.bias[l + 64 * i];
    }
  }
  v4i head = {0, 0, 0, 0};
  if (tid == 0) head = ld16<CP_DEV>(rsrc(p.guard, 16), 0);
  constexpr int XPT = G::NKS * 4 * 64 / THREADS;  // B-operand pieces per thread
  static_assert(G::NKS * 4 * 64 % THREADS == 0, "B operand staging split");
  v4i xv[XPT];
  {
    const __amdgpu_buffer_rsrc_t rx = rsrc(p.x, (uint32_t)R * H * 2);
#pragma unroll
    for (int k = 0; k < XPT; ++k) {
      const int i = tid + THREADS * k, ln = i & 63, sd = i >> 6;
      xv[k] = ld16<CP_NONE>(
          rx, (uint32_t)(((ln & 15) * H + 128 * (sd >> 2) + 32 * (ln >> 4) + 8 * (sd & 3)) * 2));
    }
  }
  for (int i = tid; i < MOE_NDIST; i += THREADS) rl.mask[i] = 0;
  if (tid == 0) ok_s = 1;
  __syncthreads();

  // ---------------------------------------------------------------- stage 0: routing
  stamp(p.timeline, MONO_TL_STAGED);
  if (w < R) {
    float sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sc[i] = 1.0f / (1.0f + expf(-lg[i]));
    const bool out0 = b == 0;
    route_row(rl, w, sc, bs, p.route_scale, out0 ? p.scores : nullptr, out0 ? p.ids : nullptr,
              out0 ? p.weights : nullptr, p.n_group, p.topk_group);
  }
#pragma unroll
  for (int k = 0; k < XPT; ++k) x_lds[tid + THREADS * k] = xv[k];
  if (tid == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) head_s[i] = (uint32_t)head[i];
  }
  __syncthreads();
  const uint32_t tag = tag_after(head_s[MONO_GUARD_EPOCH]);
  Guard guard;
  guard.init(p.guard, p.host_err, p.fault_site, head_s, (uint32_t)p.fault_after);
  if (w == 0) build_experts(rl, R);  // the slot tables follow the first weight loads
  __syncthreads();
  const int nd = rl.nd;

  // ---------------------------------------------------------------- stage 1: up/gate
  stamp(p.timeline, MONO_TL_ROUTED);
  {
    const int ntask = nd * NUG;
    const uint32_t cv = W13::code_v(l);
    // operands of a task for this wave; a task past the end reads through empty
    // buffers (loads return 0, no memory traffic), so refills need no branch. Step j's
    // scale word sits in slot S13::slot(j) (a wave's K slice starts at an even step)
    static_assert(KSW % 2 == 0, "paired scale words within a wave's K slice");
    auto issue = [&](int task, int j, v4i& wv, uint32_t& code) {
      const bool live = task < ntask;
      const int tk = live ? task : 0;
      const int u = tk / NUG, cc = tk % NUG;
      const int e = __builtin_amdgcn_readfirstlane(rl.uexp[u]);
      const int rg = half * (I / 16) + 2 * cc + rsub;
      const int s = kq * KSW + j;
      const __amdgpu_buffer_rsrc_t rc =
          rsrc(p.w13 + (size_t)e * W13::code_bytes(2 * I), live ? W13::code_bytes(2 * I) : 0u);
      const __amdgpu_buffer_rsrc_t rs =
          rsrc(p.s13 + (size_t)e * W13::scale_bytes(2 * I), live ? W13::scale_bytes(2 * I) : 0u);
      wv = ld16s<CP_NT>(rc, cv, W13::code_s(rg, s));
      if (S13::loads(j, KSW)) code = S13::load(rs, l, rg, s);
    };
    // two tasks of weights in flight per wave
    v4i w0[KSW], w1[KSW];
    uint32_t c0[KSW], c1[KSW];
#pragma unroll
    for (int j = 0; j < KSW; ++j) issue(b, j, w0[j], c0[j]);
#pragma unroll
    for (int j = 0; j < KSW; ++j) issue(b + nblk, j, w1[j], c1[j]);

    // the (expert, row) slot tables and each slot's route weight, built while the first
    // two tasks' weights are in flight
    if (w == 0) build_slots(rl, R);
    __syncthreads();
    for (int s = tid; s < R * MOE_SLOTS; s += THREADS) {
      const int ut = rl.slot_ut[s];
      wslot[s] = route_weight(rl, ut & 255, rl.uexp[ut >> 8]);
    }
    __syncthreads();

    int k = 0;  // tasks this CTA ran (the parity of the reduction buffer)
    auto run = [&](int task, v4i (&wv)[KSW], uint32_t (&code)[KSW]) {
      const int u = task / NUG, cc = task % NUG;
      const int par = k & 1;
      ++k;
      // the B operands: the same LDS words every task, read through an opaque base so
      // they are not hoisted out of the task loop (they would hold 96 VGPRs)
      const int xo = opaque_v(kq * KSW * 256 + l);
      v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < KSW; ++j) {
        v4i B[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) B[d] = x_lds[xo + (j * 4 + d) * 64];
        acc = fp4_step(wv[j], S13::of(code[S13::slot(j, KSW)], rsub, j), B, acc);
        issue(task + 2 * nblk, j, wv[j], code[j]);
        __builtin_amdgcn_sched_barrier(0);
      }
      red[par][w][l] = acc;
      __syncthreads();
      if (w < 2) {
        // wave r finishes 16-row group r of the pair: lane l holds rows 4 (l / 16) + v,
        // batch row l % 16; the gate and up partials of the four K slices summed in order
        const int g0 = 4 * w, u0 = 8 + 4 * w;
        v4f gs = red[par][g0][l], us = red[par][u0][l];
#pragma unroll
        for (int i = 1; i < QK; ++i) {
          gs += red[par][g0 + i][l];
          us += red[par][u0 + i][l];
        }
        const uint32_t mask = rl.umask[u];
        if (t < R && ((mask >> t) & 1u)) {
          uint32_t h[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) h[v] = bf16_bits(gs[v] / (1.0f + expf(-gs[v])) * us[v]);
          const int sl = slot_of(rl, u, mask, t);
          st_dev64(reinterpret_cast<uint64_t*>(mid + (size_t)sl * I + (2 * cc + w) * 16 + 4 * grp),
                   (uint64_t)(h[0] | (h[1] << 16)) | ((uint64_t)(h[2] | (h[3] << 16)) << 32));
        }
      }
    };
    for (int task = b; task < ntask; task += 2 * nblk) {
      run(task, w0, c0);
      if (task + nblk < ntask) run(task + nblk, w1, c1);
    }
    // waves 0 and 1 made every mid store of this CTA: once they completed, the CTA's
    // done word takes the launch tag (the one wait for stores in the stage)
    if (w < 2) drain();
    __syncthreads();
    if (tid == 0) st_dev(&done[b], tag);
  }

  // ---------------------------------------------------------------- stage 2: down
  stamp(p.timeline, MONO_TL_UPGATE);
  bool ok = true;
  {
    // CTA b runs down task nblk - 1 - b (the CTAs with the fewest up/gate tasks, the
    // highest b, take the down tasks first; the host refuses a grid below NDN CTAs)
    const int f = nblk - 1 - b;
    const bool has = f < G::NDN;
    const uint32_t cv = W2::code_v(l);
    // the NDS steps of distinct expert u's 16-row group f (no task or an expert past the
    // end: empty buffers, no memory traffic)
    auto issue = [&](int u, v4i (&wv)[NDS], uint32_t (&code)[NDS]) {
      const bool live = has && u < nd;
      const int e = __builtin_amdgcn_readfirstlane(rl.uexp[live ? u : 0]);
      const int fr = live ? f : 0;
      const __amdgpu_buffer_rsrc_t rc =
          rsrc(p.w2 + (size_t)e * W2::code_bytes(H), live ? W2::code_bytes(H) : 0u);
      const __amdgpu_buffer_rsrc_t rs =
          rsrc(p.s2 + (size_t)e * W2::scale_bytes(H), live ? W2::scale_bytes(H) : 0u);
#pragma unroll
      for (int s = 0; s < NDS; ++s) {
        wv[s] = ld16s<CP_NT>(rc, cv, W2::code_s(fr, s));
        if (S2::loads(s, NDS)) code[s] = S2::load(rs, l, fr, s);
      }
    };
    // waves 0..DW-1 take experts u = w, w + DW, ...: their first RING experts' weights
    // are issued now, with no branch (so each expert waits only for its own loads), and
    // each expert is computed as soon as its weights are in
    v4i dw[RING][NDS];
    uint32_t dc[RING][NDS];
    const int wu = w < DW ? w : MOE_NDIST;  // the last wave takes no expert
#pragma unroll
    for (int q = 0; q < RING; ++q) issue(wu + DW * q, dw[q], dc[q]);
    // the last wave, with no load of its own in flight (loads complete in order), polls
    // every CTA's done word, then copies the R x 9 mid slot rows into LDS in 1 KiB pieces
    // and waits for them; the streaming waves wait at the barrier only, not for their
    // weights
    if (w == DW)
      ok = wait_until(guard, MONO_SITE_MID, [&]() {
        bool all = true;
        for (int i = l; i < nblk; i += WAVE) all &= ld_dev(&done[i]) == tag;
        return __all(all);
      });
    ok = cta_all(ok, ok_s);
    if (ok && has && w == DW) {
      const uint32_t nbytes = (uint32_t)R * MOE_SLOTS * I * 2;
      const __amdgpu_buffer_rsrc_t rm = rsrc(mid, nbytes);
      for (uint32_t off = 0; off < nbytes; off += 1024)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rm, (__attribute__((address_space(3))) void*)(mid_lds + off), 16, l * 16 + off, 0,
            0, CP_DEV);
      drain();
    }
    __syncthreads();
    stamp(p.timeline, MONO_TL_MIDQ);
    if (ok && has) {
      v4f acc = {0.f, 0.f, 0.f, 0.f};
      // expert u from its weights in the ring slot (wv, code)
      auto expert = [&](int u, const v4i (&wv)[NDS], const uint32_t (&code)[NDS]) {
        const int sl = slot_of(rl, u, rl.umask[u], t);
        const bool on = sl >= 0;
        const float wt = on ? wslot[sl] : 0.f;
        // a row t not routed to u reads slot row 0 (always a written, finite mid): its
        // output column t is then scaled by wt = 0, which adds exactly nothing
        const uint8_t* mrow = mid_lds + (on ? sl : 0) * I * 2 + 64 * grp;
        v4f d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < NDS; ++s) {
          v4i B[4];
#pragma unroll
          for (int dd = 0; dd < 4; ++dd)
            B[dd] = *reinterpret_cast<const v4i*>(mrow + s * 256 + dd * 16);
          d = fp4_step(wv[s], S2::of(code[S2::slot(s, NDS)], f, s), B, d);
        }
        acc += d * wt;
      };
      // the first ring in straight-line code (each expert waits for its own loads only),
      // then rings of RING more experts (over 60 distinct experts), issued and computed
#pragma unroll
      for (int q = 0; q < RING; ++q)
        if (wu + DW * q < nd) expert(wu + DW * q, dw[q], dc[q]);
      for (int k0 = RING; wu + DW * k0 < nd; k0 += RING) {
#pragma unroll
        for (int q = 0; q < RING; ++q) issue(wu + DW * (k0 + q), dw[q], dc[q]);
#pragma unroll
        for (int q = 0; q < RING; ++q)
          if (wu + DW * (k0 + q) < nd) expert(wu + DW * (k0 + q), dw[q], dc[q]);
      }
      red[0][w][l] = acc;
    }
    __syncthreads();
    if (ok && has && w == 0) {
      v4f ys = red[0][0][l];
#pragma unroll
      for (int i = 1; i < DW; ++i) ys += red[0][i][l];
      if (t < R) {
        const int col = f * 16 + 4 * grp;
        uint32_t h[4];
#pragma unroll
        for (int v = 0; v < 4; ++v)
          h[v] = bf16_bits((p.res ? bf16_lo(p.res[t * H + col + v]) : 0.f) + ys[v]);
        // write-through: a failed launch's NaN fill must not meet a dirty line
        const v2i hv = {(int32_t)(h[0] | (h[1] << 16)), (int32_t)(h[2] | (h[3] << 16))};
        __builtin_amdgcn_raw_buffer_store_b64(hv, rsrc(p.out, (uint32_t)R * H * 2u),
                                              (uint32_t)(t * H + col) * 2u, 0, CP_DEV);
        if (p.y)
          st16<CP_DEV>(rsrc(p.y, (uint32_t)R * H * 4u), (uint32_t)(t * H + col) * 4u,
                       __builtin_bit_cast(v4i, ys));
      }
    }
    __syncthreads();
  }

  // ---------------------------------------------------------------- exit
  stamp(p.timeline, MONO_TL_DOWN);
  launch_end(sh, p.guard, tag, p.scratch, (uint32_t)G::BYTES,
             Poison{p.out, (uint32_t)R * H * 2u, NAN_BF16X2},
             Poison{p.y, (uint32_t)R * H * 4u, NAN_F32}, []() {});
  stamp(p.timeline, MONO_TL_END);
}

}  // namespace mono

using namespace mono;

extern "C" size_t mono_moe_mxfp4_scratch_bytes(int32_t hidden, int32_t inter, int32_t experts) {
  if (experts != MOE_NEXP) return 0;
  if (hidden == 3072 && inter == 384) return MoeMxGeom<3072, 384>::BYTES;
  return 0;
}

extern "C" int mono_moe_mxfp4_launch(const MonoMoeMxfp4Args* a, mono_stream_t stream) {
  if (!a) return set_error(MONO_E_ARG, "mono_moe_mxfp4_launch: null args");
  if (a->rows < 1 || a->rows > MOE_MAXR)
    return set_error(MONO_E_ARG, "mono_moe_mxfp4_launch: rows must be 1..16");
  if (a->experts != MOE_NEXP)
    return set_error(MONO_E_ARG, "mono_moe_mxfp4_launch: experts must be 256");
  if (!a->x || !a->out || !a->logits || !a->bias || !a->w13 || !a->s13 || !a->w2 || !a->s2 ||
      !a->scratch || !a->guard)
    return set_error(MONO_E_ARG, "mono_moe_mxfp4_launch: null tensor");
  if (a->layout != MONO_LAYOUT_ROWMAJOR && a->layout != MONO_LAYOUT_AITER16)
    return set_error(MONO_E_ARG, "mono_moe_mxfp4_launch: unknown weight layout");
  if (!route_groups_ok(a->n_group, a->topk_group))
    return set_error(MONO_E_ARG, "mono_moe_mxfp4_launch: n_group / topk_group: 2..16 groups "
                                 "dividing 256, keeping >= 8 experts");
  MoeMxParams p;
  p.rows = a->rows;
  p.route_scale = a->route_scale;
  p.n_group = a->n_group;
  p.topk_group = a->topk_group;
  p.x = static_cast<const uint16_t*>(a->x);
  p.res = static_cast<const uint16_t*>(a->res);
  p.out = static_cast<uint16_t*>(a->out);
  p.logits = a->logits;
  p.bias = a->bias;
  p.w13 = a->w13;
  p.s13 = a->s13;
  p.w2 = a->w2;
  p.s2 = a->s2;
  p.y = a->y;
  p.scores = a->scores;
  p.ids = a->ids;
  p.weights = a->weights;
  p.scratch = static_cast<uint8_t*>(a->scratch);
  p.guard = a->guard;
  p.host_err = nullptr;
  if (a->host_error) {
    void* dptr = nullptr;
    if (hipHostGetDevicePointer(&dptr, a->host_error, 0) != hipSuccess || !dptr)
      return set_error(MONO_E_ARG, "mono_moe_mxfp4_launch: host_error is not pinned host memory");
    p.host_err = static_cast<uint32_t*>(dptr);
  }
  p.fault_site = a->fault_site;
  p.fault_after = a->fault_after;
  p.timeline = a->timeline;
  int grid = 0;
  int rc = monokernel_grid(&grid);
  if (rc) return rc;
  if (grid > MoeMxGeom<3072, 384>::MAX_GRID)
    return set_error(MONO_E_DEVICE, "mono_moe_mxfp4_launch: more CUs than done words");
  if (grid < MoeMxGeom<3072, 384>::NDN)
    return set_error(MONO_E_DEVICE, "mono_moe_mxfp4_launch: fewer CUs than down tasks");
  if (a->hidden == 3072 && a->inter == 384) {
    auto k = a->layout == MONO_LAYOUT_AITER16 ? moe_mxfp4_kernel<3072, 384, true>
                                              : moe_mxfp4_kernel<3072, 384, false>;
    rc = check_coresident(k, 1024, 0,
                          "mono_moe_mxfp4_launch: one 1024-thread CTA per CU does not fit");
    if (rc) return rc;
    hipLaunchKernelGGL(k, dim3(grid), dim3(1024), 0, (hipStream_t)stream, p);
  } else {
    return set_error(MONO_E_ARG, "mono_moe_mxfp4_launch: unsupported hidden/inter");
  }
  return check_launch("mono_moe_mxfp4_launch");
}
