// FP8 routed MoE as one persistent gfx950 launch (the FFN half of the DSA layer).
//
// Stages, every CTA in order (task t of a stage runs on CTA t mod grid):
//   0  the rows' RMSNorm factors (every CTA, from L2), then one task a CTA: a router
//      tile (16 experts x 512 K of W_r x bf16(rmsnorm(a)) as a bf16 MFMA; 224 tiles,
//      partial logits out), or a publisher (8 of the 56 128-K chunks: per-128 E4M3
//      quant of every row straight into the MFMA B-operand image, scales out). The
//      normalised rows are quantised once, not on every CTA.
//   1  every CTA copies the published image into LDS (buffer -> LDS). Row r is routed
//      by one CTA (NTASK0 + r mod grid): the 14 partials of its 256 logits summed in a
//      fixed order, sigmoid + bias top-8, the 8 ids and weights out; every CTA reads
//      the R routes and compacts the distinct experts, shared first. Every hand-off is
//      complemented words in one of two scratch buffers (by the tag's parity), zero
//      meaning "not written yet"; the launch clears the other.
//   2  up/gate: task (u, c) = 16 gate + 16 up rows of distinct expert u over all of
//      K, the 8 waves splitting K. W8A8 16x16x128 MFMA per 128-chunk, then the
//      chunk's weight block scale x activation scale into the f32 accumulator.
//      Weight chunks stream through a register ring that already holds the next
//      task's chunks while this one finishes. mid = silu(g) * u goes out as tagged
//      pairs, so no wave ever drains its loads to publish.
//   3  mid quant: task (u, kb) polls a 128-block of mid, quantises it per row to
//      E4M3 with coefficient scale * route weight, publishes, then a ready tag.
//   4  down: task f = 32 output rows over every distinct expert (wave w takes
//      experts u = w mod 8), prefetching the next expert's weights, then a fixed
//      order reduction across waves and out = bf16(a + y).
// The tag of a launch is the guard block's epoch + 1; the last CTA out advances the
// epoch. Every wait polls under the guard's deadline.
//
// Reference: sgl_amd_mono/glm53/gfx950/kernel.py:4199-4330 (router + quant),
// :1575-1629 (route_top8), :4352-4999 (up/gate), :5001-5187 (down), :1440-1450
// (quant_scaled), :1665-1669 (W == 1 residual add).
#pragma once

#include <hip/hip_runtime.h>
#include <stdio.h>

#include <mutex>

#include "moe_common.h"
#include "mono_abi.h"
#include "mx_common.h"
#include "phase.h"

namespace mono {

// MX: MXFP4 experts (A16W4: E2M1 + E8M0 per 32 weights on bf16 rows, the layer launch
// only, at most MXR rows), else FP8 W8A8 experts
template <int H, int I, bool MX = false>
struct MoeFp8Geom {
  static constexpr int WAVES = 16;
  static constexpr int MXR = 8;            // rows of an MXFP4-expert launch, at most
  static constexpr int MQB = MX ? 2 : 1;   // bytes of a mid value as the down stage reads it
  static constexpr int THREADS = WAVES * WAVE;
  static constexpr int QW = 8;             // waves that own a K slice (stage 0, B operands)
  static constexpr int NKC = H / 128;      // 128-K chunks of the hidden dim
  static constexpr int KCW = NKC / QW;     // chunks a K slice holds
  static constexpr int NUG = I / 16;       // up/gate tasks per expert
  static constexpr int NKB = I / 128;      // 128-blocks of the intermediate
  static constexpr int DNT = 16;           // output rows of a down task
  static constexpr int NDN = H / DNT;
  static_assert(NKC % QW == 0, "hidden must split into 8 slices of 128-chunks");
  static_assert(I % 128 == 0, "intermediate must be whole 128-blocks");
  static_assert(H % 128 == 0, "hidden must be whole 128-blocks");

  // scratch layout (bytes)
  static constexpr size_t OFF_MID = 0;
  static constexpr size_t SZ_MID = (size_t)MOE_NDIST * MOE_MAXR * I * 8;
  static constexpr size_t OFF_MQ = OFF_MID + SZ_MID;
  // room for bf16 mids whichever the format: both formats keep one scratch layout, so
  // launches of either kind can share a runtime (counters and hand-off words line up)
  static constexpr size_t SZ_MQ = (size_t)MOE_NDIST * MOE_MAXR * I * 2;
  static constexpr size_t OFF_MCOEF = OFF_MQ + SZ_MQ;
  static constexpr size_t SZ_MCOEF = (size_t)MOE_NDIST * MOE_MAXR * NKB * 4;
  static constexpr size_t OFF_READY = OFF_MCOEF + SZ_MCOEF;
  static constexpr size_t SZ_READY = (size_t)MOE_NDIST * NKB * 4;
  // work-queue counters (zero at launch entry; the last CTA out re-zeroes them)
  static constexpr size_t OFF_QUEUE = (OFF_READY + SZ_READY + 255) & ~(size_t)255;
  static constexpr int NQUEUE = 4;
  // stage 0 tasks: router tiles (16 experts x 512 K), then publishers (8 of the 128-K
  // chunks each); the row routers (one a row) follow them
  static constexpr int NKS = H / 512, NRT = MOE_NEXP / 16, NROUTER = NRT * NKS;
  static constexpr int NPUB = NKC / 8, NTASK0 = NROUTER + NPUB;
  static_assert(H % 1024 == 0 && NKC % 8 == 0, "hidden must be whole 1024-blocks");
  // two parities of hand-offs (complemented words): the B image [NKC][2][64] x 16 B,
  // its scales [NKC][16] f32, the partial logits [NKS][16 rows][256] f32, then the
  // routes [NREP][16 rows][8 ids, 8 weights] in NREP copies 4 KB apart (CTA b reads
  // copy b mod NREP: no line is polled by the whole grid)
  static constexpr int NREP = 8;
  static constexpr size_t REP_STRIDE = 4096;
  static constexpr size_t SZ_XQ = (size_t)NKC * 2 * 64 * 16;
  // MX: the image is bf16 rows as MFMA B operands, [chunk][d][K group][row < MXR] x 16 B
  // (8 bf16 of the row at K 128 chunk + 32 group + 8 d), the same size
  static_assert(!MX || (size_t)NKC * 4 * 4 * MXR * 16 == SZ_XQ, "the bf16 image's size");
  static constexpr size_t SZ_XS = (size_t)NKC * 16 * 4;
  static constexpr size_t SZ_RP = (size_t)NKS * MOE_MAXR * MOE_NEXP * 4;
  static constexpr size_t SZ_RT = NREP * REP_STRIDE;
  static_assert(MOE_MAXR * 16 * 4 <= REP_STRIDE, "a route copy fits its stride");
  static constexpr size_t OFF_XS = SZ_XQ, OFF_RP = OFF_XS + SZ_XS, OFF_RT = OFF_RP + SZ_RP;
  static constexpr size_t SZ_HPAR = (OFF_RT + SZ_RT + 255) & ~(size_t)255;
  static constexpr size_t OFF_H = (OFF_QUEUE + NQUEUE * 4 + 255) & ~(size_t)255;
  static constexpr size_t BYTES = OFF_H + 2 * SZ_HPAR;
};

struct MoeFp8Params {
  int rows;
  float eps, route_scale;
  int n_group, topk_group;  // group-limited routing (n_group <= 1: none)
  const uint16_t* a;
  // fused: a's per-row sums of squares per 16-column tile, f32 [H / 16][16], stored by
  // the output block before its barrier (the norm then reads no whole row of a)
  const float* ssq;
  uint16_t* out;
  const uint16_t* g_post;
  const uint16_t* w_r;
  const float* bias;
  const uint8_t* w13;
  const float* s13;
  const uint8_t* w2;
  const float* s2;
  const uint8_t* e13;  // MX: E8M0 scales of w13 / w2 (w13, w2 then E2M1 codes)
  const uint8_t* e2;
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

// bf16 x 8 in a dword4 -> 8 f32
__device__ inline void bf16x8(v4i v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_lo((uint32_t)v[i]);
    f[2 * i + 1] = bf16_hi((uint32_t)v[i]);
  }
}

typedef __bf16 v8bfm __attribute__((ext_vector_type(8)));

__device__ inline v8i cat8(v4i a, v4i b) {
  return v8i{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// SHUF: expert weights in AITER's (16, 16) layout, [rows / 16, K / 32, 2, 16 rows, 16 B]
// (what SGLang's gfx950 MoE load leaves in place): a 16-row x 128-K MFMA tile is then one
// contiguous 2 KB, and each load instruction reads 8 whole cache lines
// LDS of the MoE phase (offsets in bytes)
template <int H, int I, bool MX = false>
struct MoeLds {
  using G = MoeFp8Geom<H, I, MX>;
  static constexpr int RL = 0;  // RouteLds
  static constexpr int XQ = (int)((sizeof(RouteLds) + 15) & ~(size_t)15);  // v4i [QW KCW 2 64]
  static constexpr int XS = XQ + G::QW * G::KCW * 2 * 64 * 16;   // f32 [QW KCW][16]
  static constexpr int RED = XS + G::QW * G::KCW * 16 * 4;       // v4f [16][64]
  static constexpr int RSTD = RED + G::WAVES * 64 * 16;          // f32 [16]
  static constexpr int NEXT = RSTD + MOE_MAXR * 4;               // int
  static constexpr int N1 = NEXT + 4;                            // int
  static constexpr int ORW = N1 + 4;                             // int: a CTA-wide OR
  static constexpr int HEAD = N1 + 12;                           // u32 [4], 16-byte aligned
  static constexpr int BYTES = HEAD + 16;
  static_assert(XS % 16 == 0 && RED % 16 == 0 && HEAD % 16 == 0, "aligned LDS carving");
};

// The MoE in one CTA of a launch. Standalone it reads the guard head itself, behind its
// first row loads, and sets `guard` and `tag`. FUSED: it is the layer launch's last phase
// (`guard` and `tag` given): it issues the norm weight and its router tile's weights,
// waits at `ready` (the output block's barrier), then reads the stream `a` the output
// block stored, device coherent.
template <int H, int I, bool SHUF, bool FUSED, bool MX = false, class Ready>
__device__ __attribute__((always_inline)) inline void moe_phase(const MoeFp8Params& p,
                                                                uint8_t* lds, Guard& guard,
                                                                uint32_t& tag, int& ok_s,
                                                                Ready ready) {
  using G = MoeFp8Geom<H, I, MX>;
  using LO = MoeLds<H, I, MX>;
  using W13 = MxOperand<SHUF, H>;  // MX: w13 [2 I, H] and w2 [H, I] as E2M1 + E8M0
  using W2 = MxOperand<SHUF, I>;
  using S2 = MxScales<SHUF, I>;
  constexpr int KCW = G::KCW, NUG = G::NUG, NKB = G::NKB, QW = G::QW;
  // the stream a is read through L2 in both forms: fused, its lines are only stored
  // (write-through) before the barrier in this launch, so no cache holds a stale copy
  constexpr int XCP = CP_NONE;
  const int tid = threadIdx.x, l = tid & 63;
  // the wave index in an SGPR: every per-wave address term stays scalar
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = l & 15, grp = l >> 4;  // MFMA column (row of the batch) and K group
  const int half = w / QW, wq = w % QW;  // gate / up (or row group) half, K slice
  const int R = p.rows;
  const int nblk = gridDim.x, b = blockIdx.x;

  RouteLds& rl = *reinterpret_cast<RouteLds*>(lds + LO::RL);
  // the E4M3 activations as each lane's MFMA B operand: [slice][chunk][half][lane]
  v4i* xq_lds = reinterpret_cast<v4i*>(lds + LO::XQ);
  float (*xs_lds)[16] = reinterpret_cast<float (*)[16]>(lds + LO::XS);  // scale per (chunk, row)
  v4f (*red)[64] = reinterpret_cast<v4f (*)[64]>(lds + LO::RED);
  int& next_s = *reinterpret_cast<int*>(lds + LO::NEXT);
  float* rstd_s = reinterpret_cast<float*>(lds + LO::RSTD);
  uint32_t* head_s = reinterpret_cast<uint32_t*>(lds + LO::HEAD);

  uint64_t* mid_pairs = reinterpret_cast<uint64_t*>(p.scratch + G::OFF_MID);
  uint8_t* mq = p.scratch + G::OFF_MQ;
  float* mcoef = reinterpret_cast<float*>(p.scratch + G::OFF_MCOEF);
  uint32_t* ready_w = reinterpret_cast<uint32_t*>(p.scratch + G::OFF_READY);
  uint32_t* queue = reinterpret_cast<uint32_t*>(p.scratch + G::OFF_QUEUE);

  // The rows' sums of squares, in one order whichever the form, so a fused launch's rstd
  // has the bits of a launch of its own: per 16-column tile of a row the balanced
  // pairwise tree of its 16 squares (the output block's 16-lane butterfly, in the fused
  // form), tile t on thread t (H / 16 of them; the rest add zeros), the wave's tiles
  // summed by the wave butterfly, then the 16 waves in order. Fused, the output block
  // stored the tile sums (rows 0-7, f32 [H / 16][16]); standalone, thread t loads its
  // tile of rows row0 .. row0 + 7 (32 bytes a row), issued first so they fly with the
  // staging and guard loads.
  constexpr int NSQT = H / 16;
  static_assert(NSQT <= G::THREADS, "a tile a thread");
  v4i sq0 = {0, 0, 0, 0}, sq1 = {0, 0, 0, 0};  // fused: tile tid's sums of rows 0-7
  v4i at[8][2];                                 // standalone: tile tid of 8 rows
  auto load_tiles = [&](int row0) {
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
      const int r = row0 + rr;
      const bool live = r < R && tid < NSQT;
      const __amdgpu_buffer_rsrc_t rar = rsrc(p.a + (size_t)(r < R ? r : 0) * H, live ? H * 2 : 0);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) at[rr][hh] = ld16<XCP>(rar, (uint32_t)(tid * 16 + 8 * hh) * 2u);
    }
  };
  auto load_ssq = [&]() {
    const __amdgpu_buffer_rsrc_t rq = rsrc(p.ssq, (uint32_t)NSQT * 16u * 4u);
    const uint32_t o = tid < NSQT ? (uint32_t)tid * 64u : 0x80000000u;
    sq0 = ld16<XCP>(rq, o);
    sq1 = ld16<XCP>(rq, o + 16u);
  };
  if constexpr (!FUSED) load_tiles(0);
  // the post-attention norm weight, the same for every row, goes to LDS (over the
  // reduction buffer, idle until stage 2); every load of the prologue is issued before
  // the first is waited on, none under a branch (absent ones read through an empty
  // range), so the one barrier below waits for a single round trip
  v4i* g_lds = reinterpret_cast<v4i*>(&red[0][0]);
  static_assert(H * 2 <= G::WAVES * 64 * 16, "norm weight staging");
  static_assert(H / 8 <= G::THREADS, "one norm-weight piece a thread");
  const v4i gv = ld16<CP_NONE>(rsrc(p.g_post, H * 2), tid < H / 8 ? (uint32_t)tid * 16u : 0x80000000u);
  // this CTA's stage-0 task (the first of them: a grid below NTASK0 loops, unprefetched):
  // router tile (et, ks), wave w takes K [ks 512 + 32 w, + 32); lane l the A operand of
  // expert 16 et + l % 16 at K + 8 (l / 16) and the B operand of row l % 16 there
  auto router_w = [&](int task) {
    const bool on = task < G::NROUTER;
    const int et = on ? task / G::NKS : 0, ks = on ? task % G::NKS : 0;
    const int k = ks * 512 + 32 * w + 8 * grp;
    return ld16<CP_NT>(rsrc(p.w_r, on ? MOE_NEXP * H * 2 : 0u),
                       (uint32_t)((et * 16 + t) * H + k) * 2u);
  };
  auto router_x = [&](int task) {
    const bool on = task < G::NROUTER;
    const int ks = on ? task % G::NKS : 0;
    const int k = ks * 512 + 32 * w + 8 * grp;
    return ld16<XCP>(rsrc(p.a, on ? (uint32_t)R * H * 2 : 0u),
                     t < R ? (uint32_t)(t * H + k) * 2u : 0x80000000u);
  };
  // publisher pt: thread tid the 8 values at 128 kc + 8 m of rows r and r + 8, with
  // kc = 8 pt + tid / 128, r = (tid / 16) % 8, m = tid % 16
  auto pub_loads = [&](int task, v4i (&pa)[2]) {
    const int pt = task - G::NROUTER;
    const bool on = task >= G::NROUTER && task < G::NTASK0;
    const int kc = (on ? pt : 0) * 8 + (tid >> 7), r = (tid >> 4) & 7, m = tid & 15;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int row = r + 8 * hh;
      pa[hh] = ld16<XCP>(rsrc(p.a, on ? (uint32_t)R * H * 2 : 0u),
                         row < R ? (uint32_t)(row * H + kc * 128 + 8 * m) * 2u : 0x80000000u);
    }
  };
  v4i wa0, xa0, pa0[2];
  bool ok = true;
  wa0 = router_w(b);
  if constexpr (FUSED) {
    ok = ready();
    load_ssq();
    xa0 = router_x(b);
    pub_loads(b, pa0);
    if (tid < H / 8) g_lds[tid] = gv;
    for (int i = tid; i < MOE_NDIST; i += G::THREADS) rl.mask[i] = 0;
    if (tid == 0) ok_s = ok ? 1 : 0;
    __syncthreads();
  } else {
    xa0 = router_x(b);
    pub_loads(b, pa0);
    const v4i hd = ld16<CP_DEV>(rsrc(p.guard, 16), tid == 0 ? 0u : 0x80000000u);
    if (tid < H / 8) g_lds[tid] = gv;
    if (tid == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) head_s[i] = (uint32_t)hd[i];
    }
    for (int i = tid; i < MOE_NDIST; i += G::THREADS) rl.mask[i] = 0;
    if (tid == 0) ok_s = 1;
    __syncthreads();
    tag = tag_after(head_s[MONO_GUARD_EPOCH]);
    guard.init(p.guard, p.host_err, p.fault_site, head_s, (uint32_t)p.fault_after);
  }
  uint8_t* hcur = p.scratch + G::OFF_H + (tag & 1u) * G::SZ_HPAR;
  uint8_t* hnxt = p.scratch + G::OFF_H + ((tag + 1u) & 1u) * G::SZ_HPAR;
  uint32_t* hxq = reinterpret_cast<uint32_t*>(hcur);
  uint32_t* hxs = reinterpret_cast<uint32_t*>(hcur + G::OFF_XS);
  uint32_t* hrp = reinterpret_cast<uint32_t*>(hcur + G::OFF_RP);
  uint32_t* hrt = reinterpret_cast<uint32_t*>(hcur + G::OFF_RT);

  // ---------------------------------------------------------------- stage 0
  // the rows' rstd (the sums' order above; a second pass for rows 8-15, standalone)
  {
    float* ssr = &xs_lds[0][0];  // [16 waves][8 rows], over the scale table (idle until stage 1)
    static_assert(G::QW * G::KCW * 16 >= G::WAVES * 8, "the row sums fit the scale table");
    // the waves holding tiles (the others' zeros would add nothing); rows past R skipped
    constexpr int SQW = (NSQT + WAVE - 1) / WAVE;
    // v[rr]: this thread's tile sum of row row0 + rr
    auto reduce_rows = [&](int row0, float (&v)[8]) {
      if (w < SQW) {
#pragma unroll
        for (int r = 0; r < 8; ++r)
          if (row0 + r < R) v[r] = wave_sum(v[r]);
        if (l == 0)
#pragma unroll
          for (int r = 0; r < 8; ++r) ssr[w * 8 + r] = v[r];
      }
      __syncthreads();
      if (tid < 8) {
        float tot = 0.f;
#pragma unroll
        for (int ww = 0; ww < SQW; ++ww) tot += ssr[ww * 8 + tid];
        const int rr = row0 + tid;
        rstd_s[rr] = rr < R ? 1.0f / sqrtf(tot / (float)H + p.eps) : 0.f;
      }
      __syncthreads();
    };
    auto tree_pass = [&](int row0) {
      float v[8];
#pragma unroll
      for (int rr = 0; rr < 8; ++rr)
        v[rr] = w < SQW && row0 + rr < R ? sq_tree16(at[rr][0], at[rr][1]) : 0.f;
      reduce_rows(row0, v);
    };
    if constexpr (FUSED) {
      float v[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[i] = __int_as_float(sq0[i]);
        v[4 + i] = __int_as_float(sq1[i]);
      }
      reduce_rows(0, v);
      if (tid >= 8 && tid < 16) rstd_s[tid] = 0.f;
    } else {
      tree_pass(0);
      if (R > 8) {
        load_tiles(8);
        tree_pass(8);
      } else if (tid >= 8 && tid < 16) {
        rstd_s[tid] = 0.f;
      }
    }
  }
  // the task(s): router tiles publish partial logits, publishers the B image and scales
  for (int task = b; task < (ok ? G::NTASK0 : 0); task += nblk) {
    v4i wa = wa0, xa = xa0, pa[2] = {pa0[0], pa0[1]};
    if (task != b) {
      wa = router_w(task);
      xa = router_x(task);
      pub_loads(task, pa);
      // a previous router tile's reduction overwrote the norm weight (red overlays it)
      __syncthreads();
      if (tid < H / 8) g_lds[tid] = ld16<CP_NONE>(rsrc(p.g_post, H * 2), (uint32_t)tid * 16u);
    }
    __syncthreads();
    if (task < G::NROUTER) {
      const int et = task / G::NKS, ks = task % G::NKS;
      const int k = ks * 512 + 32 * w + 8 * grp;
      // B: bf16(a rstd g) of row t at K k .. k + 7 (rows past R: zeros)
      const float rs = rstd_s[t];
      float fa[8], fg[8];
      bf16x8(xa, fa);
      bf16x8(g_lds[k / 8], fg);
      v4i xb;
#pragma unroll
      for (int d = 0; d < 4; ++d)
        xb[d] = (int)bf16x2_bits(fa[2 * d] * rs * fg[2 * d], fa[2 * d + 1] * rs * fg[2 * d + 1]);
      const v4f z = {0.f, 0.f, 0.f, 0.f};
      const v4f dd = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(v8bfm, wa), __builtin_bit_cast(v8bfm, xb), z, 0, 0, 0);
      __syncthreads();  // every wave read g_lds: red (which it overlays) is free
      red[w][l] = dd;
      __syncthreads();
      if (tid < 256) {
        const int i = tid & 15, r = tid >> 4;
        const int L = r + 16 * (i >> 2), v = i & 3;
        float sum = 0.f;
#pragma unroll
        for (int ww = 0; ww < G::WAVES; ++ww) sum += red[ww][L][v];
        if (r < R) st_dev(&hrp[(ks * MOE_MAXR + r) * MOE_NEXP + et * 16 + i], enc_word(__float_as_uint(sum)));
      }
    } else if constexpr (MX) {
      // the bf16 image: thread tid the 8 values of row r at K 128 kc + 8 m (rows past R
      // read zeros), the MFMA B operand of K group m / 4, d = m % 4
      const int pt = task - G::NROUTER;
      const int kc = pt * 8 + (tid >> 7), r = (tid >> 4) & 7, m = tid & 15;
      float fg[8], fa[8];
      bf16x8(g_lds[kc * 16 + m], fg);
      bf16x8(pa[0], fa);
      const float rs = rstd_s[r];
      v4i o;
#pragma unroll
      for (int d = 0; d < 4; ++d)
        o[d] = (int)enc_word(bf16x2_bits(fa[2 * d] * rs * fg[2 * d], fa[2 * d + 1] * rs * fg[2 * d + 1]));
      st16<CP_DEV>(rsrc(hxq, (uint32_t)G::SZ_XQ),
                   (uint32_t)((((kc * 4 + (m & 3)) * 4 + (m >> 2)) * G::MXR + r) * 16), o);
    } else {
      const int pt = task - G::NROUTER;
      const int kc = pt * 8 + (tid >> 7), r = (tid >> 4) & 7, m = tid & 15;
      const int g4 = m >> 2, hf = (m & 3) >> 1;
      float fg[8];
      bf16x8(g_lds[kc * 16 + m], fg);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int row = r + 8 * hh;
        const float rs = rstd_s[row];
        float fa[8], xn[8];
        bf16x8(pa[hh], fa);
        float am = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          xn[i] = fa[i] * rs * fg[i];
          am = fmaxf(am, fabsf(xn[i]));
        }
        am = row16_max(am);
        const bool nz = am > 0.f;
        const float inv = nz ? FP8_MAX / am : 1.f;
        const uint32_t q0 = pack_fp8x4(clamp_fp8(xn[0] * inv), clamp_fp8(xn[1] * inv),
                                       clamp_fp8(xn[2] * inv), clamp_fp8(xn[3] * inv));
        const uint32_t q1 = pack_fp8x4(clamp_fp8(xn[4] * inv), clamp_fp8(xn[5] * inv),
                                       clamp_fp8(xn[6] * inv), clamp_fp8(xn[7] * inv));
        // rows past R read zeros: zero codes, unit scale
        const size_t at = ((size_t)(kc * 2 + hf) * 64 + row + 16 * g4) * 4 + (m & 1) * 2;
        st_dev64(reinterpret_cast<uint64_t*>(hxq + at),
                 (uint64_t)enc_word(q0) | ((uint64_t)enc_word(q1) << 32));
        if (m == 0) st_dev(&hxs[kc * 16 + row], enc_word(__float_as_uint(nz ? am * INV_FP8_MAX : 1.f)));
      }
    }
  }
  __syncthreads();  // g_lds (under red) is read by every task above
  // clear this CTA's slice of the next launch's hand-off buffers (from the last wave:
  // wave 0's polls below do not queue behind these stores)
  {
    constexpr uint32_t PB = (uint32_t)G::SZ_HPAR;
    const uint32_t slice = (PB / 16 + nblk - 1) / nblk * 16;
    const __amdgpu_buffer_rsrc_t rn = rsrc(hnxt, PB);
    const int ct = G::THREADS - 1 - tid;
    for (uint32_t i = (uint32_t)ct * 16u; i < slice; i += (uint32_t)G::THREADS * 16u)
      st16<CP_DEV>(rn, b * slice + i, v4i{0, 0, 0, 0});
  }

  // ---------------------------------------------------------------- stage 1
  stamp(p.timeline, MONO_TL_STAGED);
  // The B image (buffer -> LDS, 1 KiB a wave instruction). Waves 1-15 first wait for
  // the scale words of the chunks they copy (sc1 polls of 2 words a lane), then copy
  // through L2: one CU of an XCD fetches a line, the others hit it. A line fetched
  // before all of its words were written holds zeros, which the check below finds;
  // the re-copy then reads device-coherent (sc1) data.
  static_assert(G::SZ_XQ / 1024 == 2 * G::NKC, "two 1 KiB chunks a 128-K chunk");
  static_assert(LO::XQ + (int)G::SZ_XQ <= LDS_DMA_END, "the image's copies below 128 KB");
  const __amdgpu_buffer_rsrc_t rxq = rsrc(hxq, (uint32_t)G::SZ_XQ);
  auto copy_image = [&](int w0, int nw, bool coherent) {
    for (int c = w - w0; c < (int)(G::SZ_XQ / 1024); c += nw) {
      auto* dst = (__attribute__((address_space(3))) void*)(reinterpret_cast<uint8_t*>(xq_lds) + c * 1024);
      if (coherent)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rxq, dst, 16, (uint32_t)(c * 1024 + l * 16), 0, 0, CP_DEV);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rxq, dst, 16, (uint32_t)(c * 1024 + l * 16), 0, 0, CP_NONE);
    }
  };
  // a CTA that routes a row copies the image only after routing: LDS writes queued behind
  // the copy's would hold up the router's own LDS traffic
  bool routes_row = false;
  for (int row = 0; row < R; ++row) routes_row |= (G::NTASK0 + row) % nblk == b;
  constexpr int NCW = (int)(G::SZ_XQ / 1024) / (G::WAVES - 1) + 1;  // chunks a wave, at most
  if (MX && w >= 1) {
    // no scale words: lanes 2 j and 2 j + 1 poll the first and the last word of the wave's
    // chunk j (written by the publisher's two waves of that chunk)
    static_assert(2 * NCW <= WAVE, "a lane a polled word");
    const __amdgpu_buffer_rsrc_t rxw = rsrc(hxq, (uint32_t)G::SZ_XQ);
    ok = wait_until(guard, MONO_SITE_LOGITS, [&]() {
      const int c = (w - 1) + (G::WAVES - 1) * (l >> 1);
      const bool on = l < 2 * NCW && c < 2 * G::NKC;
      const uint32_t v = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
          rxw, on ? (uint32_t)(c * 1024 + (l & 1) * 1020) : 0x80000000u, 0, CP_DEV);
      return !__any(on && v == 0u);
    });
    if (!routes_row) copy_image(1, G::WAVES - 1, false);
  } else if (w >= 1) {
    const __amdgpu_buffer_rsrc_t rxs = rsrc(hxs, (uint32_t)G::SZ_XS);
    static_assert(NCW * 16 <= 2 * WAVE, "a wave's scale words fit two loads a lane");
    // lane l: the scale word of chunk (w - 1) + 15 (l / 16 + 4 h), row l % 16
    uint32_t sv[2];
    ok = wait_until(guard, MONO_SITE_LOGITS, [&]() {
      uint32_t v[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = (w - 1) + (G::WAVES - 1) * ((l >> 4) + 4 * h);
        v[h] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
            rxs, c < 2 * G::NKC ? (uint32_t)(((c >> 1) * 16 + (l & 15)) * 4) : 0x80000000u, 0,
            CP_DEV);
      }
      __builtin_amdgcn_sched_barrier(0);
      uint32_t missing = 0;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = (w - 1) + (G::WAVES - 1) * ((l >> 4) + 4 * h);
        missing |= (uint32_t)(c < 2 * G::NKC) & (uint32_t)(v[h] == 0u);
        sv[h] = v[h];
      }
      return !__any(missing);
    });
    if (!routes_row) copy_image(1, G::WAVES - 1, false);
    // the scales polled above are final: both chunks of a 128-K chunk hold the same
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = (w - 1) + (G::WAVES - 1) * ((l >> 4) + 4 * h);
      if (ok && c < 2 * G::NKC) xs_lds[c >> 1][l & 15] = __uint_as_float(~sv[h]);
    }
  }
  // Up/gate task b (b < NUG) is the shared expert's and CTA b's first, whatever the
  // routing: its weights are pulled into L2 now, while the rows are routed (buffer -> LDS
  // copies, every wave's into the first 1 KB of the reduction buffer, idle until stage
  // 2's first epilogue and below 128 KB like every copy target here; stage 2's image
  // check waits for them, long done by then), so that task's ring loads hit L2
  if (MX && b < NUG && !routes_row) {
    const __amdgpu_buffer_rsrc_t r = rsrc(p.w13 + (size_t)MOE_SHARED * W13::code_bytes(2 * I),
                                          ok ? W13::code_bytes(2 * I) : 0u);
    auto* dst = (__attribute__((address_space(3))) void*)(&red[0][0]);
    static_assert(LO::RED + 1024 <= LDS_DMA_END, "the pull's copies below 128 KB");
    const int rg = half * (I / 16) + b;
    const uint32_t cv = W13::code_v(l);
#pragma unroll
    for (int j = 0; j < KCW; ++j) {
      const uint32_t cs = W13::code_s(rg, wq * KCW + j);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, cv, cs, 0, CP_NONE);
    }
  } else if (b < NUG && !routes_row) {
    const uint32_t vo = SHUF ? (uint32_t)(grp * 512 + t * 16) : (uint32_t)(t * H + 32 * grp);
    constexpr uint32_t HO = SHUF ? 256 : 16, CS = SHUF ? 2048 : 128;
    const int row0 = half * I + b * 16;
    const uint32_t so = SHUF ? (uint32_t)((row0 / 16) * (H / 32) * 512 + wq * KCW * CS)
                             : (uint32_t)(row0 * H + wq * KCW * 128);
    const __amdgpu_buffer_rsrc_t r =
        rsrc(p.w13 + (size_t)MOE_SHARED * (2 * I) * H, ok ? 2u * I * H : 0u);
    auto* dst = (__attribute__((address_space(3))) void*)(&red[0][0]);
    static_assert(LO::RED + 1024 <= LDS_DMA_END, "the pull's copies below 128 KB");
#pragma unroll
    for (int j = 0; j < KCW; ++j) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, vo, so + j * CS, 0, CP_NONE);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, vo + HO, so + j * CS, 0, CP_NONE);
    }
  }
  // Row r is routed once, by wave 0 of CTA (NTASK0 + r) mod grid: its 256 logits (the
  // 14 partials summed in a fixed order; a poll that finds an unwritten word is
  // discarded whole), sigmoid, bias top-8; the 8 ids and weights go out as
  // complemented words. Wave 0 of every CTA (which has no image copy queued ahead of
  // its polls) then reads the R routes (4 words a lane) into its slot tables.
  if (w == 0) {
    const __amdgpu_buffer_rsrc_t rrp = rsrc(hrp, (uint32_t)G::SZ_RP);
    for (int row = 0; row < R && ok; ++row) {
      if ((G::NTASK0 + row) % nblk != b) continue;
      // the biases ahead of the poll: loaded after it, they would add a round trip
      // (held here: left to the compiler, the loads sink past the poll into their use)
      float bs[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bs[i] = p.bias[l + 64 * i];
        asm volatile("" : "+v"(bs[i]));
      }
      float lg[4];
      ok = wait_until(guard, MONO_SITE_LOGITS, [&]() {
        // every load issued before the first is used: one round trip a poll
        uint32_t v[G::NKS][4];
#pragma unroll
        for (int ks = 0; ks < G::NKS; ++ks)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            // lane offset in a VGPR, the rest a scalar offset: no per-load address
            v[ks][i] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                rrp, (uint32_t)l * 4u, (uint32_t)((ks * MOE_MAXR + row) * MOE_NEXP + 64 * i) * 4u,
                CP_DEV);
        __builtin_amdgcn_sched_barrier(0);
        uint32_t mn = 0xFFFFFFFFu;
#pragma unroll
        for (int i = 0; i < 4; ++i) lg[i] = __uint_as_float(~v[0][i]);
#pragma unroll
        for (int ks = 0; ks < G::NKS; ++ks)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            mn = min(mn, v[ks][i]);
            if (ks) lg[i] += __uint_as_float(~v[ks][i]);
          }
        return __all(mn != 0u);
      });
      if (ok) {
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[i] = 1.0f / (1.0f + expf(-lg[i]));
        route_row(rl, row, sc, bs, p.route_scale, p.scores, p.ids, p.weights, p.n_group,
                  p.topk_group);
        // lanes l < 8 wrote slots 1 + l (LDS accesses of one wave complete in order)
        __builtin_amdgcn_wave_barrier();
        const int j = l & (MOE_TOPK - 1), c = l >> 3;
        const uint32_t id = enc_word((uint32_t)rl.id[row][1 + j]);
        const uint32_t wt = enc_word(__float_as_uint(rl.w[row][1 + j]));
        static_assert(G::NREP * MOE_TOPK == WAVE, "a lane a (copy, slot)");
        uint32_t* dst = hrt + c * (G::REP_STRIDE / 4) + row * 16;
        st_dev(dst + j, id);
        st_dev(dst + MOE_TOPK + j, wt);
      }
    }
    if (ok) {
      const __amdgpu_buffer_rsrc_t rrt =
          rsrc(hrt + (b % G::NREP) * (G::REP_STRIDE / 4), (uint32_t)G::REP_STRIDE);
      uint32_t rv[4];
      // 256 CTAs poll here for the slowest row's route: a longer sleep between polls
      ok = wait_until<8>(guard, MONO_SITE_LOGITS, [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          rv[i] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rrt, (uint32_t)(l + 64 * i) * 4u,
                                                                 0, CP_DEV);
        __builtin_amdgcn_sched_barrier(0);
        uint32_t missing = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          missing |= (uint32_t)(((l + 64 * i) >> 4) < R) & (uint32_t)(rv[i] == 0u);
        return !__any(missing);
      });
      if (ok) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int idx = l + 64 * i, tt = idx >> 4, j = idx & 15;
          const uint32_t u = ~rv[i];
          if (tt < R) {
            if (j < MOE_TOPK) {
              const int e = (int)min(u, (uint32_t)(MOE_NEXP - 1));
              rl.id[tt][1 + j] = e;
              atomicOr(&rl.mask[e], 1u << tt);
            } else {
              rl.w[tt][1 + j - MOE_TOPK] = __uint_as_float(u);
            }
          }
        }
        if (l < R) {
          rl.id[l][0] = MOE_SHARED;
          rl.w[l][0] = 1.f;
        }
      }
    }
  }
  if (!ok) ok_s = 0;
  __syncthreads();
  if (w == 0) build_experts(rl, R);  // the slot tables follow the first ring's loads
  __syncthreads();
  if (routes_row) copy_image(0, G::WAVES, false);
  ok = ok_s != 0;
  const int nd = rl.nd;

  // ---------------------------------------------------------------- stage 2
  stamp(p.timeline, MONO_TL_ROUTED);
  // waves 0-7: the 16 gate rows of the task, waves 8-15 the 16 up rows; wave wq's
  // K slice is chunks [KCW wq, KCW (wq + 1)). Its ring holds one task's KCW chunks:
  // a slot is refilled with the next task's chunk as soon as its MFMA issued.
  {
    int ntask = ok ? nd * NUG : 0;
    // FP8: a chunk is 32 bytes a lane; MX: a 128-K step is 16 code bytes and a scale byte
    v4i ring[KCW][MX ? 1 : 2];
    uint32_t rsc[MX ? KCW : 1];
    // this lane's row and K group; the second 16 bytes of a lane's 32 sit 16 bytes on
    // (row major) or a 16-row half-tile on (shuffled); a 128-K chunk is CS bytes on
    const uint32_t vo = SHUF ? (uint32_t)(grp * 512 + t * 16) : (uint32_t)(t * H + 32 * grp);
    constexpr uint32_t HO = SHUF ? 256 : 16, CS = SHUF ? 2048 : 128;
    // a task past the end issues through an empty buffer: its loads return 0 with no
    // memory traffic, so the refill needs no branch
    auto task_src = [&](int task, uint32_t& so) {
      const bool live = task < ntask;
      const int tk = live ? task : 0;
      const int u = tk / NUG, cc = tk % NUG;
      const int e = __builtin_amdgcn_readfirstlane(rl.uexp[u]);
      const int row0 = half * I + cc * 16;
      so = SHUF ? (uint32_t)((row0 / 16) * (H / 32) * 512 + wq * KCW * CS)
                : (uint32_t)(row0 * H + wq * KCW * 128);
      return rsrc(p.w13 + (size_t)e * (2 * I) * H, live ? 2u * I * H : 0u);
    };
    // MX: task `task`'s 128-K step j of its 16-row group of expert uexp[u]: codes, scale
    // (one byte load a step: a wave's K slice of KCW = 7 steps starts at either parity,
    // so paired scale words would need a code path per parity)
    auto mx_issue = [&](int task, int j) {
      const bool live = task < ntask;
      const int tk = live ? task : 0;
      const int u = tk / NUG, cc = tk % NUG;
      const int e = __builtin_amdgcn_readfirstlane(rl.uexp[u]);
      const int rg = half * (I / 16) + cc, st = wq * KCW + j;
      ring[j][0] = ld16s<CP_NT>(
          rsrc(p.w13 + (size_t)e * W13::code_bytes(2 * I), live ? W13::code_bytes(2 * I) : 0u),
          W13::code_v(l), W13::code_s(rg, st));
      rsc[j] = ld1(
          rsrc(p.e13 + (size_t)e * W13::scale_bytes(2 * I), live ? W13::scale_bytes(2 * I) : 0u),
          W13::scale_v(l), W13::scale_s(rg, st));
    };
    // Task hand-out: CTA b runs tasks b and b + nblk first; later tasks come from a
    // device-wide counter in order (2 nblk, 2 nblk + 1, ...), each grabbed one task ahead
    // so the ring can be refilled with the next task while this one runs. The first grab
    // is issued inside the first task: every CTA's grab hits the one counter at about the
    // same moment and the replies return one after another over microseconds, which a
    // grab ahead of the first ring would add to the first task's wait (the wave's loads
    // retire in order). Tasks run the same arithmetic on whichever CTA takes them, so
    // results do not depend on the hand-out.
    int task = b;
    if constexpr (MX) {
#pragma unroll
      for (int j = 0; j < KCW; ++j) mx_issue(task, j);
    } else {
      uint32_t so;
      const __amdgpu_buffer_rsrc_t r = task_src(task, so);
#pragma unroll
      for (int j = 0; j < KCW; ++j) {
        ring[j][0] = ld16s<CP_NT>(r, vo, so + j * CS);
        ring[j][1] = ld16s<CP_NT>(r, vo + HO, so + j * CS);
      }
    }
    // the (expert, row) slot tables, needed from the mid quant on: built while the first
    // ring is in flight (the image check's barrier publishes them)
    if (w == 0) build_slots(rl, R);
    // The image, checked while the first task's weights are in flight: every word
    // written (a line fetched early may hold zeros: copy it again, device-coherent). One
    // pass checks and un-complements: a failed check re-copies all. The first pass waits
    // for the image copy only (the 2 KCW ring loads issued after it stay in flight) and
    // sits outside the retry loop: an LDS access reached from a re-copy issued behind the
    // ring would make the compiler wait for every load, the whole ring, before it.
    {
      uint32_t* xw = reinterpret_cast<uint32_t*>(xq_lds);
      bool got = ok_s != 0;  // set before the barrier above (CTA-uniform)
      // a CTA-wide OR through an LDS word (zero on entry, left zero). Not
      // __syncthreads_or: it reads the dispatch packet, and so waits for every load in
      // flight, the whole ring
      int& orw = *reinterpret_cast<int*>(lds + LO::ORW);
      auto cta_or = [&](bool v) {
        if (__ballot(v) && l == 0) atomicOr(&orw, 1);
        __syncthreads();
        const bool r = orw != 0;
        __syncthreads();
        if (tid == 0) orw = 0;
        return r;
      };
      auto check = [&]() {
        int zero = 0;
        static_assert(G::SZ_XQ / 4 % G::THREADS == 0, "whole passes over the image");
#pragma unroll 7
        for (int i = tid; i < (int)(G::SZ_XQ / 4); i += G::THREADS) {
          const uint32_t v = xw[i];
          zero |= v == 0u;
          xw[i] = ~v;
        }
        return cta_or(zero != 0);
      };
      if (tid == 0) orw = 0;
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * KCW));
      asm volatile("" ::: "memory");
      __syncthreads();
      bool bad = got && check();
      int polls = 0;
      uint64_t start = 0;
      while (bad) {
        // bounded like every wait: the guard's deadline and abort flag
        if ((++polls & 15) == 0) {
          if (guard.aborted()) got = false;
          const uint64_t now = wall_clock64();
          if (start == 0) start = now;
          if (got && now - start > guard.deadline * (guard.fault_site ? guard.slack : 1)) {
            if (tid == 0) guard.fail(MONO_SITE_LOGITS);
            got = false;
          }
        }
        got = !cta_or(!got) && got;
        if (!got) break;
        copy_image(0, G::WAVES, true);
        drain();
        asm volatile("" ::: "memory");
        __syncthreads();
        bad = check();
      }
      if (!got) ok_s = 0;
    }
    __syncthreads();
    if (ok_s == 0) {
      ok = false;
      ntask = 0;
    }
    int next = b + nblk < ntask ? b + nblk : ntask;
    while (task < ntask) {
      const int u = task / NUG, cc = task % NUG;
      const int e = __builtin_amdgcn_readfirstlane(rl.uexp[u]);
      const uint32_t mask = rl.umask[u];
      const float tok_on = ((mask >> t) & 1u) ? 1.f : 0.f;
      const int sbase = __builtin_amdgcn_readfirstlane(
          (e * (2 * I / 128) + (half * I + cc * 16) / 128) * (H / 128) + wq * KCW);
      // the task after next (its value lands in LDS before the epilogue barrier). Lane 0
      // of wave 0 grabs it, the other lanes are out of range: with a branch around the
      // atomic the compiler waits for its reply (and so for every load before it, the
      // whole ring) right after the branch, before this task's MFMAs
      const bool grab_on = next < ntask;
      const uint32_t grabbed = (uint32_t)__builtin_amdgcn_raw_ptr_buffer_atomic_add_i32(
          1, rsrc(queue, grab_on ? 4u : 0u), tid == 0 ? 0u : 0x80000000u, 0, 0);
      v4f acc = {0.f, 0.f, 0.f, 0.f};
      if constexpr (MX) {
        // B operands of row t (rows t >= 8 reread row t - 8: their output columns are
        // never stored), through an opaque base as below
        const int xo = opaque_v(wq * KCW * 128 + grp * G::MXR + (t & (G::MXR - 1)));
#pragma unroll
        for (int j = 0; j < KCW; ++j) {
          v4i B[4];
#pragma unroll
          for (int d = 0; d < 4; ++d) B[d] = xq_lds[xo + j * 128 + d * 32];
          acc = fp4_step(ring[j][0], rsc[j], B, acc);
          mx_issue(next, j);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
        uint32_t son;
        const __amdgpu_buffer_rsrc_t rn = task_src(next, son);
        // B operands and scales: the same LDS words every task, read through an opaque
        // base so they are not hoisted out of the loop (they would hold 56 VGPRs)
        const int xb = opaque_v(wq * KCW * 2 * 64 + l);
        const int sb = opaque_v(wq * KCW * 16 + t);
#pragma unroll
        for (int j = 0; j < KCW; ++j) {
          const v8i B = cat8(xq_lds[xb + j * 128], xq_lds[xb + j * 128 + 64]);
          const v4f zero = {0.f, 0.f, 0.f, 0.f};
          const v4f d = mfma_fp8(cat8(ring[j][0], ring[j][1]), B, zero);
          // the slot is free once its MFMA issued: refill it with the next task's chunk
          ring[j][0] = ld16s<CP_NT>(rn, vo, son + j * CS);
          ring[j][1] = ld16s<CP_NT>(rn, vo + HO, son + j * CS);
          acc += d * (sld(p.s13, sbase + j) * ((&xs_lds[0][0])[sb + j * 16] * tok_on));
          // one chunk per scheduling region keeps the live set to the ring
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      red[w][l] = acc;
      if (tid == 0) next_s = grab_on ? 2 * nblk + (int)grabbed : ntask;
      __syncthreads();
      const int after = next_s;
      if (tid < 256) {
        const int row = tid & 15, tok = tid >> 4;  // adjacent threads, adjacent features
        const int L = tok + 16 * (row >> 2), v = row & 3;
        float gs = 0.f, us = 0.f;
#pragma unroll
        for (int i = 0; i < QW; ++i) {
          gs += red[i][L][v];
          us += red[QW + i][L][v];
        }
        if (tok < R && ((mask >> tok) & 1u)) {
          const float m = gs / (1.0f + expf(-gs)) * us;
          st_dev64(&mid_pairs[((size_t)u * MOE_MAXR + tok) * I + cc * 16 + row],
                   pair(__float_as_uint(m), tag));
        }
      }
      __syncthreads();
      task = next;
      next = after;
    }
  }

  // ---------------------------------------------------------------- stage 3
  stamp(p.timeline, MONO_TL_UPGATE);
  // mid quant: task (u, kb), one wave a row, handed out in (u, kb) order from a
  // device-wide counter: the CTAs that leave up/gate first quantise the experts whose
  // tiles finished first, so the down stage can start on them. Trip counts stay
  // CTA-uniform (barriers per task); a failed wait only skips work.
  {
    const int nq = ok ? nd * NKB : 0;
    auto grab = [&]() {
      if (tid == 0) next_s = nq ? (int)add_dev(&queue[1], 1u) : nq;
      __syncthreads();
      const int q = next_s;
      __syncthreads();  // next_s is rewritten by the next grab
      return q;
    };
    for (int q = grab(); q < nq; q = grab()) {
      const int u = q / NKB, kb = q % NKB;
      const int e = rl.uexp[u];
      const uint32_t mask = rl.umask[u];
      const int tok = w;
      if (tok < R && ((mask >> tok) & 1u) && ok) {
        const size_t base = ((size_t)u * MOE_MAXR + tok) * I + kb * 128 + 2 * l;
        uint64_t p0 = 0, p1 = 0;
        ok = wait_until(guard, MONO_SITE_MID, [&]() {
          p0 = ld_dev64(&mid_pairs[base]);
          p1 = ld_dev64(&mid_pairs[base + 1]);
          return __all((uint32_t)(p0 >> 32) == tag && (uint32_t)(p1 >> 32) == tag);
        });
        if (MX && ok) {
          // A16W4: the mid rounds to bf16; its down coefficient is the route weight
          const float v0 = __uint_as_float((uint32_t)p0), v1 = __uint_as_float((uint32_t)p1);
          st_dev(reinterpret_cast<uint32_t*>(
                     mq + (((size_t)u * MOE_MAXR + tok) * I + kb * 128 + 2 * l) * 2),
                 bf16x2_bits(v0, v1));
          if (l == 0)
            st_devf(&mcoef[((size_t)u * MOE_MAXR + tok) * NKB + kb], route_weight(rl, tok, e));
        } else if (ok) {
          const float v0 = __uint_as_float((uint32_t)p0), v1 = __uint_as_float((uint32_t)p1);
          const float am = wave_max(fmaxf(fabsf(v0), fabsf(v1)));
          const bool nz = am > 0.f;
          const float sc = nz ? am * INV_FP8_MAX : 1.f;
          const float inv = nz ? FP8_MAX / am : 1.f;
          const uint32_t h = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(
                                 clamp_fp8(v0 * inv), clamp_fp8(v1 * inv), 0, false) &
                             0xFFFFu;
          const uint32_t hn = dpp_u<DPP_XOR1>(h);
          if ((l & 1) == 0)
            st_dev(reinterpret_cast<uint32_t*>(mq + ((size_t)u * MOE_MAXR + tok) * I + kb * 128 +
                                               2 * l),
                   h | (hn << 16));
          if (l == 0)
            st_devf(&mcoef[((size_t)u * MOE_MAXR + tok) * NKB + kb],
                    sc * route_weight(rl, tok, e));
        }
      }
      drain();
      const bool all_ok = cta_ok(ok, guard, ok_s);
      if (tid == 0 && all_ok) st_dev(&ready_w[u * NKB + kb], tag);
    }
    ok = cta_ok(ok, guard, ok_s);
  }

  // ---------------------------------------------------------------- stage 4
  stamp(p.timeline, MONO_TL_MIDQ);
  // down: task f = output rows [16 f, 16 f + 16); wave w takes experts u = w, w + 16, ...
  // in order. CTA b runs task b, then tasks from a device-wide counter (nblk, nblk + 1,
  // ...): its second is grabbed on arrival here, each later one in its wave 0's last step
  // of the task before, so a CTA that leaves up/gate early takes two tasks and one that
  // leaves late takes one, and the stage ends together. The (expert, row) mid
  // rows are copied into LDS over the dead activation operands, so the expert loop
  // streams weights with no poll and no other global load: first those of the experts
  // already quantised when the CTA gets here (one pass over the ready words, the first
  // weight tile already in flight), which it streams while the rest are quantised, then,
  // after one wait, the others. Each wave still takes its experts in the same order.
  {
    const int ntask = ok ? G::NDN : 0;
    constexpr int DW = G::WAVES;  // a wave's expert stride
    static_assert(G::NDN >= 256, "a first task for every CTA of a full grid");
    // [9 R slots][I] E4M3 (MX: bf16, at most MXR rows), then f32 [slots][NKB]
    constexpr int SLOTR = MX ? G::MXR : MOE_MAXR, ROWB = I * G::MQB;
    uint8_t* mql = reinterpret_cast<uint8_t*>(xq_lds);
    float* mcl = reinterpret_cast<float*>(mql + SLOTR * MOE_SLOTS * ROWB);
    static_assert(SLOTR * MOE_SLOTS * (ROWB + NKB * 4) <= LO::XS - LO::XQ, "mid slots");
    static_assert(LO::XQ + SLOTR * MOE_SLOTS * ROWB <= LDS_DMA_END, "mid copies below 128 KB");
    // one tile of weight chunks a wave; each chunk is refilled with the next step's as
    // soon as its MFMA issued, the last expert of a task running into the next task
    // (MX: a 128-K step is 16 code bytes and a scale byte a lane)
    v4i buf[NKB][MX ? 1 : 2];
    uint32_t bsc[MX ? NKB : 1];
    const uint32_t vo = SHUF ? (uint32_t)(grp * 512 + t * 16) : (uint32_t)t * I + 32 * grp;
    constexpr uint32_t HO = SHUF ? 256 : 16, CS = SHUF ? 2048 : 128;
    auto src_of = [&](int f, int u, uint32_t& so) {
      const bool live = f < ntask && u < nd;
      const int e = __builtin_amdgcn_readfirstlane(rl.uexp[live ? u : 0]);
      const int row0 = (live ? f : 0) * G::DNT;
      so = SHUF ? (uint32_t)((row0 / 16) * (I / 32) * 512) : (uint32_t)row0 * I;
      return rsrc(p.w2 + (size_t)e * H * I, live ? (uint32_t)H * I : 0u);
    };
    // MX: step kb of expert uexp[u]'s 16-row group f: codes, scale
    auto mx_issue = [&](int f, int u, int kb) {
      const bool live = f < ntask && u < nd;
      const int e = __builtin_amdgcn_readfirstlane(rl.uexp[live ? u : 0]);
      const int fr = live ? f : 0;
      buf[kb][0] = ld16s<CP_NT>(
          rsrc(p.w2 + (size_t)e * W2::code_bytes(H), live ? W2::code_bytes(H) : 0u),
          W2::code_v(l), W2::code_s(fr, kb));
      if (S2::loads(kb, NKB))
        bsc[kb] = S2::load(
            rsrc(p.e2 + (size_t)e * W2::scale_bytes(H), live ? W2::scale_bytes(H) : 0u), l, fr, kb);
    };
    if constexpr (MX) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) mx_issue(b, w, kb);
    } else {
      uint32_t so;
      const __amdgpu_buffer_rsrc_t r = src_of(b, w, so);
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        buf[kb][0] = ld16s<CP_NT>(r, vo, so + kb * CS);
        buf[kb][1] = ld16s<CP_NT>(r, vo, so + kb * CS + HO);
      }
    }
    // mid rows + coefficients of slots [s0, s1) into LDS (slots are in expert order):
    // the rows by buffer -> LDS copies (2 rows of 512 B a wave instruction, no
    // registers), the coefficients one a thread; then every wave drains (the copies
    // land behind its weight tile in flight, which its next MFMA waits for anyway)
    const int nsl = R * MOE_SLOTS;
    static_assert(I == 512, "a wave's 1 KiB copy is two mid rows (MX: one)");
    auto copy_slots = [&](int s0, int s1) {
      const __amdgpu_buffer_rsrc_t rmq = rsrc(mq, (uint32_t)G::SZ_MQ);
      const __amdgpu_buffer_rsrc_t rmc = rsrc(mcoef, (uint32_t)G::SZ_MCOEF);
      for (int c = w; MX && c < s1 - s0; c += G::WAVES) {
        const int ut = rl.slot_ut[s0 + c];
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rmq, (__attribute__((address_space(3))) void*)(mql + (s0 + c) * ROWB), 16,
            (uint32_t)((((ut >> 8) * MOE_MAXR + (ut & 255)) * I) * 2 + l * 16), 0, 0, CP_DEV);
      }
      for (int c = w; !MX && 2 * c < s1 - s0; c += G::WAVES) {
        const int sl = s0 + 2 * c + (l >> 5);
        if (sl < s1) {  // an odd count: the last copy's upper half-wave writes nothing
          const int ut = rl.slot_ut[sl];
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rmq, (__attribute__((address_space(3))) void*)(mql + (s0 + 2 * c) * I), 16,
              (uint32_t)(((ut >> 8) * MOE_MAXR + (ut & 255)) * I + (l & 31) * 16), 0, 0, CP_DEV);
        }
      }
      static_assert(MOE_MAXR * MOE_SLOTS * NKB <= G::THREADS, "a coefficient a thread");
      const int nc = (s1 - s0) * NKB;
      const int sc_ = s0 + (tid < nc ? tid / NKB : 0), kc = tid % NKB;
      const int utc = rl.slot_ut[sc_];
      const uint32_t cw = (uint32_t)ld4<CP_DEV>(
          rmc, tid < nc ? (uint32_t)((((utc >> 8) * MOE_MAXR + (utc & 255)) * NKB + kc) * 4)
                        : 0x80000000u);
      if (tid < nc) mcl[s0 * NKB + tid] = __uint_as_float(cw);
      drain();
      asm volatile("" ::: "memory");  // the LDS reads after the barrier stay after it
    };
    // the leading experts already quantised: one pass over the ready words
    int& n1_s = *reinterpret_cast<int*>(lds + LO::N1);
    if (tid == 0) n1_s = nd;
    __syncthreads();
    if (ntask) {
      // the second task, with the ready words' round trip
      if (tid == 0) {
        const uint32_t g = add_dev(&queue[2], 1u);
        next_s = nblk + (int)g < ntask ? nblk + (int)g : ntask;
      }
      const int i = tid;
      static_assert(MOE_NDIST * NKB <= 2 * G::THREADS, "two ready words a thread");
      const uint32_t r0 = ld4<CP_DEV>(rsrc(ready_w, (uint32_t)(nd * NKB) * 4u), (uint32_t)i * 4u);
      const uint32_t r1 = ld4<CP_DEV>(rsrc(ready_w, (uint32_t)(nd * NKB) * 4u),
                                      (uint32_t)(i + G::THREADS) * 4u);
      if (i < nd * NKB && r0 != tag) atomicMin(&n1_s, i / NKB);
      if (i + G::THREADS < nd * NKB && r1 != tag) atomicMin(&n1_s, (i + G::THREADS) / NKB);
    }
    __syncthreads();
    const int n1 = ntask ? n1_s : nd;
    int next = ntask ? next_s : 0;
    const int s_split = n1 < nd ? rl.uslot[n1] : nsl;
    if (ok && ntask) copy_slots(0, s_split);
    __syncthreads();
    bool rest = n1 < nd;  // the experts from n1 on are still to be copied
    for (int f = b; f < (ok ? ntask : 0);) {
      const int rg0 = f * G::DNT;
      v4f acc = {0.f, 0.f, 0.f, 0.f};
      int u = w;
      uint32_t grabbed = 0;
      auto step = [&]() {
        int fn = f, un = u + DW;
        const bool last = un >= nd;
        if (last) {
          fn = next;
          un = w;
        }
        // the task after next: lane 0 of wave 0 in its last step (wave 0 has the most
        // steps); the other lanes and steps are out of range, with no branch (a branch
        // around the atomic would make the compiler wait for its reply right after it)
        const bool grab_on = last && next < ntask;
        grabbed = (uint32_t)__builtin_amdgcn_raw_ptr_buffer_atomic_add_i32(
            1, rsrc(queue + 2, grab_on ? 4u : 0u), tid == 0 ? 0u : 0x80000000u, 0, 0);
        uint32_t son;
        const __amdgpu_buffer_rsrc_t rn = src_of(fn, un, son);
        const int e = __builtin_amdgcn_readfirstlane(rl.uexp[u]);
        const int sl = slot_of(rl, u, rl.umask[u], t);
        const bool on = sl >= 0;
        if constexpr (MX) {
          // lane l: the mid row's bf16 at K 128 kb + 32 (l / 16) + 8 d, d < 4
          // a row t not routed to u reads slot row 0 (copied before any expert is
          // computed, a finite mid): its output column is scaled by cf = 0, adding
          // exactly nothing (no masked LDS reads)
          const uint8_t* mrow = mql + (on ? sl : 0) * ROWB + 64 * grp;
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) {
            v4i B[4];
#pragma unroll
            for (int d = 0; d < 4; ++d) B[d] = *reinterpret_cast<const v4i*>(mrow + kb * 256 + d * 16);
            const float cf = on ? mcl[(on ? sl : 0) * NKB + kb] : 0.f;
            const v4f zero = {0.f, 0.f, 0.f, 0.f};
            const v4f d = fp4_step(buf[kb][0], S2::of(bsc[S2::slot(kb, NKB)], f, kb), B, zero);
            mx_issue(fn, un, kb);
            acc += d * cf;
            __builtin_amdgcn_sched_barrier(0);
          }
          u += DW;
          return;
        }
        const int bb = (on ? sl : 0) * I + 32 * grp;
        const int s2b =
            __builtin_amdgcn_readfirstlane((e * (H / 128) + rg0 / 128) * (I / 128));
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          // a row t not routed to u reads slot row 0, scaled by cf = 0 (as above)
          const v4i b0 = *reinterpret_cast<const v4i*>(mql + bb + kb * 128);
          const v4i b1 = *reinterpret_cast<const v4i*>(mql + bb + kb * 128 + 16);
          const float cf = on ? mcl[(on ? sl : 0) * NKB + kb] : 0.f;
          const v4f zero = {0.f, 0.f, 0.f, 0.f};
          const v4f d = mfma_fp8(cat8(buf[kb][0], buf[kb][1]), cat8(b0, b1), zero);
          buf[kb][0] = ld16s<CP_NT>(rn, vo, son + kb * CS);
          buf[kb][1] = ld16s<CP_NT>(rn, vo, son + kb * CS + HO);
          acc += d * (sld(p.s2, s2b + kb) * cf);
          __builtin_amdgcn_sched_barrier(0);
        }
        u += DW;
      };
      while (u < (rest ? n1 : nd)) step();
      if (rest) {
        // the other experts: every wave waits for their ready words (its polls return
        // behind its weight tiles in flight), then their mid rows into LDS
        rest = false;
        const int i = w * 64 + l;
        ok = wait_until(guard, MONO_SITE_MQ, [&]() {
          const uint32_t rv = i < nd * NKB && i >= n1 * NKB ? ld_dev(&ready_w[i]) : tag;
          return __all(rv == tag);
        });
        ok = cta_all(ok, ok_s);
        if (ok) copy_slots(s_split, nsl);
        __syncthreads();
        if (!ok) break;
        while (u < nd) step();
      }
      // fixed-order reduction over the 16 waves, then the residual add
      red[w][l] = acc;
      if (tid == 0) next_s = next < ntask ? nblk + (int)grabbed : ntask;
      __syncthreads();
      const int after = next_s < ntask ? next_s : ntask;
      if (tid < 256) {
        const int row = tid & 15, tok = tid >> 4;  // 16 rows x 16 columns, rows fastest
        const int L = tok + 16 * (row >> 2), v = row & 3;
        float ys = 0.f;
#pragma unroll
        for (int i = 0; i < G::WAVES; ++i) ys += red[i][L][v];
        if (tok < R) {
          const int col = f * G::DNT + row;
          const float av = bf16_lo((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(
              rsrc(p.a, (uint32_t)R * H * 2u), (uint32_t)(tok * H + col) * 2u, 0, XCP));
          // write-through: a failed launch's NaN fill must not meet a dirty line
          __builtin_amdgcn_raw_buffer_store_b16((uint16_t)bf16_bits(av + ys),
                                                rsrc(p.out, (uint32_t)R * H * 2u),
                                                (uint32_t)(tok * H + col) * 2u, 0, CP_DEV);
          if (p.y)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(ys),
                                                  rsrc(p.y, (uint32_t)R * H * 4u),
                                                  (uint32_t)(tok * H + col) * 4u, 0, CP_DEV);
        }
      }
      __syncthreads();
      f = next;
      next = after;
    }
  }

}

// the MoE's work-queue counters, which the launch's last CTA out zeroes for the next
template <int H, int I>
__device__ inline void moe_reset_queues(const MoeFp8Params& p) {
  using G = MoeFp8Geom<H, I>;
  uint32_t* queue = reinterpret_cast<uint32_t*>(p.scratch + G::OFF_QUEUE);
#pragma unroll
  for (int i = 0; i < G::NQUEUE; ++i) st_dev(queue + i, 0u);
}

}  // namespace mono
