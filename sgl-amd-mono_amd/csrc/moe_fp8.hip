// FP8 routed MoE as one persistent gfx950 launch (the FFN half of the DSA layer).
//
// Stages, every CTA in order (task t of a stage runs on CTA t mod grid):
//   0  RMSNorm of the R rows (every CTA, from L2), per-128 E4M3 quant of its wave's
//      K slice straight into MFMA B-operand registers, and the router logit of its
//      expert(s), published as (value, tag) pairs.
//   1  routing: each CTA polls the 256 x R logits and runs sigmoid + bias top-8
//      itself (one wave a row), then compacts the distinct experts, shared first.
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
#include <hip/hip_runtime.h>

#include <type_traits>

#include "moe_common.h"
#include "mono_abi.h"

namespace mono {

template <int H, int I>
struct MoeFp8Geom {
  static constexpr int WAVES = 16;
  static constexpr int THREADS = WAVES * WAVE;
  static constexpr int QW = 8;             // waves that own a K slice (stage 0, B operands)
  static constexpr int NKC = H / 128;      // 128-K chunks of the hidden dim
  static constexpr int KCW = NKC / QW;     // chunks a K slice holds
  static constexpr int NUG = I / 16;       // up/gate tasks per expert
  static constexpr int NKB = I / 128;      // 128-blocks of the intermediate
  static constexpr int DNT = 32;           // output rows of a down task
  static constexpr int NDN = H / DNT;
  static_assert(NKC % QW == 0, "hidden must split into 8 slices of 128-chunks");
  static_assert(I % 128 == 0, "intermediate must be whole 128-blocks");
  static_assert(H % 128 == 0, "hidden must be whole 128-blocks");

  // scratch layout (bytes)
  static constexpr size_t OFF_LOGIT = 0;
  static constexpr size_t SZ_LOGIT = (size_t)MOE_MAXR * MOE_NEXP * 8;
  static constexpr size_t OFF_MID = OFF_LOGIT + SZ_LOGIT;
  static constexpr size_t SZ_MID = (size_t)MOE_NDIST * MOE_MAXR * I * 8;
  static constexpr size_t OFF_MQ = OFF_MID + SZ_MID;
  static constexpr size_t SZ_MQ = (size_t)MOE_NDIST * MOE_MAXR * I;
  static constexpr size_t OFF_MCOEF = OFF_MQ + SZ_MQ;
  static constexpr size_t SZ_MCOEF = (size_t)MOE_NDIST * MOE_MAXR * NKB * 4;
  static constexpr size_t OFF_READY = OFF_MCOEF + SZ_MCOEF;
  static constexpr size_t SZ_READY = (size_t)MOE_NDIST * NKB * 4;
  // work-queue counters (zero at launch entry; the last CTA out re-zeroes them)
  static constexpr size_t OFF_QUEUE = (OFF_READY + SZ_READY + 255) & ~(size_t)255;
  static constexpr int NQUEUE = 4;
  static constexpr size_t BYTES = (OFF_QUEUE + NQUEUE * 4 + 255) & ~(size_t)255;
};

struct MoeFp8Params {
  int rows;
  float eps, route_scale;
  const uint16_t* a;
  uint16_t* out;
  const uint16_t* g_post;
  const uint16_t* w_r;
  const float* bias;
  const uint8_t* w13;
  const float* s13;
  const uint8_t* w2;
  const float* s2;
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

__device__ inline v8i cat8(v4i a, v4i b) {
  return v8i{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// SHUF: expert weights in AITER's (16, 16) layout, [rows / 16, K / 32, 2, 16 rows, 16 B]
// (what SGLang's gfx950 MoE load leaves in place): a 16-row x 128-K MFMA tile is then one
// contiguous 2 KB, and each load instruction reads 8 whole cache lines
template <int H, int I, bool SHUF>
__global__ void __launch_bounds__(1024, 1) moe_fp8_kernel(MoeFp8Params p) {
  using G = MoeFp8Geom<H, I>;
  constexpr int KCW = G::KCW, NUG = G::NUG, NKB = G::NKB, QW = G::QW;
  const int tid = threadIdx.x, l = tid & 63;
  // the wave index in an SGPR: every per-wave address term stays scalar
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = l & 15, grp = l >> 4;  // MFMA column (row of the batch) and K group
  const int half = w / QW, wq = w % QW;  // gate / up (or row group) half, K slice
  const int R = p.rows;
  const int nblk = gridDim.x, b = blockIdx.x;

  __shared__ RouteLds rl;
  // the E4M3 activations as each lane's MFMA B operand: [slice][chunk][half][lane]
  __shared__ v4i xq_lds[QW * KCW * 2 * 64];
  __shared__ float xs_lds[QW * KCW][16];  // activation block scale per (chunk, row)
  __shared__ v4f red[G::WAVES][64];
  __shared__ float red_small[2][2][16];
  __shared__ v4i wr_lds[H / 8];  // this CTA's router row (bf16), staged like the norm weight
  __shared__ int next_s;
  __shared__ float rstd_s[MOE_MAXR];
  __shared__ int ok_s;

  uint64_t* logit_pairs = reinterpret_cast<uint64_t*>(p.scratch + G::OFF_LOGIT);
  uint64_t* mid_pairs = reinterpret_cast<uint64_t*>(p.scratch + G::OFF_MID);
  uint8_t* mq = p.scratch + G::OFF_MQ;
  float* mcoef = reinterpret_cast<float*>(p.scratch + G::OFF_MCOEF);
  uint32_t* ready = reinterpret_cast<uint32_t*>(p.scratch + G::OFF_READY);
  uint32_t* queue = reinterpret_cast<uint32_t*>(p.scratch + G::OFF_QUEUE);

  __shared__ uint32_t head_s[4];
  stamp(p.timeline, MONO_TL_START);
  // the first eight rows: two waves a row, lane l the 8 values at q * 512 + l * 8 of its
  // half's 7 slices; issued first so they fly with the staging and guard loads below
  constexpr int NQ0 = H / 1024;
  v4i av0[NQ0];
  {
    const int r = w / 2, ch = w % 2;
    const bool live = r < R;
    const __amdgpu_buffer_rsrc_t rar = rsrc(p.a + (size_t)(live ? r : 0) * H, live ? H * 2 : 0);
    const uint32_t base = (uint32_t)(ch * NQ0 * 512 + l * 8) * 2;
#pragma unroll
    for (int q = 0; q < NQ0; ++q) av0[q] = ld16<CP_NONE>(rar, base + q * 1024);
  }
  const __amdgpu_buffer_rsrc_t rg = rsrc(p.g_post, H * 2);
  // the post-attention norm weight, the same for every row, into LDS (over the
  // reduction buffer, idle until stage 2), ahead of the guard read so both overlap
  v4i* g_lds = reinterpret_cast<v4i*>(&red[0][0]);
  static_assert(H * 2 <= (int)sizeof(red), "norm weight staging");
  for (int i = tid; i < H / 8; i += G::THREADS) g_lds[i] = ld16<CP_NONE>(rg, i * 16);
  {
    const bool has = b < MOE_NEXP;
    const __amdgpu_buffer_rsrc_t rw0 =
        rsrc(p.w_r + (size_t)(has ? b : 0) * H, has ? H * 2 : 0);
    for (int i = tid; i < H / 8; i += G::THREADS) wr_lds[i] = ld16<CP_NT>(rw0, i * 16);
  }
  if (tid == 0) {
    const v4i h = ld16<CP_DEV>(rsrc(p.guard, 16), 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) head_s[i] = (uint32_t)h[i];
  }
  for (int i = tid; i < MOE_NDIST; i += G::THREADS) rl.mask[i] = 0;
  if (tid == 0) ok_s = 1;
  __syncthreads();
  const uint32_t tag = head_s[MONO_GUARD_EPOCH] + 1u;
  Guard guard;
  guard.init(p.guard, p.host_err, p.fault_site, head_s, (uint32_t)p.fault_after);
  bool ok = true;


  // ---------------------------------------------------------------- stage 0
  // Each row is owned by WPR waves (2 for R <= 8, else 1), each holding NQ 512-value
  // slices of it: lane l holds the 8 values at q * 512 + l * 8. One round trip brings the
  // row; the norm weight and this CTA's router row wait in LDS. The E4M3 codes go to
  // xq_lds in the MFMA B-operand image of stage 2 (chunk kc = q * 4 + l / 16; K group
  // (l % 16) / 4; byte (l % 4) * 8).
  {
    // the row values of pass `row0` (issued at the top of the kernel for the first)
    auto rows_pass = [&](auto nq_tag, int row0, v4i* av) {
      constexpr int NQ = decltype(nq_tag)::value;
      constexpr int WPR = H / 512 / NQ;
      const int r = row0 + w / WPR, ch = w % WPR;
      const bool live = r < R;
      float ss = 0.f;
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        float f[8];
        bf16x8(av[q], f);
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += f[i] * f[i];
      }
      ss = wave_sum(ss);
      if (l == 0 && r < 16) red_small[0][ch][r] = ss;
      __syncthreads();
      float tot = 0.f;
      if (r < 16) {
#pragma unroll
        for (int c = 0; c < WPR; ++c) tot += red_small[0][c][r];
      }
      const float rstd = live ? 1.0f / sqrtf(tot / (float)H + p.eps) : 0.f;
      // widen the packed row again below rather than keep the 8 NQ f32 values of the
      // sum of squares alive across the barrier
#pragma unroll
      for (int q = 0; q < NQ; ++q) asm volatile("" : "+v"(av[q]));
      float rp = 0.f;
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int sl = ch * NQ + q;
        float fa[8], fg[8], xn[8];
        bf16x8(av[q], fa);
        bf16x8(g_lds[sl * 64 + l], fg);
        const v4i wv = wr_lds[sl * 64 + l];
        float am = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          xn[i] = fa[i] * rstd * fg[i];
          am = fmaxf(am, fabsf(xn[i]));
        }
        // router: the normalised row rounded to bf16 pairs, dotted with the bf16 weights
#pragma unroll
        for (int d = 0; d < 4; ++d) rp = dot2_bf16(xn[2 * d], xn[2 * d + 1], (uint32_t)wv[d], rp);
        am = row16_max(am);
        const bool nz = am > 0.f;
        const float inv = nz ? FP8_MAX / am : 1.f;
        const int kc = sl * 4 + (l >> 4);
        if (live) {
          v2i qq;
          qq[0] = (int)pack_fp8x4(clamp_fp8(xn[0] * inv), clamp_fp8(xn[1] * inv),
                                  clamp_fp8(xn[2] * inv), clamp_fp8(xn[3] * inv));
          qq[1] = (int)pack_fp8x4(clamp_fp8(xn[4] * inv), clamp_fp8(xn[5] * inv),
                                  clamp_fp8(xn[6] * inv), clamp_fp8(xn[7] * inv));
          const int g4 = (l & 15) >> 2, h = (l & 3) >> 1;
          char* dst = reinterpret_cast<char*>(xq_lds) +
                      ((kc * 2 + h) * 64 + r + 16 * g4) * 16 + (l & 1) * 8;
          *reinterpret_cast<v2i*>(dst) = qq;
          if ((l & 15) == 0) xs_lds[kc][r] = nz ? am * INV_FP8_MAX : 1.f;
        }
        // one slice per scheduling region: the LDS operands are not hoisted ahead
        __builtin_amdgcn_sched_barrier(0);
      }
      rp = wave_sum(rp);
      if (l == 0 && r < 16) red_small[1][ch][r] = rp;
      __syncthreads();
      if (ch == 0 && l == 0 && live && b < MOE_NEXP) {
        float lg = 0.f;
#pragma unroll
        for (int c = 0; c < WPR; ++c) lg += red_small[1][c][r];
        st_dev64(&logit_pairs[r * MOE_NEXP + b], pair(__float_as_uint(lg), tag));
      }
    };
    static_assert(H % 1024 == 0, "hidden must split into two halves of 512-slices");
    // two waves a row, eight rows a pass (the second pass only when R > 8)
    rows_pass(std::integral_constant<int, NQ0>(), 0, av0);
    if (R > 8) {
      __syncthreads();
      const int r = 8 + w / 2, ch = w % 2;
      const bool live = r < R;
      const __amdgpu_buffer_rsrc_t rar =
          rsrc(p.a + (size_t)(live ? r : 0) * H, live ? H * 2 : 0);
      const uint32_t base = (uint32_t)(ch * NQ0 * 512 + l * 8) * 2;
      v4i av1[NQ0];
#pragma unroll
      for (int q = 0; q < NQ0; ++q) av1[q] = ld16<CP_NONE>(rar, base + q * 1024);
      rows_pass(std::integral_constant<int, NQ0>(), 8, av1);
    }
    const int ch = w / 8, wr = w % 8;
    constexpr int NQ = H / 1024;
    // rows past R: zero B operands, unit scales (stage 2 reads all 16 columns)
    for (int i = tid; i < G::NKC * 16; i += G::THREADS) {
      const int kc = i / 16, r = i % 16;
      if (r >= R) {
        xs_lds[kc][r] = 1.f;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) xq_lds[(kc * 2 + h) * 64 + r + 16 * g4] = v4i{0, 0, 0, 0};
      }
    }
    // a grid smaller than the expert count: this CTA's further router experts
    for (int e = b + nblk; e < MOE_NEXP; e += nblk) {
      for (int pass = 0; pass * 8 < R; ++pass) {
        const int r = pass * 8 + wr;
        const bool live = r < R;
        const __amdgpu_buffer_rsrc_t rar =
            rsrc(p.a + (size_t)(live ? r : 0) * H, live ? H * 2 : 0);
        const __amdgpu_buffer_rsrc_t rwr = rsrc(p.w_r + (size_t)e * H, live ? H * 2 : 0);
        const uint32_t base = (uint32_t)(ch * NQ * 512 + l * 8) * 2;
        __syncthreads();
        float ss = 0.f, rp = 0.f;
        for (int q = 0; q < NQ; ++q) {
          float f[8];
          bf16x8(ld16<CP_NONE>(rar, base + q * 1024), f);
          for (int i = 0; i < 8; ++i) ss += f[i] * f[i];
        }
        ss = wave_sum(ss);
        if (l == 0) red_small[0][ch][wr] = ss;
        __syncthreads();
        const float rstd = live ? 1.0f / sqrtf((red_small[0][0][wr] + red_small[0][1][wr]) /
                                               (float)H + p.eps)
                                : 0.f;
        for (int q = 0; q < NQ; ++q) {
          float fa[8], fg[8], fw[8];
          bf16x8(ld16<CP_NONE>(rar, base + q * 1024), fa);
          bf16x8(g_lds[ch * NQ * 64 + q * 64 + l], fg);
          bf16x8(ld16<CP_NT>(rwr, base + q * 1024), fw);
          for (int i = 0; i < 8; ++i) rp += bf16_round(fa[i] * rstd * fg[i]) * fw[i];
        }
        rp = wave_sum(rp);
        if (l == 0) red_small[1][ch][wr] = rp;
        __syncthreads();
        if (ch == 0 && l == 0 && live)
          st_dev64(&logit_pairs[r * MOE_NEXP + e],
                   pair(__float_as_uint(red_small[1][0][wr] + red_small[1][1][wr]), tag));
      }
    }
  }
  __syncthreads();

  // ---------------------------------------------------------------- stage 1
  stamp(p.timeline, MONO_TL_STAGED);
  // one wave a row: poll the row's 256 logits, sigmoid, top-8
  if (w < R) {
    const int row = w;
    uint64_t pr[4];
    ok = wait_until(guard, MONO_SITE_LOGITS, [&]() {
      bool all = true;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pr[i] = ld_dev64(&logit_pairs[row * MOE_NEXP + l + 64 * i]);
        all &= (uint32_t)(pr[i] >> 32) == tag;
      }
      return __all(all);
    });
    if (ok) {
      float sc[4], bs[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lg = __uint_as_float((uint32_t)pr[i]);
        sc[i] = 1.0f / (1.0f + expf(-lg));
        bs[i] = p.bias[l + 64 * i];
      }
      const bool out0 = b == 0;
      route_row(rl, row, sc, bs, p.route_scale, out0 ? p.scores : nullptr,
                out0 ? p.ids : nullptr, out0 ? p.weights : nullptr);
    }
  }
  if (!ok) ok_s = 0;
  __syncthreads();
  if (w == 0) build_distinct(rl, R);
  __syncthreads();
  ok = ok_s != 0;
  const int nd = rl.nd;

  // ---------------------------------------------------------------- stage 2
  stamp(p.timeline, MONO_TL_ROUTED);
  // waves 0-7: the 16 gate rows of the task, waves 8-15 the 16 up rows; wave wq's
  // K slice is chunks [KCW wq, KCW (wq + 1)). Its ring holds one task's KCW chunks:
  // a slot is refilled with the next task's chunk as soon as its MFMA issued.
  {
    const int ntask = ok ? nd * NUG : 0;
    v4i ring[KCW][2];
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
    // Task hand-out: CTA b starts on task b; later tasks come from a device-wide
    // counter in order (nblk, nblk + 1, ...), grabbed one task ahead so the ring can be
    // refilled with the next task while this one runs. Tasks run the same arithmetic on
    // whichever CTA takes them, so results do not depend on the hand-out.
    int task = b;
    {
      uint32_t so;
      const __amdgpu_buffer_rsrc_t r = task_src(task, so);
#pragma unroll
      for (int j = 0; j < KCW; ++j) {
        ring[j][0] = ld16s<CP_NT>(r, vo, so + j * CS);
        ring[j][1] = ld16s<CP_NT>(r, vo + HO, so + j * CS);
      }
    }
    if (tid == 0) next_s = task < ntask ? nblk + (int)add_dev(&queue[0], 1u) : ntask;
    __syncthreads();
    int next = next_s;
    while (task < ntask) {
      const int u = task / NUG, cc = task % NUG;
      const int e = __builtin_amdgcn_readfirstlane(rl.uexp[u]);
      const uint32_t mask = rl.umask[u];
      const float tok_on = ((mask >> t) & 1u) ? 1.f : 0.f;
      const int sbase = __builtin_amdgcn_readfirstlane(
          (e * (2 * I / 128) + (half * I + cc * 16) / 128) * (H / 128) + wq * KCW);
      // the task after next (its value lands in LDS before the epilogue barrier)
      int nn = ntask;
      if (tid == 0 && next < ntask) nn = nblk + (int)add_dev(&queue[0], 1u);
      uint32_t son;
      const __amdgpu_buffer_rsrc_t rn = task_src(next, son);
      // B operands and scales: the same LDS words every task, read through an opaque
      // base so they are not hoisted out of the loop (they would hold 56 VGPRs)
      const int xb = opaque_v(wq * KCW * 2 * 64 + l);
      const int sb = opaque_v(wq * KCW * 16 + t);
      v4f acc = {0.f, 0.f, 0.f, 0.f};
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
      red[w][l] = acc;
      if (tid == 0) next_s = nn;
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
  // mid quant: task (u, kb), one wave a row. Trip counts stay CTA-uniform (barriers
  // per task); a failed wait only skips work.
  {
    const int nq = ok ? nd * NKB : 0;
    for (int q = b; q < nq; q += nblk) {
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
        if (ok) {
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
      if (tid == 0 && all_ok) st_dev(&ready[u * NKB + kb], tag);
    }
    ok = cta_ok(ok, guard, ok_s);
  }

  // ---------------------------------------------------------------- stage 4
  stamp(p.timeline, MONO_TL_MIDQ);
  // down: task f = output rows [32 f, 32 f + 32); waves 0-7 the first 16 rows, 8-15 the
  // next 16; wave wq takes experts u = wq, wq + 8, ... One wait for every quantised mid
  // block (the first weight tile already in flight), then the 9 R (expert, row) mid rows
  // are copied into LDS over the dead activation operands, so the expert loop streams
  // weights with no poll and no other global load.
  {
    const int ntask = ok ? G::NDN : 0;
    uint8_t* mql = reinterpret_cast<uint8_t*>(xq_lds);  // [9 R slots][I] E4M3
    float* mcl = reinterpret_cast<float*>(mql + MOE_MAXR * MOE_SLOTS * I);  // [slots][NKB]
    static_assert(MOE_MAXR * MOE_SLOTS * (I + NKB * 4) <= (int)sizeof(xq_lds), "mid slots");
    // one tile of weight chunks a wave; each chunk is refilled with the next step's as
    // soon as its MFMA issued, the last expert of a task running into the next task
    v4i buf[NKB][2];
    const uint32_t vo = SHUF ? (uint32_t)(grp * 512 + t * 16) : (uint32_t)t * I + 32 * grp;
    constexpr uint32_t HO = SHUF ? 256 : 16, CS = SHUF ? 2048 : 128;
    auto src_of = [&](int f, int u, uint32_t& so) {
      const bool live = f < ntask && u < nd;
      const int e = __builtin_amdgcn_readfirstlane(rl.uexp[live ? u : 0]);
      const int row0 = (live ? f : 0) * G::DNT + 16 * half;
      so = SHUF ? (uint32_t)((row0 / 16) * (I / 32) * 512) : (uint32_t)row0 * I;
      return rsrc(p.w2 + (size_t)e * H * I, live ? (uint32_t)H * I : 0u);
    };
    {
      uint32_t so;
      const __amdgpu_buffer_rsrc_t r = src_of(b, wq, so);
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        buf[kb][0] = ld16s<CP_NT>(r, vo, so + kb * CS);
        buf[kb][1] = ld16s<CP_NT>(r, vo, so + kb * CS + HO);
      }
    }
    // every quantised mid block of this launch
    if (ntask) {
      const int i = w * 64 + l;
      ok = wait_until(guard, MONO_SITE_MQ, [&]() {
        const uint32_t rv = i < nd * NKB ? ld_dev(&ready[i]) : tag;
        return __all(rv == tag);
      });
    }
    ok = cta_all(ok, ok_s);
    if (ok && ntask) {
      // mid rows + coefficients into LDS: 32 lanes of 16 B a slot row
      const __amdgpu_buffer_rsrc_t rmq = rsrc(mq, (uint32_t)G::SZ_MQ);
      const int nsl = R * MOE_SLOTS;
      constexpr int CPR = I / 16;  // 16-byte pieces of a mid row
      for (int i = tid; i < nsl * CPR; i += G::THREADS) {
        const int s = i / CPR, c = i % CPR;
        const int ut = rl.slot_ut[s];
        const uint32_t src_off = (uint32_t)(((ut >> 8) * MOE_MAXR + (ut & 255)) * I + c * 16);
        *reinterpret_cast<v4i*>(mql + s * I + c * 16) = ld16<CP_DEV>(rmq, src_off);
      }
      for (int i = tid; i < nsl * NKB; i += G::THREADS) {
        const int s = i / NKB, kb = i % NKB;
        const int ut = rl.slot_ut[s];
        mcl[i] = __uint_as_float(ld_dev(reinterpret_cast<const uint32_t*>(
            &mcoef[((size_t)(ut >> 8) * MOE_MAXR + (ut & 255)) * NKB + kb])));
      }
    }
    __syncthreads();
    for (int f = b; f < (ok ? ntask : 0); f += nblk) {
      const int rg0 = f * G::DNT + 16 * half;
      v4f acc = {0.f, 0.f, 0.f, 0.f};
      for (int u = wq; u < nd; u += QW) {
        int fn = f, un = u + QW;
        if (un >= nd) {
          fn = f + nblk;
          un = wq;
        }
        uint32_t son;
        const __amdgpu_buffer_rsrc_t rn = src_of(fn, un, son);
        const int e = __builtin_amdgcn_readfirstlane(rl.uexp[u]);
        const int sl = slot_of(rl, u, rl.umask[u], t);
        const bool on = sl >= 0;
        const int bb = (on ? sl : 0) * I + 32 * grp;
        const int s2b =
            __builtin_amdgcn_readfirstlane((e * (H / 128) + rg0 / 128) * (I / 128));
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          const v4i z = {0, 0, 0, 0};
          const v4i b0 = on ? *reinterpret_cast<const v4i*>(mql + bb + kb * 128) : z;
          const v4i b1 = on ? *reinterpret_cast<const v4i*>(mql + bb + kb * 128 + 16) : z;
          const float cf = on ? mcl[(on ? sl : 0) * NKB + kb] : 0.f;
          const v4f zero = {0.f, 0.f, 0.f, 0.f};
          const v4f d = mfma_fp8(cat8(buf[kb][0], buf[kb][1]), cat8(b0, b1), zero);
          buf[kb][0] = ld16s<CP_NT>(rn, vo, son + kb * CS);
          buf[kb][1] = ld16s<CP_NT>(rn, vo, son + kb * CS + HO);
          acc += d * (sld(p.s2, s2b + kb) * cf);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      // fixed-order reduction over each half's 8 waves, then the residual add
      red[w][l] = acc;
      __syncthreads();
      if (tid < 512) {
        const int row = tid & 31, tok = tid >> 5;  // 32 rows x 16 columns, rows fastest
        const int h = row >> 4, rr = row & 15;
        const int L = tok + 16 * (rr >> 2), v = rr & 3;
        float ys = 0.f;
#pragma unroll
        for (int i = 0; i < QW; ++i) ys += red[h * QW + i][L][v];
        if (tok < R) {
          const int col = f * G::DNT + row;
          const float av = bf16_lo(p.a[tok * H + col]);
          p.out[tok * H + col] = (uint16_t)bf16_bits(av + ys);
          if (p.y) p.y[tok * H + col] = ys;
        }
      }
      __syncthreads();
    }
  }

  // ---------------------------------------------------------------- exit
  stamp(p.timeline, MONO_TL_DOWN);
  __syncthreads();
  if (tid == 0) {
    uint32_t* gw = reinterpret_cast<uint32_t*>(p.guard);
    drain();
    const uint32_t old = add_dev(gw + MONO_GUARD_EXIT, 1u);
    if (old == (uint32_t)nblk - 1u) {
      // every other CTA is past its last queue grab: the counters restart at zero
#pragma unroll
      for (int i = 0; i < G::NQUEUE; ++i) st_dev(queue + i, 0u);
      st_dev(gw + MONO_GUARD_EXIT, 0u);
      st_dev(gw + MONO_GUARD_EPOCH, tag);
    }
  }
  stamp(p.timeline, MONO_TL_END);
}

}  // namespace mono

using namespace mono;

extern "C" size_t mono_moe_fp8_scratch_bytes(int32_t hidden, int32_t inter, int32_t experts) {
  if (experts != MOE_NEXP) return 0;
  if (hidden == 7168 && inter == 512) return MoeFp8Geom<7168, 512>::BYTES;
  return 0;
}

extern "C" int mono_moe_fp8_launch(const MonoMoeFp8Args* a, mono_stream_t stream) {
  if (!a) return set_error(MONO_E_ARG, "mono_moe_fp8_launch: null args");
  if (a->rows < 1 || a->rows > MOE_MAXR)
    return set_error(MONO_E_ARG, "mono_moe_fp8_launch: rows must be 1..16");
  if (a->experts != MOE_NEXP)
    return set_error(MONO_E_ARG, "mono_moe_fp8_launch: experts must be 256");
  if (!a->a || !a->out || !a->g_post || !a->w_r || !a->bias || !a->w13 || !a->s13 || !a->w2 ||
      !a->s2 || !a->scratch || !a->guard)
    return set_error(MONO_E_ARG, "mono_moe_fp8_launch: null tensor");
  MoeFp8Params p;
  p.rows = a->rows;
  p.eps = a->eps;
  p.route_scale = a->route_scale;
  p.a = static_cast<const uint16_t*>(a->a);
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
  p.scratch = static_cast<uint8_t*>(a->scratch);
  p.guard = a->guard;
  p.host_err = nullptr;
  if (a->host_error) {
    void* dptr = nullptr;
    if (hipHostGetDevicePointer(&dptr, a->host_error, 0) != hipSuccess || !dptr)
      return set_error(MONO_E_ARG, "mono_moe_fp8_launch: host_error is not pinned host memory");
    p.host_err = static_cast<uint32_t*>(dptr);
  }
  p.fault_site = a->fault_site;
  p.fault_after = a->fault_after;
  p.timeline = a->timeline;
  int grid = 0;
  int rc = monokernel_grid(&grid);
  if (rc) return rc;
  if (a->layout != MONO_LAYOUT_ROWMAJOR && a->layout != MONO_LAYOUT_AITER16)
    return set_error(MONO_E_ARG, "mono_moe_fp8_launch: unknown weight layout");
  if (a->hidden == 7168 && a->inter == 512) {
    auto k = a->layout == MONO_LAYOUT_AITER16 ? moe_fp8_kernel<7168, 512, true>
                                              : moe_fp8_kernel<7168, 512, false>;
    rc = check_coresident(k, 1024, 0,
                          "mono_moe_fp8_launch: one 1024-thread CTA per CU does not fit");
    if (rc) return rc;
    hipLaunchKernelGGL(k, dim3(grid), dim3(1024), 0, (hipStream_t)stream, p);
  } else {
    return set_error(MONO_E_ARG, "mono_moe_fp8_launch: unsupported hidden/inter");
  }
  return check_launch("mono_moe_fp8_launch");
}
