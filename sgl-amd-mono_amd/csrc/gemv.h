// W8A16 GEMV tiles for the dense projections of the layer: y[r, n] = sum_k x[r, k]
// W[n, k] s[n / 128, k / 128] for up to 16 rows r (the MFMA columns), with W in E4M3
// read in place (row-major, or AITER's (16, 16) shuffle) and widened exactly to bf16,
// x in bf16, f32 accumulation (sgl_amd_mono/glm53/gfx950/kernel.py:823-875 unit_fp8x2,
// :1061-1213 units and row reduction).
//
// A tile is RG 16-row groups of one group g (per-head GEMVs are G independent groups);
// KS x RG waves of the CTA take it, RG row groups x KS K-splits, each wave STEPS steps of
// 64 K. A lane's 16 weight bytes are row l % 16, K k0 + 16 (l / 16) .. + 15 (in the
// shuffle, a 16-row x 64-K tile is 1 KiB contiguous with lane l at 16 l); they feed two
// 16x16x32 bf16 MFMAs whose B operands are x[l % 16][k0 + 16 (l / 16) + 8 m ..] (m = 0,
// 1). Each step's partial is scaled by its block's f32 scale. The KS partials of a row
// group are summed in a fixed order through LDS.
//
// The phases are separate so a launch can put a tile's weights in flight long before its
// x exists (issue), load x once for several tiles of one group (load_x: x depends on the
// wave's K range only), and reduce several tiles behind one barrier (dot, epilogue).
#pragma once

#include "mono_device.h"

namespace mono {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// 8 E4M3 (two dwords) -> 8 bf16 (exact)
__device__ inline v8bf fp8x8_bf16(uint32_t lo, uint32_t hi) {
  const v2bf a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
  const v2bf b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
  const v2bf c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
  const v2bf d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
  return v8bf{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

__device__ inline v4f mfma_bf16(v8bf a, v8bf b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

struct GemvJob {
  const uint16_t* x;  // bf16: x[r][k] of group g at x + g * x_gstride + r * x_stride + k
  int x_stride, x_gstride;
  const uint8_t* w;   // E4M3 [G][N][K]
  const float* s;     // f32 [G][N / 128][K / 128]
  int N, K, G;
  int shuf;           // AITER (16, 16) layout
  // epilogue: out[g][r][n] at out + g * out_gstride + r * out_stride + n, bf16 (with the
  // residual res[r][g * N + n] added, if given) or f32
  uint16_t* out_bf;
  float* out_f;
  int out_stride, out_gstride;
  const uint16_t* res;
  int res_stride;
  // bf16 pairs are stored XOR out_xor (a hand-off whose zero words mean "not written
  // yet" stores the complement); out_plain, if given, gets the plain pairs as well
  uint32_t out_xor;
  uint16_t* out_plain;
  // with bf16 outputs: each output row's sum of the squares of a 16-column tile's bf16
  // values, ssq[column tile][16] (f32, device coherent), if given
  float* ssq;
};

template <int KS, int RG, int STEPS>
struct Gemv {
  static_assert(KS * RG <= 16, "16 waves a CTA");
  static constexpr int ROWS = 16 * RG;  // rows of a tile
  int l, w, rg, ks, t, grp;
  bool on;  // this wave takes part (w < KS * RG)

  __device__ explicit Gemv(int tid) {
    l = tid & 63;
    w = __builtin_amdgcn_readfirstlane(tid >> 6);
    rg = w / KS;
    ks = w % KS;
    t = l & 15;
    grp = l >> 4;
    on = KS * RG == 16 || w < KS * RG;
  }
  __device__ int k0(int s) const { return (ks * STEPS + s) * 64; }

  // put the wave's weight bytes of tile `tile` of group g in flight (a tile that is not
  // `valid` reads zeros without memory traffic: no branch, so the loads that follow keep
  // static wait counts)
  // Both layouts put row group rgg at byte 16 rgg K; within it the shuffle's 64-K step
  // is 1 KiB (lane l at 16 l) and the row-major one 64 B (lane at t K + 16 grp): one
  // formula, so the unrolled loads carry no branch. Waves beyond KS x RG read zeros.
  // The steps' block scales are read here too, as vector loads issued with the weights
  // (they return in order with them): a scalar load at the dot would cost a round trip
  // of its own after the data arrived, and a constant load may sink to its use.
  __device__ void issue(const GemvJob& j, int g, int tile, v4i (&wv)[STEPS],
                        float (&sc)[STEPS], bool valid = true) const {
    const uint32_t wbytes = (uint32_t)j.N * (uint32_t)j.K;
    const __amdgpu_buffer_rsrc_t rw =
        rsrc(j.w + (size_t)g * wbytes, valid && on ? wbytes : 0u);
    const int rgg = tile * RG + rg;
    const uint32_t vo = j.shuf ? (uint32_t)l * 16 : (uint32_t)(t * j.K + 16 * grp);
    const int sh = j.shuf ? 4 : 0;
#pragma unroll
    for (int s = 0; s < STEPS; ++s)
      wv[s] = ld16s<CP_NT>(rw, vo, (uint32_t)(rgg * 16 * j.K) + ((uint32_t)k0(s) << sh));
    // (an absent tile reads zeros; with STEPS even, steps 2i and 2i + 1 share a block)
    const int sbase = (g * (j.N / 128) + rgg / 8) * (j.K / 128);
    const __amdgpu_buffer_rsrc_t rs =
        rsrc(j.s, valid && on ? (uint32_t)(j.G * (j.N / 128) * (j.K / 128)) * 4u : 0u);
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      if (STEPS % 2 == 0 && (s & 1))
        sc[s] = sc[s - 1];
      else
        sc[s] = __int_as_float(ld4<CP_NONE>(rs, (uint32_t)(sbase + k0(s) / 128) * 4u));
    }
  }

  // the wave's x operands of group g (rows >= R read zeros); XCP: cache policy (CP_DEV
  // when another CTA of this launch wrote x)
  template <int XCP>
  __device__ void load_x(const GemvJob& j, int g, int R, v4i (&xa)[STEPS][2],
                         bool valid = true) const {
    const uint16_t* xg = j.x + (size_t)g * j.x_gstride;
    const __amdgpu_buffer_rsrc_t rx =
        rsrc(xg, valid && on ? (uint32_t)((R - 1) * j.x_stride + j.K) * 2u : 0u);
#pragma unroll
    for (int s = 0; s < STEPS; ++s)
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const uint32_t off = t < R ? (uint32_t)(t * j.x_stride + k0(s) + 16 * grp + 8 * m) * 2u
                                   : 0x80000000u;
        xa[s][m] = ld16<XCP>(rx, off);
      }
  }

  // the wave's scaled partial of tile `tile`, into red[w] (a barrier must follow)
  __device__ void dot(const v4i (&wv)[STEPS], const float (&sc)[STEPS],
                      const v4i (&xa)[STEPS][2], v4f (*red)[64]) const {
    if (!on) return;
    v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      v4f d = {0.f, 0.f, 0.f, 0.f};
      d = mfma_bf16(fp8x8_bf16((uint32_t)wv[s][0], (uint32_t)wv[s][1]),
                    __builtin_bit_cast(v8bf, xa[s][0]), d);
      d = mfma_bf16(fp8x8_bf16((uint32_t)wv[s][2], (uint32_t)wv[s][3]),
                    __builtin_bit_cast(v8bf, xa[s][1]), d);
      acc += d * sc[s];
    }
    red[w][l] = acc;
  }

  // sum the KS partials of tile `tile` and store it: threads e in [0, RG * 256) of the
  // CTA (whole waves), row = e % 16 (adjacent threads, adjacent rows), token e / 16 % 16
  // (`hres`: the residual's bits for this thread's output, if the caller loaded it ahead;
  // else j.res is read here)
  __device__ static void epilogue(const GemvJob& j, int g, int tile, int R, int e,
                                  v4f (*red)[64], int hres = -1) {
    const int rge = e >> 8, row = e & 15, tok = (e >> 4) & 15;
    const int L = tok + 16 * (row >> 2), v = row & 3;
    float y = 0.f;
#pragma unroll
    for (int i = 0; i < KS; ++i) y += red[rge * KS + i][L][v];
    const int n = (tile * RG + rge) * 16 + row;
    if (j.out_f) {
      if (tok < R) st_devf(j.out_f + (size_t)g * j.out_gstride + tok * j.out_stride + n, y);
    } else {
      if (j.res && tok < R)
        y += bf16_lo(hres >= 0 ? (uint32_t)hres : j.res[tok * j.res_stride + g * j.N + n]);
      const uint32_t h = bf16_bits(y);
      const uint32_t hn = dpp_u<DPP_XOR1>(h);  // the next row's bits (same token)
      uint32_t pair = h | (hn << 16);
      if (pair == 0xFFFFFFFFu) pair = 0xFFC0FFC0u;  // two NaNs; keeps ~pair nonzero
      // through buffer resources (scalar bases; device coherent like st_dev): a 64-bit
      // per-lane address would be built ahead of the phase and held in registers
      const uint32_t at = (uint32_t)(g * j.out_gstride + tok * j.out_stride + n) * 2u;
      if (tok < R && (row & 1) == 0) {
        __builtin_amdgcn_raw_buffer_store_b32(pair ^ j.out_xor, rsrc(j.out_bf, 0xFFFFFFFFu), at, 0,
                                              CP_DEV);
        if (j.out_plain)
          __builtin_amdgcn_raw_buffer_store_b32(pair, rsrc(j.out_plain, 0xFFFFFFFFu), at, 0, CP_DEV);
      }
      if (j.ssq) {
        // the squares of the stored bf16 values over the row of 16 lanes (the tile's 16
        // columns of one output row), in the pairwise tree of `pair_sq_tree`
        const float sq = pair_sq_tree(h, tok < R);
        if (tok < R && row == 0)
          __builtin_amdgcn_raw_buffer_store_b32(
              __float_as_uint(sq), rsrc(j.ssq, (uint32_t)j.N * 4u),
              (uint32_t)(((tile * RG + rge) * 16 + tok) * 4), 0, CP_DEV);
      }
    }
  }
};

// Run every tile of `j` this CTA owns (tasks b, b + nblk, ... over G x N / (16 RG)),
// one at a time. `before_x` runs once, after the first task's weight loads are issued
// and before its x loads: the place to wait for x. Returns false if before_x reported a
// failure (the CTA then skips its tasks).
template <int KS, int RG, int STEPS, int XCP, class BeforeX>
__device__ inline bool gemv_tasks(const GemvJob& j, int R, int b, int nblk, int tid,
                                  v4f (*red)[64], BeforeX before_x) {
  const Gemv<KS, RG, STEPS> gv(tid);
  const int tiles = j.N / Gemv<KS, RG, STEPS>::ROWS;
  const int ntask = j.G * tiles;
  bool ok = true, first = true;
  for (int task = b; task < ntask; task += nblk) {
    const int g = task / tiles, tile = task % tiles;
    v4i wv[STEPS];
    float sc[STEPS];
    gv.issue(j, g, tile, wv, sc);
    if (first) {
      first = false;
      ok = before_x();
      if (!ok) break;
    }
    v4i xa[STEPS][2];
    gv.template load_x<XCP>(j, g, R, xa);
    gv.dot(wv, sc, xa, red);
    __syncthreads();
    if (tid < RG * 256) Gemv<KS, RG, STEPS>::epilogue(j, g, tile, R, tid, red);
    __syncthreads();
  }
  return ok;
}

// W_UV of one (token, head), the same arithmetic wherever it runs (the output block's own
// launch, or the attention's merge in the one-launch layer, so both give the same bits):
// o[v] = bf16(sum_c W[v][c] x[c] s[c / 128]) for the head's 128 rows v, W in E4M3
// [128][512] (row-major or AITER's (16, 16) shuffle), s the head's four f32 block scales,
// x the 512 latents in bf16 in LDS. Wave w takes rows 16 (w % 8) .. + 15 and K [256
// (w / 8), + 256) as 4 steps of 64 K with Gemv's lane map (lane l: row l % 16, K + 16
// (l / 16) .. + 15), two 16x16x32 bf16 MFMAs a step whose B operand is x in column 0
// (the other columns zero), each step scaled by its block's scale; the two K halves of a
// row are then summed in a fixed order.
struct UvUnit {
  static constexpr int THREADS = 1024;
  v4i w[4];
  float s[4];

  // this wave's weight bytes and block scales of head h (on = false: zeros, no traffic)
  __device__ void load(const uint8_t* w_uv, const float* s_uv, int shuf, int h, int tid,
                       bool on) {
    const int l = tid & 63, wv = tid >> 6, rt = wv & 7, kh = wv >> 3;
    const __amdgpu_buffer_rsrc_t r = rsrc(w_uv + (size_t)h * 128 * 512, on ? 128u * 512u : 0u);
    const uint32_t vo = shuf ? (uint32_t)l * 16 : (uint32_t)((l & 15) * 512 + 16 * (l >> 4));
    const int sh = shuf ? 4 : 0;
#pragma unroll
    for (int st = 0; st < 4; ++st)
      w[st] = ld16s<CP_NONE>(r, vo, (uint32_t)(rt * 16 * 512) + ((uint32_t)(256 * kh + 64 * st) << sh));
    const __amdgpu_buffer_rsrc_t rs = rsrc(s_uv + h * 4, on ? 16u : 0u);
    s[0] = s[1] = __int_as_float(ld4<CP_NONE>(rs, (uint32_t)(2 * kh) * 4u));
    s[2] = s[3] = __int_as_float(ld4<CP_NONE>(rs, (uint32_t)(2 * kh + 1) * 4u));
  }
  // the wave's scaled partial into red[w] (16 x 64 v4f of LDS; a barrier must follow)
  __device__ void dot(const uint16_t* x, v4f (*red)[64], int tid) const {
    const int l = tid & 63, wv = tid >> 6, kh = wv >> 3;
    const bool col0 = (l & 15) == 0;
    v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int k0 = 256 * kh + 64 * st + 16 * (l >> 4);
      const v4i z = {0, 0, 0, 0};
      const v4i x0 = col0 ? *reinterpret_cast<const v4i*>(x + k0) : z;
      const v4i x1 = col0 ? *reinterpret_cast<const v4i*>(x + k0 + 8) : z;
      v4f d = {0.f, 0.f, 0.f, 0.f};
      d = mfma_bf16(fp8x8_bf16((uint32_t)w[st][0], (uint32_t)w[st][1]), __builtin_bit_cast(v8bf, x0), d);
      d = mfma_bf16(fp8x8_bf16((uint32_t)w[st][2], (uint32_t)w[st][3]), __builtin_bit_cast(v8bf, x1), d);
      acc += d * s[st];
    }
    red[wv][l] = acc;
  }
  // row v (< 128) after the barrier: its K halves in order
  __device__ static float row(const v4f (*red)[64], int v) {
    const int rt = v >> 4, L = 16 * ((v & 15) >> 2), j = v & 3;
    return red[rt][L][j] + red[rt + 8][L][j];
  }
  // rows -> bf16 pairs: thread t < 64 stores pair t (rows 2t, 2t + 1, from ob: u16 [128]
  // in LDS) XOR `xr` at dst[t] (device coherent), and plainly at plain[t] if given. A pair
  // of all-ones bits becomes two NaNs whose complement stays nonzero (a hand-off reads zero
  // as "not written yet").
  __device__ static void store(const uint16_t* ob, int tid, uint32_t* dst, uint32_t xr,
                               uint32_t* plain) {
    if (tid < 64) {
      uint32_t pair = reinterpret_cast<const uint32_t*>(ob)[tid];
      if (pair == 0xFFFFFFFFu) pair = 0xFFC0FFC0u;
      st_dev(dst + tid, pair ^ xr);
      if (plain) st_dev(plain + tid, pair);
    }
  }
};

}  // namespace mono
