// W8A16 GEMV tasks for the dense projections of the layer: y[r, n] = sum_k x[r, k]
// W[n, k] s[n / 128, k / 128] for up to 16 rows r (the MFMA columns), with W in E4M3
// read in place (row-major, or AITER's (16, 16) shuffle) and widened exactly to bf16,
// x in bf16, f32 accumulation (sgl_amd_mono/glm53/gfx950/kernel.py:823-875 unit_fp8x2,
// :1061-1213 units and row reduction).
//
// A task is RG 16-row groups of one group g (per-head GEMVs are G independent groups);
// its 16 waves are RG row groups x KS K-splits, each wave STEPS steps of 64 K. A lane's
// 16 weight bytes are row l % 16, K k0 + 16 (l / 16) .. + 15 (in the shuffle, a 16-row x
// 64-K tile is 1 KiB contiguous with lane l at 16 l); they feed two 16x16x32 bf16 MFMAs
// whose B operands are x[l % 16][k0 + 16 (l / 16) + 8 m ..] (m = 0, 1). Each step's
// partial is scaled by its block's f32 scale. The KS partials of a row group are summed
// in a fixed order through LDS.
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
};

// Run every task of `j` this CTA owns (tasks b, b + nblk, ...). XCP: cache policy of the x
// loads (CP_DEV when another CTA of this launch wrote x). `before_x` runs once, after the
// first task's weight loads are issued and before its x loads: the place to wait for x.
// Returns false if before_x reported a failure (the CTA then skips its tasks).
template <int KS, int STEPS, int XCP, class BeforeX>
__device__ inline bool gemv_tasks(const GemvJob& j, int R, int b, int nblk, int tid, v4f (*red)[64],
                                  BeforeX before_x) {
  constexpr int RG = 16 / KS;
  static_assert(KS * RG == 16, "16 waves: KS K-splits x RG row groups");
  const int l = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = w / KS, ks = w % KS;
  const int t = l & 15, grp = l >> 4;
  const int tiles = j.N / (16 * RG);
  const int ntask = j.G * tiles;
  const uint32_t wbytes = (uint32_t)j.N * (uint32_t)j.K;
  const uint32_t vo = j.shuf ? (uint32_t)l * 16 : (uint32_t)(t * j.K + 16 * grp);
  bool ok = true, first = true;
  for (int task = b; task < ntask; task += nblk) {
    const int g = task / tiles, tile = task % tiles;
    const int rgg = tile * RG + rg;  // this wave's 16-row group within the group's N rows
    const __amdgpu_buffer_rsrc_t rw = rsrc(j.w + (size_t)g * wbytes, wbytes);
    v4i wv[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int k0 = (ks * STEPS + s) * 64;
      const uint32_t so = j.shuf ? (uint32_t)(rgg * (j.K / 32) + k0 / 32) * 512u
                                 : (uint32_t)(rgg * 16 * j.K + k0);
      wv[s] = ld16s<CP_NT>(rw, vo, so);
    }
    if (first) {
      first = false;
      ok = before_x();
      if (!ok) break;
    }
    const uint16_t* xg = j.x + (size_t)g * j.x_gstride;
    const __amdgpu_buffer_rsrc_t rx =
        rsrc(xg, (uint32_t)((R - 1) * j.x_stride + j.K) * 2u);  // rows >= R read zeros
    v4i xa[STEPS][2];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int k0 = (ks * STEPS + s) * 64;
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const uint32_t off = t < R ? (uint32_t)(t * j.x_stride + k0 + 16 * grp + 8 * m) * 2u
                                   : 0x80000000u;
        xa[s][m] = ld16<XCP>(rx, off);
      }
    }
    const int sbase = (g * (j.N / 128) + rgg / 8) * (j.K / 128);
    v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int k0 = (ks * STEPS + s) * 64;
      v4f d = {0.f, 0.f, 0.f, 0.f};
      d = mfma_bf16(fp8x8_bf16((uint32_t)wv[s][0], (uint32_t)wv[s][1]),
                    __builtin_bit_cast(v8bf, xa[s][0]), d);
      d = mfma_bf16(fp8x8_bf16((uint32_t)wv[s][2], (uint32_t)wv[s][3]),
                    __builtin_bit_cast(v8bf, xa[s][1]), d);
      acc += d * sld(j.s, sbase + k0 / 128);
    }
    red[w][l] = acc;
    __syncthreads();
    // 256 threads a row group: row = e % 16 (adjacent threads, adjacent rows), token e / 16
    if (tid < RG * 256) {
      const int rge = tid >> 8, e = tid & 255;
      const int row = e & 15, tok = e >> 4;
      const int L = tok + 16 * (row >> 2), v = row & 3;
      float y = 0.f;
#pragma unroll
      for (int i = 0; i < KS; ++i) y += red[rge * KS + i][L][v];
      const int n = (tile * RG + rge) * 16 + row;
      if (j.out_f) {
        if (tok < R) st_devf(j.out_f + (size_t)g * j.out_gstride + tok * j.out_stride + n, y);
      } else {
        if (j.res && tok < R) y += bf16_lo(j.res[tok * j.res_stride + g * j.N + n]);
        const uint32_t h = bf16_bits(y);
        const uint32_t hn = dpp_u<DPP_XOR1>(h);  // the next row's bits (same token)
        if (tok < R && (row & 1) == 0)
          st_dev(reinterpret_cast<uint32_t*>(j.out_bf + (size_t)g * j.out_gstride +
                                             tok * j.out_stride + n),
                 h | (hn << 16));
      }
    }
    __syncthreads();
  }
  return ok;
}

}  // namespace mono
