// The attention output block as one persistent gfx950 launch: the merged latent o_lat
// through W_UV per head, then o_proj and the residual add of the W == 1 reduce.
//   W_UV  o[r][h * 128 + v] = sum_c W_UV[h][v][c] o_lat[r][h][c], handed over in bf16 (the
//         reference rounds o to bf16 before o_proj, kernel.py:4080-4123): a task a (token,
//         head) on the vector units (UvUnit), issued before anything else so it leads
//         every CU's queue. In the one-launch layer the attention's merge runs these tasks
//         instead, on the latents it has just merged (same arithmetic, same bits), and
//         this phase starts with o_proj, waiting for nothing but o itself.
//   o_proj a[r][n] = bf16(h[r][n] + sum_k W_o[n][k] o[r][k]): 448 tiles of 16 rows, two
//         at a time a CTA: the first tile's weights and h in flight from the launch's
//         start, the second's from the moment W_UV's outputs are stored.
// The hand-off of o needs no flag, drain or poll: W_UV stores the complement of each bf16
// pair into one of two scratch buffers (by the launch tag's parity), and clears the other
// for the next launch; a zero word is "not written yet". o_proj's x loads are its wait:
// issued right behind the weights, they return right behind them (a wave's loads return
// in order) and are loaded again only if a word is still zero. Every prefetch is
// unconditional (absent tiles read zeros through a zero-size buffer resource), so the
// compiler keeps exact wait counts instead of waiting for everything after a branch.
// Reference: sgl_amd_mono/glm53/gfx950/kernel.py:3975-4123 (W_UV), :4125-4197 (o_proj,
// residual), :1665-1669 (W == 1 reduce).
#pragma once

#include <hip/hip_runtime.h>

#include "gemv.h"
#include "mono_abi.h"
#include "phase.h"

namespace mono {

constexpr int PO_HEADS = 32, PO_V = 128, PO_LAT = 512, PO_HID = 7168;
constexpr int PO_O = PO_HEADS * PO_V;
constexpr int PO_MAXR = 16;
constexpr int PO_MAX_GRID = 1024;
constexpr int PO_TILES = PO_HID / 16;   // o_proj tiles of 16 rows

using GemvO = Gemv<16, 1, 4>;   // 16 rows: 16 K-splits of 256

struct PostScratch {
  // two hand-off buffers of o, u32 [16][4096 / 2] complemented bf16 pairs
  static constexpr size_t OBUF = (size_t)PO_MAXR * PO_O * 2;
  static constexpr size_t BYTES = 2 * OBUF;
};

struct PostParams {
  int rows, shuf;
  const uint16_t* o_lat;
  const uint16_t* h;
  const uint8_t* w_uv;
  const float* s_uv;
  const uint8_t* w_o;
  const float* s_o;
  uint16_t* out;
  uint16_t* o;  // bf16 [R][4096]: the caller's, or scratch
  // the one-launch layer: each row's sum of squares of out's bf16 values per 16-column
  // tile, f32 [448][16], for the MoE phase's RMSNorm (null: not written)
  float* ssq;
  uint8_t* scratch;
  int32_t* guard;
  uint32_t* host_err;
  int fault_site, fault_after;
  uint64_t* timeline;
};

// red[32][64] of o_proj's two tiles, then W_UV's partials [16][64], x and rows
constexpr int PO_LDS_BYTES = 48 * 64 * 16 + 512 * 2 + 128 * 2;

// The output block in one CTA of a launch. FUSED: it runs after the attention phase in
// the same launch, whose merge stored o; `ready` is called once the weight prefetch and
// the residual rows are in flight (the layer passes NoWait: o's complemented words are
// their own hand-off).
template <bool FUSED, class Ready>
__device__ __attribute__((always_inline)) inline void post_phase(const PostParams& p, uint8_t* lds,
                                                                 Guard& guard, uint32_t tag,
                                                                 int& ok_s, Ready ready) {
  const int b = blockIdx.x, nblk = gridDim.x, R = p.rows;
  v4f (*red)[64] = reinterpret_cast<v4f (*)[64]>(lds);
  uint16_t* obuf = reinterpret_cast<uint16_t*>(p.scratch + (tag & 1u) * PostScratch::OBUF);
  uint8_t* onext = p.scratch + ((tag + 1u) & 1u) * PostScratch::OBUF;

  const int tid = opaque_v((int)threadIdx.x);
  const int l = tid & 63, w = tid >> 6;
  GemvJob jo{};
  jo.x = obuf;
  jo.x_stride = PO_O;
  jo.w = p.w_o;
  jo.s = p.s_o;
  jo.N = PO_HID;
  jo.K = PO_O;
  jo.G = 1;
  jo.shuf = p.shuf;
  jo.out_bf = p.out;
  jo.out_stride = PO_HID;
  jo.res = p.h;
  jo.res_stride = PO_HID;
  jo.ssq = FUSED ? p.ssq : nullptr;  // a launch of its own has no MoE to feed
  const GemvO go(tid);
  const __amdgpu_buffer_rsrc_t rh = rsrc(p.h, (uint32_t)R * PO_HID * 2u);
  const int etok = (tid >> 4) & 15, erow = tid & 15;     // o_proj epilogue coordinates

  int a0 = b, a1 = b + nblk;
  v4i w0[4], w1[4];
  float s0[4], s1[4];
  auto load_h = [&](int t0, int t1) -> int {
    const int t = tid < 256 ? t0 : t1;
    const bool v = etok < R && tid < 512 && t < PO_TILES;
    return __builtin_amdgcn_raw_buffer_load_b16(
        rh, v ? (uint32_t)(etok * PO_HID + t * 16 + erow) * 2u : 0x80000000u, 0, 0);
  };
  int hres;
  bool ok = true;
  // W_UV tasks (token r, head h) = u = r * 32 + h, CTA b taking u = b, b + nblk, ...
  // (UvUnit). In the one-launch layer the attention's merge runs them (FUSED: none here).
  UvUnit uu;
  v4i xv = {0, 0, 0, 0};
  const int nuv = FUSED ? 0 : R * PO_HEADS;
  v4f (*uvred)[64] = red + 32;                                       // [16][64], past o_proj's
  uint16_t* uvx = reinterpret_cast<uint16_t*>(lds + 48 * 64 * 16);  // [512]
  uint16_t* uob = uvx + PO_LAT;                                      // [128]
  static_assert(48 * 64 * 16 + PO_LAT * 2 + PO_V * 2 <= PO_LDS_BYTES, "W_UV LDS");
  auto uv_x = [&](int u) -> v4i {  // token r's latents of head h: 64 threads x 8 bf16
    const int r = u / PO_HEADS, h = u % PO_HEADS;
    return ld16<CP_NONE>(
        rsrc(p.o_lat + ((size_t)r * PO_HEADS + h) * PO_LAT, u < nuv && tid < 64 ? PO_LAT * 2 : 0),
        (uint32_t)(tid & 63) * 16u);
  };
  auto uv_run = [&](int u) {
    const int r = u / PO_HEADS, h = u % PO_HEADS;
    if (tid < 64) reinterpret_cast<v4i*>(uvx)[tid] = xv;
    __syncthreads();
    uu.dot(uvx, uvred, tid);
    __syncthreads();
    if (tid < PO_V) uob[tid] = (uint16_t)bf16_bits(UvUnit::row(uvred, tid));
    __syncthreads();
    UvUnit::store(uob, tid, reinterpret_cast<uint32_t*>(obuf + (size_t)r * PO_O + h * PO_V),
                  0xFFFFFFFFu,
                  p.o ? reinterpret_cast<uint32_t*>(p.o + (size_t)r * PO_O + h * PO_V) : nullptr);
  };

  // ---------------------------------------------------------------- prefetch
  // W_UV task b's weights and latents, then o_proj tile b (all waves) and h; o_proj tile
  // b + nblk only once W_UV's outputs are stored. The barrier puts every W_UV load of the
  // CU ahead of every o_proj load: the CU's vector memory path serves its waves' requests
  // in issue order, stores included, and drains a prefetch at the CU's share of HBM
  // bandwidth (~23 KB/us), so a store issued behind both tiles (128 KB) would wait ~4 us
  // and hold back the o hand-off; one tile keeps HBM busy through W_UV.
  if constexpr (!FUSED) {
    uu.load(p.w_uv, p.s_uv, p.shuf, b % PO_HEADS, tid, b < nuv);
    xv = uv_x(b);
    __syncthreads();
  }
  go.issue(jo, 0, a0, w0, s0, a0 < PO_TILES);
  hres = load_h(a0, a1);
  if constexpr (FUSED) ok = ready();

  // ---------------------------------------------------------------- W_UV
  if constexpr (!FUSED) {
    if (b < nuv) {
      // W_UV's loads retire here; 7 follow them: the o_proj tile's 4 weight and 2 scale
      // loads, and h
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(7));
      uv_run(b);
    }
    // more W_UV tasks than CTAs: the rest without prefetch
    for (int u = b + nblk; u < nuv; u += nblk) {
      __syncthreads();
      uu.load(p.w_uv, p.s_uv, p.shuf, u % PO_HEADS, tid, true);
      xv = uv_x(u);
      uv_run(u);
    }
  }
  go.issue(jo, 0, a1, w1, s1, a1 < PO_TILES);
  // clear this CTA's slice of the next launch's hand-off buffer
  {
    constexpr uint32_t OB = (uint32_t)PostScratch::OBUF;
    const uint32_t slice = (OB / 16 + nblk - 1) / nblk * 16;
    const __amdgpu_buffer_rsrc_t rn = rsrc(onext, OB);
    for (uint32_t i = (uint32_t)tid * 16; i < slice; i += 1024 * 16)
      st16<CP_DEV>(rn, b * slice + i, v4i{0, 0, 0, 0});
  }
  stamp(p.timeline, MONO_TL_STAGED);

  // ---------------------------------------------------------------- o_proj
  for (int pass = 0; ok && a0 < PO_TILES; ++pass, a0 += 2 * nblk, a1 += 2 * nblk) {
    if (pass > 0) {
      go.issue(jo, 0, a0, w0, s0);
      go.issue(jo, 0, a1, w1, s1, a1 < PO_TILES);
      hres = load_h(a0, a1);
    }
    // o in this wave's K range, for rows t < R; complemented: zero = not written yet
    v4i xa[4][2];
    const __amdgpu_buffer_rsrc_t rx = rsrc(obuf, (uint32_t)PostScratch::OBUF);
    const int t = l & 15, grp = l >> 4;
    ok = wait_until(guard, MONO_SITE_O, [&]() {
      uint32_t mn = 0xFFFFFFFFu;
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          const uint32_t off =
              t < R ? (uint32_t)(t * PO_O + go.k0(st) + 16 * grp + 8 * m) * 2u : 0x80000000u;
          xa[st][m] = ld16<CP_DEV>(rx, off);
#pragma unroll
          for (int q = 0; q < 4; ++q) mn = __builtin_elementwise_min(mn, (uint32_t)xa[st][m][q]);
        }
      return __all(t >= R || mn != 0u);
    });
    ok = cta_all(ok, ok_s);
    if (!ok) break;
    stamp(p.timeline, MONO_TL_UPGATE);
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int m = 0; m < 2; ++m) xa[st][m] = ~xa[st][m];
    const bool two = a1 < PO_TILES;
    go.dot(w0, s0, xa, red);
    if (two) go.dot(w1, s1, xa, red + 16);
    __syncthreads();
    if (tid < 256)
      GemvO::epilogue(jo, 0, a0, R, tid, red, hres);
    else if (two && tid < 512)
      GemvO::epilogue(jo, 0, a1, R, tid - 256, red + 16, hres);
    __syncthreads();
    stamp(p.timeline, MONO_TL_MIDQ);
  }

}

}  // namespace mono
