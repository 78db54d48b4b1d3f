// The front of the layer as one persistent gfx950 launch: from the layer input h to the
// attention launch's inputs, with the row's KV and index-key cache writes.
//   X   x = bf16(rmsnorm(h) g_in) of row r built once, by CTA 168 + r (a CTA with no
//       stage-A task), and handed to every stage-A CTA as complemented bf16 pairs;
//   A   q_a | kv_a (W_qkv_a [2112, 7168]) and the index key (W_k [128, 7168]) as
//       140 FP8 16-row tiles over the whole K, the head weights (W_w [64, 7168] bf16) as
//       28 tasks of 16 rows x 1024 K (partials summed in a fixed order by their reader)
//       (sgl_amd_mono/glm53/gfx950/kernel.py:1781-1970, stage_x_rmsnorm :1367-1402);
//   A'  tasks (row, kind) on the last 4R CTAs, which hold no B or C tile when the rest
//       of the grid can hold them all: the KV row, kv_n = bf16(rmsnorm(kv_a[:512]) g_kv)
//       and k_pe = bf16(rope(kv_a[512:]))
//       as E4M3 with a power-of-two per-token scale (:2005-2101); the index key,
//       LayerNorm, RoPE on dims 0..63, FWHT-128, each rounded to bf16, FP4 (e2m1 + e8m0
//       per 32) into SGLang's index plane (:2103-2180, deepseek_v4 indexer.py:143-151,
//       242-254); the head weights,
//       bf16(w) 128^-1/2 64^-1/2 (indexer.py:400-406);
//   B   q_an = bf16(rmsnorm(q_a) g_q) (:1978-2003), built in LDS by every B CTA from
//       A's q_a (no hand-off through A'), then q_b (W_qb [6144, 1536]) and the index
//       query (W_iq [8192, 1536]) over it: 448 tiles of 32 rows; q_b's nope rows go on in
//       bf16, its rope rows are rotated in the epilogue (adjacent rows in adjacent lanes,
//       factors read from the cos / sin tables) into q[.., 512:] (:2183-2353);
//   B'  the index query, RoPE, FWHT-128, FP4 per head (one wave a head, lane l holding
//       dims 2l, 2l + 1), the rotated half and the transform's output rounded to bf16
//       (indexer.py:311-338);
//   C   the absorbed query q_lat = bf16(W_UK q_nope), 4 tiles of 128 latent rows a head
//       into q[.., :512] (:2355-2443).
// Hand-offs between stages are complemented words in one of two scratch buffers (by the
// launch tag's parity; the launch clears the other one for the next launch): a zero word
// is "not written yet", so a reader's loads are its wait and no flag, drain or poll is
// needed. Every prefetch is unconditional where a later wait depends on its count (absent
// tiles read zeros through a zero-size buffer resource).
#pragma once

#include <hip/hip_runtime.h>

#include "gemv.h"
#include "mono_abi.h"
#include "phase.h"

namespace mono {

constexpr int FR_H = 7168, FR_QL = 1536, FR_KVL = 512, FR_PE = 64, FR_KVA = 576;
constexpr int FR_QKVA = FR_QL + FR_KVA;          // 2112 rows of W_qkv_a
constexpr int FR_IK = 128, FR_IH = 64;           // index key dims, index heads
constexpr int FR_HEADS = 32, FR_NOPE = 128, FR_QHD = 192;
constexpr int FR_QB = FR_HEADS * FR_QHD;         // 6144
constexpr int FR_IQ = FR_IH * FR_IK;             // 8192
constexpr int FR_LAT = 512;
constexpr int FR_Q = FR_LAT + FR_PE;             // 576: an attention query row
constexpr uint32_t FR_DSA_PAGE = 64 * (128 + 4);  // a DSA index page: values, then scales
constexpr int FR_MAXR = 8;                       // rows: x of all of them fits in LDS
constexpr int FR_XG = 8;
constexpr int FR_XS = FR_H + 8;                  // LDS row stride of x (bf16): 16 B of pad
constexpr int FR_AST = FR_H / 64 / 16;           // 7 steps of 64 K a wave in stage A
constexpr int FR_QKT = FR_QKVA / 16;             // 132 tiles of W_qkv_a
constexpr int FR_A8 = FR_QKT + FR_IK / 16;       // 140 FP8 tiles
constexpr int FR_WCH = 7;                        // head-weight K chunks of 1024
constexpr int FR_ATASKS = FR_A8 + FR_IH / 16 * FR_WCH;  // 168
constexpr int FR_BT = (FR_QB + FR_IQ) / 32;      // 448 tiles (q_b: 192, then W_iq)
constexpr int FR_QBT = FR_QB / 32;               // 192
constexpr int FR_CT = FR_HEADS * 4;              // 128 W_UK tiles
constexpr int FR_HA = FR_QKVA + FR_IK;           // 2240 stage A outputs a row
constexpr int FR_MAX_GRID = 1024;
// timeline marks of the front beyond MONO_TL_STAGED (A / A' done) and MONO_TL_ROUTED (B
// done): a stage-A CTA's guard set up (its weights issued), x in its LDS, its MFMAs done;
// a B CTA's q_a in, its MFMAs done
constexpr int FR_TL_BEGUN = 3, FR_TL_XIN = 4, FR_TL_AMFMA = 5, FR_TL_QAIN = 6, FR_TL_BMFMA = 7;

using GemvB = Gemv<8, 2, 3>;   // 32 rows over K 1536: 2 row groups x 8 K-splits of 192
using GemvC = Gemv<2, 8, 1>;   // 128 rows over K 128: 8 row groups x 2 K-splits of 64

struct FrontScratch {
  // one parity's hand-off buffers (complemented words)
  static constexpr size_t HA = 0;                                           // f32 [8][2240]
  static constexpr size_t HW = HA + (size_t)FR_MAXR * FR_HA * 4;            // f32 [7][8][64]
  static constexpr size_t HN = HW + (size_t)FR_WCH * FR_MAXR * FR_IH * 4;   // bf16 [8][32][128]
  static constexpr size_t HI = HN + (size_t)FR_MAXR * FR_HEADS * FR_NOPE * 2;  // bf16 [8][8192]
  static constexpr size_t HX = HI + (size_t)FR_MAXR * FR_IQ * 2;            // bf16 [8][7168]
  static constexpr size_t PARITY = (HX + (size_t)FR_MAXR * FR_H * 2 + 255) & ~(size_t)255;
  static constexpr size_t BYTES = 2 * PARITY;
};

struct FrontParams {
  int rows, shuf, rope_rows;
  int index_fmt;  // MONO_INDEX_*: the index key's cache and the index query's form
  uint32_t kv_slots, plane_pages;
  float eps;
  const uint16_t* h;
  const uint16_t* g_in;
  const uint16_t* g_q;
  const uint16_t* g_kv;
  const uint8_t* w_qkv_a;
  const float* s_qkv_a;
  const uint8_t* w_k;
  const float* s_k;
  const uint16_t* w_w;
  const float* g_k;
  const float* b_k;
  const uint8_t* w_qb;
  const float* s_qb;
  const uint8_t* w_iq;
  const float* s_iq;
  const uint8_t* w_uk;
  const float* s_uk;
  const uint16_t* cos;
  const uint16_t* sin;
  const int64_t* positions;
  const int64_t* slots;
  uint8_t* kv;
  float* kv_scale;
  uint8_t* plane;
  uint8_t* plane_scale;
  uint16_t* q;
  uint8_t* iq;
  uint8_t* iqs;
  float* iw;
  float* ik_raw;
  uint16_t* iq_raw;
  uint8_t* scratch;
  int32_t* guard;
  uint32_t* host_err;
  int fault_site, fault_after;
  uint64_t* timeline;
};

// complemented hand-off words: never zero once written (an all-ones f32 or bf16 pair is
// a NaN, kept a NaN by clearing its lowest mantissa bit)
__device__ inline uint32_t enc_f(float v) {
  const uint32_t u = __float_as_uint(v);
  return ~(u == 0xFFFFFFFFu ? 0xFFFFFFFEu : u);
}
__device__ inline uint32_t enc_pair(uint32_t pr) { return ~(pr == 0xFFFFFFFFu ? 0xFFFEFFFFu : pr); }
__device__ inline float dec_f(uint32_t w) { return __uint_as_float(~w); }

// smallest power of two >= x (x positive and normal): 2^e, and its inverse 2^-e
__device__ inline void pow2_ceil(float x, float& sc, float& inv) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t e = ((u >> 23) & 0xFFu) + ((u & 0x7FFFFFu) != 0u);
  sc = __uint_as_float(e << 23);
  inv = __uint_as_float((254u - e) << 23);
}

// one butterfly over lanes l and l ^ M (`up`: lane l holds the upper one): the lower lane
// gets lo + hi, the upper lo - hi. On the VALU: DPP quad_perm for M = 1, 2, two DPP
// mirrors for 4 (half-row mirror, then quad reversal) and 8 (row mirror, then half-row
// mirror), v_permlane16_swap / v_permlane32_swap for 16, 32 (which hand every lane its
// pair's lower and upper value).
template <int M>
__device__ inline float bfly(float v, bool up) {
  if constexpr (M == 16 || M == 32) {
    const uint32_t u = __float_as_uint(v);
    const auto s = M == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                           : __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const float lo = __uint_as_float(s[0]), hi = __uint_as_float(s[1]);
    return up ? lo - hi : lo + hi;
  } else {
    float p;
    if constexpr (M == 1) p = dpp_f<DPP_XOR1>(v);
    else if constexpr (M == 2) p = dpp_f<DPP_XOR2>(v);
    else if constexpr (M == 4) p = dpp_f<DPP_REV4>(dpp_f<DPP_HALF_MIRROR>(v));
    else p = dpp_f<DPP_HALF_MIRROR>(dpp_f<DPP_MIRROR>(v));
    return up ? p - v : v + p;
  }
}

// the orthonormal 128-point Sylvester Hadamard transform of the values a wave holds,
// lane l holding entries 2l and 2l + 1
__device__ inline void fwht128(float& v0, float& v1, int l) {
  const float a = v0 + v1, b = v0 - v1;
  v0 = a;
  v1 = b;
  auto stage = [&](auto m_c) {
    constexpr int M = decltype(m_c)::value;
    const bool up = (l & M) != 0;
    v0 = bfly<M>(v0, up);
    v1 = bfly<M>(v1, up);
  };
  stage(std::integral_constant<int, 1>());
  stage(std::integral_constant<int, 2>());
  stage(std::integral_constant<int, 4>());
  stage(std::integral_constant<int, 8>());
  stage(std::integral_constant<int, 16>());
  stage(std::integral_constant<int, 32>());
  constexpr float S = 0.08838834764831845f;  // 128^-1/2
  v0 *= S;
  v1 *= S;
}

// FP4 of a wave's 128 values (lane l: entries 2l, 2l + 1) in blocks of 32 (16 lanes):
// returns this lane's code byte (entry 2l in the low nibble) and sets `e8` to the block's
// E8M0 scale byte. scale = pow2_ceil(max(amax, 6 * 2^-126) / 6), codes = E2M1(v / scale)
// round to nearest even.
__device__ inline uint32_t fp4_pair(float v0, float v1, uint32_t& e8) {
  const float amax = red16(fmaxf(fabsf(v0), fabsf(v1)), OpMax());
  float sc, inv;
  pow2_ceil(fmaxf(amax, 6.0f * 1.1754944e-38f) * (1.0f / 6.0f), sc, inv);
  const float q0 = __builtin_amdgcn_fmed3f(v0 * inv, -6.0f, 6.0f);
  const float q1 = __builtin_amdgcn_fmed3f(v1 * inv, -6.0f, 6.0f);
  e8 = (__float_as_uint(sc) >> 23) & 0xFFu;
  return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, q0, q1, 1.0f, 0) & 0xFFu;
}

// 4 lanes' bytes (lanes 4k .. 4k + 3) into one word, valid in lane 4k
__device__ inline uint32_t gather4(uint32_t byte, int l) {
  uint32_t w = byte << (8 * (l & 3));
  w |= dpp_u<DPP_XOR1>(w);
  w |= dpp_u<DPP_XOR2>(w);
  return w;
}

// CTA-wide sum / max of one value a thread, in a fixed order (all threads get it)
__device__ inline float block_red(float v, float* sred, bool is_max) {
  v = is_max ? wave_max(v) : wave_sum(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) sred[w] = v;
  __syncthreads();
  float s = sred[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) s = is_max ? fmaxf(s, sred[i]) : s + sred[i];
  __syncthreads();
  return s;
}

// LDS of the front: x (or q_an) rows, the reduction tiles, small sums
constexpr int FR_LDS_XS = 0;                                   // bf16 [8][FR_XS]
constexpr int FR_LDS_RED = FR_LDS_XS + FR_XG * FR_XS * 2;      // v4f [32][64]
constexpr int FR_LDS_SRED = FR_LDS_RED + 32 * 64 * 16;         // f32 [8 * 16]
constexpr int FR_LDS_RS = FR_LDS_SRED + 8 * 16 * 4;            // f32 [8]
constexpr int FR_LDS_BYTES = FR_LDS_RS + FR_XG * 4;
static_assert(FR_LDS_RED % 16 == 0, "16-byte aligned reduction tiles");

// The front in one CTA of a launch (the layer launch's first phase: nothing to wait for).
// Its outputs (q, iq, iqs, iw, the rows' KV and index-key cache entries) are stored
// device coherent, so the attention phase of the same launch can read them. `begin`
// (every thread, once) sets up the guard and returns the launch tag: it is called after
// the CTA's first loads are issued, so they are in flight while the guard head arrives.
// Returns the tag.
template <class Begin>
__device__ __attribute__((always_inline)) inline uint32_t front_phase(const FrontParams& p,
                                                                      uint8_t* lds,
                                                                      Guard& guard, int& ok_s,
                                                                      Begin begin) {
  const int b = blockIdx.x, G = gridDim.x, R = p.rows;
  uint16_t* xs = reinterpret_cast<uint16_t*>(lds + FR_LDS_XS);
  v4f (*red)[64] = reinterpret_cast<v4f (*)[64]>(lds + FR_LDS_RED);
  float* sred = reinterpret_cast<float*>(lds + FR_LDS_SRED);
  float* rs_s = reinterpret_cast<float*>(lds + FR_LDS_RS);

  uint32_t tag = 0;
  uint8_t* cur = nullptr;
  uint8_t* nxt = nullptr;
  auto start = [&]() {
    tag = begin();
    cur = p.scratch + (tag & 1u) * FrontScratch::PARITY;
    nxt = p.scratch + ((tag + 1u) & 1u) * FrontScratch::PARITY;
  };
  // the hand-off buffers of this launch
  auto rHA = [&]() { return rsrc(cur + FrontScratch::HA, FR_MAXR * FR_HA * 4); };
  auto rHW = [&]() { return rsrc(cur + FrontScratch::HW, FR_WCH * FR_MAXR * FR_IH * 4); };
  auto rHN = [&]() { return rsrc(cur + FrontScratch::HN, FR_MAXR * FR_HEADS * FR_NOPE * 2); };
  auto rHI = [&]() { return rsrc(cur + FrontScratch::HI, FR_MAXR * FR_IQ * 2); };
  auto rHX = [&]() { return rsrc(cur + FrontScratch::HX, FR_MAXR * FR_H * 2); };
  // the RoPE factors of row r's position, pair j, from the bf16 tables (as A' kind 1)
  auto rope_at = [&](int r, int j, float& cs, float& sn) {
    const int64_t pos = p.positions[r];
    const uint32_t po = pos >= 0 && pos < p.rope_rows ? (uint32_t)(pos * 32 + j) * 2u : 0x80000000u;
    cs = bf16_lo((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rsrc(p.cos, (uint32_t)p.rope_rows * 64u), po, 0, 0));
    sn = bf16_lo((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rsrc(p.sin, (uint32_t)p.rope_rows * 64u), po, 0, 0));
  };
  const int nap = 4 * R;            // A' tasks: the last nap CTAs
  const bool is_a = b < FR_ATASKS;
  const bool is_ap = b >= G - nap;

  // ---------------------------------------------------------------- B / C jobs
  // B and C tiles go to the CTAs without an A' task when those hold them all (two B
  // tiles each): a tile placed behind an A' task (index key, KV row) would wait for it,
  // and B', C and the end of the launch for the tile
  const int nbc = 2 * (G - nap) >= FR_BT ? G - nap : G;
  const bool bc = b < nbc;
  const int jb0 = bc ? b : FR_BT, jb1 = bc ? b + nbc : FR_BT;
  auto bjob = [&](int j) {
    GemvJob jb{};
    const bool qb = j < FR_QBT;
    jb.x = nullptr;
    jb.w = qb ? p.w_qb : p.w_iq;
    jb.s = qb ? p.s_qb : p.s_iq;
    jb.N = qb ? FR_QB : FR_IQ;
    jb.K = FR_QL;
    jb.G = 1;
    jb.shuf = p.shuf;
    return jb;
  };
  const GemvJob jB0 = bjob(jb0), jB1 = bjob(jb1);
  const int tb0 = jb0 < FR_QBT ? jb0 : jb0 - FR_QBT, tb1 = jb1 < FR_QBT ? jb1 : jb1 - FR_QBT;
  const int cidx = bc ? nbc - 1 - b : -1;  // this CTA's W_UK tile (if 0 .. 127)
  GemvJob jC{};
  jC.w = p.w_uk;
  jC.s = p.s_uk;
  jC.N = FR_LAT;
  jC.K = FR_NOPE;
  jC.G = FR_HEADS;
  jC.shuf = p.shuf;
  v4i wb0[3], wb1[3], wc[1];
  float sb0[3], sb1[3], sc_[1];

  // ---------------------------------------------------------------- A, or A'
  {
    const int tid = opaque_v((int)threadIdx.x);
    const int l = tid & 63, w = tid >> 6;
    const GemvB gb(tid);
    const GemvC gc(tid);
    auto issue_b0 = [&]() { gb.issue(jB0, 0, tb0, wb0, sb0, jb0 < FR_BT); };
    auto issue_b1c = [&]() {
      gb.issue(jB1, 0, tb1, wb1, sb1, jb1 < FR_BT);
      gc.issue(jC, cidx / 4, cidx % 4, wc, sc_, cidx >= 0 && cidx < FR_CT);
    };
    if (is_a) {
      // ------------------------------------------ stage A: the task's weights first,
      // then x (polled), then stage B and C's weights
      const bool a8 = b < FR_A8, qkv = b < FR_QKT;
      const int ta = qkv ? b : b - FR_QKT;          // FP8 16-row tile
      const int tw = (b - FR_A8) / FR_WCH, cw = (b - FR_A8) % FR_WCH;  // bf16 task
      const int ck = tid < FR_H / 8 ? tid : 0;       // thread's 8-K chunk of x
      const bool xk = tid < FR_H / 8;
      // the task's weights: an FP8 tile's 7 steps of the wave's K range, or a bf16 task's
      // two 16-byte pieces (rows 16 tw + t16, K c 1024 + 64 w + 16 grp + 8 m) in steps 0-1
      const uint8_t* wa = qkv ? p.w_qkv_a : p.w_k;
      const float* sa = qkv ? p.s_qkv_a : p.s_k;
      const int na = qkv ? FR_QKVA : FR_IK;
      const int t16 = l & 15, grp = l >> 4;
      v4i wa8[FR_AST];
      float sa8[FR_AST];
      {
        const __amdgpu_buffer_rsrc_t rwa =
            a8 ? rsrc(wa, (uint32_t)na * FR_H) : rsrc(p.w_w, (uint32_t)FR_IH * FR_H * 2u);
        const __amdgpu_buffer_rsrc_t rsa =
            rsrc(sa, a8 ? (uint32_t)((na + 127) / 128) * (FR_H / 128) * 4u : 0u);
        const uint32_t vo = !a8 ? (uint32_t)((tw * 16 + t16) * FR_H + cw * 1024 + 64 * w + 16 * grp) * 2u
                            : p.shuf ? (uint32_t)l * 16 : (uint32_t)(t16 * FR_H + 16 * grp);
        const int sh = p.shuf ? 4 : 0;
#pragma unroll
        for (int s = 0; s < FR_AST; ++s) {
          const int k0 = (w * FR_AST + s) * 64;
          const uint32_t so = !a8 ? (s < 2 ? (uint32_t)(16 * s) : 0x80000000u)
                                  : (uint32_t)(ta * 16 * FR_H) + ((uint32_t)k0 << sh);
          wa8[s] = ld16s<CP_NT>(rwa, vo, so);
        }
#pragma unroll
        for (int s = 0; s < FR_AST; ++s) {
          const int k0 = (w * FR_AST + s) * 64;
          sa8[s] = __int_as_float(
              ld4<CP_NONE>(rsa, (uint32_t)((ta / 8) * (FR_H / 128) + k0 / 128) * 4u));
        }
      }
      start();
      stamp(p.timeline, FR_TL_BEGUN);

      // x of the rows into LDS (built once a row by CTA FR_ATASKS + r as complemented bf16
      // pairs: the loads are the wait; rows past R are zeros), then the MFMAs over it and
      // the outputs
      auto run_group = [&](int g) {
        {
          const __amdgpu_buffer_rsrc_t rx = rHX();
          v4i xv[FR_XG];
          bool okx = wait_until(guard, MONO_SITE_X, [&]() {
            uint32_t mn = 0xFFFFFFFFu;
#pragma unroll
            for (int t = 0; t < FR_XG; ++t) {
              const bool on = xk && g * FR_XG + t < R;
              xv[t] = ld16<CP_DEV>(rx, on ? (uint32_t)(((g * FR_XG + t) * FR_H + 8 * ck) * 2) : 0x80000000u);
#pragma unroll
              for (int q = 0; q < 4; ++q) mn = on ? min(mn, (uint32_t)xv[t][q]) : mn;
            }
            return __all(mn != 0u);
          });
          if (!cta_all(okx, ok_s)) return;
#pragma unroll
          for (int t = 0; t < FR_XG; ++t)
            if (xk)
              *reinterpret_cast<v4i*>(&xs[t * FR_XS + 8 * ck]) =
                  g * FR_XG + t < R ? ~xv[t] : v4i{0, 0, 0, 0};
        }
        __syncthreads();
        stamp(p.timeline, FR_TL_XIN);
        issue_b0();  // the rows are in: stage B's first tile now
        // MFMAs: lanes t16 < 8 take row t16 of the group; the others multiply zeros
        v4f acc = {0.f, 0.f, 0.f, 0.f};
        if (a8) {
#pragma unroll
          for (int s = 0; s < FR_AST; ++s) {
            // one step's LDS reads at a time: hoisting all 14 would need 56 more registers
            __builtin_amdgcn_sched_barrier(0);
            const int k = (w * FR_AST + s) * 64 + 16 * grp;
            const v4i* px = reinterpret_cast<const v4i*>(&xs[(t16 & 7) * FR_XS + k]);
            const v4i zero = {0, 0, 0, 0};
            const v4i x0 = t16 < FR_XG ? px[0] : zero, x1 = t16 < FR_XG ? px[1] : zero;
            v4f d = {0.f, 0.f, 0.f, 0.f};
            d = mfma_bf16(fp8x8_bf16((uint32_t)wa8[s][0], (uint32_t)wa8[s][1]),
                          __builtin_bit_cast(v8bf, x0), d);
            d = mfma_bf16(fp8x8_bf16((uint32_t)wa8[s][2], (uint32_t)wa8[s][3]),
                          __builtin_bit_cast(v8bf, x1), d);
            acc += d * sa8[s];
          }
        } else {
          const int k = cw * 1024 + 64 * w + 16 * grp;
          const v4i* px = reinterpret_cast<const v4i*>(&xs[(t16 & 7) * FR_XS + k]);
          const v4i zero = {0, 0, 0, 0};
          const v4i x0 = t16 < FR_XG ? px[0] : zero, x1 = t16 < FR_XG ? px[1] : zero;
          acc = mfma_bf16(__builtin_bit_cast(v8bf, wa8[0]), __builtin_bit_cast(v8bf, x0), acc);
          acc = mfma_bf16(__builtin_bit_cast(v8bf, wa8[1]), __builtin_bit_cast(v8bf, x1), acc);
        }
        issue_b1c();  // this stage's weights are consumed: B's second tile and C's
        red[w][l] = acc;
        stamp(p.timeline, FR_TL_AMFMA);
        __syncthreads();
        if (tid < 256) {
          const int row = tid & 15, tok = (tid >> 4) & 15;
          const int L = tok + 16 * (row >> 2), v = row & 3;
          float y = 0.f;
#pragma unroll
          for (int i = 0; i < 16; ++i) y += red[i][L][v];
          const int r = g * FR_XG + tok;
          if (tok < FR_XG && r < R) {
            if (a8) {
              const int n = (qkv ? 0 : FR_QKVA) + ta * 16 + row;
              st_dev(reinterpret_cast<uint32_t*>(cur + FrontScratch::HA) + r * FR_HA + n, enc_f(y));
              if (!qkv && p.ik_raw) p.ik_raw[r * FR_IK + ta * 16 + row] = y;
            } else {
              st_dev(reinterpret_cast<uint32_t*>(cur + FrontScratch::HW) +
                         (cw * FR_MAXR + r) * FR_IH + tw * 16 + row,
                     enc_f(y));
            }
          }
        }
        __syncthreads();
      };
      run_group(0);
    } else {
      // ------------------------------------------ x of row xr = b - FR_ATASKS, once for
      // every stage-A task: bf16(rmsnorm(h) g_in), the sum of squares in the order each
      // task used when it built x itself (a thread's 8 values by dot2, the wave, the 16
      // waves in order), as complemented bf16 pairs
      const int xr = b - FR_ATASKS;
      const bool xb = xr >= 0 && xr < R;
      const int ck = tid < FR_H / 8 ? tid : 0;
      const bool xk = tid < FR_H / 8;
      const v4i hw = ld16<CP_NONE>(rsrc(p.h, (uint32_t)R * FR_H * 2u),
                                   xb && xk ? (uint32_t)((xr * FR_H + 8 * ck) * 2) : 0x80000000u);
      const v4i gv = ld16<CP_NONE>(rsrc(p.g_in, xb ? FR_H * 2 : 0u), (uint32_t)(8 * ck) * 2u);
      start();
      if (xb) {
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) s = dot2_bf16_sq((uint32_t)hw[q], s);
        s = wave_sum(s);
        if (l == 0) sred[w] = s;
        __syncthreads();
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) ss += sred[i];
        const float rs = __builtin_amdgcn_rsqf(ss * (1.0f / FR_H) + p.eps);
        if (xk) {
          v4i o;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t hq = (uint32_t)hw[q], gq = (uint32_t)gv[q];
            o[q] = (int)enc_pair(bf16x2_bits(bf16_lo(hq) * rs * bf16_lo(gq), bf16_hi(hq) * rs * bf16_hi(gq)));
          }
          st16<CP_DEV>(rHX(), (uint32_t)((xr * FR_H + 8 * ck) * 2), o);
        }
        __syncthreads();  // sred is reused
      }
      if (is_ap) {
        // ------------------------------------------ A': task (row, kind)
        const int u = b - (G - nap), r = u >> 2, kind = u & 3;
        bool ok = true;
        if (kind == 0) {
          // q_an is built by every stage-B CTA from q_a: nothing to do
        } else if (kind == 1) {
          // the KV row -> cache (E4M3 + power-of-two scale)
          const int64_t pos = sld(p.positions, r), slot = sld(p.slots, r);
          const bool on = tid < FR_KVA / 2;       // pair i = tid
          const bool pe = tid >= FR_KVL / 2 && on;
          const int j = pe ? tid - FR_KVL / 2 : (tid & 31);
          const __amdgpu_buffer_rsrc_t rc = rsrc(p.cos, (uint32_t)p.rope_rows * 64u);
          const __amdgpu_buffer_rsrc_t rsn = rsrc(p.sin, (uint32_t)p.rope_rows * 64u);
          const uint32_t po = pos >= 0 && pos < p.rope_rows ? (uint32_t)(pos * 32 + j) * 2u : 0x80000000u;
          const float cs = bf16_lo((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rc, po, 0, 0));
          const float sn = bf16_lo((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rsn, po, 0, 0));
          v2i v;
          ok = wait_until(guard, MONO_SITE_FRONT_A, [&]() {
            v = ld8<CP_DEV>(rHA(), on ? (uint32_t)(r * FR_HA + FR_QL + 2 * tid) * 4u : 0x80000000u);
            return __all(!on || min((uint32_t)v[0], (uint32_t)v[1]) != 0u);
          });
          ok = cta_all(ok, ok_s);
          if (ok) {
            const float a = on ? dec_f((uint32_t)v[0]) : 0.f, c = on ? dec_f((uint32_t)v[1]) : 0.f;
            const float ss = block_red(pe || !on ? 0.f : fmaf(a, a, c * c), sred, false);
            const float rs = __builtin_amdgcn_rsqf(ss * (1.0f / FR_KVL) + p.eps);
            float x0, x1;
            if (pe) {
              x0 = bf16_round(a * cs - c * sn);
              x1 = bf16_round(a * sn + c * cs);
            } else {
              const uint32_t gw = on ? (uint32_t)ld4<CP_NONE>(rsrc(p.g_kv, FR_KVL * 2), (uint32_t)tid * 4u) : 0u;
              x0 = bf16_round(a * rs * bf16_lo(gw));
              x1 = bf16_round(c * rs * bf16_hi(gw));
            }
            // with per-token scales: scale = pow2_ceil(max(amax, 1e-4) / 448); without (the
            // pool's raw E4M3 rows, SGLang's layout): scale 1, values saturating at +-448
            float sc = 1.0f, inv = 1.0f;
            if (p.kv_scale) {
              const float amax = block_red(on ? fmaxf(fabsf(x0), fabsf(x1)) : 0.f, sred, true);
              pow2_ceil(fmaxf(amax, 1e-4f) * (1.0f / 448.0f), sc, inv);
            }
            const uint32_t c16 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(
                                     clamp_fp8(x0 * inv), clamp_fp8(x1 * inv), 0, false) & 0xFFFFu;
            const uint32_t word = c16 | (dpp_u<DPP_XOR1>(c16) << 16);
            const bool live = slot >= 0 && (uint64_t)slot < (uint64_t)p.kv_slots;
            if (live && on && (tid & 1) == 0)
              __builtin_amdgcn_raw_buffer_store_b32((int)word, rsrc(p.kv, p.kv_slots * (uint32_t)FR_KVA),
                                                    (uint32_t)slot * FR_KVA + 2u * tid, 0, CP_DEV);
            if (live && tid == 0 && p.kv_scale) st_devf(p.kv_scale + slot, sc);
          }
        } else if (kind == 2) {
          // the index key -> LayerNorm, RoPE, FWHT -> FP4 into the index plane or E4M3
          // into a DSA page (wave 0)
          const int64_t pos = sld(p.positions, r), slot = sld(p.slots, r);
          const bool on = w == 0;
          const __amdgpu_buffer_rsrc_t rc = rsrc(p.cos, (uint32_t)p.rope_rows * 64u);
          const __amdgpu_buffer_rsrc_t rsn = rsrc(p.sin, (uint32_t)p.rope_rows * 64u);
          const uint32_t po = pos >= 0 && pos < p.rope_rows ? (uint32_t)(pos * 32 + (l & 31)) * 2u : 0x80000000u;
          const float cs = bf16_lo((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rc, po, 0, 0));
          const float sn = bf16_lo((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rsn, po, 0, 0));
          const v2f gk = __builtin_bit_cast(v2f, ld8<CP_NONE>(rsrc(p.g_k, FR_IK * 4), (uint32_t)(2 * l) * 4u));
          const v2f bk = __builtin_bit_cast(v2f, ld8<CP_NONE>(rsrc(p.b_k, FR_IK * 4), (uint32_t)(2 * l) * 4u));
          v2i v;
          ok = wait_until(guard, MONO_SITE_FRONT_A, [&]() {
            v = ld8<CP_DEV>(rHA(), on ? (uint32_t)(r * FR_HA + FR_QKVA + 2 * l) * 4u : 0x80000000u);
            return __all(!on || min((uint32_t)v[0], (uint32_t)v[1]) != 0u);
          });
          ok = cta_all(ok, ok_s);
          if (ok && on) {
            const float k0 = dec_f((uint32_t)v[0]), k1 = dec_f((uint32_t)v[1]);
            const float mean = wave_sum(k0 + k1) * (1.0f / FR_IK);
            const float c0 = k0 - mean, c1 = k1 - mean;
            const float rstd = __builtin_amdgcn_rsqf(wave_sum(fmaf(c0, c0, c1 * c1)) * (1.0f / FR_IK) + 1e-6f);
            const bool live = slot >= 0 && (uint64_t)slot < (uint64_t)p.plane_pages * 64u;
            if (p.index_fmt == MONO_INDEX_FP4_PLANE) {
              // bf16 after the norm, after the rotation and after the transform, then FP4
              // (the reference's FP4 key path, deepseek_v4 indexer.py:242-254)
              float v0 = bf16_round(fmaf(c0 * rstd, gk[0], bk[0]));
              float v1 = bf16_round(fmaf(c1 * rstd, gk[1], bk[1]));
              if (l < FR_PE / 2) {
                const float r0 = v0 * cs - v1 * sn, r1 = v0 * sn + v1 * cs;
                v0 = bf16_round(r0);
                v1 = bf16_round(r1);
              }
              fwht128(v0, v1, l);
              v0 = bf16_round(v0);
              v1 = bf16_round(v1);
              uint32_t e8;
              const uint32_t byte = fp4_pair(v0, v1, e8);
              const uint32_t word = gather4(byte, l);
              if (live) {
                const uint32_t page = (uint32_t)(slot >> 6), s = (uint32_t)(slot & 63), c = (uint32_t)(l >> 4);
                if ((l & 3) == 0)
                  __builtin_amdgcn_raw_buffer_store_b32(
                      (int)word, rsrc(p.plane, p.plane_pages * 4096u),
                      ((page * 4 + c) * 64 + s) * 16 + (uint32_t)(l & 15), 0, CP_DEV);
                if ((l & 15) == 0)
                  __builtin_amdgcn_raw_buffer_store_b8(
                      (uint8_t)e8, rsrc(p.plane_scale, p.plane_pages * 256u),
                      (page * 4 + c) * 64 + (s % 16) * 4 + s / 16, 0, CP_DEV);
              }
            } else {
              // a DSA index page (kernel.py:2103-2168): the norm, the rotation and the
              // transform in f32, then E4M3 at a power-of-two per-token scale
              float v0 = fmaf(c0 * rstd, gk[0], bk[0]);
              float v1 = fmaf(c1 * rstd, gk[1], bk[1]);
              if (l < FR_PE / 2) {
                const float r0 = v0 * cs - v1 * sn, r1 = v0 * sn + v1 * cs;
                v0 = r0;
                v1 = r1;
              }
              fwht128(v0, v1, l);
              float sc, inv;
              pow2_ceil(__fdiv_rn(fmaxf(wave_max(fmaxf(fabsf(v0), fabsf(v1))), 1e-4f), 448.0f), sc, inv);
              // lanes 2 k, 2 k + 1 hold dims 4 k .. 4 k + 3: one dword of codes
              const uint32_t c2 =
                  (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v0 * inv, v1 * inv, 0, false) & 0xFFFFu;
              const uint32_t word = c2 | (dpp_u<DPP_XOR1>(c2) << 16);
              if (live) {
                const uint32_t s = (uint32_t)(slot & 63), d = 2u * (uint32_t)l;
                const __amdgpu_buffer_rsrc_t rp =
                    rsrc(p.plane + (size_t)(slot >> 6) * FR_DSA_PAGE, FR_DSA_PAGE);
                const uint32_t at = p.index_fmt == MONO_INDEX_FP8_PAGE
                                        ? (s >> 4) * 2048u + (d >> 4) * 256u + (s & 15u) * 16u + (d & 15u)
                                        : s * 128u + d;
                if ((l & 1) == 0) __builtin_amdgcn_raw_buffer_store_b32((int)word, rp, at, 0, CP_DEV);
                if (l == 0)
                  __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(sc), rp, 8192u + 4u * s, 0, CP_DEV);
              }
            }
          }
        } else {
          // the head weights: bf16(sum of the 7 partials) 128^-1/2 64^-1/2
          const bool on = tid < FR_IH;
          uint32_t pw[FR_WCH];
          ok = wait_until(guard, MONO_SITE_FRONT_A, [&]() {
            uint32_t mn = 0xFFFFFFFFu;
#pragma unroll
            for (int c = 0; c < FR_WCH; ++c) {
              pw[c] = (uint32_t)ld4<CP_DEV>(rHW(), on ? (uint32_t)((c * FR_MAXR + r) * FR_IH + tid) * 4u
                                                    : 0x80000000u);
              mn = min(mn, pw[c]);
            }
            return __all(!on || mn != 0u);
          });
          ok = cta_all(ok, ok_s);
          if (ok && on) {
            float s = dec_f(pw[0]);
#pragma unroll
            for (int c = 1; c < FR_WCH; ++c) s += dec_f(pw[c]);
            st_devf(p.iw + r * FR_IH + tid, bf16_round(s) * (0.08838834764831845f * 0.125f));
          }
        }
        (void)ok;
      }
      issue_b0();
      issue_b1c();
    }
  }
  stamp(p.timeline, MONO_TL_STAGED);

  // ---------------------------------------------------------------- clear the next buffers
  {
    constexpr uint32_t PB = (uint32_t)FrontScratch::PARITY;
    const uint32_t slice = (PB / 16 + G - 1) / G * 16;
    const __amdgpu_buffer_rsrc_t rn = rsrc(nxt, PB);
    for (uint32_t i = threadIdx.x * 16u; i < slice; i += 1024u * 16u)
      st16<CP_DEV>(rn, b * slice + i, v4i{0, 0, 0, 0});
  }

  // ---------------------------------------------------------------- B: q_b, W_iq
  bool okb = true;
  if (jb0 < FR_BT) {
    const int tid = opaque_v((int)threadIdx.x);
    const int l = tid & 63, w = tid >> 6;
    const GemvB gb(tid);
    const int t = l & 15, grp = l >> 4;
    // the epilogue thread's RoPE factors (q_b rope tiles): row tok, pair (n % 192 - 128) / 2
    const int e = tid & 511, rge = e >> 8, erow = e & 15, etok = (e >> 4) & 15;
    const int ej = tid < 512 ? jb0 : jb1;
    const int en = ((ej < FR_QBT ? ej : ej - FR_QBT) * 2 + rge) * 16 + erow;
    const bool epe = ej < FR_QBT && en % FR_QHD >= FR_NOPE && etok < R && ej < FR_BT;
    const int epair = (en % FR_QHD - FR_NOPE) >> 1;
    // the epilogue's RoPE factors (row etok, pair epair) from the bf16 tables
    float ecs = 0.f, esn = 0.f;
    if (epe) rope_at(etok, epair, ecs, esn);
    // q_an = bf16(rmsnorm(q_a) g_q) of every row, built by this CTA: thread tid holds 12
    // q_a values of row tid / 128 (A's f32 outputs, complemented words: the loads are the
    // wait), the row's sum of squares over its two waves in a fixed order, then the
    // products into LDS (stage A's x buffer), where the MFMA operands are read from
    constexpr int QNS = FR_QL + 8;  // LDS row stride of q_an (bf16)
    static_assert(FR_MAXR * QNS <= FR_XG * FR_XS, "q_an fits the x buffer");
    const int qr = tid >> 7, qc = (tid & 127) * 12;
    const bool qon = qr < R;
    const __amdgpu_buffer_rsrc_t rg = rsrc(p.g_q, FR_QL * 2);
    const v4i g0 = ld16<CP_NONE>(rg, (uint32_t)qc * 2u);
    const v2i g1 = ld8<CP_NONE>(rg, (uint32_t)qc * 2u + 16u);
    v4i qv[3];
    okb = wait_until(guard, MONO_SITE_QAN, [&]() {
      uint32_t mn = 0xFFFFFFFFu;
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        qv[i] = ld16<CP_DEV>(rHA(), qon ? (uint32_t)(qr * FR_HA + qc + 4 * i) * 4u : 0x80000000u);
#pragma unroll
        for (int q = 0; q < 4; ++q) mn = min(mn, (uint32_t)qv[i][q]);
      }
      return __all(!qon || mn != 0u);
    });
    okb = cta_all(okb, ok_s);
    stamp(p.timeline, FR_TL_QAIN);
    v4i xa[3][2];
    if (okb) {
      float a[12], s = 0.f;
#pragma unroll
      for (int i = 0; i < 12; ++i) {
        a[i] = qon ? dec_f((uint32_t)qv[i / 4][i % 4]) : 0.f;
        s = fmaf(a[i], a[i], s);
      }
      s = wave_sum(s);
      if (l == 0) sred[w] = s;
      __syncthreads();
      const float rs = __builtin_amdgcn_rsqf((sred[2 * qr] + sred[2 * qr + 1]) * (1.0f / FR_QL) + p.eps);
      if (qon) {
        const uint32_t gw[6] = {(uint32_t)g0[0], (uint32_t)g0[1], (uint32_t)g0[2], (uint32_t)g0[3],
                                (uint32_t)g1[0], (uint32_t)g1[1]};
        uint32_t pr[6];
#pragma unroll
        for (int j = 0; j < 6; ++j)
          pr[j] = bf16_bits(a[2 * j] * rs * bf16_lo(gw[j])) |
                  (bf16_bits(a[2 * j + 1] * rs * bf16_hi(gw[j])) << 16);
        uint32_t* dst = reinterpret_cast<uint32_t*>(&xs[qr * QNS + qc]);
#pragma unroll
        for (int j = 0; j < 3; ++j)
          *reinterpret_cast<v2i*>(dst + 2 * j) = v2i{(int)pr[2 * j], (int)pr[2 * j + 1]};
      }
      __syncthreads();
      const v4i zero = {0, 0, 0, 0};
#pragma unroll
      for (int s2 = 0; s2 < 3; ++s2)
#pragma unroll
        for (int m = 0; m < 2; ++m)
          xa[s2][m] = t < R ? *reinterpret_cast<const v4i*>(&xs[t * QNS + gb.k0(s2) + 16 * grp + 8 * m])
                            : zero;
      const bool two = jb1 < FR_BT;
      if (jb0 < FR_BT) gb.dot(wb0, sb0, xa, red);
      if (two) gb.dot(wb1, sb1, xa, red + 16);
      __syncthreads();
      stamp(p.timeline, FR_TL_BMFMA);
      const bool mine = tid < 512 ? jb0 < FR_BT : two;
      if (mine) {
        v4f (*rd)[64] = red + (tid < 512 ? 0 : 16);
        const int L = etok + 16 * (erow >> 2), v = erow & 3;
        float y = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) y += rd[rge * 8 + i][L][v];
        const bool qb = ej < FR_QBT;
        const int head = en / FR_QHD, d = en % FR_QHD;
        if (qb && d >= FR_NOPE) {
          const float cs = ecs, sn = esn;
          const float yp = dpp_f<DPP_XOR1>(y);  // the pair's other row
          y = (erow & 1) == 0 ? y * cs - yp * sn : yp * sn + y * cs;
        }
        const uint32_t h16 = bf16_bits(y);
        const uint32_t hn = dpp_u<DPP_XOR1>(h16);
        const uint32_t pr = h16 | (hn << 16);
        if (etok < R && (erow & 1) == 0) {
          if (!qb) {
            const int at = (etok * FR_IQ + (ej - FR_QBT) * 32 + rge * 16 + erow) / 2;
            st_dev(reinterpret_cast<uint32_t*>(cur + FrontScratch::HI) + at, enc_pair(pr));
            if (p.iq_raw) reinterpret_cast<uint32_t*>(p.iq_raw)[at] = pr;
          } else if (d < FR_NOPE)
            st_dev(reinterpret_cast<uint32_t*>(cur + FrontScratch::HN) + ((etok * FR_HEADS + head) * FR_NOPE + d) / 2,
                   enc_pair(pr));
          else
            st_dev(reinterpret_cast<uint32_t*>(p.q + (etok * FR_HEADS + head) * FR_Q + FR_LAT + d - FR_NOPE), pr);
        }
      }
      __syncthreads();
    }
  }
  stamp(p.timeline, MONO_TL_ROUTED);

  // ---------------------------------------------------------------- B': index query
  if (okb && b < nap) {
    const int tid = opaque_v((int)threadIdx.x);
    const int l = tid & 63, w = tid >> 6;
    const int r = b >> 2, hi = (b & 3) * 16 + w;
    uint32_t xw = 0;
    const bool rp = l < FR_PE / 2;
    float cs = 0.f, sn = 0.f;
    rope_at(r, l & 31, cs, sn);
    bool ok = wait_until(guard, MONO_SITE_QB, [&]() {
      xw = (uint32_t)ld4<CP_DEV>(rHI(), (uint32_t)((r * FR_IH + hi) * 64 + l) * 4u);
      return __all(xw != 0u);
    });
    ok = cta_all(ok, ok_s);
    if (ok && p.index_fmt != MONO_INDEX_FP4_PLANE) {
      // a DSA index page's query (kernel.py:2928-2944): the rotation and the transform in
      // f32, then bf16 once, into iq bf16 [R, 64, 128]
      const uint32_t pr = ~xw;
      float v0 = bf16_lo(pr), v1 = bf16_hi(pr);
      if (rp) {
        const float r0 = v0 * cs - v1 * sn, r1 = v0 * sn + v1 * cs;
        v0 = r0;
        v1 = r1;
      }
      fwht128(v0, v1, l);
      st_dev(reinterpret_cast<uint32_t*>(p.iq) + (r * FR_IH + hi) * 64 + l,
             bf16_bits(v0) | (bf16_bits(v1) << 16));
    } else if (ok) {
      const uint32_t pr = ~xw;
      float v0 = bf16_lo(pr), v1 = bf16_hi(pr);
      // the rotated half rounded to bf16 before the transform, the transform's output
      // rounded to bf16 before FP4 (deepseek_v4 indexer.py:330-335)
      if (rp) {
        const float r0 = v0 * cs - v1 * sn, r1 = v0 * sn + v1 * cs;
        v0 = bf16_round(r0);
        v1 = bf16_round(r1);
      }
      fwht128(v0, v1, l);
      v0 = bf16_round(v0);
      v1 = bf16_round(v1);
      uint32_t e8;
      const uint32_t byte = fp4_pair(v0, v1, e8);
      const uint32_t word = gather4(byte, l);
      if ((l & 3) == 0) st_dev(reinterpret_cast<uint32_t*>(p.iq + (r * FR_IH + hi) * 64 + l), word);
      if ((l & 15) == 0)
        __builtin_amdgcn_raw_buffer_store_b8((uint8_t)e8, rsrc(p.iqs, (uint32_t)R * 256u),
                                             ((r * 4 + (l >> 4)) * 16 + hi % 16) * 4 + hi / 16,
                                             0, CP_DEV);
    }
  }

  // ---------------------------------------------------------------- C: W_UK absorb
  if (okb && cidx >= 0 && cidx < FR_CT) {
    const int tid = opaque_v((int)threadIdx.x);
    const int l = tid & 63;
    const GemvC gc(tid);
    const int hc = cidx / 4, tc = cidx % 4;
    const int t = l & 15, grp = l >> 4;
    v4i xa[1][2];
    bool ok = wait_until(guard, MONO_SITE_QB, [&]() {
      uint32_t mn = 0xFFFFFFFFu;
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const uint32_t off = t < R ? (uint32_t)((t * FR_HEADS + hc) * FR_NOPE + gc.k0(0) + 16 * grp + 8 * m) * 2u
                                   : 0x80000000u;
        xa[0][m] = ld16<CP_DEV>(rHN(), off);
#pragma unroll
        for (int q = 0; q < 4; ++q) mn = min(mn, (uint32_t)xa[0][m][q]);
      }
      return __all(t >= R || mn != 0u);
    });
    ok = cta_all(ok, ok_s);
    if (ok) {
      xa[0][0] = ~xa[0][0];
      xa[0][1] = ~xa[0][1];
      gc.dot(wc, sc_, xa, red);
      __syncthreads();
      GemvJob jo{};
      jo.N = FR_LAT;
      jo.out_bf = p.q;
      jo.out_stride = FR_HEADS * FR_Q;
      jo.out_gstride = FR_Q;
      for (int e = tid; e < GemvC::ROWS * 16; e += 1024) GemvC::epilogue(jo, hc, tc, R, e, red);
      __syncthreads();
    }
  }
  return tag;
}

}  // namespace mono
