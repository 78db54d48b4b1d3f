// MXFP4 (E2M1 codes + E8M0 scales per 32) weight operands of the bf16 MFMA path (A16W4),
// shared by the MXFP4 MoE launch and the layer launch's MXFP4 experts.
//
// Reference: A16W4 operands sgl_amd_mono/minimax_m31/a16w4.py:26-92 (lane = one row's
// 32-group, scale folded into the fp4 -> bf16 convert); MXFP4 units
// sgl_amd_mono/glm53/gfx950/kernel.py:906-995; the e8m0 shuffle index
// sgl_amd_mono/common/mx.py:40-44.
#pragma once

#include "mono_device.h"

namespace mono {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// Operand addressing of one MXFP4 weight matrix [N, K] (one expert): a lane's 16 code
// bytes are row 16 rg + l % 16, K 128 s + 32 (l / 16) .. + 31; its scale is that row's
// E8M0 of column 4 s + l / 16. Offsets split into a per-lane part (VGPR) and a
// wave-uniform part (SGPR).
//   row-major: codes [N, K / 2], scales [N, K / 32];
//   SHUF: codes in AITER's (16, 16) shuffle, [N / 16, K / 64, 2, 16 rows, 16 B], where a
//   16-row x 128-K tile is 1 KiB contiguous with lane l at 16 l; scales in the e8m0
//   shuffle of sgl_amd_mono/common/mx.py:40-44 over CP = K / 32 rounded up to 8 columns:
//   byte ((((r32 CP/8 + c8) 4 + e) 16 + b) 2 + d) 2 + a for row 32 r32 + 16 a + b and
//   column 8 c8 + 4 d + e, so lane l's byte of step s sits in dword
//   (r32 CP/8 + s / 2) 64 + l at byte 2 (s % 2) + rg % 2.
template <bool SHUF, int K>
struct MxOperand {
  static constexpr int C = K / 32;
  static constexpr int CP = SHUF ? (C + 7) / 8 * 8 : C;
  static constexpr uint32_t code_bytes(int n) { return (uint32_t)n * (K / 2); }
  static constexpr uint32_t scale_bytes(int n) { return (uint32_t)n * CP; }
  __device__ static uint32_t code_v(int l) {
    return SHUF ? (uint32_t)l * 16 : (uint32_t)((l & 15) * (K / 2) + (l >> 4) * 16);
  }
  __device__ static uint32_t code_s(int rg, int s) {
    return (uint32_t)rg * 8 * K + (uint32_t)s * (SHUF ? 1024 : 64);
  }
  __device__ static uint32_t scale_v(int l) {
    return SHUF ? (uint32_t)l * 4 : (uint32_t)((l & 15) * C + (l >> 4));
  }
  __device__ static uint32_t scale_s(int rg, int s) {
    return SHUF ? (uint32_t)((((rg >> 1) * (CP / 8) + (s >> 1)) * 256) + (s & 1) * 2 + (rg & 1))
                : (uint32_t)(rg * 16 * C + 4 * s);
  }
};

__device__ inline uint32_t ld1(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b8(r, voff, soff, CP_NT);
}

// Scale loads of an n-step run of one 16-row group (steps s = 0 .. n - 1 of 128 K, the
// first at absolute step parity p0). Row-major: one byte load a step. SHUF: absolute
// steps 2i and 2i + 1 of a lane share one dword (bytes 2 (step % 2) + rg % 2), so one
// dword load serves both: it is made with the later of the two that lies in the run (the
// earlier one consumes the word before that slot is refilled), and the scale of absolute
// step a is that dword shifted right by 8 (2 (a % 2) + rg % 2); fp4_step reads the low
// byte.
template <bool SHUF, int K>
struct MxScales {
  using Op = MxOperand<SHUF, K>;
  // the slot holding run step s's scale word
  static constexpr int slot(int s, int n, int p0 = 0) {
    return SHUF && ((p0 + s) & 1) == 0 && s + 1 < n ? s + 1 : s;
  }
  // run step s loads a scale word into its own slot
  static constexpr bool loads(int s, int n, int p0 = 0) { return slot(s, n, p0) == s; }
  // scale loads of a run
  static constexpr int count(int n, int p0 = 0) {
    int c = 0;
    for (int s = 0; s < n; ++s) c += loads(s, n, p0) ? 1 : 0;
    return c;
  }
  // the scale word of absolute step a of group rg
  __device__ static uint32_t load(__amdgpu_buffer_rsrc_t r, int l, int rg, int a) {
    if constexpr (SHUF)
      return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
          r, (uint32_t)l * 4, (uint32_t)(((rg >> 1) * (Op::CP / 8) + (a >> 1)) * 256), CP_NT);
    else
      return ld1(r, Op::scale_v(l), Op::scale_s(rg, a));
  }
  // the scale of absolute step a, from the word in its slot
  __device__ static uint32_t of(uint32_t word, int rg, int a) {
    return SHUF ? word >> (8 * (2 * (a & 1) + (rg & 1))) : word;
  }
};

// acc += one 128-K step: the lane's 16 code bytes (E8M0 `code`) dequantised to bf16 and
// multiplied with the four B operands of the step (8 bf16 each, K 8 d .. of the lane's
// 32-group). The fp4 -> bf16 conversion with the power-of-two scale is exact.
__device__ inline v4f fp4_step(v4i wv, uint32_t code, const v4i (&B)[4], v4f acc) {
  const float sc = __uint_as_float((code & 0xFFu) << 23);
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t wd = (uint32_t)wv[d];
    const v2bf p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, sc, 0);
    const v2bf p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, sc, 1);
    const v2bf p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, sc, 2);
    const v2bf p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, sc, 3);
    const v8bf a = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(v8bf, B[d]), acc, 0, 0,
                                                  0);
  }
  return acc;
}

}  // namespace mono
