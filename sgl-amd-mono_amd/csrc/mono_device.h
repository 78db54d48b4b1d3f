// Device helpers shared by the gfx950 monokernel stages.
//
// Everything here is CDNA4 (gfx950) specific: wave64, the f8f6f4 matrix cores, buffer
// resources with CDNA cache-policy bits, and the 100 MHz s_memrealtime clock.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mono_amd.h"

namespace mono {

typedef int32_t v8i __attribute__((ext_vector_type(8)));
typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v2i __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));

constexpr int WAVE = 64;
constexpr float FP8_MAX = 448.0f;
constexpr float INV_FP8_MAX = 1.0f / 448.0f;

// ------------------------------------------------------------------ cache policies
// aux bits of the buffer intrinsics on gfx950: sc0 = 1, nt = 2, sc1 = 16
constexpr int CP_NONE = 0;
constexpr int CP_NT = 2;    // streamed once: weights
constexpr int CP_DEV = 16;  // device coherent (sc1): mailboxes written by other CTAs

// raw buffer resource over [base, base + bytes); loads past the end return 0
__device__ inline __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

template <int CP>
__device__ inline v4i ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CP);
}
template <int CP>
__device__ inline void st16(__amdgpu_buffer_rsrc_t r, uint32_t off, v4i v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, CP);
}
// per-lane offset `voff` (VGPR) + wave-uniform offset `soff` (SGPR)
template <int CP>
__device__ inline v4i ld16s(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, CP);
}
// a wave-uniform read through the constant address space: an s_load, counted by
// lgkmcnt, so waiting for it never waits on the vector loads in flight
template <class T>
__device__ inline T sld(const T* p, int i) {
  typedef const __attribute__((address_space(4))) T* cptr;
  return ((cptr)(p))[i];
}

// The LDS a buffer -> LDS copy (buffer_load ... lds) may write: the bytes below 128 KiB.
// gfx950 has 160 KiB of LDS, but the DMA path's LDS address (M0 plus the instruction
// offset) has 17 significant bits here: copies reaching past 128 KiB read back wrong, as
// if they had landed 128 KiB lower (over the start of the arena). Every kernel keeps its
// LDS in one arena starting at address 0 (``LdsArena``), and every copy site checks at
// compile time that its target ends at or below this bound.
constexpr int LDS_DMA_END = 128 * 1024;

// an int the compiler cannot see through (kept in a VGPR): indexing LDS from it keeps
// a load inside its loop while the constant parts fold into the instruction offset
__device__ inline int opaque_v(int v) {
  asm volatile("" : "+v"(v));
  return v;
}
// a constant vector made where it is stored: the compiler would otherwise build it once,
// ahead of the loops around the store, and hold (or spill) its registers meanwhile
__device__ inline v4i opaque_v4(int a, int b, int c, int d) {
  v4i v{a, b, c, d};
  asm volatile("" : "+v"(v));
  return v;
}
__device__ inline v2i opaque_v2(int a, int b) {
  v2i v{a, b};
  asm volatile("" : "+v"(v));
  return v;
}
template <int CP>
__device__ inline v2i ld8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, CP);
}
template <int CP>
__device__ inline int32_t ld4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CP);
}

// device-coherent (sc1) scalar-width accesses through the memory model
__device__ inline uint32_t ld_dev(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint64_t ld_dev64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_dev(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_dev64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_devf(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t add_dev(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// wait until this wave's earlier memory operations (sc1 stores included) completed
__device__ inline void drain() { __builtin_amdgcn_s_waitcnt(0); }
// s_waitcnt immediate waiting for vmcnt <= n only (gfx9 encoding: vmcnt bits 3:0 and
// 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima)
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// a complemented hand-off word: never zero once written (an all-ones word, a NaN in any
// of the float formats carried, is stored as another NaN), so zero means "not written"
__device__ inline uint32_t enc_word(uint32_t u) { return ~(u == 0xFFFFFFFFu ? 0xFFFFFFFEu : u); }

// (value, tag) pair: one 8-byte store publishes a 32-bit word with its launch tag
__device__ inline uint64_t pair(uint32_t v, uint32_t tag) {
  return (uint64_t)v | ((uint64_t)tag << 32);
}

// ------------------------------------------------------------------ wave ops
// a zero the compiler cannot see through: indexing with it keeps a load inside its loop
__device__ inline int opaque_zero() {
  int z;
  asm volatile("s_mov_b32 %0, 0" : "=s"(z));
  return z;
}

__device__ inline int lane_id() { return __lane_id(); }


// Butterfly reductions on the VALU (no LDS crossbar): DPP quad_perm pairs lanes i^1 and
// i^2, row_half_mirror i <-> 7-i and row_mirror i <-> 15-i within each row of 16 lanes,
// then v_permlane16_swap / v_permlane32_swap exchange rows. Every lane of a group ends
// with the same bits (each step combines the same two operands, commutatively).
template <int CTRL>
__device__ inline uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ inline float dpp_f(float v) {
  return __uint_as_float(dpp_u<CTRL>(__float_as_uint(v)));
}
constexpr int DPP_XOR1 = 0xB1;       // quad_perm [1, 0, 3, 2]
constexpr int DPP_XOR2 = 0x4E;       // quad_perm [2, 3, 0, 1]
constexpr int DPP_REV4 = 0x1B;       // quad_perm [3, 2, 1, 0]
constexpr int DPP_HALF_MIRROR = 0x141;
constexpr int DPP_MIRROR = 0x140;

// the partner row's value (rows of 16 lanes paired as 0-1, 2-3), or the other half
__device__ inline void swap16(float v, float& a, float& b) {
  auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  a = __uint_as_float(s[0]);
  b = __uint_as_float(s[1]);
}
__device__ inline void swap32(float v, float& a, float& b) {
  auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  a = __uint_as_float(s[0]);
  b = __uint_as_float(s[1]);
}

// reduction over each row of 16 lanes
template <class Op>
__device__ inline float red16(float v, Op op) {
  v = op(v, dpp_f<DPP_XOR1>(v));
  v = op(v, dpp_f<DPP_XOR2>(v));
  v = op(v, dpp_f<DPP_HALF_MIRROR>(v));
  v = op(v, dpp_f<DPP_MIRROR>(v));
  return v;
}
// reduction over the wave
template <class Op>
__device__ inline float red64(float v, Op op) {
  v = red16(v, op);
  float a, b;
  swap16(v, a, b);
  v = op(a, b);
  swap32(v, a, b);
  return op(a, b);
}
struct OpAdd {
  __device__ float operator()(float a, float b) const { return a + b; }
};
struct OpMax {
  __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
__device__ inline float wave_sum(float v) { return red64(v, OpAdd()); }
__device__ inline float wave_max(float v) { return red64(v, OpMax()); }
__device__ inline float row16_max(float v) { return red16(v, OpMax()); }

// maximum of a u32 over the wave (every lane ends with it)
__device__ inline uint32_t wave_max_u32(uint32_t v) {
  auto mx = [](uint32_t a, uint32_t b) { return a > b ? a : b; };
  v = mx(v, dpp_u<DPP_XOR1>(v));
  v = mx(v, dpp_u<DPP_XOR2>(v));
  v = mx(v, dpp_u<DPP_HALF_MIRROR>(v));
  v = mx(v, dpp_u<DPP_MIRROR>(v));
  auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = mx(a[0], a[1]);
  auto c = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return mx(c[0], c[1]);
}

// minimum of a u32 over the wave (every lane ends with it)
__device__ inline uint32_t wave_min_u32(uint32_t v) {
  auto mn = [](uint32_t a, uint32_t b) { return a < b ? a : b; };
  v = mn(v, dpp_u<DPP_XOR1>(v));
  v = mn(v, dpp_u<DPP_XOR2>(v));
  v = mn(v, dpp_u<DPP_HALF_MIRROR>(v));
  v = mn(v, dpp_u<DPP_MIRROR>(v));
  auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = mn(a[0], a[1]);
  auto c = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return mn(c[0], c[1]);
}

// ------------------------------------------------------------------ number formats
// f32 -> bf16 bits, round to nearest even (finite inputs)
__device__ inline uint32_t bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ inline float bf16_round(float f) { return __uint_as_float(bf16_bits(f) << 16); }
__device__ inline float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// 4 f32 (already within +-448) -> 4 E4M3 bytes in one dword, round to nearest even
__device__ inline uint32_t pack_fp8x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}
// E4M3 byte pair (low or high 16 bits of w) -> 2 f32, exact
__device__ inline v2f fp8x2_lo(uint32_t w) { return __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false); }
__device__ inline v2f fp8x2_hi(uint32_t w) { return __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true); }

__device__ inline float clamp_fp8(float v) { return __builtin_amdgcn_fmed3f(v, -FP8_MAX, FP8_MAX); }

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
// two f32 -> two bf16 (lo in bits 0-15), round to nearest even: one v_cvt_pk_bf16_f32,
// equal to bf16_bits on every non-NaN input (denormals included)
__device__ inline uint32_t bf16x2_bits(float lo, float hi) {
  const v2f f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, v2bf));
}
// acc + w.lo^2 + w.hi^2 for a bf16 pair w, by v_dot2c_f32_bf16
__device__ inline float dot2_bf16_sq(uint32_t w, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, w), __builtin_bit_cast(v2bf, w),
                                        acc, false);
}
// The squares of 16 bf16 values (lo: values 0-7, hi: 8-15, two a dword, the low half
// first) summed as a balanced pairwise tree: each adjacent pair (a dword) by
// v_dot2c_f32_bf16 with a zero accumulator, then ((p0 + p1) + (p2 + p3)) + ... The same
// bits as `pair_sq_tree` summing one value a lane over a 16-lane row (the dot2 rounds a
// pair's sum once, which two separately rounded squares do not match when a square is
// denormal, so both forms take the pair through it).
__device__ inline float sq_tree16(v4i lo, v4i hi) {
  float s[8];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    s[q] = dot2_bf16_sq((uint32_t)lo[q], 0.f);
    s[4 + q] = dot2_bf16_sq((uint32_t)hi[q], 0.f);
  }
#pragma unroll
  for (int n = 4; n >= 1; n /= 2)
#pragma unroll
    for (int k = 0; k < n; ++k) s[k] = s[2 * k] + s[2 * k + 1];
  return s[0];
}
// One bf16 value a lane (bits h, low half), a 16-lane row holding 16 consecutive values:
// the sum of their squares in `sq_tree16`'s order and bits (lanes 2k, 2k + 1 form the
// pair's dword, low half first, for v_dot2c_f32_bf16; then the butterfly over the
// pairs). `live` (uniform over the row): false gives the row zero. Every lane of the
// row ends with its sum; call from every lane of the wave.
__device__ inline float pair_sq_tree(uint32_t h, bool live) {
  h &= 0xFFFFu;
  const uint32_t hn = dpp_u<DPP_XOR1>(h);
  const uint32_t w = (lane_id() & 1) ? (hn | (h << 16)) : (h | (hn << 16));
  float v = live ? dot2_bf16_sq(w, 0.f) : 0.f;
  v += dpp_f<DPP_XOR2>(v);
  v += dpp_f<DPP_HALF_MIRROR>(v);
  v += dpp_f<DPP_MIRROR>(v);
  return v;
}
// acc + bf16(a) * w.lo + bf16(b) * w.hi, with a, b rounded to bf16 (nearest even) by
// v_cvt_pk_bf16_f32 and the products summed by v_dot2c_f32_bf16
__device__ inline float dot2_bf16(float a, float b, uint32_t w, float acc) {
  const v2f f = {a, b};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_convertvector(f, v2bf),
                                        __builtin_bit_cast(v2bf, w), acc, false);
}

// radix order key of f32 bits: larger key ranks first (+0 above -0)
__device__ inline uint32_t radix_key(float f) {
  uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b ^ 0x80000000u);
}

// ------------------------------------------------------------------ matrix cores
// 16x16x128 E4M3 x E4M3 -> f32 (the scaled form at unit E8M0 scales). Lane l holds
// row l % 16 of A (column l % 16 of B) and 32 K values of group l / 16; D lane l
// holds rows 4 (l / 16) + v, column l % 16.
__device__ inline v4f mfma_fp8(v8i a, v8i b, v4f c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}
// 16x16x128 E2M1 x E2M1 with E8M0 scales per 32 K (lane l: row/column l % 16, K
// group l / 16); only the low 4 dwords of a and b carry data
__device__ inline v4f mfma_fp4_scaled(v8i a, v8i b, v4f c, int sa, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 4, 4, 0, sa, 0, sb);
}

// ------------------------------------------------------------------ guard
// The guard block (int32 words, runtime owned): see mono_amd.h MONO_GUARD_*.
// Every field is CTA-uniform and kept in scalar registers (the LDS-read ones through
// readfirstlane): vector registers held for the whole launch would crowd every phase.
struct Guard {
  int32_t* words;
  uint32_t* host_err;  // pinned host mirror of the first error (may be null)
  uint64_t deadline;   // ticks of the 100 MHz clock
  int fault_site;      // test fault injection: this wait site never completes
  uint64_t slack;      // deadline multiple of the other waits while a fault is injected

  // `head` = guard words 0-3 as read once by the CTA (one coherent load, shared in LDS:
  // every thread reading the block itself would pile thousands of requests on one line)
  __device__ void init(int32_t* w, uint32_t* he, int fsite, const uint32_t* head, uint32_t fafter) {
    words = w;
    host_err = he;
    const uint32_t epoch = __builtin_amdgcn_readfirstlane(head[MONO_GUARD_EPOCH]);
    deadline = ((uint64_t)__builtin_amdgcn_readfirstlane(head[MONO_GUARD_DEADLINE_HI]) << 32) |
               __builtin_amdgcn_readfirstlane(head[MONO_GUARD_DEADLINE_LO]);
    // a block nobody set a deadline on (the library's static block starts zeroed): 10 s
    if (deadline == 0) deadline = 10ull * MONO_CLOCK_HZ;
    fault_site = (fsite > 0 && epoch >= fafter) ? fsite : 0;
    // the injected wait times out first: waits downstream of it (which stall as a
    // consequence) get four times as long, so the error word names the injected site
    slack = fault_site ? 4 : 1;
  }
  __device__ bool aborted() const {
    return ld_dev(reinterpret_cast<uint32_t*>(words) + MONO_GUARD_ABORT) != 0;
  }
  // a wait at `site` passed its deadline: record 1 + site (first failure sticks),
  // raise the abort flag every other wait checks, mirror the word to the host
  // (its stored constants are made here, opaque: hoisted to the launch's top they would
  // hold registers through every phase for a path that runs at most once)
  __device__ void fail(int site) {
    uint32_t* w = reinterpret_cast<uint32_t*>(words);
    uint32_t expect = (uint32_t)opaque_v(0);
    const uint32_t one = (uint32_t)opaque_v(1), code = (uint32_t)opaque_v(site + 1);
    __hip_atomic_compare_exchange_strong(w + MONO_GUARD_ERR_DEADLINE, &expect, code,
                                         __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    int fs = fault_site;
    asm volatile("" : "+s"(fs));
    if (fs) st_dev(w + MONO_GUARD_ERR_FAULT, one);
    st_dev(w + MONO_GUARD_ABORT, one);
    if (host_err)
      __hip_atomic_store(host_err, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    drain();
  }
};

// timeline stamp: thread 0 of the CTA writes the 100 MHz clock at mark k
__device__ inline void stamp(uint64_t* tl, int k) {
  if (tl && threadIdx.x == 0) tl[blockIdx.x * MONO_TL_COLS + k] = wall_clock64();
}

// CTA-uniform success: false if any thread of the CTA failed or the launch aborted.
// Call from every thread (three barriers); `ok_s` is a __shared__ int.
__device__ inline bool cta_ok(bool mine, Guard& g, int& ok_s) {
  __syncthreads();
  if (threadIdx.x == 0) ok_s = g.aborted() ? 0 : 1;
  __syncthreads();
  if (!mine) ok_s = 0;
  __syncthreads();
  return ok_s != 0;
}

// CTA-uniform AND of the threads' flags, without reading the global abort flag
__device__ inline bool cta_all(bool mine, int& ok_s) {
  __syncthreads();
  if (threadIdx.x == 0) ok_s = 1;
  __syncthreads();
  if (!mine) ok_s = 0;
  __syncthreads();
  return ok_s != 0;
}

// Poll `ready()` (wave-uniform result expected) until true, sleeping SLEEP x 64 clocks
// between polls. Every 64 polls: check the abort flag and the deadline. Returns false if
// the launch is failing; the caller then skips its remaining work so every wave still
// reaches the end of the kernel.
template <int SLEEP = 1, class F>
__device__ inline bool wait_until(Guard& g, int site, F ready) {
  const bool stalled = (site == g.fault_site);
  uint32_t polls = 0;
  uint64_t start = 0;
  while (true) {
    if (!stalled && ready()) return true;
    if ((++polls & 63) == 0) {
      if (g.aborted()) return false;
      uint64_t now = wall_clock64();
      if (start == 0) start = now;
      if (now - start > (stalled ? g.deadline : g.deadline * g.slack)) {
        g.fail(site);
        return false;
      }
    }
    __builtin_amdgcn_s_sleep(SLEEP);
  }
}

}  // namespace mono
