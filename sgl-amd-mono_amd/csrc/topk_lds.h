// Exact top-k selection of one row in one CTA's LDS (the attention launch's stage 2).
// Rule (sgl_amd_mono/glm53/gfx950/kernel.py:3002-3636; glm53/check.py:94-117): rank by
// the radix order key of the f32 score bits, larger first, ties to the lower position;
// the selection in ascending position order.
//
// A row of up to AT_TKBLOCK keys is ranked by one CTA: from its chunks' candidate lists
// (chunk_list, topk_lists) when they decide it, else from every score (topk_select). Every
// key a chunk leaves out lies below its cut; when every cut lies at or below the low edge
// of the final bin of the lists' ranking, every key left out ranks below every selected
// one, so the lists' selection is the row's. A longer row is cut
// into blocks of AT_TKBLOCK keys, each ranked by a CTA of its own; since every element of
// the row's top-TOPK is in its own block's top-TOPK (fewer than TOPK elements of the row,
// so of the block, rank above it), one more CTA ranks the blocks' selections (topk_final)
// and its result is exactly the row's.
#pragma once

#include <type_traits>

#include "mono_device.h"

namespace mono {

constexpr int AT_TOPK = 2048;
constexpr int AT_TKBLOCK = 32768;  // keys one CTA ranks (its LDS image): a block
constexpr int AT_MAXBLK = 5;       // blocks a row may span
constexpr int AT_MAXCTX = AT_TKBLOCK * AT_MAXBLK;  // keys a row may see: 163840
constexpr int AT_THREADS = 1024;
constexpr int AT_WAVES = AT_THREADS / WAVE;
constexpr int CAND = 256;  // a threshold bin this small is ranked directly
// a scored chunk of AT_THREADS keys lists its candidates for the row's top-TOPK: at most
// TK_LIST, at least TK_LIST_MIN where one histogram pass can cut there
constexpr int TK_LIST = 256;
constexpr int TK_LIST_MIN = 128;
constexpr int TK_NLIST = AT_TKBLOCK / AT_THREADS;  // chunks of a one-block row
// LDS words topk_select needs: the padded key image, then the histogram
constexpr int TOPK_ARENA_WORDS = AT_THREADS * 33 + 4096;

// inclusive prefix sum over the wave: DPP row shifts scan each row of 16 lanes, then
// the row totals (read from lanes 15, 31, 47) are added to the rows above them
__device__ inline int wave_scan(int v) {
  auto shr = [](int x, auto ctrl_c) {
    constexpr int CTRL = decltype(ctrl_c)::value;
    return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, true);
  };
  v += shr(v, std::integral_constant<int, 0x111>());  // row_shr:1
  v += shr(v, std::integral_constant<int, 0x112>());  // row_shr:2
  v += shr(v, std::integral_constant<int, 0x114>());  // row_shr:4
  v += shr(v, std::integral_constant<int, 0x118>());  // row_shr:8
  const int r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31),
            r2 = __builtin_amdgcn_readlane(v, 47);
  const int row = lane_id() >> 4;
  return v + (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
}

// exclusive prefix sum over the CTA's 1024 threads. `wsum` is 2 x 16 ints of LDS (16-byte
// aligned) used alternately by successive calls (`phase` flips), so one barrier suffices:
// a call's buffer is not rewritten until the call after next, behind the next barrier.
__device__ inline int block_scan(int v, int* wsum, int& phase, int& total) {
  const int l = lane_id(), w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int* buf = wsum + AT_WAVES * phase;
  phase ^= 1;
  const int x = wave_scan(v);
  if (l == WAVE - 1) buf[w] = x;
  __syncthreads();
  const v4i* ws = reinterpret_cast<const v4i*>(buf);
  const v4i a = ws[0], b = ws[1], c = ws[2], d = ws[3];
  const int s[16] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3],
                     c[0], c[1], c[2], c[3], d[0], d[1], d[2], d[3]};
  int pre = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < AT_WAVES; ++i) {
    pre += i < w ? s[i] : 0;
    tot += s[i];
  }
  total = tot;
  return pre + x - v;
}

// (hist must be zero on entry; select_pass leaves it zero)
template <int NK>
__device__ inline void select_pass(int tid, const uint32_t (&key)[NK], uint32_t lo, uint32_t hi,
                                   int shift, int kk, uint32_t* hist, int* wsum, int& phase,
                                   int* res) {
  constexpr int NB = 4096;
#pragma unroll
  for (int j = 0; j < NK; ++j) {
    const uint32_t k = key[j];
    if (k >= lo && k <= hi) atomicAdd(&hist[(k - lo) >> shift], 1u);
  }
  __syncthreads();
  // thread t owns bins [NB - 4 (t + 1), NB - 4 t): the scan runs from the top bin down;
  // the thread clears its bins once read (no other thread reads them)
  constexpr int G = NB / AT_THREADS;
  v4i* mine = reinterpret_cast<v4i*>(hist + NB - G * (tid + 1));
  const v4i h4 = *mine;
  *mine = opaque_v4(0, 0, 0, 0);
  const int s = h4[0] + h4[1] + h4[2] + h4[3];
  int tot;
  const int pre = block_scan(s, wsum, phase, tot);
  if (tid == 0) res[3] = tot;
  if (pre < kk && kk <= pre + s) {
    int cum = pre;
#pragma unroll
    for (int g = G - 1; g >= 0; --g) {
      const int c = h4[g];
      if (cum < kk && kk <= cum + c) {
        res[0] = NB - G * (tid + 1) + g;
        res[1] = cum;
        res[2] = c;
      }
      cum += c;
    }
  }
  __syncthreads();
}

// The selection from keys held in registers, NK (<= 32) a thread, thread order then index
// order being position order (pos_of(j) gives the position of key[j]). `cnt` keys lie in
// [lo, hi]; the first pass bins [plo0, hi] and, with `check0`, is redone over [lo, hi] if
// that range holds fewer than TOPK keys. Histogram passes (4096 bins) keep the bin holding
// the TOPK-th key until it holds few keys or one key value. The selection is every key
// above that bin plus the first kk of the bin's keys in (key descending, position
// ascending) order: few candidates rank themselves, one shared value takes its first kk
// positions. A thread's picks are a 32-bit mask; the scan of the pick counts places them,
// in ascending position order, at sel[0 .. TOPK). `hist` (4096 words, zero on entry) holds
// the passes' bins, then the candidates and the masks of the candidates' owners.
// With `floor_out`, thread 0 stores there the low edge of the final bin: no selected key
// lies below it.
template <int NK, class PosF>
__device__ inline void topk_refine(int tid, const uint32_t (&key)[NK], PosF pos_of, uint32_t lo,
                                   uint32_t hi, int cnt, uint32_t plo0, bool check0,
                                   uint32_t* hist, int* wsum, int& phase, int* res_s,
                                   int32_t* sel, uint32_t* floor_out = nullptr) {
  static_assert(NK <= 32, "a thread's picks fit one 32-bit mask");
  uint32_t* ck = hist;                                       // candidates, after the passes
  int32_t* cp = reinterpret_cast<int32_t*>(hist + CAND);     // their positions
  uint32_t* co = hist + 2 * CAND;                            // their (thread, index)
  uint32_t* pmask = hist + 3 * CAND;                         // [AT_THREADS] picked candidates
  static_assert(3 * CAND + AT_THREADS <= 4096, "candidates and masks fit the histogram");
  int kk = AT_TOPK, shift = 1;
#pragma unroll 1
  for (int pass = 0; shift > 0 && cnt > CAND; ++pass) {
    const uint32_t plo = pass == 0 ? plo0 : lo;
    const uint32_t span = hi - plo;
    const int bits = span ? 32 - __clz((int)span) : 0;
    shift = bits > 12 ? bits - 12 : 0;
    select_pass<NK>(tid, key, plo, hi, shift, kk, hist, wsum, phase, res_s);
    if (check0 && pass == 0 && res_s[3] < AT_TOPK) {  // the first range holds too few keys
      shift = 1;
      continue;
    }
    const uint32_t bin = (uint32_t)res_s[0];
    kk -= res_s[1];
    cnt = res_s[2];
    const uint32_t nlo = plo + (bin << shift);
    const uint64_t top = (uint64_t)nlo + ((1ull << shift) - 1ull);
    hi = top < (uint64_t)hi ? (uint32_t)top : hi;
    lo = nlo;
  }
  // every wave has read the last pass's results before res_s[0] is reused; the passes left
  // the histogram (masks included) zero
  __syncthreads();
  if (tid == 0) {
    res_s[0] = 0;
    if (floor_out) *floor_out = lo;
  }
  __syncthreads();
  // bit j: key[j] is selected. Masks are built a shift at a time from the top bit down:
  // a constant 1 << j would be a literal each, which gfx9's VOP3 forms cannot encode, so
  // the compiler would hold them in registers through the stage.
  uint32_t pick = 0;
#pragma unroll
  for (int j = NK - 1; j >= 0; --j) pick = (pick << 1) | (uint32_t)(key[j] > hi);
  if (cnt <= CAND) {
    // the bin's candidates gathered in one pass
#pragma unroll
    for (int j = 0; j < NK; ++j) {
      if (key[j] >= lo && key[j] <= hi) {
        const int at = atomicAdd(&res_s[0], 1);
        ck[at] = key[j];
        cp[at] = pos_of(j);
        co[at] = ((uint32_t)tid << 5) | (uint32_t)j;
      }
    }
    __syncthreads();
    // each candidate finds its rank among them; the first kk are picked
    if (tid < cnt) {
      const uint32_t mk = ck[tid];
      const int mp = cp[tid];
      int rank = 0;
      for (int m = 0; m < cnt; ++m) rank += (ck[m] > mk) | ((ck[m] == mk) & (cp[m] < mp));
      if (rank < kk) {
        const uint32_t o = co[tid];
        atomicOr(&pmask[o >> 5], 1u << (o & 31u));
      }
    }
  } else {
    // one key value (lo == hi) shared by many positions: the first kk of them
    int c = 0;
#pragma unroll
    for (int j = 0; j < NK; ++j) c += key[j] == lo;
    int tot;
    int seen = block_scan(c, wsum, phase, tot);
    // the tied keys taken, in index order (seen counts them), then their mask top down
    bool take[NK];
#pragma unroll
    for (int j = 0; j < NK; ++j) {
      const bool e = key[j] == lo;
      take[j] = e && seen < kk;
      seen += e;
    }
    uint32_t tmask = 0;
#pragma unroll
    for (int j = NK - 1; j >= 0; --j) tmask = (tmask << 1) | (uint32_t)take[j];
    pick |= tmask;
  }
  __syncthreads();
  pick |= pmask[tid];
  int tot;
  int at = block_scan(__popc(pick), wsum, phase, tot);
  // the picks in position order: only the set bits are visited
  for (uint32_t m = pick; m; m &= m - 1u) sel[at++] = pos_of(__builtin_ctz(m));
  __syncthreads();
}

// The exact top-TOPK of one block's n scores (TOPK < n <= AT_TKBLOCK), in LDS: returns the
// selected positions in ascending order (sel[0 .. TOPK)). Ranked by the radix key of
// the f32 score, larger first, ties to the lower position. `rs` covers the n scores (f32,
// read through L2: the caller has seen their done words, and within the launch the
// scores are only stored, write-through, before them, so no L2 holds a stale copy);
// `arena` holds TOPK_ARENA_WORDS words. Every thread of the
// CTA calls it. With `ts` non-null, thread 0 records the shader clock after each step.
//
// Thread t keeps the keys of positions 32 t .. 32 t + 31 in registers (loaded through a
// padded LDS image, 33 words a thread, so both the coalesced writes and the per-thread
// reads are conflict-free). A sample (every 32nd position) narrows the key range to one
// holding about 1.5 TOPK keys, where topk_refine's first pass starts.
// Always inlined: called from more than one kernel, it would otherwise become a real call
// (registers saved through scratch around it, no scheduling across it), which measured
// ~4 us slower a row.
__device__ __attribute__((always_inline)) inline int32_t* topk_select(
    int tid, __amdgpu_buffer_rsrc_t rs, int n, uint8_t* arena, int* wsum, uint32_t* mm,
    int* res_s, uint64_t* ts = nullptr) {
  int phase = 0;
  auto mark = [&](int k) {
    if (ts && tid == 0) ts[k] = __builtin_amdgcn_s_memtime();
  };
  mark(0);
  uint32_t* kl = reinterpret_cast<uint32_t*>(arena);  // [1024][33] image
  uint32_t* hist = kl + AT_THREADS * 33;               // [4096]; candidates after the passes
  // [TOPK], past the candidates and masks of topk_refine (dead when it is written)
  int32_t* sel = reinterpret_cast<int32_t*>(hist + 3 * CAND + AT_THREADS);
  static_assert(3 * CAND + AT_THREADS + AT_TOPK <= 4096, "the selection fits the histogram");
  constexpr int NLD = AT_TKBLOCK / 4 / AT_THREADS;
  v4i raw[NLD];
#pragma unroll
  for (int q = 0; q < NLD; ++q) raw[q] = ld16<CP_NONE>(rs, (uint32_t)(4 * (tid + AT_THREADS * q)) * 4);
  reinterpret_cast<v4i*>(hist)[tid] = opaque_v4(0, 0, 0, 0);  // select_pass expects it zero
  // a position past the row holds key 0, below every real key (a score keeps key >= 1:
  // only the all-ones NaN would map to 0, and it ranks next to it)
  uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
#pragma unroll
  for (int q = 0; q < NLD; ++q) {
    const int i = 4 * (tid + AT_THREADS * q);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint32_t k = radix_key(__int_as_float(raw[q][e]));
      k = i + e < n ? (k > 1u ? k : 1u) : 0u;
      kl[((i + e) >> 5) * 33 + ((i + e) & 31)] = k;
      kmin = (k && k < kmin) ? k : kmin;
      kmax = k > kmax ? k : kmax;
    }
  }
  // the CTA's minimum and maximum key: a wave reduction, then one LDS atomic a wave into
  // mm[0], mm[1] (set to ~0 and 0 by the caller before its last barrier)
  kmax = wave_max_u32(kmax);
  kmin = ~wave_max_u32(~kmin);
  if ((tid & (WAVE - 1)) == 0) {
    atomicMin(&mm[0], kmin);
    atomicMax(&mm[1], kmax);
  }
  __syncthreads();
  uint32_t key[32];
#pragma unroll
  for (int j = 0; j < 32; ++j) key[j] = kl[33 * tid + j];
  kmin = mm[0];
  kmax = mm[1];
  mark(1);
  mark(2);
  // Sample the range first: position 32 t is thread t's sample. The bin of the sample
  // ranked SR from the top bounds a range [cut, kmax] expected to hold about 1.5 TOPK
  // keys; if it holds fewer than TOPK the first pass is redone over the whole range.
  uint32_t cut = kmin;
  bool sampled = false;
  {
    const int ns = (n + 31) / 32;
    const int sr = (3 * AT_TOPK * ns + 2 * n - 1) / (2 * n);
    if (sr >= 1 && sr <= ns) {
      const uint32_t span = kmax - kmin;
      const int bits = span ? 32 - __clz((int)span) : 0;
      const int sh = bits > 12 ? bits - 12 : 0;
      const uint32_t one[1] = {key[0]};
      select_pass<1>(tid, one, kmin, kmax, sh, sr, hist, wsum, phase, res_s);
      cut = kmin + ((uint32_t)res_s[0] << sh);
      sampled = true;
    }
  }
  mark(3);
  topk_refine<32>(tid, key, [&](int j) { return 32 * tid + j; }, kmin, kmax, n, cut, sampled,
                  hist, wsum, phase, res_s, sel);
  mark(7);
  return sel;
}

// After topk_select: the order key it ranked block position `pos` by (its LDS image)
__device__ inline uint32_t topk_key_at(const uint8_t* arena, int pos) {
  return reinterpret_cast<const uint32_t*>(arena)[(pos >> 5) * 33 + (pos & 31)];
}

// The exact top-TOPK of a row that spans several blocks, from the C candidates of its
// blocks' selections: `rc` covers them as u64 (position | order key << 32), block after
// block and each block's in ascending position order, so the whole list is in ascending
// position order. Thread t holds candidates NK t .. NK t + NK - 1 (past C: key 0, below
// every real key, which is >= 1); topk_refine ranks them as topk_select ranks a block.
// Their positions wait in LDS past the histogram (a register array indexed at run time
// would live in scratch memory). `mm` is set to ~0 and 0 by the caller before its last
// barrier. Returns the selected positions of the row, ascending, at sel[0 .. TOPK).
template <int NK>
__device__ __attribute__((always_inline)) inline int32_t* topk_final(
    int tid, __amdgpu_buffer_rsrc_t rc, int C, uint8_t* arena, int* wsum, uint32_t* mm,
    int* res_s) {
  static_assert(NK * AT_THREADS >= AT_MAXBLK * AT_TOPK, "every candidate has a thread");
  int phase = 0;
  uint32_t* hist = reinterpret_cast<uint32_t*>(arena);
  int32_t* sel = reinterpret_cast<int32_t*>(hist + 3 * CAND + AT_THREADS);
  int32_t* cpos = reinterpret_cast<int32_t*>(hist + 4096);  // [NK x 1024]
  static_assert((4096 + NK * AT_THREADS) * 4 <= TOPK_ARENA_WORDS * 4, "positions fit the arena");
  v2i raw[NK];
#pragma unroll
  for (int j = 0; j < NK; ++j) raw[j] = ld8<CP_DEV>(rc, (uint32_t)(NK * tid + j) * 8u);
  reinterpret_cast<v4i*>(hist)[tid] = opaque_v4(0, 0, 0, 0);  // select_pass expects it zero
  uint32_t key[NK];
  uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
#pragma unroll
  for (int j = 0; j < NK; ++j) {
    cpos[NK * tid + j] = raw[j][0];
    const uint32_t k = NK * tid + j < C ? (uint32_t)raw[j][1] : 0u;
    key[j] = k;
    kmin = (k && k < kmin) ? k : kmin;
    kmax = k > kmax ? k : kmax;
  }
  kmax = wave_max_u32(kmax);
  kmin = ~wave_max_u32(~kmin);
  if ((tid & (WAVE - 1)) == 0) {
    atomicMin(&mm[0], kmin);
    atomicMax(&mm[1], kmax);
  }
  __syncthreads();
  kmin = mm[0];
  kmax = mm[1];
  topk_refine<NK>(tid, key, [&](int j) { return cpos[NK * tid + j]; }, kmin, kmax, C, kmin,
                  false, hist, wsum, phase, res_s, sel);
  return sel;
}

// One chunk of a row (thread t: the chunk's position t, its order key k; 0: no key) lists
// its candidates for the row's top-TOPK: every key at or above a cut, in ascending position
// order, as u64 (row position | key << 32) at out[0 .. TK_LIST) through `rout` (the tail
// zeroed). The cut comes from 256-bin histograms, each scanned by wave 0 from the top: the
// low edge of the bin holding the TK_LIST_MIN-th key when that lists at most TK_LIST keys,
// else a finer pass inside that bin, down to single key values (then just above the
// value: fewer keys). A chunk of at most TK_LIST keys lists them all (cut 1). Returns the
// cut: every key of the chunk below it is left out. `mm` (4 words) is set to ~0, 0, 0, 0
// and `hist` (256 words) to zero by the caller before its last barrier; `wsum` holds 16
// words. No __syncthreads_count (it reads the dispatch packet, so it waits for every
// memory access in flight).
__device__ inline uint32_t chunk_list(int tid, uint32_t k, int pos0, uint32_t* hist, int* wsum,
                                      uint32_t* mm, __amdgpu_buffer_rsrc_t rout) {
  const int l = tid & (WAVE - 1), w = tid >> 6;
  const uint32_t kmx = wave_max_u32(k), kmn = ~wave_max_u32(k ? ~k : 0u);
  const int wv = __popcll(__ballot(k != 0u));
  if (l == 0) {
    atomicMin(&mm[0], kmn);
    atomicMax(&mm[1], kmx);
    atomicAdd(&mm[3], (uint32_t)wv);
  }
  __syncthreads();
  const int nv = (int)mm[3];
  const uint32_t lo = mm[0], hi = mm[1];
  uint32_t cut = 1u;
  if (nv > TK_LIST) {  // CTA-uniform
    // passes of 256 bins over [rlo, rhi], `above` keys above it, until the bin holding the
    // TK_LIST_MIN-th key lists at most TK_LIST keys or is one key value wide: then the cut
    // is its low edge, or just above it. The state crosses the barriers in mm (every
    // thread read mm after the first barrier; wave 0 rewrites it after the next one).
    uint32_t rlo = lo, rhi = hi;
    int above0 = 0;
    const uint32_t span = hi - lo;
    const int bits = span ? 32 - __clz((int)span) : 0;
    int sh = bits > 8 ? bits - 8 : 0;
#pragma unroll 1
    for (;;) {
      if (k >= rlo && k <= rhi) atomicAdd(&hist[(k - rlo) >> sh], 1u);
      __syncthreads();
      if (w == 0) {
        // lane l: bins 255 - 4 l .. 252 - 4 l (from the top), then an inclusive scan
        const v4i h4 = reinterpret_cast<const v4i*>(hist)[63 - l];
        reinterpret_cast<v4i*>(hist)[63 - l] = opaque_v4(0, 0, 0, 0);
        const int c4 = h4[0] + h4[1] + h4[2] + h4[3];
        int above = above0 + wave_scan(c4) - c4;  // keys above the lane's four bins
        int bin = -1, ab = 0, nb = 0;
#pragma unroll
        for (int g = 3; g >= 0; --g) {
          const int n_b = h4[g];
          if (bin < 0 && above < TK_LIST_MIN && TK_LIST_MIN <= above + n_b) {
            bin = 4 * (63 - l) + g;
            ab = above;
            nb = n_b;
          }
          above += n_b;
        }
        // one lane finds it (the range holds the TK_LIST_MIN-th key)
        const uint64_t fb = __ballot(bin >= 0);
        const int src = fb ? (int)__ffsll((long long)fb) - 1 : 0;
        const int fbin = __builtin_amdgcn_readlane(bin, src);
        const int fab = __builtin_amdgcn_readlane(ab, src), fnb = __builtin_amdgcn_readlane(nb, src);
        if (l == 0) {
          const uint64_t edge = (uint64_t)rlo + ((uint64_t)(uint32_t)fbin << sh);
          uint32_t st = 1u;  // bit 0: done
          if (!fb) {
            mm[2] = 0xFFFFFFFFu;
          } else if (fab + fnb <= TK_LIST) {
            mm[2] = (uint32_t)edge;
          } else if (sh == 0) {
            mm[2] = edge + 1ull > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)(edge + 1ull);
          } else {  // refine inside the bin
            const uint64_t top = edge + (1ull << sh) - 1ull;
            mm[0] = (uint32_t)edge;
            mm[1] = top > (uint64_t)rhi ? rhi : (uint32_t)top;
            st = (uint32_t)fab << 1;
          }
          mm[3] = st;
        }
      }
      __syncthreads();
      const uint32_t st = mm[3];
      if (st & 1u) break;
      rlo = mm[0];
      rhi = mm[1];
      above0 = (int)(st >> 1);
      sh = sh > 8 ? sh - 8 : 0;
    }
    cut = mm[2];
  }
  // ascending position order: the wave's prefix by ballot, the waves' totals through LDS
  const bool on = k != 0u && k >= cut;
  const uint64_t bal = __ballot(on);
  const int pre = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
  if (l == 0) wsum[w] = __popcll(bal);
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < AT_WAVES; ++i) {
    const int v = wsum[i];
    base += i < w ? v : 0;
    tot += v;
  }
  if (on)
    __builtin_amdgcn_raw_buffer_store_b64(v2i{pos0 + tid, (int32_t)k}, rout,
                                          (uint32_t)(base + pre) * 8u, 0, CP_DEV);
  if (tid >= tot && tid < TK_LIST)
    __builtin_amdgcn_raw_buffer_store_b64(opaque_v2(0, 0), rout, (uint32_t)tid * 8u, 0, CP_DEV);
  return cut;
}

// The exact top-TOPK of a one-block row from its nch chunks' lists (chunk_list), or nullptr
// when the lists cannot decide it. `rl` covers the lists ([nch][TK_LIST] u64, read through
// L2 like the scores), `rcut` the chunks' cuts. Thread t holds entries 8 t .. 8 t + 7 (of
// chunk t / 32), so the candidates run in ascending position order; their positions wait
// in LDS past the histogram. Wave w first waits for its chunks 2 w and 2 w + 1 (`wait`:
// wave-uniform, false when the launch fails, then `ok` turns false CTA-wide and it
// returns nullptr), so the loads of chunks already done are in flight while later ones
// are still being scored. The lists decide the selection when they hold at least TOPK
// keys and no chunk's cut lies above the final bin's low edge: every key a chunk left out
// then ranks below every selected key. `mm` (4 words) is set to ~0, 0, 0, 0 by the caller
// before its last barrier. Returns the selected positions, ascending, at sel[0 .. TOPK).
template <class WaitChunks>
__device__ __attribute__((always_inline)) inline int32_t* topk_lists(
    int tid, __amdgpu_buffer_rsrc_t rl, __amdgpu_buffer_rsrc_t rcut, int nch, uint8_t* arena,
    int* wsum, uint32_t* mm, int* res_s, WaitChunks wait, bool& ok) {
  constexpr int NK = TK_NLIST * TK_LIST / AT_THREADS;
  static_assert(NK * AT_THREADS == TK_NLIST * TK_LIST && TK_LIST % NK == 0, "list map");
  int phase = 0;
  uint32_t* hist = reinterpret_cast<uint32_t*>(arena);
  int32_t* sel = reinterpret_cast<int32_t*>(hist + 3 * CAND + AT_THREADS);
  int32_t* cpos = reinterpret_cast<int32_t*>(hist + 4096);  // [NK x 1024]
  static_assert((4096 + NK * AT_THREADS) * 4 <= TOPK_ARENA_WORDS * 4, "positions fit the arena");
  const int ch = tid / (TK_LIST / NK);
  static_assert(WAVE / (TK_LIST / NK) == 2, "two chunks a wave");
  const int w2 = 2 * (tid >> 6);
  if (!wait(w2, w2 + 1) && (tid & (WAVE - 1)) == 0) atomicOr(&mm[2], 2u);
  v2i raw[NK];
#pragma unroll
  for (int j = 0; j < NK; ++j) raw[j] = ld8<CP_NONE>(rl, (uint32_t)(NK * tid + j) * 8u);
  const uint32_t mycut =
      (uint32_t)ld4<CP_NONE>(rcut, ch < nch && tid % (TK_LIST / NK) == 0 ? (uint32_t)ch * 4u
                                                                          : 0x80000000u);
  reinterpret_cast<v4i*>(hist)[tid] = opaque_v4(0, 0, 0, 0);  // select_pass expects it zero
  uint32_t key[NK];
  uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
  int cnt = 0;
#pragma unroll
  for (int j = 0; j < NK; ++j) {
    cpos[NK * tid + j] = raw[j][0];
    const uint32_t k = (uint32_t)raw[j][1];
    key[j] = k;
    cnt += k != 0u;
    kmin = (k && k < kmin) ? k : kmin;
    kmax = k > kmax ? k : kmax;
  }
  kmax = wave_max_u32(kmax);
  kmin = ~wave_max_u32(~kmin);
  if ((tid & (WAVE - 1)) == 0) {
    atomicMin(&mm[0], kmin);
    atomicMax(&mm[1], kmax);
  }
  int total;
  (void)block_scan(cnt, wsum, phase, total);  // its barrier also publishes mm
  if (mm[2] & 2u) {
    ok = false;
    return nullptr;
  }
  if (total < AT_TOPK) return nullptr;
  kmin = mm[0];
  kmax = mm[1];
  topk_refine<NK>(tid, key, [&](int j) { return cpos[NK * tid + j]; }, kmin, kmax, total, kmin,
                  false, hist, wsum, phase, res_s, sel, &mm[1]);
  if (mycut > mm[1]) atomicOr(&mm[2], 1u);
  __syncthreads();
  return (mm[2] & 1u) ? nullptr : sel;
}

}  // namespace mono
