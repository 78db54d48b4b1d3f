// The attention phase of the DSA layer as one persistent gfx950 launch: the FP4
// indexer's scores, their exact top-2048, and sparse MLA decode over the selected
// tokens' FP8 cache rows.
//
// Stages, every CTA in order (task t of a stage runs on CTA (t + offset) mod grid):
//   1  scores: task (row, 1024-token chunk), one 64-token page a wave. Per 16-token
//      tile and 16-head group one scaled 16x16x128 MFMA with E2M1 operands and their
//      E8M0 scales (query rows = heads, key columns = tokens, K = the 128 dims); relu,
//      the head weights and the sum over heads stay in the lane, then two permlane
//      swaps sum the lane groups. Scores go to scratch; the chunk's done word follows.
//      A row within one top-k block also gets each chunk's candidate list (chunk_list:
//      its keys at or above a histogram cut, 128-256 of them, with the cut).
//   2  top-k: task = row (one block, topk_lds.h): the chunks' lists ranked by one CTA
//      (topk_lists); where they cannot decide it (too few keys listed, or a chunk's cut
//      above the lists' threshold), or for a longer row, the scores themselves: task =
//      (row, 32768-key block), thread t holds the radix keys of block positions 32 t ..
//      in registers; a sample narrows the range, histograms over the live range keep the
//      bin of the 2048th key until its few candidates rank themselves; the selection
//      (every element up to the threshold element of the order key descending, position
//      ascending) is published as (position, tag) pairs. A row longer than one block
//      publishes each block's selection as candidates with their keys, and one more task
//      ranks the candidates of the row's blocks the same way.
//   3  split: task (row, SPLIT-key split), all 32 heads (SPLIT 64 when the rows' 32
//      splits each fill the grid once, else 128). The split's tokens (through the
//      page table) are gathered as E4M3 rows into LDS; S = q K^T on bf16 MFMAs (E4M3
//      widened exactly), times the token's scale and the softmax scale; per head the
//      split's max m and sum l; P, with the token's scale folded in, as bf16; O = P V on
//      MFMAs, V read from the same rows. O (in bf16), m and l go to scratch.
//   4  merge: task (row, head): o = sum_s exp(m_s - M) O_s / sum_s exp(m_s - M) l_s,
//      rounded to bf16.
// Every hand-off is a (word = launch tag) wait under the guard's deadline.
//
// Reference: FP4 scores sgl_amd_mono/deepseek_v41/gfx950/indexer/score_fp4.py:1-20,
// 254-296 (plane layout, formula); exact top-k sgl_amd_mono/glm53/gfx950/kernel.py:
// 3002-3636 (rule: glm53/check.py:94-117); sparse MLA split and merge kernel.py:
// 3638-4123; softmax scale glm53/gfx950/config.py:180-181.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "gemv.h"
#include "mono_abi.h"
#include "mono_device.h"
#include "phase.h"
#include "topk_lds.h"

namespace mono {

constexpr int AT_HEADS = 32;     // attention heads of one GPU's TP=4 share
constexpr int AT_IHEADS = 64;    // index heads
constexpr int AT_KV = 576;       // cached row: latent 512 + rope 64
constexpr int AT_LAT = 512;
constexpr int AT_PAGE = 64;
constexpr int AT_CHUNK = 1024;    // tokens of a score task
constexpr int AT_NCHUNK = AT_MAXCTX / AT_CHUNK;
// keys of a split task: 64 when the rows' splits (32 a row) fill the grid once, else 128
// (16 a row); scratch is laid out for the most splits a row
constexpr int AT_NSPLIT = AT_TOPK / 64;
constexpr int AT_MAXR = 48;

constexpr size_t at_align(size_t v) { return (v + 255) & ~(size_t)255; }

// scratch of a runtime sized for `rm` rows (every launch on it passes the same rm, so a
// word keeps its meaning from launch to launch and a stale tag can never match)
struct AttnScratch {
  size_t scores;      // f32 [rm][MAXCTX]
  size_t score_done;  // u32 [rm][NCHUNK]
  size_t topk;        // the selection as (position, tag) pairs [rm][TOPK]
  size_t cand;        // a long row's block selections: u64 (position | key << 32) [rm][MAXBLK][TOPK]
  size_t blk_done;    // u32 [rm][MAXBLK]
  size_t lists;       // a one-block row's chunk candidates: u64 [rm][TK_NLIST][TK_LIST]
  size_t cuts;        // u32 [rm][TK_NLIST]: each chunk's cut
  size_t acc;         // bf16 [rm][split][h][512]: a split's unnormalised P V
  size_t ml;          // f32 [rm][split][h][2]
  size_t split_done;  // u32 [rm][split]
  size_t bytes;
  __host__ __device__ explicit AttnScratch(int rm) {
    const size_t r = (size_t)rm;
    scores = 0;
    score_done = at_align(scores + r * AT_MAXCTX * 4);
    topk = at_align(score_done + r * AT_NCHUNK * 4);
    cand = at_align(topk + r * AT_TOPK * 8);
    blk_done = at_align(cand + r * AT_MAXBLK * AT_TOPK * 8);
    lists = at_align(blk_done + r * AT_MAXBLK * 4);
    cuts = at_align(lists + r * TK_NLIST * TK_LIST * 8);
    acc = at_align(cuts + r * TK_NLIST * 4);
    ml = at_align(acc + r * AT_NSPLIT * AT_HEADS * AT_LAT * 2);
    split_done = at_align(ml + r * AT_NSPLIT * AT_HEADS * 8);
    bytes = at_align(split_done + r * AT_NSPLIT * 4);
  }
};

struct AttnParams {
  int rows, rows_max, ctx_max, pt_stride, pt_rows;
  int index_fmt;  // MONO_INDEX_*: the FP4 plane, or a DSA (FP8) page (tiled or token-major)
  float sm_scale;
  uint32_t plane_pages, kv_slots;
  const int64_t* positions;
  const int32_t* req_ids;
  const int32_t* page_table;
  const uint16_t* q;
  const uint8_t* iq;
  const uint8_t* iqs;
  const float* iw;
  const uint8_t* plane;
  const uint8_t* plane_scale;
  const uint8_t* kv;
  const float* kv_scale;
  uint16_t* out;
  float* scores_out;
  int32_t* topk_out;
  uint8_t* scratch;
  int32_t* guard;
  uint32_t* host_err;
  int fault_site, fault_after;
  uint64_t* timeline;
  // the one-launch layer (FUSED): W_UV runs in the merge (UvUnit) on the latents it has
  // just merged, storing o as complemented bf16 pairs [16][4096] into the output block's
  // hand-off buffer of the launch tag's parity (unused by a launch of its own)
  const uint8_t* uv_w;
  const float* uv_s;
  int uv_shuf;
  uint16_t* uv_obuf[2];
};

// 16x16x128 E2M1 x E2M1 -> f32, each operand's E8M0 scale the byte OA / OB of its dword
template <int OA, int OB>
__device__ inline v4f mfma_fp4(v4i a, v4i b, int sa, int sb) {
  const v8i A = {a[0], a[1], a[2], a[3], 0, 0, 0, 0};
  const v8i B = {b[0], b[1], b[2], b[3], 0, 0, 0, 0};
  const v4f z = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, z, 4, 4, OA, sa, OB, sb);
}


// LDS of the attention phase: the top-k arena (carved per stage), then small words
// a DSA (FP8) index page: 64 x 128 E4M3 values, then 64 f32 scales; the score task's
// bf16 query in LDS, a head a row of 256 + 16 bytes, then the 64 head weights
constexpr uint32_t AT_DSA_PAGE = 64 * (128 + 4);
constexpr int AT_LDS_IQ8 = 8192;
constexpr int AT_IQ8_ROW = 272;
static_assert(AT_LDS_IQ8 + 64 * AT_IQ8_ROW + 256 <= TOPK_ARENA_WORDS * 4, "in the arena");
constexpr int AT_LDS_WSUM = TOPK_ARENA_WORDS * 4;         // int [2][16], 16-byte aligned
constexpr int AT_LDS_RES = AT_LDS_WSUM + 2 * AT_WAVES * 4;  // int [4]
constexpr int AT_LDS_MM = AT_LDS_RES + 16;                  // u32 [4]
constexpr int AT_LDS_BYTES = AT_LDS_MM + 16;

// The attention phase (stages 1-4) in one CTA of a launch. LONG: rows may span more than
// one top-k block (a context bound above AT_TKBLOCK); the launch picks it, so a launch
// within one block carries none of the multi-block code. DSA: the index keys are DSA (FP8)
// pages (the launch picks it by its index format). FUSED: it runs after the front
// in the same launch, so its inputs (q, iq, iqs, iw and the rows' own cache entries) are
// read device-coherent, after `ready` (the front's barrier), which it calls once, after
// its first index-page loads are in flight. Always inlined: it is instantiated in more
// than one kernel, and as a real call it would spill around the call.
template <int SPLIT, bool FUSED, bool LONG, bool DSA, class Ready>
__device__ __attribute__((always_inline)) inline void attn_phase(const AttnParams& p,
                                                                 uint8_t* lds, Guard& guard,
                                                                 uint32_t tag, int& ok_s,
                                                                 Ready ready) {
  const AttnScratch S(p.rows_max);
  static_assert(SPLIT == 64 || SPLIT == 128, "64- or 128-key splits");
  constexpr int NSP = AT_TOPK / SPLIT;  // splits a row
  // the front's outputs (q, iq, iqs, iw) are read after the barrier through L2: their
  // lines are only stored (write-through) before it in this launch, so no cache holds a
  // stale copy (phase.h)
  constexpr int XCP = CP_NONE;
  const int tid = threadIdx.x, l = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int R = p.rows;
  const int nblk = gridDim.x, b = blockIdx.x;

  uint8_t* smem = lds;
  int* wsum = reinterpret_cast<int*>(lds + AT_LDS_WSUM);
  int* res_s = reinterpret_cast<int*>(lds + AT_LDS_RES);
  uint32_t* mm_s = reinterpret_cast<uint32_t*>(lds + AT_LDS_MM);

  float* scores = reinterpret_cast<float*>(p.scratch + S.scores);
  uint32_t* score_done = reinterpret_cast<uint32_t*>(p.scratch + S.score_done);
  uint64_t* topk = reinterpret_cast<uint64_t*>(p.scratch + S.topk);
  uint64_t* cands = reinterpret_cast<uint64_t*>(p.scratch + S.cand);
  uint32_t* blk_done = reinterpret_cast<uint32_t*>(p.scratch + S.blk_done);
  uint64_t* lists = reinterpret_cast<uint64_t*>(p.scratch + S.lists);
  uint32_t* cuts = reinterpret_cast<uint32_t*>(p.scratch + S.cuts);
  uint16_t* accs = reinterpret_cast<uint16_t*>(p.scratch + S.acc);
  float* mls = reinterpret_cast<float*>(p.scratch + S.ml);
  uint32_t* split_done = reinterpret_cast<uint32_t*>(p.scratch + S.split_done);
  bool ok = true;
  // the wait for the phase before (fused), once a CTA: CTA-uniform
  bool waited = !FUSED;
  auto enter = [&]() {
    if (!waited) {
      waited = true;
      ok = ready() && ok;
    }
  };

  // keys a row sees (its position + 1, within the launch's context bound)
  auto row_n = [&](int r) -> int {
    const int64_t pos = p.positions[r];
    return (int)(pos < 0 ? 0 : (pos + 1 > p.ctx_max ? p.ctx_max : pos + 1));
  };
  // the page table through a bounded resource: an entry past it reads page 0
  const __amdgpu_buffer_rsrc_t rpt =
      rsrc(p.page_table, (uint32_t)p.pt_rows * (uint32_t)p.pt_stride * 4u);
  auto page_of = [&](int r, int pg) -> int {
    return ld4<CP_NONE>(rpt, ((uint32_t)p.req_ids[r] * (uint32_t)p.pt_stride + (uint32_t)pg) * 4u);
  };
  const __amdgpu_buffer_rsrc_t rplane = rsrc(p.plane, p.plane_pages * 4096u);
  const __amdgpu_buffer_rsrc_t rpsc = rsrc(p.plane_scale, p.plane_pages * 256u);

  // XCD-local placement (up to 8 rows on 256 CTAs; the hardware hands CTA b to XCD
  // (b + c) % 8 for a launch-wide c, so CTAs b and b + 8 share an XCD):
  // row r's score tasks, its top-k tasks, its 32 splits and its 32 merges all run on XCD r,
  // so the scores, the row's q and the split partials each cross HBM once and are then read
  // from that XCD's L2: task t of a stage belongs to row t % 8 (`rs8` = 8). Otherwise task
  // t of a 32-task-a-row stage is task t % 32 of row t / 32, and a stage with a run-time
  // task count numbers row-fastest (`rs8` = rows). CTA b takes tasks b, b + grid, ...
  const bool xcd = R <= 8 && nblk == 8 * 32;
  const int ntask32 = xcd ? nblk : R * 32;
  const int rs8 = xcd ? 8 : R;
  auto task_of = [&](int t, int& r, int& i) {
    r = xcd ? (t & 7) : t / 32;
    i = xcd ? (t >> 3) : t % 32;
  };

  // ---------------------------------------------------------------- 1: scores
  // Each stage takes the thread index through an opaque copy: conditions on it are then
  // computed inside the stage, not hoisted to the kernel's top where they would hold
  // registers through every stage.
  // tasks (row, 1024-key chunk), as many chunks a row as the launch's context bound needs.
  // A row within one top-k block that keeps fewer keys than it has also gets each chunk's
  // candidate list (chunk_list): the chunk's order keys go through LDS (ckey).
  static_assert(AT_CHUNK == AT_THREADS && TK_NLIST * AT_CHUNK == AT_TKBLOCK, "a key a thread");
  static_assert((AT_CHUNK + 256 + AT_WAVES) * 4 <= AT_LDS_IQ8, "the query clear of the keys");
  static_assert(AT_IHEADS * 256 == AT_THREADS * 16, "a DSA row's query: 16 bytes a thread");
  uint32_t* ckey = reinterpret_cast<uint32_t*>(smem);   // [AT_CHUNK]
  uint32_t* chist = ckey + AT_CHUNK;                     // [256]
  int* cwsum = reinterpret_cast<int*>(chist + 256);      // [AT_WAVES]
  uint8_t* iq8 = smem + AT_LDS_IQ8;                      // a DSA row's bf16 query
  const int nchr = (p.ctx_max + AT_CHUNK - 1) / AT_CHUNK;
  // chunk lists only while every CTA holds at most one score task: a list costs its task
  // ~2 us of VALU work, which several tasks a CTA would pay in series
  const bool lists_on = !LONG && rs8 * nchr <= nblk;
  // This CTA's score tasks: with XCD-local rows, tasks b, b + nblk, .. (all of row b % 8);
  // otherwise a contiguous run of the row-major task list (task t: row t / nchr, chunk
  // t % nchr), so that consecutive tasks mostly share a row and its query
  const int ntask = rs8 * nchr;
  int t_first = b, t_step = nblk, t_count = b < ntask ? (ntask - 1 - b) / nblk + 1 : 0;
  if (!xcd) {
    const int q = ntask / nblk, rem = ntask % nblk;
    t_first = b * q + (b < rem ? b : rem);
    t_step = 1;
    t_count = q + (b < rem ? 1 : 0);
  }
  auto task_rc = [&](int t, int& r, int& c) {
    r = xcd ? t % rs8 : t / nchr;
    c = xcd ? t / rs8 : t % nchr;
  };
  // the keys each row sees, lane r holding row r's, loaded ahead of every key (a later
  // read would wait for the keys in flight)
  static_assert(AT_MAXR <= 64, "a lane a row");
  const int nrow = l < R ? row_n(l) : 0;
  // FP4 plane: the page ids of this CTA's tasks, one a lane (lane i: the wave's page of
  // its task i; -1: none), loaded at once, so that a task's keys are requested while the
  // task before computes
  static_assert(AT_MAXR * ((AT_MAXCTX + AT_CHUNK - 1) / AT_CHUNK) <= 64 * 256, "a lane a task");
  int tpage = -1;
  if constexpr (!DSA) {
    int ri, ci;
    task_rc(t_first + l * t_step, ri, ci);
    const int pgi = ci * (AT_CHUNK / AT_PAGE) + w;
    if (l < t_count && ri < R && pgi * AT_PAGE < row_n(ri)) tpage = page_of(ri, pgi);
  }
  // task i's key tiles (B operands): tile nt, lane l: slot 16 nt + l % 16, dims 32 (l / 16)
  // ..; the key scales of the four tiles: bytes of one dword
  auto fp4_keys = [&](int i, v4i (&kb)[4], int& ks, bool dev) {
    const int pid = __builtin_amdgcn_readlane(tpage, i < 64 ? i : 63);
    const uint32_t kofs = pid >= 0 ? (uint32_t)pid * 4096u : 0x80000000u;
    const uint32_t sofs = pid >= 0 ? (uint32_t)pid * 256u : 0x80000000u;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const uint32_t o = kofs + (uint32_t)((l >> 4) * 1024 + (16 * nt + (l & 15)) * 16);
      kb[nt] = dev ? ld16<CP_DEV>(rplane, o) : ld16<CP_NT>(rplane, o);
    }
    ks = dev ? ld4<CP_DEV>(rpsc, sofs + (uint32_t)l * 4) : ld4<CP_NT>(rpsc, sofs + (uint32_t)l * 4);
  };
  // the next task's keys (FP4 plane), in flight while a task computes
  v4i kbn[4];
  int ksn = 0;
  if constexpr (!DSA) fp4_keys(0, kbn, ksn, false);
  // the row whose query (FP4: in registers; DSA: in LDS) the CTA holds
  int qrow = -1;
  v4i qa[4];
  int qs = 0;
  v4f wv[4];
  // row r's head weights of the lane's D rows: heads 16 mi + 4 (l / 16) + e
  auto load_wv = [&](int r, v4f (&wv)[4]) {
    const __amdgpu_buffer_rsrc_t rw = rsrc(p.iw + (size_t)r * AT_IHEADS, AT_IHEADS * 4);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
      wv[mi] = __builtin_bit_cast(v4f, ld16<XCP>(rw, (uint32_t)(16 * mi + 4 * (l >> 4)) * 4));
  };
  // One task; false: the launch is failing (every later task skipped).
  auto score_task = [&](int ti, v4i (&kb)[4], int& ks, v4i (&kbn)[4], int& ksn) -> bool {
    const int tid = opaque_v((int)threadIdx.x), l = tid & 63;
    int r, c;
    task_rc(t_first + ti * t_step, r, c);
    const int n = r < R ? __builtin_amdgcn_readlane(nrow, r) : 0;
    const bool valid = r < R && c * AT_CHUNK < n;
    if constexpr (!DSA) {
      // after the wait for the front: the row's query when the wave's task changes rows,
      // then the next task's keys (the newest loads: this task's MFMAs wait for neither)
      enter();
      if (!ok) return false;
      if (valid && (c * (AT_CHUNK / AT_PAGE) + w) * AT_PAGE < n && r != qrow) {
        // the query as A operands: head tile mi, lane l: head 16 mi + l % 16, dims
        // 32 (l / 16) .. (16 bytes); its scales: the dword of lane l holds tile mi's byte mi
        const __amdgpu_buffer_rsrc_t rq = rsrc(p.iq + (size_t)r * AT_IHEADS * 64, AT_IHEADS * 64);
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
          qa[mi] = ld16<XCP>(rq, (uint32_t)((16 * mi + (l & 15)) * 64 + 16 * (l >> 4)));
        qs = ld4<XCP>(rsrc(p.iqs + (size_t)r * 256, 256), (uint32_t)l * 4);
        load_wv(r, wv);
        qrow = r;
      }
      if (ti + 1 < t_count) fp4_keys(ti + 1, kbn, ksn, false);
    }
    if (!valid) return true;
    const bool listed = lists_on && n > AT_TOPK;
    if (listed) {
      if (tid < 64) reinterpret_cast<v4i*>(chist)[tid] = opaque_v4(0, 0, 0, 0);
      if (tid == 0) *reinterpret_cast<v4i*>(mm_s) = opaque_v4(-1, 0, 0, 0);
    }
    const int pg = c * (AT_CHUNK / AT_PAGE) + w;
    const bool live = pg * AT_PAGE < n;
    float sco[4];  // a listed chunk's scores (lanes < 16), stored after its list
    // (a DSA page's id, looked up by its task)
    const int pid = DSA && live ? __builtin_amdgcn_readfirstlane(page_of(r, pg)) : 0;
    // token tile nt's sums (one a lane: heads 4 (l / 16) .. of token 16 nt + l % 16) to
    // the tile's scores: the four lane groups summed, lane l < 16 keeping token l's. A
    // listed chunk's scores are stored after its list is made (a store in flight would
    // hold up the list making's waits)
    float* dst = scores + (size_t)r * AT_MAXCTX + pg * AT_PAGE;
    auto emit = [&](int nt, float acc) {
      float a, bb;
      swap16(acc, a, bb);
      acc = a + bb;
      swap32(acc, a, bb);
      acc = a + bb;
      sco[nt] = acc;
      if (l < 16) {
        const int tok = pg * AT_PAGE + 16 * nt + l;
        if (listed) {
          const uint32_t k = radix_key(acc);
          ckey[w * AT_PAGE + 16 * nt + l] = tok < n ? (k > 1u ? k : 1u) : 0u;
        } else {
          st_devf(dst + 16 * nt + l, acc);
          if (p.scores_out && tok < n) p.scores_out[(size_t)r * p.ctx_max + tok] = acc;
        }
      }
    };
    // The wave's page from the FP4 index plane. False: the launch is failing.
    // The wave's page from the FP4 index plane (its keys requested a task ahead, before
    // the wait for the front: only the row's own key, its last, is written this launch).
    // False: the launch is failing.
    auto fp4_page = [&]() -> bool {
      if (!live) return true;
      // the row's own key (the last page of the row) is the front's store of this
      // launch: read it again, device coherent
      if (FUSED && pg == (n - 1) / AT_PAGE) fp4_keys(ti, kb, ks, true);
      auto tile = [&](auto nt_c) {
        constexpr int NT = decltype(nt_c)::value;
        float acc = 0.f;
        auto head_tile = [&](auto mi_c) {
          constexpr int MI = decltype(mi_c)::value;
          const v4f d = mfma_fp4<MI, NT>(qa[MI], kb[NT], qs, ks);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc = fmaf(fmaxf(d[e], 0.f), wv[MI][e], acc);
        };
        head_tile(std::integral_constant<int, 0>());
        head_tile(std::integral_constant<int, 1>());
        head_tile(std::integral_constant<int, 2>());
        head_tile(std::integral_constant<int, 3>());
        emit(NT, acc);
      };
      tile(std::integral_constant<int, 0>());
      tile(std::integral_constant<int, 1>());
      tile(std::integral_constant<int, 2>());
      tile(std::integral_constant<int, 3>());
      return true;
    };
    // The wave's page from a DSA (FP8) index page: 64 x 128 E4M3 values (16-token x
    // 16-byte tiles, or token-major), then 64 f32 scales. Token tile nt, K steps 2 m and
    // 2 m + 1: lane l's 16 bytes are token 16 nt + l % 16's dims 64 m + 16 (l / 16) .. (the
    // first 8 for step 2 m, the next 8 for 2 m + 1; the query's A operands take the same
    // dims). The query is the row's bf16 [64][128], staged in LDS. False: the launch is
    // failing.
    auto fp8_page = [&]() -> bool {
      const bool tiled = p.index_fmt == MONO_INDEX_FP8_PAGE;
      // a page-table entry outside the pages reads zeros, as the FP4 plane's bounded reads
      const bool inside = (uint32_t)pid < p.plane_pages;
      const __amdgpu_buffer_rsrc_t rpg =
          rsrc(p.plane + (inside ? (size_t)pid * AT_DSA_PAGE : 0), live && inside ? AT_DSA_PAGE : 0u);
      auto vofs = [&](int nt, int m) -> uint32_t {
        const int t = 16 * nt + (l & 15), d = 64 * m + 16 * (l >> 4);
        return (uint32_t)(tiled ? (t >> 4) * 2048 + (d >> 4) * 256 + (t & 15) * 16 : t * 128 + d);
      };
      v4i kb[8];
      int ks[4];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
#pragma unroll
        for (int m = 0; m < 2; ++m) kb[2 * nt + m] = ld16<CP_NT>(rpg, vofs(nt, m));
        ks[nt] = ld4<CP_NT>(rpg, 8192u + (uint32_t)(16 * nt + (l & 15)) * 4u);
      }
      enter();
      if (!ok) return false;
      // the row's query into LDS rows of AT_IQ8_ROW bytes (A-operand reads conflict free),
      // its head weights after them, when the CTA's task changes rows (after the last
      // task's readers)
      if (r != qrow) {
        __syncthreads();
        *reinterpret_cast<v4i*>(iq8 + (tid >> 4) * AT_IQ8_ROW + (tid & 15) * 16) =
            ld16<XCP>(rsrc(p.iq + (size_t)r * AT_IHEADS * 256, AT_IHEADS * 256), (uint32_t)tid * 16u);
        if (tid < AT_IHEADS / 4)
          *reinterpret_cast<v4i*>(iq8 + AT_IHEADS * AT_IQ8_ROW + tid * 16) =
              ld16<XCP>(rsrc(p.iw + (size_t)r * AT_IHEADS, AT_IHEADS * 4), (uint32_t)tid * 16u);
        __syncthreads();
        qrow = r;
      }
      if (!live) return true;
      if (FUSED && pg == (n - 1) / AT_PAGE) {
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
#pragma unroll
          for (int m = 0; m < 2; ++m) kb[2 * nt + m] = ld16<CP_DEV>(rpg, vofs(nt, m));
          ks[nt] = ld4<CP_DEV>(rpg, 8192u + (uint32_t)(16 * nt + (l & 15)) * 4u);
        }
      }
      // two head tiles at a time: the four token tiles' accumulators of both over the four
      // K steps, each key step widened exactly to bf16 (B operand) once for the pair. The
      // second pair widens the keys again: an opaque copy of the raw keys keeps the
      // compiler from reusing the first pair's widened keys, whose 64 registers beside
      // the raw keys and accumulators would spill
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int hp = 0; hp < 2; ++hp) {
        __builtin_amdgcn_sched_barrier(0);
        if (hp == 1) {
#pragma unroll
          for (int i = 0; i < 8; ++i) asm volatile("" : "+v"(kb[i]));
        }
        // A operands of head tile 2 hp + j: head 16 (2 hp + j) + l % 16, K step 2 m + s
        const uint8_t* qrow = iq8 + (32 * hp + (l & 15)) * AT_IQ8_ROW + 32 * (l >> 4);
        v4f d[2][4];
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) d[0][nt] = d[1][nt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const int qo = 128 * (st >> 1) + 16 * (st & 1);
          const v8bf qa0 = *reinterpret_cast<const v8bf*>(qrow + qo);
          const v8bf qa1 = *reinterpret_cast<const v8bf*>(qrow + 16 * AT_IQ8_ROW + qo);
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) {
            const v4i& k = kb[2 * nt + (st >> 1)];
            const v8bf kw = (st & 1) ? fp8x8_bf16((uint32_t)k[2], (uint32_t)k[3])
                                     : fp8x8_bf16((uint32_t)k[0], (uint32_t)k[1]);
            d[0][nt] = mfma_bf16(qa0, kw, d[0][nt]);
            d[1][nt] = mfma_bf16(qa1, kw, d[1][nt]);
          }
        }
        // head weights of the lane's D rows: heads 16 (2 hp + j) + 4 (l / 16) + e, the
        // tiles summed in head order
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const v4f wv = *reinterpret_cast<const v4f*>(iq8 + AT_IHEADS * AT_IQ8_ROW +
                                                       (16 * (2 * hp + j) + 4 * (l >> 4)) * 4);
#pragma unroll
          for (int nt = 0; nt < 4; ++nt)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              acc[nt] = fmaf(fmaxf(d[j][nt][e], 0.f), wv[e], acc[nt]);
        }
      }
      // the key's power-of-two scale after the heads' sums (the ReLU commutes with it)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) emit(nt, acc[nt] * __int_as_float(ks[nt]));
      return true;
    };
    bool going;
    if constexpr (DSA)
      going = fp8_page();
    else
      going = fp4_page();
    if (!going) return false;
    if (!live && listed) ckey[w * AT_PAGE + l] = 0u;
    if (listed) {
      __syncthreads();
      const uint32_t cut =
          chunk_list(tid, ckey[tid], c * AT_CHUNK, chist, cwsum, mm_s,
                     rsrc(lists + ((size_t)r * TK_NLIST + c) * TK_LIST, TK_LIST * 8));
      if (tid == 0) st_dev(&cuts[r * TK_NLIST + c], cut);
      if (live && l < 16) {
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          st_devf(dst + 16 * nt + l, sco[nt]);
          const int tok = pg * AT_PAGE + 16 * nt + l;
          if (p.scores_out && tok < n) p.scores_out[(size_t)r * p.ctx_max + tok] = sco[nt];
        }
      }
    }
    // a listed chunk's LDS is reused by the next task
    if (listed) __syncthreads();
    return true;
  };
  for (int ti = 0; ti < t_count; ++ti) {
    v4i kb[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) kb[nt] = kbn[nt];
    int ks = ksn;
    if (!score_task(ti, kb, ks, kbn, ksn)) break;
  }
  enter();  // a CTA without a score task
  // every task's stores acknowledged, then their done words (one drain a CTA, not a task)
  if (ok && t_count > 0) {
    drain();
    __syncthreads();
    const int tid = opaque_v((int)threadIdx.x);
    if (tid < t_count) {
      int r, c;
      task_rc(t_first + tid * t_step, r, c);
      if (r < R) st_dev(&score_done[r * AT_NCHUNK + c], tag);
    }
  }

  // ---------------------------------------------------------------- 2: top-k
  stamp(p.timeline, MONO_TL_STAGED);
  // a row's selection as (position, tag) pairs, and the caller's copy of it
  auto publish = [&](int tid, int r, const int32_t* sel_l) {
    uint64_t* sel = topk + (size_t)r * AT_TOPK;
    for (int i = tid; i < AT_TOPK; i += AT_THREADS) {
      const int v = sel_l[i];
      st_dev64(sel + i, pair((uint32_t)v, tag));
      if (p.topk_out) p.topk_out[(size_t)r * AT_TOPK + i] = v;
    }
  };
  if constexpr (!LONG) {
    // every row within one block: task = row (XCD-local: row r on CTA r)
    for (int r = b; r < (ok ? R : 0); r += nblk) {
      const int tid = opaque_v((int)threadIdx.x), l = tid & 63;
      const int n = row_n(r);
      if (n <= AT_TOPK) {
        // every key of the row, in position order
        uint64_t* sel = topk + (size_t)r * AT_TOPK;
        for (int i = tid; i < AT_TOPK; i += AT_THREADS) {
          if (i < n) st_dev64(sel + i, pair((uint32_t)i, tag));
          if (p.topk_out) p.topk_out[(size_t)r * AT_TOPK + i] = i < n ? i : -1;
        }
      } else {
        const int nch = (n + AT_CHUNK - 1) / AT_CHUNK;
        // topk_lists' / topk_select's minimum, maximum and flag words, set before a barrier
        if (tid == 0) *reinterpret_cast<v4i*>(mm_s) = opaque_v4(-1, 0, 0, 0);
        __syncthreads();
        // each wave waits for its own chunks' done words (then loads their lists at once)
        const uint32_t* dw = score_done + r * AT_NCHUNK;
        auto wait_chunks = [&](int c0, int c1) {
          return wait_until(guard, MONO_SITE_SCORES, [&]() {
            return __all((c0 >= nch || ld_dev(&dw[c0]) == tag) &&
                         (c1 >= nch || ld_dev(&dw[c1]) == tag));
          });
        };
        int32_t* sel = nullptr;
        if (lists_on) {
          sel = topk_lists(
              tid, rsrc(lists + (size_t)r * TK_NLIST * TK_LIST, (uint32_t)(nch * TK_LIST * 8)),
              rsrc(cuts + r * TK_NLIST, (uint32_t)nch * 4u), nch, smem, wsum, mm_s, res_s,
              wait_chunks, ok);
        } else {
          ok = cta_all(wait_chunks(2 * w, 2 * w + 1) && ok, ok_s);
        }
        if (ok) {
          // without lists, or where they cannot decide it (every chunk is done: each wave
          // saw its own), every score
          if (!sel) {
            if (tid == 0) *reinterpret_cast<v2i*>(mm_s) = opaque_v2(-1, 0);
            __syncthreads();
            const __amdgpu_buffer_rsrc_t rs = rsrc(scores + (size_t)r * AT_MAXCTX, (uint32_t)n * 4);
            sel = topk_select(tid, rs, n, smem, wsum, mm_s, res_s);
          }
          publish(tid, r, sel);
        }
      }
      __syncthreads();  // the LDS arena is reused by the next row
    }
  } else {
    const int nbr = (p.ctx_max + AT_TKBLOCK - 1) / AT_TKBLOCK;  // blocks of the longest row
    // tasks: (row, block) for every block of the longest row, then one final task a row.
    // Every final task comes after every block task in the numbering, so no CTA waits on
    // a task it has yet to run.
    for (int task = b; task < (ok ? rs8 * (nbr + 1) : 0); task += nblk) {
      const int tid = opaque_v((int)threadIdx.x), l = tid & 63;
      const int r = task % rs8, blk = task / rs8;
      if (r >= R) continue;
      const int n = row_n(r);
      // blocks of this row (a row seeing no key has one, empty: its selection is all -1)
      const int nb = n > AT_TKBLOCK ? (n + AT_TKBLOCK - 1) / AT_TKBLOCK : 1;
      if (blk < nbr) {
        // ---- a block task
        if (blk >= nb) continue;
        const int b0 = blk * AT_TKBLOCK;
        const int nk = n - b0 < AT_TKBLOCK ? n - b0 : AT_TKBLOCK;
        const bool last = nb == 1;  // the block's selection is the row's
        if (last && n <= AT_TOPK) {
          uint64_t* sel = topk + (size_t)r * AT_TOPK;
          for (int i = tid; i < AT_TOPK; i += AT_THREADS) {
            if (i < n) st_dev64(sel + i, pair((uint32_t)i, tag));
            if (p.topk_out) p.topk_out[(size_t)r * AT_TOPK + i] = i < n ? i : -1;
          }
        } else {
          const int nch = (nk + AT_CHUNK - 1) / AT_CHUNK;
          const int c0 = b0 / AT_CHUNK;
          if (w == 0)
            ok = wait_until(guard, MONO_SITE_SCORES, [&]() {
              return __all(l >= nch || ld_dev(&score_done[r * AT_NCHUNK + c0 + l]) == tag);
            });
          if (tid == 0) *reinterpret_cast<v2i*>(mm_s) = opaque_v2(-1, 0);
          ok = cta_all(ok, ok_s);
          if (!ok) break;
          const __amdgpu_buffer_rsrc_t rs =
              rsrc(scores + (size_t)r * AT_MAXCTX + b0, (uint32_t)nk * 4);
          uint64_t* cand = cands + ((size_t)r * AT_MAXBLK + blk) * AT_TOPK;
          if (nk > AT_TOPK) {
            const int32_t* sel_l = topk_select(tid, rs, nk, smem, wsum, mm_s, res_s);
            if (last) {
              publish(tid, r, sel_l);
            } else {
              for (int i = tid; i < AT_TOPK; i += AT_THREADS) {
                const int v = sel_l[i];
                st_dev64(cand + i, (uint64_t)(uint32_t)(b0 + v) |
                                       ((uint64_t)topk_key_at(smem, v) << 32));
              }
            }
          } else {
            // a short last block: every key is a candidate (keys as topk_select makes them)
            for (int i = tid; i < nk; i += AT_THREADS) {
              const uint32_t k = radix_key(__int_as_float(ld4<CP_NONE>(rs, (uint32_t)i * 4u)));
              st_dev64(cand + i, (uint64_t)(uint32_t)(b0 + i) | ((uint64_t)(k > 1u ? k : 1u) << 32));
            }
          }
          if (!last) {
            drain();
            __syncthreads();
            if (tid == 0) st_dev(&blk_done[r * AT_MAXBLK + blk], tag);
          }
        }
      } else {
        // ---- the final task of a row spanning several blocks
        if (nb < 2) continue;
        const int nl = n - (nb - 1) * AT_TKBLOCK;
        const int C = AT_TOPK * (nb - 1) + (nl < AT_TOPK ? nl : AT_TOPK);
        if (w == 0)
          ok = wait_until(guard, MONO_SITE_BLOCKS, [&]() {
            return __all(l >= nb || ld_dev(&blk_done[r * AT_MAXBLK + l]) == tag);
          });
        if (tid == 0) *reinterpret_cast<v2i*>(mm_s) = opaque_v2(-1, 0);
        ok = cta_all(ok, ok_s);
        if (!ok) break;
        const __amdgpu_buffer_rsrc_t rc =
            rsrc(cands + (size_t)r * AT_MAXBLK * AT_TOPK, (uint32_t)C * 8u);
        publish(tid, r,
                topk_final<AT_MAXBLK * AT_TOPK / AT_THREADS>(tid, rc, C, smem, wsum, mm_s, res_s));
      }
      __syncthreads();  // the LDS arena is reused by the next task
    }
  }

  // ---------------------------------------------------------------- 3: split
  stamp(p.timeline, MONO_TL_ROUTED);
  {
    // LDS: K rows (E4M3, 576 + 16 bytes apart), q (bf16, 1152 + 16), S (f32), P (bf16),
    // the split's slots and token scales, the row's page-table entries
    constexpr int KSTR = AT_KV + 16, QSTR = AT_KV * 2 + 16, SSTR = SPLIT + 4,
                  PSTR = SPLIT * 2 + 16;
    constexpr int NSB = SPLIT == 64 ? 2 : 1;  // S buffers: the two K chains (64), or summed
    constexpr int NPG = (LONG ? AT_MAXCTX : AT_TKBLOCK) / AT_PAGE;
    uint8_t* kbuf = smem;
    uint8_t* qbuf = kbuf + SPLIT * KSTR;
    float* sbuf = reinterpret_cast<float*>(qbuf + AT_HEADS * QSTR);
    uint8_t* pbuf = reinterpret_cast<uint8_t*>(sbuf + NSB * AT_HEADS * SSTR);
    int32_t* slot_s = reinterpret_cast<int32_t*>(pbuf + AT_HEADS * PSTR);
    float* ksc = reinterpret_cast<float*>(slot_s + SPLIT);
    int32_t* pt_s = reinterpret_cast<int32_t*>(ksc + SPLIT);
    static_assert(SPLIT * KSTR + AT_HEADS * QSTR + NSB * AT_HEADS * SSTR * 4 + AT_HEADS * PSTR +
                          SPLIT * 8 + NPG * 4 <=
                      TOPK_ARENA_WORDS * 4,
                  "split LDS");
    constexpr int NPT = (NPG + AT_THREADS - 1) / AT_THREADS;  // page-table entries a thread
    constexpr int QP = AT_HEADS * AT_KV / 8;  // 16-byte pieces of a row's q
    constexpr int NQP = (QP + AT_THREADS - 1) / AT_THREADS;
    const __amdgpu_buffer_rsrc_t rkv = rsrc(p.kv, p.kv_slots * (uint32_t)AT_KV);
    // without per-token scales every row is raw E4M3 (scale 1)
    const bool scaled = p.kv_scale != nullptr;
    const __amdgpu_buffer_rsrc_t rks = rsrc(p.kv_scale, scaled ? p.kv_slots * 4u : 0u);
    const bool xsp = xcd && NSP == 32;
    const int nt = ok ? (xsp ? nblk : R * NSP) : 0;
    for (int t0 = 0; t0 < nt; t0 += nblk) {
      const int tid = opaque_v((int)threadIdx.x), l = tid & 63;
      // XCD-local (task b / 8 of row b % 8), else task t0 + b with the rows' top-k CTAs last
      const int task = xsp ? b : t0 + (b + nblk - (R % nblk)) % nblk;
      if (task >= nt) continue;
      const int r = xsp ? (task & 7) : task / NSP, sp = xsp ? (task >> 3) : task % NSP;
      if (r >= R) continue;
      const int n = row_n(r);
      const int k = n < AT_TOPK ? n : AT_TOPK;
      const int kcnt = k - sp * SPLIT < SPLIT ? k - sp * SPLIT : SPLIT;
      if (kcnt <= 0) continue;
      // ahead of the wait (neither depends on the selection): the row's q, all heads
      // ([32][576] bf16), and its page-table entries
      const __amdgpu_buffer_rsrc_t rq = rsrc(p.q + (size_t)r * AT_HEADS * AT_KV, AT_HEADS * AT_KV * 2);
      v4i qv[NQP];
#pragma unroll
      for (int i = 0; i < NQP; ++i) {
        const int pc = tid + AT_THREADS * i;
        qv[i] = ld16<XCP>(rq, pc < QP ? (uint32_t)pc * 16u : 0x80000000u);
      }
      const int npg = (n + AT_PAGE - 1) / AT_PAGE;
      int pgv[NPT];
#pragma unroll
      for (int i = 0; i < NPT; ++i) {
        const int pi = tid + AT_THREADS * i;
        pgv[i] = ld4<CP_NONE>(
            rpt, pi < npg ? ((uint32_t)p.req_ids[r] * (uint32_t)p.pt_stride + (uint32_t)pi) * 4u
                          : 0x80000000u);
      }
      // the split's tokens, polled as (position, tag) pairs
      int pos = -1;
      if (tid < SPLIT) {
        uint64_t v = 0;
        const uint64_t* src = topk + (size_t)r * AT_TOPK + sp * SPLIT + tid;
        ok = wait_until(guard, MONO_SITE_TOPK, [&]() {
          v = tid < kcnt ? ld_dev64(src) : pair(0u, tag);
          return __all((uint32_t)(v >> 32) == tag);
        });
        if (ok && tid < kcnt) pos = (int)(uint32_t)v;
      }
#pragma unroll
      for (int i = 0; i < NQP; ++i) {
        const int pc = tid + AT_THREADS * i;
        if (pc < QP)
          *reinterpret_cast<v4i*>(qbuf + (pc / (AT_KV / 8)) * QSTR + (pc % (AT_KV / 8)) * 16) = qv[i];
      }
#pragma unroll
      for (int i = 0; i < NPT; ++i)
        if (tid + AT_THREADS * i < NPG) pt_s[tid + AT_THREADS * i] = pgv[i];
      ok = cta_all(ok, ok_s);
      if (!ok) break;
      // position -> cache slot through the page table in LDS
      if (tid < SPLIT) slot_s[tid] = pos >= 0 ? pt_s[pos >> 6] * AT_PAGE + (pos & 63) : -1;
      __syncthreads();
      // gather the rows: 36 pieces of 16 bytes a row (a dead slot reads zeros), and the
      // token scales, in one round trip
      {
        constexpr int GP = SPLIT * (AT_KV / 16);
        constexpr int NGP = (GP + AT_THREADS - 1) / AT_THREADS;
        const int slot = tid < SPLIT ? slot_s[tid] : -1;
        // the row's own KV row is the front's store of this launch (fused): coherent
        const int own = FUSED ? pt_s[(n - 1) >> 6] * AT_PAGE + ((n - 1) & 63) : -2;
        const uint32_t so = slot >= 0 ? (uint32_t)slot * 4u : 0x80000000u;
        const float sc = __int_as_float(slot == own ? ld4<CP_DEV>(rks, so) : ld4<CP_NONE>(rks, so));
        // every load issued before the first is stored (a load-store loop would wait
        // one round trip an iteration)
        v4i gv[NGP];
#pragma unroll
        for (int i = 0; i < NGP; ++i) {
          const int idx = tid + AT_THREADS * i;
          const int j = idx / (AT_KV / 16), c = idx % (AT_KV / 16);
          const int sj = idx < GP ? slot_s[j] : -1;
          const uint32_t go = sj >= 0 ? (uint32_t)sj * AT_KV + c * 16 : 0x80000000u;
          gv[i] = (FUSED && sj == own) ? ld16<CP_DEV>(rkv, go) : ld16<CP_NT>(rkv, go);
        }
#pragma unroll
        for (int i = 0; i < NGP; ++i) {
          const int idx = tid + AT_THREADS * i;
          const int j = idx / (AT_KV / 16), c = idx % (AT_KV / 16);
          if (idx < GP) *reinterpret_cast<v4i*>(kbuf + j * KSTR + c * 16) = gv[i];
        }
        if (tid < SPLIT) ksc[tid] = slot >= 0 ? (scaled ? sc : 1.0f) : 0.f;
      }
      __syncthreads();
      // S = q K^T: wave w takes heads 16 (w / 8) .., keys 16 (w % 4) .. and the even (w / 4
      // even) or odd K steps: two MFMA chains a tile, summed (even + odd) by the softmax
      if constexpr (SPLIT == 64) {
        const int h0 = 16 * (w >> 3), j0 = 16 * (w & 3), odd = (w >> 2) & 1;
        v4f d = {0.f, 0.f, 0.f, 0.f};
        const uint8_t* qa = qbuf + (h0 + (l & 15)) * QSTR + 16 * (l >> 4) + odd * 64;
        const uint8_t* kr = kbuf + (j0 + (l & 15)) * KSTR + 8 * (l >> 4) + odd * 32;
        static_assert(AT_KV / 32 % 2 == 0, "K steps in pairs");
#pragma unroll 3
        for (int ks = 0; ks < AT_KV / 32; ks += 2) {
          const v8bf a0 = *reinterpret_cast<const v8bf*>(qa + ks * 64);
          const v2i k0 = *reinterpret_cast<const v2i*>(kr + ks * 32);
          d = mfma_bf16(a0, fp8x8_bf16((uint32_t)k0[0], (uint32_t)k0[1]), d);
        }
        float* sb = sbuf + odd * AT_HEADS * SSTR;
#pragma unroll
        for (int e = 0; e < 4; ++e) sb[(h0 + 4 * (l >> 4) + e) * SSTR + j0 + (l & 15)] = d[e];
      } else {
        // wave w takes heads 16 (w / 8) .. and keys 16 (w % 8) ..; two accumulators (even
        // and odd K steps): two MFMA chains in flight, summed, then scaled
        const int h0 = 16 * (w >> 3), j0 = 16 * (w & 7);
        v4f d = {0.f, 0.f, 0.f, 0.f}, d1 = d;
        const uint8_t* qa = qbuf + (h0 + (l & 15)) * QSTR + 16 * (l >> 4);
        const uint8_t* kr = kbuf + (j0 + (l & 15)) * KSTR + 8 * (l >> 4);
#pragma unroll 3
        for (int ks = 0; ks < AT_KV / 32; ks += 2) {
          const v8bf a0 = *reinterpret_cast<const v8bf*>(qa + ks * 64);
          const v2i k0 = *reinterpret_cast<const v2i*>(kr + ks * 32);
          const v8bf a1 = *reinterpret_cast<const v8bf*>(qa + ks * 64 + 64);
          const v2i k1 = *reinterpret_cast<const v2i*>(kr + ks * 32 + 32);
          d = mfma_bf16(a0, fp8x8_bf16((uint32_t)k0[0], (uint32_t)k0[1]), d);
          d1 = mfma_bf16(a1, fp8x8_bf16((uint32_t)k1[0], (uint32_t)k1[1]), d1);
        }
        d += d1;
        const float f = ksc[j0 + (l & 15)] * p.sm_scale;
#pragma unroll
        for (int e = 0; e < 4; ++e) sbuf[(h0 + 4 * (l >> 4) + e) * SSTR + j0 + (l & 15)] = d[e] * f;
      }
      __syncthreads();
      // softmax of the split, per head: wave w takes heads 2w, 2w + 1; lane l keys l (and
      // l + 64 in a 128-key split)
      float* ml = mls + ((size_t)(r * AT_NSPLIT + sp) * AT_HEADS) * 2;
      const float f0 = ksc[l] * p.sm_scale;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int h = 2 * w + hh;
        const bool v0 = l < kcnt, v1 = SPLIT == 128 && l + 64 < kcnt;
        float s0, s1 = -INFINITY;
        if constexpr (SPLIT == 64) {
          s0 = v0 ? (sbuf[h * SSTR + l] + sbuf[(AT_HEADS + h) * SSTR + l]) * f0 : -INFINITY;
        } else {
          s0 = v0 ? sbuf[h * SSTR + l] : -INFINITY;
          s1 = v1 ? sbuf[h * SSTR + l + 64] : -INFINITY;
        }
        const float m = wave_max(fmaxf(s0, s1));
        const float p0 = v0 ? expf(s0 - m) : 0.f, p1 = v1 ? expf(s1 - m) : 0.f;
        const float lsum = wave_sum(p0 + p1);
        // P with the token's scale folded in (V = E4M3 value x scale)
        reinterpret_cast<uint16_t*>(pbuf + h * PSTR)[l] = (uint16_t)bf16_bits(p0 * ksc[l]);
        if constexpr (SPLIT == 128)
          reinterpret_cast<uint16_t*>(pbuf + h * PSTR)[l + 64] = (uint16_t)bf16_bits(p1 * ksc[l + 64]);
        if (l == 0) {
          st_devf(ml + 2 * h, m);
          st_devf(ml + 2 * h + 1, lsum);
        }
      }
      __syncthreads();
      // O = P V: wave w takes heads 16 (w / 8) .. and dims 64 (w % 8) ..; MFMA j4 covers
      // dims d0 + 4 c + j4 (column c), so one dword of a row feeds four MFMAs
      {
        const int h0 = 16 * (w >> 3), d0 = 64 * (w & 7);
        const int c = l & 15, g = l >> 4;
        v4f o0 = {0.f, 0.f, 0.f, 0.f}, o1 = o0, o2 = o0, o3 = o0;
        const uint8_t* pa = pbuf + (h0 + c) * PSTR + 16 * g;
#pragma unroll
        for (int kst = 0; kst < SPLIT / 32; ++kst) {
          const v8bf a = *reinterpret_cast<const v8bf*>(pa + kst * 64);
          uint32_t dv[8];
#pragma unroll
          for (int i = 0; i < 8; ++i)
            dv[i] = *reinterpret_cast<const uint32_t*>(kbuf + (32 * kst + 8 * g + i) * KSTR + d0 +
                                                       4 * c);
          // byte j of keys (2i, 2i + 1): perm picks bytes j and j + 1 of both dwords
          uint32_t pr[4][2];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            pr[i][0] = __builtin_amdgcn_perm(dv[2 * i + 1], dv[2 * i], 0x05010400u);  // j 0, 1
            pr[i][1] = __builtin_amdgcn_perm(dv[2 * i + 1], dv[2 * i], 0x07030602u);  // j 2, 3
          }
          auto gather = [&](auto hi_c, int which) {
            constexpr bool HI = decltype(hi_c)::value;
            const v2bf q0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(pr[0][which], 1.0f, HI);
            const v2bf q1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(pr[1][which], 1.0f, HI);
            const v2bf q2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(pr[2][which], 1.0f, HI);
            const v2bf q3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(pr[3][which], 1.0f, HI);
            return v8bf{q0[0], q0[1], q1[0], q1[1], q2[0], q2[1], q3[0], q3[1]};
          };
          const v8bf bj[4] = {gather(std::false_type(), 0), gather(std::true_type(), 0),
                              gather(std::false_type(), 1), gather(std::true_type(), 1)};
          o0 = mfma_bf16(a, bj[0], o0);
          o1 = mfma_bf16(a, bj[1], o1);
          o2 = mfma_bf16(a, bj[2], o2);
          o3 = mfma_bf16(a, bj[3], o3);
        }
        // the partial in bf16 (the merge's sum of 32 of them rounds to bf16 again)
        uint16_t* acc = accs + ((size_t)(r * AT_NSPLIT + sp) * AT_HEADS) * AT_LAT;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int h = h0 + 4 * g + e;
          const v2i v = {(int32_t)(bf16_bits(o0[e]) | (bf16_bits(o1[e]) << 16)),
                         (int32_t)(bf16_bits(o2[e]) | (bf16_bits(o3[e]) << 16))};
          __builtin_amdgcn_raw_buffer_store_b64(v, rsrc(acc, AT_HEADS * AT_LAT * 2),
                                                (uint32_t)(h * AT_LAT + d0 + 4 * c) * 2, 0,
                                                CP_DEV);
        }
      }
      drain();
      __syncthreads();
      if (tid == 0) st_dev(&split_done[r * AT_NSPLIT + sp], tag);
    }
  }

  // ---------------------------------------------------------------- 4: merge
  stamp(p.timeline, MONO_TL_UPGATE);
  {
    static_assert(AT_HEADS == 32, "32 merge tasks a row");
    static_assert(AT_NSPLIT <= WAVE, "a split's (m, l) a lane");
    constexpr bool uv = FUSED;  // the one-launch layer sets uv_w
    v4f (*uvred)[64] = reinterpret_cast<v4f (*)[64]>(smem);  // [16][64]
    uint16_t* uvx = reinterpret_cast<uint16_t*>(uvred + 16);  // [512] x
    uint16_t* uob = uvx + AT_LAT;                             // [128] rows
    static_assert(16 * 64 * 16 + (AT_LAT + 128) * 2 <= TOPK_ARENA_WORDS * 4, "merge LDS");
    uint16_t* obuf = p.uv_obuf[tag & 1u];
    for (int task = b; task < ntask32; task += nblk) {
      const int tid = opaque_v((int)threadIdx.x), l = tid & 63;
      if (!ok) break;
      int r, h;
      task_of(task, r, h);
      if (r >= R) continue;
      const int n = row_n(r);
      const int k = n < AT_TOPK ? n : AT_TOPK;
      const int nsp = (k + SPLIT - 1) / SPLIT;
      // W_UV's weights of head h, ahead of the wait (they depend on nothing of the launch)
      UvUnit uu;
      if constexpr (uv) uu.load(p.uv_w, p.uv_s, p.uv_shuf, h, tid, true);
      if (w == 0 && nsp > 0)
        ok = wait_until(guard, MONO_SITE_SPLIT, [&]() {
          return __all(l >= nsp || ld_dev(&split_done[r * AT_NSPLIT + l]) == tag);
        });
      ok = cta_all(ok, ok_s);
      if (!ok) break;
      // thread d < 512: output dim d. Its 32 split terms (bf16, a wave's 64 dims of a split
      // are 128 contiguous bytes) and, in every wave, the splits' (m, l) (lane s: split s)
      // in one round trip; each wave forms the weights exp(m_s - M) itself (no LDS round
      // trip), then the terms scaled and summed in split order.
      if (tid < AT_LAT) {
        // through L2: within the launch the partials are only stored (write-through) before
        // the done words this CTA waited for, so no L2 holds a stale copy
        const __amdgpu_buffer_rsrc_t ra =
            rsrc(accs + ((size_t)r * AT_NSPLIT * AT_HEADS + h) * AT_LAT,
                 (uint32_t)(nsp * AT_HEADS * AT_LAT * 2));
        uint32_t v[AT_NSPLIT];
#pragma unroll
        for (int sp = 0; sp < AT_NSPLIT; ++sp)
          v[sp] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(
              ra, (uint32_t)(tid + sp * AT_HEADS * AT_LAT) * 2u, 0, CP_NONE);
        const float* ml = mls + (size_t)r * AT_NSPLIT * AT_HEADS * 2;
        const bool on = l < nsp;
        const v2i mlv = ld8<CP_NONE>(rsrc(ml, AT_NSPLIT * AT_HEADS * 8),
                                    on ? (uint32_t)((l * AT_HEADS + h) * 8) : 0x80000000u);
        const float m = on ? __int_as_float(mlv[0]) : -INFINITY;
        const float ls = on ? __int_as_float(mlv[1]) : 0.f;
        const float M = wave_max(m);
        const float ws = on ? expf(m - M) : 0.f;
        const float L = wave_sum(ws * ls);
        const float linv = L > 0.f ? 1.0f / L : 0.f;
        float acc = 0.f;
#pragma unroll
        for (int sp = 0; sp < AT_NSPLIT; ++sp) {
          const float wsp = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ws), sp));
          const float term = __fmul_rn(bf16_lo(v[sp]), wsp);
          acc = sp < nsp ? __fadd_rn(acc, term) : acc;
        }
        const uint32_t ob = bf16_bits(acc * linv);
        // device coherent: in the layer launch the output block reads it next
        __builtin_amdgcn_raw_buffer_store_b16(
            (uint16_t)ob, rsrc(p.out, (uint32_t)R * AT_HEADS * AT_LAT * 2u),
            (uint32_t)((r * AT_HEADS + h) * AT_LAT + tid) * 2u, 0, CP_DEV);
        if constexpr (uv) uvx[tid] = (uint16_t)ob;
      }
      __syncthreads();
      if constexpr (uv) {
        uu.dot(uvx, uvred, tid);
        __syncthreads();
        if (tid < 128) uob[tid] = (uint16_t)bf16_bits(UvUnit::row(uvred, tid));
        __syncthreads();
        UvUnit::store(uob, tid,
                      reinterpret_cast<uint32_t*>(obuf + ((size_t)r * AT_HEADS + h) * 128),
                      0xFFFFFFFFu, nullptr);
        __syncthreads();
      }
    }
  }

}

}  // namespace mono
