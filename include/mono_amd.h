/* C ABI of the MI355X (gfx950) DSA decoder-layer monokernel library, libmono_amd.so.
 *
 * Plain pointers and sizes only: every tensor is a device address the caller owns,
 * except the scratch and guard blocks a runtime allocates once (sizes from the
 * *_scratch_bytes functions). Every entry point returns 0 or a negative MONO_E* code
 * (never throws); mono_last_error() gives the message of the last failure on the
 * calling thread. Launches are asynchronous on the given HIP stream, do no host
 * synchronisation, and hold no host state between calls, so they can be captured in
 * a HIP graph.
 *
 * What each entry point replaces in the reference (yuychang/sgl-amd-mono) is cited on
 * its declaration. */
#ifndef MONO_AMD_H
#define MONO_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* an opaque HIP stream (hipStream_t); 0 is the default stream */
typedef void* mono_stream_t;

#define MONO_OK 0
#define MONO_E_ARG (-1)     /* bad argument: null pointer, shape or size */
#define MONO_E_DEVICE (-2)  /* not a gfx950 device, or the grid cannot be co-resident */
#define MONO_E_LAUNCH (-3)  /* the HIP runtime refused the launch */
#define MONO_E_FAILED (-4)  /* an earlier launch on this guard block timed out */

/* The guard block: int32 words, runtime owned, zeroed at allocation. Words 0-5 keep
 * the meaning of the reference's epoch buffer (sgl_amd_mono/common/guard.py:16-30). */
#define MONO_GUARD_EPOCH 0        /* launches completed on this block (the tag base) */
#define MONO_GUARD_DEADLINE_LO 1  /* wait deadline, 100 MHz ticks, low word */
#define MONO_GUARD_DEADLINE_HI 2  /* ... high word */
#define MONO_GUARD_ERR_DEADLINE 3 /* 1 + the site of the first wait that timed out */
#define MONO_GUARD_ERR_PEER 4     /* reserved: a failure seen on another GPU */
#define MONO_GUARD_ERR_FAULT 5    /* set when the timed-out wait was fault-injected */
#define MONO_GUARD_EXIT 6         /* CTAs of the running launch that finished */
#define MONO_GUARD_ABORT 7        /* set on a failure: every other wait gives up */
#define MONO_GUARD_WORDS 16

#define MONO_CLOCK_HZ 100000000 /* s_memrealtime */

/* Wait sites (the value in MONO_GUARD_ERR_DEADLINE is 1 + site). */
#define MONO_SITE_LOGITS 1   /* routing waits on the router's logits */
#define MONO_SITE_MID 2      /* a mid quant task waits on up/gate tiles */
#define MONO_SITE_MQ 3       /* an expert-down tile waits on a quantised mid block */
#define MONO_SITE_SCORES 4   /* a row's top-k waits on its indexer scores */
#define MONO_SITE_TOPK 5     /* a sparse-MLA split waits on its row's top-k */
#define MONO_SITE_SPLIT 6    /* a merge waits on its row's splits */
#define MONO_SITE_O 7        /* o_proj waits on the W_UV outputs */
#define MONO_SITE_FRONT_A 8  /* a row task waits on the q_a | kv_a | index-key outputs */
#define MONO_SITE_QAN 9      /* q_b / W_iq wait on the normalised q_a */
#define MONO_SITE_QB 10      /* W_UK / the index query wait on q_b / W_iq outputs */
#define MONO_SITE_PHASE 11   /* a phase of the layer launch waits for the phase before it */
#define MONO_SITE_BLOCKS 12  /* a long row's final top-k waits on its blocks' selections */
#define MONO_SITE_X 13       /* a stage-A task waits on the normalised input rows x */

int mono_version(void);
const char* mono_last_error(void);

/* Device facts the host checks at load: gfx950, CU count, LDS per CU.
 * Replaces the co-residency check of sgl_amd_mono/minimax_m31/residency.py:66-85. */
typedef struct {
  int32_t cus;
  int32_t lds_bytes;
  int32_t is_gfx950;
  int32_t grid; /* CTAs of a monokernel launch: one per CU */
} MonoDeviceInfo;
int mono_device_info(int32_t device, MonoDeviceInfo* out);

/* Write the wait deadline (seconds -> 100 MHz ticks) into a guard block.
 * Replaces Glm53Runtime.set_deadline (sgl_amd_mono/glm53/gfx950/runner.py:197-204)
 * and guard.deadline_ticks (sgl_amd_mono/common/guard.py:69-76). */
int mono_set_deadline(int32_t* guard, double seconds, mono_stream_t stream);

/* Zero a scratch and guard block with a fill kernel (graph safe): required after a
 * launch failed, since a failed launch leaves hand-off words half written. The
 * reference stops the process instead (sgl_amd_mono/common/guard.py:91-97). */
int mono_reset(void* scratch, size_t scratch_bytes, int32_t* guard, mono_stream_t stream);

/* ------------------------------------------------------------------------------
 * FP8 routed MoE: the FFN half of the layer as one persistent launch.
 * post-attention RMSNorm -> router GEMV + sigmoid -> top-8 (+ shared expert) ->
 * W8A8 expert up/gate + SiLU -> mid per-128 quant -> expert down, route weighting
 * -> out = a + y (the local residual add of the W == 1 reduce).
 * Replaces stages 8-10 of the reference layer kernel:
 * sgl_amd_mono/glm53/gfx950/kernel.py:4199-4330 (norm, router, activation quant),
 * :1575-1629 + :4332-4350 (routing), :4352-4999 (up/gate), :5001-5187 (down), and
 * the W == 1 peer_reduce branch :1665-1669. */
/* On-HBM layouts of FP8 expert weights [.., N, K] */
/* Index-key caches (the indexer's keys, one per token, read in place):
 * MONO_INDEX_FP4_PLANE  SGLang's FP4 index plane: plane [pages, 4, 64, 16] E2M1 and
 *                       plane_scale [pages, 4, 64] E8M0 (the attention launch's layout note)
 * MONO_INDEX_FP8_PAGE   SGLang's DSA index page on HIP: [pages, 8448] bytes, 64 tokens x 128
 *                       E4M3 values in 16-token x 16-byte tiles (token t, dim d at (t / 16)
 *                       * 2048 + (d / 16) * 256 + (t % 16) * 16 + d % 16), then the 64 tokens'
 *                       power-of-two f32 scales (sgl_amd_mono/glm53/gfx950/kernel.py:534-550);
 *                       plane_scale unused
 * MONO_INDEX_FP8_ROWS   the same page with token-major values (t * 128 + d)
 * With an FP8 page the index query iq is bf16 [R, 64, 128] (rotated, transformed, then
 * rounded to bf16 once) and iqs is unused. */
#define MONO_INDEX_FP4_PLANE 0
#define MONO_INDEX_FP8_PAGE 1
#define MONO_INDEX_FP8_ROWS 2

/* Expert weights of the layer launch (the reference's MoE modes W8A8 and A16W4,
 * sgl_amd_mono/glm53/gfx950/config.py:15-21,88-93):
 * MONO_EXPERTS_FP8    E4M3 w13 [257, 1024, 7168] + f32 s13 [257, 8, 56] and w2 [257, 7168,
 *                     512] + s2 [257, 56, 4] (128 x 128 blocks), W8A8 on per-128 E4M3 rows
 * MONO_EXPERTS_MXFP4  E2M1 codes (two a byte, the even K index in the low nibble) w13
 *                     [257, 1024, 3584] + E8M0 e13 [257, 1024, 224] and w2 [257, 7168, 256] +
 *                     e2 [257, 7168, 16] (one scale per 32 values), A16W4: the bf16 rows,
 *                     mid = bf16(silu(gate) up), the route weight on each expert's f32 down
 *                     sum; at most 8 rows. Layout AITER16: codes in the (16, 16) byte shuffle,
 *                     scales in the e8m0 shuffle (the MXFP4 MoE launch's layout note) */
#define MONO_EXPERTS_FP8 0
#define MONO_EXPERTS_MXFP4 1

#define MONO_LAYOUT_ROWMAJOR 0 /* plain row-major E4M3 */
#define MONO_LAYOUT_AITER16 1  /* AITER (16, 16) shuffle: [N / 16, K / 32, 2, 16, 16 B],
                                  SGLang's in-place layout on gfx950
                                  (sgl_amd_mono/glm53/gfx950/kernel.py:787-808) */

typedef struct {
  int32_t rows;            /* R, 1..16 */
  int32_t hidden;          /* 7168 */
  int32_t inter;           /* expert intermediate per GPU: 512 */
  int32_t experts;         /* routed experts: 256 (the shared one is id 256) */
  int32_t layout;          /* MONO_LAYOUT_* of w13 and w2 */
  float eps;               /* RMSNorm epsilon */
  float route_scale;       /* routed_scaling_factor, 2.5 */
  const void* a;           /* bf16 [R, H]: the stream after attention */
  void* out;               /* bf16 [R, H]: a + MoE(a) */
  const void* g_post;      /* bf16 [H]: post-attention norm weight */
  const void* w_r;         /* bf16 [E, H]: router */
  const float* bias;       /* f32 [E]: e_score_correction_bias */
  const uint8_t* w13;      /* E4M3 [E + 1, 2 I, H]: gate rows then up rows */
  const float* s13;        /* f32 [E + 1, 2 I / 128, H / 128] */
  const uint8_t* w2;       /* E4M3 [E + 1, H, I] */
  const float* s2;         /* f32 [E + 1, H / 128, I / 128] */
  float* y;                /* optional f32 [R, H]: the MoE sum alone */
  float* scores;           /* optional f32 [R, E]: sigmoid(logit) */
  int32_t* ids;            /* optional i32 [R, 9]: slot 0 shared (256), then picks */
  float* weights;          /* optional f32 [R, 9]: slot 0 1.0, then route weights */
  void* scratch;           /* runtime owned, mono_moe_fp8_scratch_bytes() */
  int32_t* guard;          /* runtime owned guard block */
  uint32_t* host_error;    /* optional pinned host word: 1 + failed site */
  int32_t fault_site;      /* test fault injection: this wait site stalls (0: none) */
  int32_t fault_after;     /* ... once the epoch reached this many launches */
  uint64_t* timeline;      /* optional u64 [grid, 8]: per-CTA s_memrealtime stamps at the
                              stage boundaries (MONO_TL_*), as the reference's timeline
                              build (sgl_amd_mono/common/stamps.py:16-33) */
  int32_t n_group;         /* group-limited routing (DeepSeek-V3's n_group): 0 or 1 none;
                              else 2..16 groups of 256 / n_group consecutive experts */
  int32_t topk_group;      /* groups kept (topk_group * 256 / n_group >= 8) */
} MonoMoeFp8Args;

/* timeline marks of the MoE launch */
#define MONO_TL_START 0
#define MONO_TL_STAGED 1  /* norm, activation quant and router logits published */
#define MONO_TL_ROUTED 2  /* routing and the distinct-expert list in LDS */
#define MONO_TL_UPGATE 3  /* this CTA's up/gate tasks done */
#define MONO_TL_MIDQ 4    /* this CTA's mid quant tasks done */
#define MONO_TL_DOWN 5    /* this CTA's down tasks done */
#define MONO_TL_END 6
#define MONO_TL_COLS 8

size_t mono_moe_fp8_scratch_bytes(int32_t hidden, int32_t inter, int32_t experts);
int mono_moe_fp8_launch(const MonoMoeFp8Args* args, mono_stream_t stream);

/* mono_moe_fp8_launch without any allocation, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. The scratch and the guard block live in
 * a static device array of this library (20.9 MiB a GPU, held until the process ends,
 * its address looked up once per device on the first call there): args->scratch and
 * args->guard must be null; hidden 7168, inter 512, 256 experts and at most 16 rows,
 * else MONO_E_ARG. Every call on one GPU shares that GPU's block and its launch tags, so
 * calls that overlap on one GPU (two streams, no ordering) race; calls ordered on one
 * stream are safe. The waits use the library's default 10 s deadline. A timed-out call
 * leaves the block unusable: pass a pinned host_error word, and a call seeing it
 * non-zero is refused with MONO_E_FAILED. That refusal happens on the host, when the
 * call is made: a launch captured in a HIP graph is not refused at replay, so after a
 * timeout every replay runs on the aborted block and only fills out (and y) with NaN.
 * Nothing resets the static block short of ending the process. */
int mono_moe_fp8_launch_static(const MonoMoeFp8Args* args, mono_stream_t stream);

/* ------------------------------------------------------------------------------
 * MXFP4 (A16W4) routed MoE as one persistent launch: the gate logits are given, the
 * rows x are bf16 and stay bf16 (no activation quant); experts are E2M1 codes (two a
 * byte, the even K index in the low nibble) with one E8M0 scale per 32 K values.
 * sigmoid(logits) + bias top-8 (+ the shared expert in slot 0) -> up/gate with each
 * 32-group dequantised exactly to bf16 -> mid = bf16(silu(g) * u) -> down, route
 * weighting -> out = bf16(res + y) (or bf16(y) without res).
 * Replaces the A16W4 expert stage of the reference's FFN launch
 * (sgl_amd_mono/minimax_m31/a16w4.py:26-92 operands; route as
 * test/kernels/test_minimax_m31_ffn.py:146-151) and the MXFP4 units of the layer
 * kernel (sgl_amd_mono/glm53/gfx950/kernel.py:906-995).
 * Layouts: MONO_LAYOUT_ROWMAJOR = codes [E + 1, N, K / 2], scales [E + 1, N, K / 32];
 * MONO_LAYOUT_AITER16 = codes in the AITER (16, 16) byte shuffle and scales in the
 * e8m0 shuffle of sgl_amd_mono/common/mx.py:40-44, [E + 1, N, C] with C = K / 32
 * rounded up to a multiple of 8 (the map groups columns by 8). One CTA a CU; the grid
 * must hold the hidden / 16 = 192 down tasks, one a CTA (MONO_E_DEVICE otherwise). */
typedef struct {
  int32_t rows;            /* R, 1..16 */
  int32_t hidden;          /* 3072 */
  int32_t inter;           /* expert intermediate per GPU: 384 */
  int32_t experts;         /* routed experts: 256 (the shared one is id 256) */
  int32_t layout;          /* MONO_LAYOUT_* of the codes and scales */
  float route_scale;       /* routed_scaling_factor */
  const void* x;           /* bf16 [R, H]: the expert input rows */
  const void* res;         /* optional bf16 [R, H]: residual added to y */
  void* out;               /* bf16 [R, H]: res + y */
  const float* logits;     /* f32 [R, E]: gate logits */
  const float* bias;       /* f32 [E]: e_score_correction_bias */
  const uint8_t* w13;      /* E2M1 x2 [E + 1, 2 I, H / 2]: gate rows then up rows */
  const uint8_t* s13;      /* E8M0 [E + 1, 2 I, H / 32] (or the AITER16 shuffle) */
  const uint8_t* w2;       /* E2M1 x2 [E + 1, H, I / 2] */
  const uint8_t* s2;       /* E8M0 [E + 1, H, I / 32] (or the AITER16 shuffle) */
  float* y;                /* optional f32 [R, H]: the MoE sum alone */
  float* scores;           /* optional f32 [R, E]: sigmoid(logit) */
  int32_t* ids;            /* optional i32 [R, 9]: slot 0 shared (256), then picks */
  float* weights;          /* optional f32 [R, 9]: slot 0 1.0, then route weights */
  void* scratch;           /* runtime owned, mono_moe_mxfp4_scratch_bytes() */
  int32_t* guard;          /* runtime owned guard block */
  uint32_t* host_error;    /* optional pinned host word: 1 + failed site */
  int32_t fault_site;      /* test fault injection (MONO_SITE_MID: the down wait) */
  int32_t fault_after;
  uint64_t* timeline;      /* optional u64 [grid, 8]: MONO_TL_* stamps (MIDQ: the wait for
                              every mid tile ended) */
  int32_t n_group;         /* group-limited routing (DeepSeek-V3's n_group): 0 or 1 none;
                              else 2..16 groups of 256 / n_group consecutive experts */
  int32_t topk_group;      /* groups kept (topk_group * 256 / n_group >= 8) */
} MonoMoeMxfp4Args;

size_t mono_moe_mxfp4_scratch_bytes(int32_t hidden, int32_t inter, int32_t experts);
int mono_moe_mxfp4_launch(const MonoMoeMxfp4Args* args, mono_stream_t stream);

/* ------------------------------------------------------------------------------
 * The attention phase as one persistent launch: FP4 indexer scores of every key a row
 * sees, their exact top-2048 (ranked by the radix order of the f32 score, ties to the
 * lower position, kept in ascending position order; every key when a row sees at
 * most 2048), and sparse MLA decode of the absorbed queries over the selected tokens'
 * FP8 cache rows, merged across splits into the latent output (before W_UV).
 * Replaces the index-score, top-k, split and merge stages of the reference layer
 * kernel: sgl_amd_mono/glm53/gfx950/kernel.py:2684-3000 (scores; FP4 form
 * sgl_amd_mono/deepseek_v41/gfx950/indexer/score_fp4.py:254-296), :3002-3636 (exact
 * top-k), :3638-3973 (split), :3975-4123 (merge, without W_UV).
 * Layouts (SGLang's FP4 index plane, sgl_amd_mono/deepseek_v41/gfx950/indexer/
 * score_fp4.py:11-14): plane [pages, 4 (32-dim chunk), 64 (slot), 16 B] E2M1, low
 * nibble first; plane_scale [pages, 4, 64] E8M0, slot s's byte at (s % 16) * 4 + s / 16;
 * iq [R, 64 heads, 64 B] E2M1; iqs [R, 4 (chunk), 16 (head % 16), 4 (head / 16)] E8M0.
 * The score of key t: sum_h iw[h] relu(sum_c 2^(qe - 127) 2^(ke - 127) iq[h, c] . k[t, c]).
 * KV: kv [slots, 576] E4M3 (latent 512, rope 64) times kv_scale[slot] (1 without
 * kv_scale: SGLang's raw E4M3 rows); a key's slot is
 * page_table[req_ids[row], pos / 64] * 64 + pos % 64. Timeline marks 1-5 of this launch:
 * scores, top-k, splits, merge done, exit. */
typedef struct {
  int32_t rows;          /* R, 1..rows_max: decode rows, row r at positions[r] of req_ids[r] */
  int32_t rows_max;      /* 1..48: the rows the scratch was sized for (mono_attn_scratch_bytes);
                            every launch on one scratch passes the same value */
  int32_t heads;         /* 32 */
  int32_t index_heads;   /* 64 */
  int32_t topk;          /* 2048 */
  int32_t page;          /* 64 */
  int32_t ctx_max;       /* keys a row may see at most (positions clamp to it): 1..163840;
                            the row stride of `scores` */
  int32_t pt_stride;     /* page_table row stride (entries), >= ceil(ctx_max / 64) */
  int32_t pt_rows;       /* page_table rows */
  uint32_t plane_pages;  /* pages of plane / plane_scale */
  uint32_t kv_slots;     /* rows of kv / kv_scale */
  float sm_scale;        /* softmax scale, (nope + rope)^-0.5 times any YaRN factor */
  const int64_t* positions;  /* i64 [R]: the row's position (keys 0..position); < 0: none */
  const int32_t* req_ids;    /* i32 [R] */
  const int32_t* page_table; /* i32 [pt_rows, pt_stride] */
  const void* q;             /* bf16 [R, 32, 576]: absorbed latent query, then rope */
  const uint8_t* iq;
  const uint8_t* iqs;
  const float* iw;           /* f32 [R, 64]: index head weights */
  const uint8_t* plane;
  const uint8_t* plane_scale;
  const uint8_t* kv;
  const float* kv_scale;     /* optional f32 [slots]: per-token scales (null: every row is
                                raw E4M3 at scale 1, the layout of SGLang's FP8 MLA pool) */
  void* out;                 /* bf16 [R, 32, 512] */
  float* scores;             /* optional f32 [R, ctx_max]: the indexer scores */
  int32_t* topk_pos;         /* optional i32 [R, 2048]: selected positions, -1 past count */
  void* scratch;             /* runtime owned, mono_attn_scratch_bytes() */
  int32_t* guard;
  uint32_t* host_error;
  int32_t fault_site;        /* test fault injection (MONO_SITE_SCORES/TOPK/SPLIT) */
  int32_t fault_after;
  uint64_t* timeline;
  int32_t index_format;      /* MONO_INDEX_*: plane / plane_scale and iq / iqs as it says */
} MonoAttnArgs;

size_t mono_attn_scratch_bytes(int32_t rows_max);
int mono_attn_launch(const MonoAttnArgs* args, mono_stream_t stream);

/* ------------------------------------------------------------------------------
 * The attention output block as one persistent launch: the merged latent o_lat through
 * W_UV per head (o, handed over in bf16), o_proj, and the residual add of the W == 1
 * reduce: out = bf16(h + W_o o). FP8 E4M3 weights with f32 128 x 128 block scales, read
 * in place (MONO_LAYOUT_*), widened exactly to bf16 against bf16 activations.
 * Replaces sgl_amd_mono/glm53/gfx950/kernel.py:3975-4123 (W_UV after the merge),
 * :4125-4197 (o_proj + residual) and the W == 1 peer_reduce branch :1665-1669. */
typedef struct {
  int32_t rows;          /* R, 1..16 */
  int32_t heads;         /* 32 */
  int32_t hidden;        /* 7168 */
  int32_t layout;        /* MONO_LAYOUT_* of w_uv and w_o */
  const void* o_lat;     /* bf16 [R, 32, 512]: the merged latent attention output */
  const void* h;         /* bf16 [R, 7168]: the residual stream */
  const uint8_t* w_uv;   /* E4M3 [32, 128, 512] */
  const float* s_uv;     /* f32 [32, 1, 4] */
  const uint8_t* w_o;    /* E4M3 [7168, 4096] */
  const float* s_o;      /* f32 [56, 32] */
  void* out;             /* bf16 [R, 7168]: h + o_proj(o) */
  void* o;               /* optional bf16 [R, 4096]: W_UV's output (else kept in scratch) */
  void* scratch;         /* runtime owned, mono_post_scratch_bytes() */
  int32_t* guard;
  uint32_t* host_error;
  int32_t fault_site;    /* test fault injection (MONO_SITE_O) */
  int32_t fault_after;
  uint64_t* timeline;    /* marks 1: W_UV done, 2: o_proj done */
} MonoPostArgs;

size_t mono_post_scratch_bytes(void);
int mono_post_launch(const MonoPostArgs* args, mono_stream_t stream);

/* ------------------------------------------------------------------------------
 * The front of the layer as one persistent launch: from the layer input h to the
 * attention launch's inputs (q, iq, iqs, iw), with the rows' KV and index-key cache
 * writes. x = bf16(rmsnorm(h) g_in); q_a | kv_a, the index key and the head weights off
 * x; q_an = bf16(rmsnorm(q_a) g_q); the KV row (kv_n = bf16(rmsnorm(kv_a[:512]) g_kv),
 * k_pe = bf16(rope(kv_a[512:]))) as E4M3 at the row's slot, with a power-of-two
 * per-token scale or, without kv_scale, raw at scale 1; the index key (LayerNorm, RoPE on dims 0..63, FWHT-128, FP4 e2m1 + e8m0
 * per 32) into the index plane at the slot; q_b over q_an (nope bf16, rope rotated),
 * q_lat = bf16(W_UK q_nope); the index query (W_iq q_an, RoPE, FWHT, FP4); the head
 * weights bf16(W_w x) 128^-1/2 64^-1/2. The index key and query are rounded to bf16 at
 * the points of the reference's FP4 indexer (after the key's LayerNorm, after RoPE and
 * after the FWHT: sgl_amd_mono/deepseek_v4/gfx950/kernels/stages/indexer.py:242-254,
 * 330-335). RoPE pairs are interleaved (x0 c - x1 s,
 * x0 s + x1 c) with bf16 tables cos/sin [rope_rows, 32] indexed by position. A slot
 * outside the caches (e.g. -1, a pad row) writes nothing. With a DSA index page
 * (MONO_INDEX_FP8_*) the index key's LayerNorm, RoPE and FWHT are not rounded and it is
 * stored as E4M3 at a power-of-two per-token scale 2^ceil(log2(max(amax, 1e-4) / 448)),
 * and the index query is rotated and transformed unrounded, then bf16 once
 * (sgl_amd_mono/glm53/gfx950/kernel.py:2103-2168, 2928-2944).
 * Replaces sgl_amd_mono/glm53/gfx950/kernel.py:1781-2443 (stages qkv_a, q_norm, cache,
 * q_b, index_q, uk) and the FP4 index paths of
 * sgl_amd_mono/deepseek_v4/gfx950/kernels/stages/indexer.py:143-151,311-338,340-408. */
typedef struct {
  int32_t rows;          /* R, 1..8 */
  int32_t hidden;        /* 7168 */
  int32_t heads;         /* 32 */
  int32_t layout;        /* MONO_LAYOUT_* of the FP8 weights */
  int32_t rope_rows;     /* rows of cos / sin */
  uint32_t kv_slots;     /* rows of kv */
  uint32_t plane_pages;  /* pages of the index plane */
  float eps;             /* RMSNorm epsilon (1e-6 for DeepSeek) */
  const void* h;         /* bf16 [R, 7168] */
  const void* g_in;      /* bf16 [7168] input RMSNorm weight */
  const void* g_q;       /* bf16 [1536] */
  const void* g_kv;      /* bf16 [512] */
  const uint8_t* w_qkv_a; const float* s_qkv_a;  /* E4M3 [2112, 7168] + f32 [17, 56] */
  const uint8_t* w_k; const float* s_k;          /* E4M3 [128, 7168] + f32 [1, 56] */
  const void* w_w;                               /* bf16 [64, 7168] */
  const float* g_k; const float* b_k;            /* f32 [128] index-key LayerNorm */
  const uint8_t* w_qb; const float* s_qb;        /* E4M3 [6144, 1536] + f32 [48, 12] */
  const uint8_t* w_iq; const float* s_iq;        /* E4M3 [8192, 1536] + f32 [64, 12] */
  const uint8_t* w_uk; const float* s_uk;        /* E4M3 [32, 512, 128] + f32 [32, 4, 1] */
  const void* cos; const void* sin;              /* bf16 [rope_rows, 32] */
  const int64_t* positions;  /* [R] */
  const int64_t* slots;      /* [R] cache slot (page * 64 + offset), -1 = none */
  uint8_t* kv;               /* E4M3 [kv_slots, 576] */
  float* kv_scale;           /* optional f32 [kv_slots]: written with a power-of-two per-token
                                scale; null: raw E4M3 at scale 1 (SGLang's pool layout),
                                values saturating at +-448 */
  uint8_t* plane;            /* [plane_pages, 4, 64, 16], or DSA pages [plane_pages, 8448] */
  uint8_t* plane_scale;      /* [plane_pages, 4, 64] (FP4 plane only) */
  void* q;                   /* out bf16 [R, 32, 576]: q_lat | q_pe */
  uint8_t* iq;               /* out [R, 64, 64] E2M1 (DSA pages: bf16 [R, 64, 128]) */
  uint8_t* iqs;              /* out [R, 4, 16, 4] E8M0 (FP4 plane only) */
  float* iw;                 /* out f32 [R, 64] */
  void* scratch;             /* runtime owned, mono_front_scratch_bytes() */
  int32_t* guard;
  uint32_t* host_error;
  int32_t fault_site;        /* test fault injection (MONO_SITE_FRONT_A / QAN / QB / X) */
  int32_t fault_after;
  uint64_t* timeline;
  float* ik_raw;             /* optional out f32 [R, 128]: the index key W_k x, before its
                                LayerNorm */
  void* iq_raw;              /* optional out bf16 [R, 64, 128]: the index query W_iq q_an,
                                before its RoPE */
  int32_t index_format;      /* MONO_INDEX_*: the index key written as it says, iq / iqs
                                made for it */
} MonoFrontArgs;

size_t mono_front_scratch_bytes(void);
int mono_front_launch(const MonoFrontArgs* args, mono_stream_t stream);

/* ------------------------------------------------------------------------------
 * The whole decoder layer as ONE persistent launch: the front, the attention phase, the
 * output block and the MoE above (FP8 or MXFP4 experts: expert_format), run back to
 * back in every CTA of one launch with a
 * deadline-guarded grid barrier between phases (each phase's input-independent loads,
 * weights and index pages, issued before it waits). out = the layer's output stream
 * (h + attention block + MoE), bf16 [R, 7168].
 * Replaces the reference's per-layer launch Glm53LayerOp.launch(h, caches, cos, sin, step)
 * (sgl_amd_mono/glm53/gfx950/runner.py:240-321) and its one-launch kernel
 * (sgl_amd_mono/glm53/gfx950/kernel.py:171-5282, arguments :5191-5234), for one GPU's
 * TP=4 share with the W == 1 reduces as local residual adds (:1665-1669). Every tensor
 * has the meaning and layout of the per-phase launches' arguments above. */
typedef struct {
  int32_t rows;          /* R, 1..rows_max */
  int32_t rows_max;      /* 1..8: the rows the scratch was sized for (mono_layer_scratch_bytes) */
  int32_t hidden;        /* 7168 */
  int32_t heads;         /* 32 */
  int32_t inter;         /* 512 */
  int32_t experts;       /* 256 */
  int32_t layout;        /* MONO_LAYOUT_* of every FP8 weight */
  int32_t ctx_max;       /* keys a row may see at most, 1..163840 */
  int32_t pt_stride;     /* page_table row stride */
  int32_t pt_rows;       /* page_table rows */
  int32_t rope_rows;     /* rows of cos / sin */
  uint32_t kv_slots;     /* rows of kv */
  uint32_t plane_pages;  /* pages of the index plane */
  float eps;             /* RMSNorm epsilon */
  float sm_scale;        /* softmax scale */
  float route_scale;     /* routed_scaling_factor */
  const void* h;         /* bf16 [R, 7168]: the layer's input stream */
  void* out;             /* bf16 [R, 7168]: the layer's output stream */
  const int64_t* positions; /* [R] */
  const int64_t* slots;     /* [R] cache slot of the row's key (-1: none) */
  const int32_t* req_ids;   /* [R] */
  const int32_t* page_table; /* [pt_rows, pt_stride] */
  uint8_t* kv; float* kv_scale;            /* E4M3 [kv_slots, 576] (+ optional per-token scales) */
  uint8_t* plane; uint8_t* plane_scale;    /* FP4 index plane [pages, 4, 64, 16] + [pages, 4, 64] */
  const void* g_in; const void* g_q; const void* g_kv;   /* bf16 RMSNorm weights */
  const uint8_t* w_qkv_a; const float* s_qkv_a;
  const uint8_t* w_k; const float* s_k;
  const void* w_w;
  const float* g_k; const float* b_k;
  const uint8_t* w_qb; const float* s_qb;
  const uint8_t* w_iq; const float* s_iq;
  const uint8_t* w_uk; const float* s_uk;
  const void* cos; const void* sin;
  const uint8_t* w_uv; const float* s_uv;
  const uint8_t* w_o; const float* s_o;
  const void* g_post; const void* w_r; const float* bias;
  const uint8_t* w13; const float* s13; const uint8_t* w2; const float* s2;
  /* optional: where the phases hand their results to each other (null: in scratch) */
  void* q;               /* bf16 [R, 32, 576] */
  uint8_t* iq;           /* [R, 64, 64] */
  uint8_t* iqs;          /* [R, 4, 16, 4] */
  float* iw;             /* f32 [R, 64] */
  void* o_lat;           /* bf16 [R, 32, 512] */
  void* a;               /* bf16 [R, 7168]: the stream after attention */
  /* optional outputs */
  float* scores;         /* f32 [R, ctx_max]: the indexer scores */
  int32_t* topk_pos;     /* i32 [R, 2048] */
  float* y;              /* f32 [R, 7168]: the MoE sum alone */
  float* moe_scores;     /* f32 [R, 256] */
  int32_t* ids;          /* i32 [R, 9] */
  float* weights;        /* f32 [R, 9] */
  void* scratch;         /* runtime owned, mono_layer_scratch_bytes(rows_max), zeroed */
  int32_t* guard;        /* runtime owned guard block */
  uint32_t* host_error;  /* optional pinned host word: 1 + failed site */
  int32_t fault_site;    /* test fault injection: any MONO_SITE_* */
  int32_t fault_after;
  uint64_t* timeline;    /* optional u64 [grid, 8]: start, front, attention, output block,
                            MoE done, exit */
  uint64_t* phase_timeline; /* optional u64 [4, grid, 8]: each phase's own stamps (the
                               marks of its launch of its own), front, attention, output
                               block, MoE */
  int32_t n_group;       /* group-limited routing: 0 or 1 none, else 2..16 groups */
  int32_t topk_group;    /* groups kept (topk_group * 256 / n_group >= 8) */
  int32_t index_format;  /* MONO_INDEX_* of plane / plane_scale (and so of iq / iqs) */
  int32_t expert_format; /* MONO_EXPERTS_*: FP8 (w13, s13, w2, s2) or MXFP4 (w13, e13, w2,
                            e2; s13 / s2 unused) experts */
  const uint8_t* e13;    /* MXFP4: E8M0 scales of w13 */
  const uint8_t* e2;     /* MXFP4: E8M0 scales of w2 */
} MonoLayerArgs;

size_t mono_layer_scratch_bytes(int32_t rows_max);
int mono_layer_launch(const MonoLayerArgs* args, mono_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* MONO_AMD_H */
