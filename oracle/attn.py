"""The attention phase of the layer, restated on the CPU (test infrastructure only).

* FP4 indexer scores over SGLang's FP4 index plane (``sgl_amd_mono/deepseek_v41/gfx950/
  indexer/score_fp4.py:1-20`` layouts; formula as the reference's fp64 check
  ``test/kernels/test_deepseek_v41_k2i.py:149-166``):
  s[t] = sum_h w_h relu(sum_c 2^(qe[h,c]-127) 2^(ke[t,c]-127) q[h,c,:] . k[t,c,:]).
  Plane: payload [pages, 4 (32-dim chunk c), 64 (slot), 16 B] E2M1 (low nibble first),
  scales [pages, 4, 64] E8M0 with slot s's byte at (s % 16) * 4 + s // 16; query
  [H, 64 B] E2M1 with scales [4 (c), 16 (h % 16), 4 (h // 16)] E8M0.
* exact top-k of those scores (``oracle/topk.py``).
* sparse MLA decode over the selected tokens (``sgl_amd_mono/glm53/gfx950/kernel.py:
  3638-4123``; softmax scale ``glm53/gfx950/config.py:180-181``): K = V = the cached
  576-value row (latent 512 + rope 64) of each selected token, E4M3 times the token's
  f32 scale; scores = q . k * sm_scale, softmax over the selected tokens, o = P V[:, :512].
* or the DSA (FP8) indexer scores (``index_scores_fp8``) over SGLang's DSA index pages:
  [pages, 64 x 128 E4M3 values (16-token x 16-byte tiles, or token-major), 64 f32
  scales], a bf16 query [64, 128] (``kernel.py:2684-2842``, layout :534-550).

Pinned by ``tests/test_oracle_attn.py``: the scores against a dense dequantisation
built slot by slot from bit fields and an independent matmul; a scale-code shift
doubling them exactly; sparse MLA against ``torch.nn.functional.scaled_dot_product_attention``
in f64; the selection of the chain against ``topk_sort``; the DSA (FP8) page keys
against a byte-by-byte decode through the reference's token formula, and their scores
against one-hot queries and keys whose scores are closed forms.
"""

from __future__ import annotations

import numpy as np
import torch

from . import formats as F
from .front import dsa_value_offset
from .topk import topk_sort

PAGE = 64
KV_DIM = 576
LATENT = 512


def plane_scale_index(slot):
    """Position of slot ``slot``'s E8M0 byte within its (page, chunk) row of 64."""
    slot = np.asarray(slot)
    return (slot % 16) * 4 + slot // 16


def index_query(q_fp4, q_scale):
    """[H, 64] E2M1 bytes + [4, 16, 4] E8M0 -> (values f32 [H, 4, 32] without scales,
    scale exponents [H, 4]: qe - 127)."""
    q = F.unpack_e2m1(np.asarray(q_fp4)).reshape(-1, 4, 32)
    h = np.arange(q.shape[0])
    qe = np.asarray(q_scale)[:, h % 16, h // 16].T.astype(np.int64) - 127  # [H, 4]
    return q, qe


def index_keys(payload, kscale, pages, n, cols=None):
    """The first n keys of a request whose pages are ``pages`` (or the positions
    ``cols``): (values f32 [n, 4, 32] without scales, scale exponents [n, 4]: ke - 127)."""
    pos = np.arange(n) if cols is None else np.asarray(cols, dtype=np.int64)
    page = np.asarray(pages)[pos // PAGE].astype(np.int64)
    slot = pos % PAGE
    raw = np.asarray(payload)[page[:, None], np.arange(4)[None], slot[:, None]]  # [n, 4, 16]
    ke = np.asarray(kscale)[page[:, None], np.arange(4)[None], plane_scale_index(slot)[:, None]]
    return F.unpack_e2m1(raw), ke.astype(np.int64) - 127


def index_scores(q_fp4, q_scale, w, payload, kscale, pages, n, cols=None):
    """f64 [n]: the indexer score of each of the row's first n tokens (or of the
    positions ``cols``, in their order). Each 32-dim chunk's
    dot product is exact in f32 (E2M1 products are multiples of 1/4 of magnitude at most
    36, so a 32-term sum stays below 2^13 quarters); the chunk scales 2^(qe + ke) and the
    rest are applied in f64."""
    q, qe = index_query(q_fp4, q_scale)
    k, ke = index_keys(payload, kscale, pages, n, cols)
    s = np.zeros((k.shape[0], q.shape[0]))
    for c in range(4):
        dot = (k[:, c, :] @ q[:, c, :].T).astype(np.float64)  # [n, H]
        s += dot * np.exp2(ke[:, c].astype(np.float64))[:, None] * np.exp2(qe[:, c].astype(np.float64))[None, :]
    return np.maximum(s, 0.0) @ np.asarray(w, dtype=np.float64)


def dsa_keys(pages_u8, pages, n, cols=None, tiled: bool = True):
    """f64 [n, 128]: the first n keys of a request whose pages are ``pages`` (or the
    positions ``cols``) from DSA index pages u8 [P, 8448]: each E4M3 value times its
    token's f32 scale (the page decode of ``sgl_amd_mono/glm53/check.py:58-66``)."""
    pos = np.arange(n) if cols is None else np.asarray(cols, dtype=np.int64)
    page = np.asarray(pages)[pos // PAGE].astype(np.int64)
    off = pos % PAGE
    pu = np.asarray(pages_u8)
    vals = pu[page[:, None], dsa_value_offset(off[:, None], np.arange(128)[None], tiled)]
    sc = pu[page[:, None], 8192 + 4 * off[:, None] + np.arange(4)[None]].copy().view(np.float32)
    return F.e4m3_to_f32(vals).astype(np.float64) * sc.astype(np.float64)


def index_scores_fp8(q, w, pages_u8, pages, n, cols=None, tiled: bool = True):
    """f64 [n]: the DSA (FP8) indexer score of each of the row's first n tokens (or of the
    positions ``cols``): s_t = sum_h w_h relu(q_h . k_t), q the bf16 query [64, 128], k_t
    the page's E4M3 key times its scale (``kernel.py:2784-2842``: a bf16 MFMA of the query
    against the E4M3 values widened exactly, each head's ReLU times its weight, times the
    key's power-of-two scale)."""
    k = dsa_keys(pages_u8, pages, n, cols, tiled)
    return np.maximum(k @ np.asarray(q, np.float64).T, 0.0) @ np.asarray(w, dtype=np.float64)


def kv_rows(kv, kv_scale, slots):
    """f64 [k, 576]: the cached rows at ``slots`` (E4M3 times the token's scale; raw E4M3
    at scale 1 when ``kv_scale`` is None, the layout of SGLang's FP8 MLA pool)."""
    slots = np.asarray(slots, dtype=np.int64)
    v = F.e4m3_to_f32(np.asarray(kv)[slots]).astype(np.float64)
    if kv_scale is None:
        return v
    return v * np.asarray(kv_scale, dtype=np.float64)[slots][:, None]


def sparse_mla(q, kv, kv_scale, slots, sm_scale):
    """q [heads, 576] (bf16 values) over the rows at ``slots`` -> (o f64 [heads, 512],
    lse f64 [heads])."""
    qf = torch.as_tensor(q).double()
    k = torch.from_numpy(kv_rows(kv, kv_scale, slots))
    s = (qf @ k.T) * sm_scale
    lse = torch.logsumexp(s, -1)
    p = torch.exp(s - lse[:, None])
    return (p @ k[:, :LATENT]).numpy(), lse.numpy()


def attention_row(q, q_fp4, q_scale, w, payload, kscale, pages, kv, kv_scale, position,
                  topk, sm_scale):
    """One decode row at ``position``: the indexer scores of keys 0..position, their
    exact top-k (all keys when there are at most ``topk``), and the sparse MLA output
    over the selected tokens. Returns dict(scores f32 [n], sel positions [m], o [32, 512])."""
    n = int(position) + 1
    sc = index_scores(q_fp4, q_scale, w, payload, kscale, pages, n).astype(np.float32)
    sel = np.arange(n, dtype=np.int32) if n <= topk else topk_sort(sc, topk)
    pages = np.asarray(pages).astype(np.int64)
    slots = pages[sel // PAGE] * PAGE + sel % PAGE
    o, lse = sparse_mla(q, kv, kv_scale, slots, sm_scale)
    return dict(scores=sc, sel=sel, o=o, lse=lse)
