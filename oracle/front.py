"""The front of the layer, restated on the CPU (test infrastructure only): everything
between the layer input h and the attention phase's inputs.

Reference stages (``sgl_amd_mono/glm53/gfx950/kernel.py``):

* x = bf16(rmsnorm(h) * g_in) (``stage_x_rmsnorm`` :1367-1402: rstd = (sum x^2 / n +
  eps)^-1/2, x * rstd * g, bf16);
* q_a | kv_a = W_qkv_a x (FP8 128x128 block scales, W8A16, f32 out; :1781-1970), index
  key k = W_k x (:1917-1937), head weights w = W_w x (bf16 weights; :1939-1947);
* q_an = bf16(rmsnorm(q_a) * g_q) (:1978-2003);
* the KV row (:2005-2101): kv_n = bf16(rmsnorm(kv_a[:512]) * g_kv); k_pe = bf16(rope(kv_a
  [512:])) with interleaved pairs (x0 c - x1 s, x0 s + x1 c) at the row's position. The
  cache takes E4M3 either with one f32 scale per token (the north star's synthetic
  format): scale = 2^ceil(log2(max(amax, 1e-4) / 448)) over the 576 values, as the
  reference's index cache quantiser (:2138-2150), codes = E4M3(value / scale) round to
  nearest even; or raw at scale 1 (SGLang's FP8 MLA pool, the GLM cache write
  :2044-2062), ``kv_quant(row, scaled=False)``;
* the index key (``index_key``): k_n = bf16((k - mean) rstd g + b) (the LayerNorm of
  :2103-2131, eps 1e-6), bf16(RoPE) on dims 0..63, the orthonormal Sylvester FWHT-128
  (``fwht128`` :556-566) rounded to bf16, then FP4 as the V4 indexer's ``fp4_block``
  (``deepseek_v4/gfx950/kernels/stages/indexer.py:143-151``): per 32 values scale =
  pow2_ceil(max(amax, 6 * 2^-126) / 6) (``ops.py:153-158``), codes = E2M1(v / scale)
  round to nearest even, written into SGLang's FP4 index plane. The bf16 rounding points
  are those of the reference's FP4 key path (``indexer.py:242-254``: the normalised key,
  the rotated half and the Hadamard output are each ``bf16_round``-ed before
  ``fp4_block``);
* q = W_qb q_an (:2183-2260): the nope part bf16, the rope part rotated then bf16; the
  absorbed query q_lat = bf16(W_UK q_nope) per head (:2355-2443);
* the index query (``index_query``): iq_raw = bf16(W_iq q_an) (:2262-2353), bf16(RoPE) on
  dims 0..63, FWHT-128 rounded to bf16, FP4 per 32: the V4 query path
  (``indexer.py:311-338``), whose rotated half is ``bf16_round``-ed before the Hadamard
  transform and whose Hadamard output is ``bf16_round``-ed before ``fp4_block``
  (:330-335);
* the head weights: bf16(w) * 128^-0.5 * 64^-0.5 (``indexer.py:400-406``);
* the DSA (FP8) index path instead of FP4 (``index_key_fp8``, ``index_query_bf16``): the
  key's LayerNorm, RoPE and FWHT unrounded, then E4M3 at a power-of-two per-token scale
  into SGLang's DSA index page (:2103-2168, layout :534-550, ``dsa_value_offset``); the
  query rotated and transformed unrounded, then bf16 once (:2928-2944).

The f32 / f64 arithmetic here is exact or correctly rounded; the launch uses f32 with
hardware rsqrt, so bf16 outputs may differ by one rounding and quantised codes only where
the value sits at a rounding boundary (the tests allow for exactly that).

Pinned by ``tests/test_oracle_front.py``: rmsnorm and layer_norm against torch's; RoPE as
a complex multiplication (and its inverse); the FWHT against scipy's Hadamard matrix
(and as an involution); the FP4 and FP8 quantisers against brute-force nearest-value
search with ties to even and the pow2 scale against frexp; the index key and query
chains' bf16 rounding points by constructed inputs whose FP4 codes flip when a rounding
is dropped (one- or two-hot pre-transform vectors, whose Hadamard outputs are closed
forms); the DSA page layout against the reference's page decode (``glm53/check.py:
58-66``), the FP8 key chain by a closed form (a one-hot key's LayerNorm and transform) and
a scale that drops a power of two when the transform's output is rounded to bf16 first,
the bf16 query's single rounding by a rotated pair whose early rounding changes its bf16
transform; the GEMVs are ``oracle/dense.py`` (pinned there).
"""

from __future__ import annotations

import numpy as np
import torch

from . import dense as D
from . import formats as F

HIDDEN, Q_LORA, KV_LORA, ROPE, NOPE = 7168, 1536, 512, 64, 128
HEADS, IHEADS, IDIM = 32, 64, 128
E2M1_GRID = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def bf16(x) -> np.ndarray:
    return D.bf16(x)


def rmsnorm(x, g, eps) -> np.ndarray:
    """f64 x * (mean(x^2) + eps)^-1/2 * g over the last axis."""
    x = np.asarray(x, np.float64)
    r = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    return x * r * np.asarray(g, np.float64)


def layernorm(x, g, b, eps=1e-6) -> np.ndarray:
    x = np.asarray(x, np.float64)
    m = x.mean(-1, keepdims=True)
    c = x - m
    r = 1.0 / np.sqrt((c * c).mean(-1, keepdims=True) + eps)
    return c * r * np.asarray(g, np.float64) + np.asarray(b, np.float64)


def rope(x, cos, sin) -> np.ndarray:
    """Interleaved pairs (x[2i], x[2i+1]) rotated by (cos[i], sin[i]) (the reference's
    x0 c - x1 s, x0 s + x1 c); x [..., 2n], cos/sin [n] or broadcastable."""
    x = np.asarray(x, np.float64)
    x0, x1 = x[..., 0::2], x[..., 1::2]
    c, s = np.asarray(cos, np.float64), np.asarray(sin, np.float64)
    out = np.empty_like(x)
    out[..., 0::2] = x0 * c - x1 * s
    out[..., 1::2] = x0 * s + x1 * c
    return out


def _sylvester(n):
    h = np.array([[1.0]])
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


_H128 = _sylvester(128) / np.sqrt(128.0)


def fwht128(x) -> np.ndarray:
    """The orthonormal Sylvester-order Hadamard transform over the last axis (128)."""
    return np.asarray(x, np.float64) @ _H128


def pow2_ceil(x) -> np.ndarray:
    """Smallest power of two >= x (x > 0, normal)."""
    m, e = np.frexp(np.asarray(x, np.float64))  # x = m 2^e, m in [0.5, 1)
    return np.where(m == 0.5, np.ldexp(1.0, e - 1), np.ldexp(1.0, e))


def _rne_grid(v, grid):
    """Nearest value of a sorted non-negative grid to |v| with ties to the even index
    (the even mantissa), sign kept; |v| beyond the grid saturates."""
    a = np.abs(np.asarray(v, np.float64))
    i = np.clip(np.searchsorted(grid, a), 1, len(grid) - 1)
    lo, hi = grid[i - 1], grid[i]
    d_lo, d_hi = a - lo, hi - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (i % 2 == 0))
    idx = np.where(pick_hi, i, i - 1)
    idx = np.where(a >= grid[-1], len(grid) - 1, idx)
    return np.sign(v) * grid[idx], idx


def fp4_codes(v) -> np.ndarray:
    """E2M1 codes (sign << 3 | index) of values already divided by their scale."""
    q, idx = _rne_grid(v, E2M1_GRID)
    sign = (np.signbit(np.asarray(v, np.float64)) & (idx > 0)).astype(np.uint8)
    return (sign << 3 | idx.astype(np.uint8)).astype(np.uint8)


def fp4_block(v):
    """FP4 of the last axis in blocks of 32: (codes u8 [..., n], e8m0 bytes [..., n/32],
    dequantised f64 [..., n])."""
    v = np.asarray(v, np.float64)
    blocks = v.reshape(*v.shape[:-1], -1, 32)
    amax = np.abs(blocks).max(-1)
    sc = pow2_ceil(np.maximum(amax, 6.0 * 2.0 ** -126) / 6.0)
    codes = fp4_codes(np.clip(blocks / sc[..., None], -6.0, 6.0))
    e8 = (np.frexp(sc)[1] - 1 + 127).astype(np.uint8)
    deq = F.unpack_e2m1(pack_nibbles(codes)).reshape(blocks.shape) * sc[..., None]
    return codes.reshape(v.shape), e8, deq.reshape(v.shape)


def pack_nibbles(codes) -> np.ndarray:
    """[..., 2n] 4-bit codes -> [..., n] bytes, the even element in the low nibble."""
    c = np.asarray(codes, np.uint8)
    return (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)


def fp8_codes(v) -> np.ndarray:
    """E4M3 (fn) codes of values within +-448, round to nearest even."""
    return F.f32_to_e4m3(np.asarray(v, np.float64))


def kv_quant(row, scaled: bool = True):
    """A cache row [576] (bf16 values) -> (E4M3 codes [576], f32 scale). Scaled: the
    power-of-two per-token scale of the index-cache quantiser (``kernel.py:2138-2150``);
    unscaled: raw E4M3 at scale 1 saturating at +-448 (the GLM cache write,
    ``kernel.py:2050-2062``: the bf16 values cast to E4M3)."""
    row = np.asarray(row, np.float64)
    if not scaled:
        return fp8_codes(np.clip(row, -448.0, 448.0)), np.float32(1.0)
    amax = np.abs(row).max()
    sc = pow2_ceil(max(amax, 1e-4) / 448.0)
    return fp8_codes(row / sc), np.float32(sc)


def front(h, g_in, g_q, g_kv, w_qkv_a, s_qkv_a, w_k, s_k, w_w, g_k, b_k, w_qb, s_qb,
          w_iq, s_iq, w_uk, s_uk, cos, sin, positions, eps=1e-6, kv_scaled=True, absorb=None):
    """One step's front for rows h [R, 7168] (bf16 values) at ``positions``; row-major
    weights (numpy E4M3 codes, f32 scales; w_w bf16 values); cos/sin [pos, 32].
    ``absorb(q_nope_h [R, 128], h) -> [R, 512]`` replaces the W_UK GEMV (w_uk / s_uk may
    then be None): a caller holding W_UK in another orientation states its product.

    Returns dict with x, q_a, kv_a, k, w (f64 GEMV outputs), q_an (bf16), kv_rows
    (bf16-valued [R, 576] before quantisation), kv_codes u8 [R, 576], kv_scale f32 [R],
    ik (f64 [R, 128] before FP4), ik_codes u8 [R, 128], ik_e8 u8 [R, 4], q bf16 [R, 32,
    576], iq_raw (bf16 [R, 64, 128]), iq_pre (f64 before FP4), iq_codes u8 [R, 64, 128],
    iq_e8 u8 [R, 64, 4], iw f32 [R, 64]; and the DSA (FP8) index path's ik8 (f64 [R, 128]
    before E4M3), ik8_codes u8 [R, 128], ik8_scale f32 [R], iq16 (bf16 values [R, 64,
    128])."""
    h = np.asarray(torch.as_tensor(h).float(), np.float64)
    R = h.shape[0]
    pos = np.asarray(positions, np.int64)
    c = np.asarray(torch.as_tensor(cos).float(), np.float64)[pos]  # [R, 32]
    s = np.asarray(torch.as_tensor(sin).float(), np.float64)[pos]
    f32 = lambda t: np.asarray(torch.as_tensor(t).float(), np.float64)
    x = bf16(rmsnorm(h, f32(g_in), eps))
    qkv = D.w8a16_gemv(x, w_qkv_a, s_qkv_a)  # [R, 2112]
    q_a, kv_a = qkv[:, :Q_LORA], qkv[:, Q_LORA:]
    k = D.w8a16_gemv(x, w_k, s_k)  # [R, 128]
    w = x @ f32(w_w).T  # [R, 64]
    q_an = bf16(rmsnorm(q_a, f32(g_q), eps))
    kv_n = bf16(rmsnorm(kv_a[:, :KV_LORA], f32(g_kv), eps))
    k_pe = bf16(rope(kv_a[:, KV_LORA:], c, s))
    kv_rows = np.concatenate([kv_n, k_pe], -1)
    kq = [kv_quant(r, kv_scaled) for r in kv_rows]
    ikd = index_key(k, f32(g_k), f32(b_k), c, s)
    qb =D.w8a16_gemv(q_an, w_qb, s_qb).reshape(R, HEADS, NOPE + ROPE)
    q_nope = bf16(qb[..., :NOPE])
    q_pe = bf16(rope(qb[..., NOPE:], c[:, None], s[:, None]))
    if absorb is None:
        absorb = lambda qn, hh: D.w8a16_gemv(qn, w_uk[hh], s_uk[hh])  # noqa: E731
    q_lat = np.stack([bf16(np.asarray(absorb(q_nope[:, hh], hh), np.float64))
                      for hh in range(HEADS)], 1)
    q = np.concatenate([q_lat, q_pe], -1)
    iq_raw = bf16(D.w8a16_gemv(q_an, w_iq, s_iq)).reshape(R, IHEADS, IDIM)
    iqd = index_query(iq_raw, c, s)
    ik8 = index_key_fp8(k, f32(g_k), f32(b_k), c, s)
    iw = (bf16(w) * (IDIM ** -0.5 * IHEADS ** -0.5)).astype(np.float32)
    return dict(x=x, q_a=q_a, kv_a=kv_a, k=k, w=w, q_an=q_an, kv_rows=kv_rows,
                kv_codes=np.stack([a for a, _ in kq]), kv_scale=np.array([b for _, b in kq]),
                ik=ikd["pre"], ik_codes=ikd["codes"], ik_e8=ikd["e8"], q=q, iq_raw=iq_raw,
                iq_pre=iqd["pre"], iq_codes=iqd["codes"], iq_e8=iqd["e8"], iw=iw,
                ik8=ik8["pre"], ik8_codes=ik8["codes"], ik8_scale=ik8["scale"],
                iq16=index_query_bf16(iq_raw, c, s))


def _rope_lead(v, cos, sin):
    """bf16(RoPE) of the first ROPE dims (interleaved pairs); the other dims unchanged."""
    return np.concatenate([bf16(rope(v[..., :ROPE], cos, sin)), v[..., ROPE:]], -1)


def index_key(k, g_k, b_k, cos, sin):
    """The index-key chain of rows k [R, 128] (the W_k outputs) with the rows' RoPE
    factors cos / sin [R, 32]: n = bf16(LayerNorm(k) g + b) (``kernel.py:2118-2131``),
    r = bf16(RoPE(n[:64])) | n[64:], t = FWHT-128(r), pre = bf16(t), then FP4 of pre: the
    rounding points of ``deepseek_v4/gfx950/kernels/stages/indexer.py:242-254``
    (``bf16_round`` after the norm, after the rotation and after the Hadamard transform,
    then ``fp4_block``).

    Returns dict(norm, rot, fwht (f64, before its rounding), pre, codes u8 [R, 128],
    e8 u8 [R, 4])."""
    n = bf16(layernorm(k, g_k, b_k))
    r = _rope_lead(n, cos, sin)
    t = fwht128(r)
    pre = bf16(t)
    codes, e8, _ = fp4_block(pre)
    return dict(norm=n, rot=r, fwht=t, pre=pre, codes=codes, e8=e8)


def index_query(iq_raw, cos, sin):
    """The index-query chain of iq_raw [R, 64, 128] (bf16 values of W_iq q_an) with the
    rows' RoPE factors cos / sin [R, 32]: r = bf16(RoPE(iq_raw[..., :64])) | iq_raw[...,
    64:], t = FWHT-128(r), pre = bf16(t), then FP4 per 32 of pre: the rounding points of
    ``deepseek_v4/gfx950/kernels/stages/indexer.py:330-335`` (the rotated half
    ``bf16_round``-ed before ``had_pair``, the Hadamard output ``bf16_round``-ed before
    ``fp4_block``).

    Returns dict(rot, fwht (f64, before its rounding), pre, codes u8 [R, 64, 128],
    e8 u8 [R, 64, 4])."""
    iq_raw = np.asarray(iq_raw, np.float64)
    c = np.asarray(cos, np.float64)[:, None]
    s = np.asarray(sin, np.float64)[:, None]
    r = _rope_lead(iq_raw, c, s)
    t = fwht128(r)
    pre = bf16(t)
    codes, e8, _ = fp4_block(pre)
    return dict(rot=r, fwht=t, pre=pre, codes=codes, e8=e8)


# ------------------------------------------------------------ the DSA (FP8) index page
DSA_PAGE_BYTES = 64 * (IDIM + 4)  # 64 tokens x 128 E4M3 values, then 64 f32 scales


def dsa_value_offset(off, d, tiled: bool = True):
    """Byte offset of value ``d`` (0..127) of token ``off`` (0..63) within a DSA index page
    (``kernel.py:534-543``, ``index_value_word``). Tiled (SGLang's HIP layout,
    ``index_shuffled``): 16-token x 16-byte tiles, (off // 16) * 2048 + (d // 16) * 256 +
    (off % 16) * 16 + d % 16; otherwise token-major, off * 128 + d. The token's f32 scale
    follows the values, at 8192 + 4 off (:545-550)."""
    off, d = np.asarray(off), np.asarray(d)
    if tiled:
        return (off // 16) * 2048 + (d // 16) * 256 + (off % 16) * 16 + d % 16
    return off * IDIM + d


def index_key_fp8(k, g_k, b_k, cos, sin):
    """The index-key chain into a DSA (FP8) index page (``kernel.py:2103-2168``, its
    ``index_paged`` branch) for rows k [R, 128] (the W_k outputs) with the rows' RoPE
    factors cos / sin [R, 32]: LayerNorm (eps 1e-6) times g plus b, RoPE on dims 0..63,
    the FWHT-128, none of them rounded; then one power-of-two scale a token, scale =
    2^ceil(log2(max(amax, 1e-4) / 448)) with the quotient rounded to f32 first (the
    kernel's ``div_rn``), and codes = E4M3(v / scale), round to nearest even.

    Returns dict(pre f64 [R, 128] before quantisation, codes u8 [R, 128], scale f32 [R])."""
    n = layernorm(k, g_k, b_k)
    r = np.concatenate([rope(n[..., :ROPE], cos, sin), n[..., ROPE:]], -1)
    t = fwht128(r)
    amax = np.maximum(np.abs(t).max(-1), 1e-4).astype(np.float32)
    sc = pow2_ceil(amax / np.float32(448.0))
    codes = fp8_codes(t / sc[:, None])
    return dict(pre=t, codes=codes, scale=sc.astype(np.float32))


def index_query_bf16(iq_raw, cos, sin):
    """The index query of the DSA (FP8) path for iq_raw [R, 64, 128] (bf16 values of W_iq
    q_an, ``kernel.py:2262-2353``) with the rows' RoPE factors cos / sin [R, 32]: the score
    stage rotates dims 0..63, applies the FWHT-128 and rounds the result to bf16 once
    (:2928-2944). Returns f64 [R, 64, 128] of bf16 values."""
    iq_raw = np.asarray(iq_raw, np.float64)
    c = np.asarray(cos, np.float64)[:, None]
    s = np.asarray(sin, np.float64)[:, None]
    r = np.concatenate([rope(iq_raw[..., :ROPE], c, s), iq_raw[..., ROPE:]], -1)
    return bf16(fwht128(r))


def dsa_page_write(pages, slot, codes, scale, tiled: bool = True):
    """Write one token's FP8 key (codes [128], f32 scale) into DSA index pages u8 [P, 8448]
    at ``slot`` (page slot // 64, token slot % 64)."""
    page, off = divmod(int(slot), 64)
    pages[page, dsa_value_offset(off, np.arange(IDIM), tiled)] = np.asarray(codes, np.uint8)
    at = 64 * IDIM + 4 * off
    pages[page, at:at + 4] = np.frombuffer(np.float32(scale).tobytes(), np.uint8)


def iq_bytes(codes, e8):
    """Index query codes [R, 64, 128] + e8m0 [R, 64, 4] -> the attention launch's inputs:
    iq u8 [R, 64, 64] (low nibble first) and iqs u8 [R, 4 (chunk), 16 (h % 16), 4 (h // 16)]."""
    iq = pack_nibbles(codes)
    R = codes.shape[0]
    iqs = np.zeros((R, 4, 16, 4), np.uint8)
    hh = np.arange(IHEADS)
    for cc in range(4):
        iqs[:, cc, hh % 16, hh // 16] = e8[:, hh, cc]
    return iq, iqs


def plane_write(plane, plane_scale, slot, codes, e8):
    """Write one token's FP4 key (codes [128], e8m0 [4]) into SGLang's FP4 index plane at
    ``slot`` (payload [pages, 4, 64, 16], scales [pages, 4, 64], the slot's scale byte at
    (s % 16) * 4 + s // 16)."""
    page, sl = divmod(int(slot), 64)
    b = pack_nibbles(codes).reshape(4, 16)
    plane[page, :, sl, :] = b
    plane_scale[page, :, (sl % 16) * 4 + sl // 16] = e8
