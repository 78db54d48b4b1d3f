"""A loaded SGLang DeepSeek-V3.2 layer bound to the launches' weight and cache structs.

The reference binds GLM-5.3 layers the same way (``sgl_amd_mono/glm53/gfx950/weights.py:
94-310``, caches ``sgl_amd_mono/glm53/spec.py:431-465``; the FP4 index pages of
``sgl_amd_mono/deepseek_v4/gfx950/runner.py:336-346``). Every FP8 projection is read in
place (its ``weight`` and ``weight_scale_inv``), and so are the norms, the indexer's head
weights and the MoE. Four kinds of tensor are copied once, because the launches read
another format, and each copy is logged in ``copies`` under (what, layer, name):

* W_UK / W_UV: SGLang's per-tensor FP8 ``w_kc`` [heads, 128, 512] / ``w_vc`` [heads,
  512, 128] transposed to the launches' [head][out][in] rows, with the scalar ``w_scale``
  as every block scale (``weights.py:145-184``), each packed once a layer;
* the index key LayerNorm weight and bias in f32 (``weights.py:187-210``);
* the RoPE table: SGLang's f32 ``cos_sin_cache`` [positions, 64] (cos | sin) as the
  bf16 [positions, 32] pair the front reads, made once for all covered layers
  (``rope_table``: every layer's MLA and indexer rotary must hold the same cache).

Mismatches raise ``ValueError`` naming the tensor, before anything launches; a cache
that does not have the launches' layout raises ``RuntimeError`` (``spec.py:446-461``).
"""

from __future__ import annotations

from typing import Optional

import torch

from .. import _lib, layouts
from .config import DSV32, LayerConfig
from .front import FrontCaches, FrontWeights
from .layer import LayerWeights
from .moe import FP8, MoeFp8Weights
from .post import PostWeights


def _layout(linear) -> str:
    """AITER's (16, 16) shuffle when SGLang marked the weight pre-shuffled."""
    shuffled = getattr(linear, "aiter_bpreshuffled", False) or getattr(
        linear.weight, "is_shuffled", False)
    return layouts.AITER16 if shuffled else layouts.ROWMAJOR


def _linear(name: str, linear, rows: int, cols: int):
    """(weight, weight_scale_inv, layout) of an FP8 block-scaled projection, in place."""
    w = linear.weight
    s = getattr(linear, "weight_scale_inv", None)
    if w.dtype != FP8 or tuple(w.shape) != (rows, cols):
        raise ValueError(f"{name}: needs E4M3 [{rows}, {cols}], got {w.dtype} {tuple(w.shape)}")
    want = ((rows + 127) // 128, cols // 128)
    if s is None or s.dtype != torch.float32 or tuple(s.shape) != want:
        got = None if s is None else f"{s.dtype} {tuple(s.shape)}"
        raise ValueError(f"{name}: needs 128 x 128 block scales f32 {list(want)}, got {got}")
    return w, s, _layout(linear)


def _same(name: str, t: torch.Tensor, shape: tuple, dtype) -> torch.Tensor:
    if t.dtype != dtype or tuple(t.shape) != shape:
        raise ValueError(f"{name}: needs {dtype} {list(shape)}, got {t.dtype} {tuple(t.shape)}")
    return t


def _one_layout(parts: dict) -> str:
    """The launches take one layout for all FP8 projections of a struct."""
    kinds = set(parts.values())
    if len(kinds) != 1:
        raise ValueError(f"mixed FP8 layouts {parts}: the launches read one layout a layer")
    return kinds.pop()


def _shuffled(t: torch.Tensor, layout: str) -> torch.Tensor:
    """An [N, K] E4M3 copy in ``layout`` (the copies follow the in-place projections)."""
    if layout == layouts.AITER16:
        return layouts.shuffle_16x16(t.view(torch.uint8)).view(FP8)
    return t.contiguous()


def _per_tensor(attn, cfg: LayerConfig):
    """SGLang's per-tensor E4M3 ``w_kc`` [heads, nope, latent], ``w_vc`` [heads, latent,
    v] and the scalar ``w_scale`` they share, checked."""
    w_kc, w_vc, w_scale = attn.w_kc, attn.w_vc, getattr(attn, "w_scale", None)
    if w_kc.dtype != FP8 or w_scale is None or w_scale.numel() != 1:
        raise ValueError(
            f"w_kc / w_vc: needs per-tensor E4M3 with a scalar w_scale, got {w_kc.dtype} and "
            f"{None if w_scale is None else tuple(w_scale.shape)}")
    _same("w_kc", w_kc, (cfg.heads, cfg.nope_dim, cfg.kv_lora), FP8)
    _same("w_vc", w_vc, (cfg.heads, cfg.kv_lora, cfg.v_dim), FP8)
    return w_kc, w_vc, float(w_scale.float().reshape(()).item())


def pack_uk(attn, idx: int, copies: dict, layout: str, cfg: LayerConfig = DSV32):
    """W_UK [heads, 512, 128] (E4M3, ``layout`` per head) and its block scales. SGLang
    absorbs as ``q_lat[h] = q_nope[h] @ w_kc[h]`` (w_kc [heads, 128, 512]); the front's
    GEMV computes y[c] = sum_n W[c][n] x[n], so W_UK[h] = w_kc[h] transposed, with the
    scalar w_scale as every block scale (``weights.py:145-184``)."""
    w_kc, _, scale = _per_tensor(attn, cfg)
    hh = cfg.heads
    uk = w_kc.transpose(1, 2).contiguous()  # [h][latent c][nope n]
    w_uk = torch.stack([_shuffled(uk[h], layout) for h in range(hh)])
    s_uk = torch.full((hh, cfg.kv_lora // 128, (cfg.nope_dim + 127) // 128), scale,
                      dtype=torch.float32, device=w_kc.device)
    copies["W_UK / W_UV packed", idx, "w_uk"] = w_uk
    copies["W_UK / W_UV packed", idx, "s_uk"] = s_uk
    return w_uk, s_uk


def pack_uv(attn, idx: int, copies: dict, layout: str, cfg: LayerConfig = DSV32):
    """W_UV [heads, 128, 512] (E4M3, ``layout`` per head) and its block scales. SGLang
    maps the latent back as ``o[h] = o_lat[h] @ w_vc[h]`` (w_vc [heads, 512, 128]); as the
    output block's GEMV rows, W_UV[h] = w_vc[h] transposed, at the scalar w_scale."""
    _, w_vc, scale = _per_tensor(attn, cfg)
    hh = cfg.heads
    uv = w_vc.transpose(1, 2).contiguous()  # [h][v][latent c]
    w_uv = torch.stack([_shuffled(uv[h], layout) for h in range(hh)])
    s_uv = torch.full((hh, cfg.v_dim // 128, cfg.kv_lora // 128), scale,
                      dtype=torch.float32, device=w_vc.device)
    copies["W_UK / W_UV packed", idx, "w_uv"] = w_uv
    copies["W_UK / W_UV packed", idx, "s_uv"] = s_uv
    return w_uv, s_uv


def _cos_sin_cache(rotary, what: str) -> torch.Tensor:
    cache = getattr(rotary, "cos_sin_cache", None)
    if cache is None or cache.dim() != 2 or cache.shape[1] != DSV32.rope_dim:
        got = None if cache is None else tuple(cache.shape)
        raise ValueError(f"{what}.cos_sin_cache: needs [positions, {DSV32.rope_dim}], got {got}")
    return cache


def rope_table(layers: dict, copies: dict):
    """The bf16 cos / sin [positions, 32] that every covered layer's front reads, made once
    from the first layer's MLA rotary: SGLang's f32 ``cos_sin_cache`` [positions, 64]
    (rotating with ``cos, sin = cache[pos].chunk(2, -1)``). The front rotates the index
    key and query with the same table, so each layer's MLA rotary and its indexer's (when
    it keeps its own) must hold the same cache (``glm53/gfx950/weights.py:323-344``).
    ``layers``: {layer index: SGLang decoder layer}."""
    first = min(layers)
    cache = _cos_sin_cache(layers[first].self_attn.rotary_emb, f"layer {first} rotary_emb")
    for i, layer in sorted(layers.items()):
        attn = layer.self_attn
        mine = _cos_sin_cache(attn.rotary_emb, f"layer {i} rotary_emb")
        ind = getattr(getattr(attn, "indexer", None), "rotary_emb", None)
        others = [mine] + ([_cos_sin_cache(ind, f"layer {i} indexer.rotary_emb")] if ind else [])
        for other in others:
            if other is not cache and (other.shape != cache.shape or not torch.equal(other, cache)):
                raise ValueError(f"layer {i}: the indexer's and every layer's rotary table "
                                 f"must equal layer {first}'s MLA one (one table is read)")
    half = DSV32.rope_dim // 2
    cos = cache[:, :half].to(torch.bfloat16).contiguous()
    sin = cache[:, half:].to(torch.bfloat16).contiguous()
    copies["RoPE table bf16", first, "cos"] = cos
    copies["RoPE table bf16", first, "sin"] = sin
    return cos, sin


def front_weights(layer, idx: int, copies: dict, cfg: LayerConfig = DSV32,
                  rope=None) -> FrontWeights:
    """The attention front of a loaded layer (``self_attn`` with its indexer); ``rope``:
    the (cos, sin) table shared by the covered layers (made from this layer if None)."""
    attn = layer.self_attn
    ind = getattr(attn, "indexer", None)
    if ind is None:
        raise ValueError("self_attn.indexer: the front is built for DSA layers with an indexer")
    H, QL, KL, PE = cfg.hidden, cfg.q_lora, cfg.kv_lora, cfg.rope_dim
    w_qkv_a, s_qkv_a, l_a = _linear("fused_qkv_a_proj_with_mqa", attn.fused_qkv_a_proj_with_mqa,
                                    QL + KL + PE, H)
    w_qb, s_qb, l_b = _linear("q_b_proj", attn.q_b_proj, cfg.heads * cfg.qk_dim, QL)
    w_k, s_k, l_k = _linear("indexer.wk", ind.wk, cfg.index_dim, H)
    w_iq, s_iq, l_q = _linear("indexer.wq_b", ind.wq_b, cfg.index_heads * cfg.index_dim, QL)
    layout = _one_layout({"fused_qkv_a_proj_with_mqa": l_a, "q_b_proj": l_b, "indexer.wk": l_k,
                          "indexer.wq_b": l_q})
    bf16 = torch.bfloat16
    g_in = _same("input_layernorm", layer.input_layernorm.weight, (H,), bf16)
    g_q = _same("q_a_layernorm", attn.q_a_layernorm.weight, (QL,), bf16)
    g_kv = _same("kv_a_layernorm", attn.kv_a_layernorm.weight, (KL,), bf16)
    w_w = _same("indexer.weights_proj", ind.weights_proj.weight, (cfg.index_heads, H), bf16)
    g_k = _same("indexer.k_norm", ind.k_norm.weight, (cfg.index_dim,), ind.k_norm.weight.dtype)
    g_k = g_k.detach().float().contiguous()
    b_k = ind.k_norm.bias.detach().float().contiguous()
    copies["indexer k LayerNorm f32", idx, "weight"] = g_k
    copies["indexer k LayerNorm f32", idx, "bias"] = b_k
    w_uk, s_uk = pack_uk(attn, idx, copies, layout, cfg)
    cos, sin = rope if rope is not None else rope_table({idx: layer}, copies)
    return FrontWeights(g_in=g_in, g_q=g_q, g_kv=g_kv, w_qkv_a=w_qkv_a, s_qkv_a=s_qkv_a,
                        w_k=w_k, s_k=s_k, w_w=w_w, g_k=g_k, b_k=b_k, w_qb=w_qb, s_qb=s_qb,
                        w_iq=w_iq, s_iq=s_iq, w_uk=w_uk, s_uk=s_uk, cos=cos, sin=sin,
                        layout=layout)


def post_weights(layer, idx: int, copies: dict, cfg: LayerConfig = DSV32) -> PostWeights:
    """The attention output block: ``o_proj`` in place, W_UV packed in its layout."""
    attn = layer.self_attn
    w_o, s_o, layout = _linear("o_proj", attn.o_proj, cfg.hidden, cfg.heads * cfg.v_dim)
    w_uv, s_uv = pack_uv(attn, idx, copies, layout, cfg)
    return PostWeights(w_uv=w_uv, s_uv=s_uv, w_o=w_o, s_o=s_o, layout=layout)


def moe_weights(layer) -> MoeFp8Weights:
    """The FFN half: the fused experts (the shared expert last), router and norm, in place."""
    mlp, ex = layer.mlp, layer.mlp.experts
    return MoeFp8Weights(
        g_post=layer.post_attention_layernorm.weight,
        w_r=mlp.gate.weight,
        bias=mlp.gate.e_score_correction_bias,
        w13=ex.w13_weight, s13=ex.w13_weight_scale_inv,
        w2=ex.w2_weight, s2=ex.w2_weight_scale_inv,
        layout=layouts.AITER16 if getattr(ex.w13_weight, "is_shuffled", False)
        else layouts.ROWMAJOR,
    )


def layer_weights(layer, idx: int, copies: dict, cfg: LayerConfig = DSV32,
                  rope=None) -> LayerWeights:
    """Every weight of a covered layer's four launches; ``rope``: the covered layers'
    shared (cos, sin) table (``rope_table``; made from this layer if None)."""
    return LayerWeights(front=front_weights(layer, idx, copies, cfg, rope),
                        post=post_weights(layer, idx, copies, cfg), moe=moe_weights(layer))


def layer_disable_reason(layer, idx: int, cfg: LayerConfig = DSV32) -> Optional[str]:
    """Why a covered layer cannot be bound in place (None: it can); nothing is kept."""
    try:
        layer_weights(layer, idx, {}, cfg)
    except (ValueError, AttributeError) as e:
        return f"layer {idx}: {e}"
    return None


def index_cache(pool, idx: int, cfg: LayerConfig = DSV32):
    """The layer's index-key cache in SGLang's pool, in place: ``(plane, plane_scale,
    index_format)``. A pool with the FP4 index plane gives its pages [pages, 1, 4, 64, 16]
    and E8M0 scales [pages, 1, 4, 64] (``get_index_k_fp4_payload_buffer`` /
    ``_scale_buffer``); DeepSeek-V3.2's NSA pool gives its DSA index pages
    (``get_index_k_with_scale_buffer``: per page 64 tokens x 128 E4M3 values then 64 f32
    scales, 8448 bytes), bound as 16-token x 16-byte tiles, the layout of SGLang's HIP DSA
    pool as the reference binds it (``glm53/spec.py:444-466``,
    ``glm53/gfx950/runner.py:177``). Any other pool raises ``RuntimeError``."""
    if hasattr(pool, "get_index_k_fp4_payload_buffer"):
        pay = pool.get_index_k_fp4_payload_buffer(idx)
        sc = pool.get_index_k_fp4_scale_buffer(idx)
        if (pay.dtype != torch.uint8 or tuple(pay.shape[1:]) != (1, 4, cfg.page, 16)
                or not pay.is_contiguous()):
            raise RuntimeError(f"layer {idx}: FP4 index pages {pay.dtype} {tuple(pay.shape)}; "
                               f"needs contiguous uint8 [pages, 1, 4, {cfg.page}, 16]")
        if (sc.dtype != torch.uint8 or tuple(sc.shape) != (pay.shape[0], 1, 4, cfg.page)
                or not sc.is_contiguous()):
            raise RuntimeError(f"layer {idx}: FP4 index scales {sc.dtype} {tuple(sc.shape)}; "
                               f"needs contiguous uint8 [{pay.shape[0]}, 1, 4, {cfg.page}]")
        pages = pay.shape[0]
        return (pay.view(pages, 4, cfg.page, 16), sc.view(pages, 4, cfg.page),
                _lib.INDEX_FP4_PLANE)
    if hasattr(pool, "get_index_k_with_scale_buffer"):
        buf = pool.get_index_k_with_scale_buffer(idx)
        per = cfg.page * (cfg.index_dim + 4)
        if (buf.dtype != torch.uint8 or buf.dim() < 2 or not buf.is_contiguous()
                or buf.numel() != buf.shape[0] * per or per != _lib.DSA_PAGE_BYTES):
            raise RuntimeError(f"layer {idx}: DSA index pages {buf.dtype} {tuple(buf.shape)}; "
                               f"needs contiguous uint8 [pages, {per}] (64 x (128 + 4) bytes "
                               f"a page)")
        return buf.view(buf.shape[0], per), None, _lib.INDEX_FP8_PAGE
    raise RuntimeError(f"layer {idx}: the KV pool has no index-key cache this build reads "
                       f"(an FP4 index plane or DSA index pages)")


def index_buffers(pool, idx: int) -> list:
    """The pool's index-key tensors of a layer, page-major (for a caller that saves and
    restores pages around SGLang's own layer)."""
    if hasattr(pool, "get_index_k_fp4_payload_buffer"):
        return [pool.get_index_k_fp4_payload_buffer(idx), pool.get_index_k_fp4_scale_buffer(idx)]
    return [pool.get_index_k_with_scale_buffer(idx)]


def caches(pool, idx: int, cfg: LayerConfig = DSV32) -> FrontCaches:
    """A layer's caches from SGLang's KV pool, in place: the MLA rows E4M3 [slots, 1, 576]
    (``get_key_buffer``) and the index-key cache (``index_cache``: the FP4 index plane or
    DSA index pages). The pool's MLA rows are raw E4M3 at scale 1 (SGLang's HIP DSA
    layout, as the reference binds it: ``glm53/spec.py:451-461``), so the launches write
    and read them with no per-token scale: a row SGLang wrote and a row the front wrote
    read the same way, whichever path serves the next step."""
    kv = pool.get_key_buffer(idx)
    row = cfg.kv_row
    if kv.element_size() != 1 or kv.shape[-1] != row or not kv.is_contiguous():
        raise RuntimeError(f"layer {idx}: MLA cache {kv.dtype} {tuple(kv.shape)}; needs "
                           f"contiguous E4M3 [slots, 1, {row}]")
    slots = kv.numel() // row
    plane, plane_scale, fmt = index_cache(pool, idx, cfg)
    return FrontCaches(kv=kv.view(torch.uint8).view(slots, row), kv_scale=None, plane=plane,
                       plane_scale=plane_scale, index_format=fmt)
