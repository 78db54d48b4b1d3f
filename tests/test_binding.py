"""Binding a loaded SGLang layer (modules with SGLang's attribute names, on the CPU) to the
launches' structs: projections read in place, the logged copies equal to the launches'
own formats, refusals naming the tensor, and the cache checks."""

from types import SimpleNamespace as NS

import numpy as np
import pytest
import torch

from sgl_amd_mono_amd import layouts
from sgl_amd_mono_amd.dsv32 import binding, synthetic
from sgl_amd_mono_amd.dsv32.config import DSV32
from sgl_amd_mono_amd.dsv32.moe import FP8

SCALE = 0.0078125  # the scalar w_scale of w_kc / w_vc


def _rowmajor(t, layout):
    return layouts.unshuffle_16x16(t.view(torch.uint8)).view(FP8) if layout == layouts.AITER16 else t


def _lin(w, s, layout):
    lin = NS(weight=w, weight_scale_inv=s)
    if layout == layouts.AITER16:
        lin.aiter_bpreshuffled = True
    return lin


def _layer(layout):
    """A DeepSeek-V3.2 layer as SGLang loads it, built from the synthetic launch weights
    (W_UK / W_UV at one scalar scale, so the copies can be compared bit for bit)."""
    fw = synthetic.front_weights("cpu", seed=3, layout=layout, rope_rows=64)
    pw = synthetic.post_weights("cpu", seed=3, layout=layout)
    hh = DSV32.heads
    uk = torch.stack([_rowmajor(fw.w_uk[h], layout) for h in range(hh)])  # [h][512][128]
    uv = torch.stack([_rowmajor(pw.w_uv[h], layout) for h in range(hh)])  # [h][128][512]
    half = DSV32.rope_dim // 2
    cache = torch.cat([fw.cos.float(), fw.sin.float()], 1)
    attn = NS(
        fused_qkv_a_proj_with_mqa=_lin(fw.w_qkv_a, fw.s_qkv_a, layout),
        q_b_proj=_lin(fw.w_qb, fw.s_qb, layout),
        o_proj=_lin(pw.w_o, pw.s_o, layout),
        q_a_layernorm=NS(weight=fw.g_q), kv_a_layernorm=NS(weight=fw.g_kv),
        w_kc=uk.transpose(1, 2).contiguous(), w_vc=uv.transpose(1, 2).contiguous(),
        w_scale=torch.tensor(SCALE),
        rotary_emb=NS(cos_sin_cache=cache),
        indexer=NS(wk=_lin(fw.w_k, fw.s_k, layout), wq_b=_lin(fw.w_iq, fw.s_iq, layout),
                   weights_proj=NS(weight=fw.w_w),
                   k_norm=NS(weight=fw.g_k.to(torch.bfloat16), bias=fw.b_k.to(torch.bfloat16))),
    )
    assert half == fw.cos.shape[1]
    return NS(self_attn=attn, input_layernorm=NS(weight=fw.g_in)), fw, pw


@pytest.mark.parametrize("layout", [layouts.ROWMAJOR, layouts.AITER16])
def test_the_front_and_output_block_bind_in_place(layout):
    layer, fw, pw = _layer(layout)
    copies = {}
    f = binding.front_weights(layer, 5, copies)
    p = binding.post_weights(layer, 5, copies)
    assert f.layout == p.layout == layout
    for name in ("w_qkv_a", "s_qkv_a", "w_qb", "s_qb", "w_k", "s_k", "w_iq", "s_iq", "w_w",
                 "g_in", "g_q", "g_kv"):
        assert getattr(f, name) is getattr(fw, name), name  # the loaded tensor itself
    assert p.w_o is pw.w_o and p.s_o is pw.s_o
    # the copies: W_UK / W_UV in the launches' layout with the scalar scale
    assert torch.equal(f.w_uk.view(torch.uint8), fw.w_uk.view(torch.uint8))
    assert torch.equal(p.w_uv.view(torch.uint8), pw.w_uv.view(torch.uint8))
    assert torch.all(f.s_uk == SCALE) and f.s_uk.shape == fw.s_uk.shape
    assert torch.all(p.s_uv == SCALE) and p.s_uv.shape == pw.s_uv.shape
    assert torch.equal(f.cos, fw.cos) and torch.equal(f.sin, fw.sin)
    assert f.g_k.dtype == torch.float32 and f.b_k.dtype == torch.float32
    f.validate(DSV32, torch.device("cpu"))
    p.validate(DSV32, torch.device("cpu"))
    logged = {(k[0], k[2]) for k in copies}
    assert logged == {("W_UK / W_UV packed", n) for n in ("w_uk", "s_uk", "w_uv", "s_uv")} | {
        ("indexer k LayerNorm f32", "weight"), ("indexer k LayerNorm f32", "bias"),
        ("RoPE table bf16", "cos"), ("RoPE table bf16", "sin")}
    assert all(k[1] == 5 for k in copies)


def test_refusals_name_the_tensor():
    layer, fw, _ = _layer(layouts.ROWMAJOR)
    assert binding.layer_disable_reason(NS(self_attn=layer.self_attn, input_layernorm=layer.input_layernorm,
                                           post_attention_layernorm=None, mlp=None), 4) is not None
    bad = NS(**vars(layer.self_attn))
    bad.q_b_proj = NS(weight=fw.w_qb.to(torch.bfloat16), weight_scale_inv=fw.s_qb)
    with pytest.raises(ValueError, match="q_b_proj"):
        binding.front_weights(NS(self_attn=bad, input_layernorm=layer.input_layernorm), 4, {})
    mixed = NS(**vars(layer.self_attn))
    mixed.q_b_proj = _lin(fw.w_qb, fw.s_qb, layouts.AITER16)
    with pytest.raises(ValueError, match="mixed FP8 layouts"):
        binding.front_weights(NS(self_attn=mixed, input_layernorm=layer.input_layernorm), 4, {})
    blocky = NS(**vars(layer.self_attn))
    blocky.w_scale = torch.ones(4)
    with pytest.raises(ValueError, match="scalar w_scale"):
        binding.post_weights(NS(self_attn=blocky), 4, {})
    no_index = NS(**vars(layer.self_attn))
    no_index.indexer = None
    with pytest.raises(ValueError, match="indexer"):
        binding.front_weights(NS(self_attn=no_index, input_layernorm=layer.input_layernorm), 4, {})


def _pool(slots=256, pages=4):
    kv = torch.zeros(slots, 1, DSV32.kv_row, dtype=FP8)
    pay = torch.zeros(pages, 1, 4, 64, 16, dtype=torch.uint8)
    sc = torch.zeros(pages, 1, 4, 64, dtype=torch.uint8)
    return NS(get_key_buffer=lambda i: kv, get_index_k_fp4_payload_buffer=lambda i: pay,
              get_index_k_fp4_scale_buffer=lambda i: sc), kv, pay, sc


def test_caches_bind_in_place_and_refuse_other_layouts():
    pool, kv, pay, sc = _pool()
    c = binding.caches(pool, 7)
    assert c.kv.data_ptr() == kv.data_ptr() and c.kv.shape == (256, 576) and c.kv.dtype == torch.uint8
    assert c.plane.data_ptr() == pay.data_ptr() and c.plane.shape == (4, 4, 64, 16)
    assert c.plane_scale.data_ptr() == sc.data_ptr() and c.plane_scale.shape == (4, 4, 64)
    # SGLang's MLA rows are raw E4M3: the launches keep no scale beside the pool, so a
    # slot that SGLang rewrites after the front wrote it reads back as SGLang wrote it
    assert c.kv_scale is None
    wide = NS(**vars(pool))
    wide.get_key_buffer = lambda i: torch.zeros(256, 1, 656, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="MLA cache"):
        binding.caches(wide, 7)
    paged = NS(**vars(pool))
    paged.get_index_k_fp4_payload_buffer = lambda i: torch.zeros(4, 1, 64, 132, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="FP4 index pages"):
        binding.caches(paged, 7)


def test_dsa_index_pages_bind_in_place():
    """DeepSeek-V3.2's NSA pool keeps its index keys in DSA pages
    (``get_index_k_with_scale_buffer``, [pages, 64 x (128 + 4)] uint8): bound in place as
    the tiled DSA format, with no scale plane; a page of another size is refused."""
    from sgl_amd_mono_amd import _lib

    kv = torch.zeros(256, 1, DSV32.kv_row, dtype=FP8)
    buf = torch.zeros(4, 64 * 132, dtype=torch.uint8)
    pool = NS(get_key_buffer=lambda i: kv, get_index_k_with_scale_buffer=lambda i: buf)
    c = binding.caches(pool, 3)
    assert c.index_format == _lib.INDEX_FP8_PAGE and c.plane_scale is None
    assert c.plane.data_ptr() == buf.data_ptr() and c.plane.shape == (4, 8448)
    assert binding.index_buffers(pool, 3) == [buf]
    odd = NS(get_key_buffer=lambda i: kv,
             get_index_k_with_scale_buffer=lambda i: torch.zeros(4, 64 * 130, dtype=torch.uint8))
    with pytest.raises(RuntimeError, match="DSA index pages"):
        binding.caches(odd, 3)
    with pytest.raises(RuntimeError, match="no index-key cache"):
        binding.caches(NS(get_key_buffer=lambda i: kv), 3)


def test_a_reused_slot_reads_back_unscaled():
    """A slot the front wrote (raw E4M3 of the row, oracle.front.kv_quant unscaled), then
    freed and rewritten by SGLang with another row: the attention's reader (oracle.attn
    kv_rows without scales, as the launch reads the bound pool) sees exactly the new
    row's E4M3 values, with no scale left over from the first writer."""
    from oracle import attn as A
    from oracle import formats as F
    from oracle import front as Fr

    pool, kv, _, _ = _pool()
    c = binding.caches(pool, 7)
    g = torch.Generator().manual_seed(5)
    first = torch.randn(576, generator=g).to(torch.bfloat16).float().numpy() * 40
    codes, sc = Fr.kv_quant(first, scaled=False)
    assert sc == 1.0
    c.kv[9] = torch.from_numpy(codes)  # the front's write
    np_first = A.kv_rows(c.kv.numpy(), c.kv_scale, [9])[0]
    assert np.allclose(np_first, F.e4m3_to_f32(codes))
    second = torch.randn(576, generator=g) * 0.01
    kv[9, 0] = second.to(FP8)  # SGLang's own write of the reused slot
    got = A.kv_rows(c.kv.numpy(), c.kv_scale, [9])[0]
    assert np.array_equal(got, second.to(FP8).float().numpy())


def test_page_tables_come_from_req_to_token():
    from sgl_amd_mono_amd.dsv32.runner import page_table

    g = torch.Generator().manual_seed(1)
    perm = torch.randperm(12, generator=g)
    req_to_token = torch.zeros(5, 4 * 64, dtype=torch.int32)
    for r in range(3):  # request r holds pages perm[4 r .. 4 r + 3], 64 slots each
        req_to_token[r] = (perm[4 * r : 4 * r + 4, None] * 64 + torch.arange(64)).reshape(-1)
    pt = page_table(req_to_token, torch.tensor([2, 0]), 2, 200)
    assert pt.dtype == torch.int32 and pt.shape == (2, 4)
    assert torch.equal(pt[0], perm[8:12].to(torch.int32)) and torch.equal(pt[1], perm[0:4].to(torch.int32))


def test_a_layer_that_cannot_bind_refuses_the_model_with_its_reason():
    from tests import fake_sglang

    fake_sglang.install()
    from sgl_amd_mono_amd.dsv32 import spec

    layer, _, _ = _layer(layouts.ROWMAJOR)
    ok = NS(self_attn=layer.self_attn, input_layernorm=layer.input_layernorm,
            post_attention_layernorm=NS(weight=torch.ones(DSV32.hidden, dtype=torch.bfloat16)),
            mlp=NS(gate=NS(weight=None, e_score_correction_bias=None),
                   experts=NS(w13_weight=torch.zeros(1, dtype=FP8), w13_weight_scale_inv=None,
                              w2_weight=None, w2_weight_scale_inv=None)))
    dense_attn = NS(**vars(layer.self_attn))
    dense_attn.indexer = None
    other = NS(**{**vars(ok), "self_attn": dense_attn})
    model = NS(model=NS(layers=[None, ok, other]))
    reasons = spec._model_disable_reasons(model, NS(first_k_dense_replace=1,
                                                    num_hidden_layers=3), {})
    assert len(reasons) == 1 and reasons[0].startswith("layer 2:") and "indexer" in reasons[0]
    assert spec._model_disable_reasons(NS(model=NS(layers=[None, ok])),
                                       NS(first_k_dense_replace=1, num_hidden_layers=2), {}) == []


def _sglang_attn(seed, positions=96):
    """SGLang's MLA tensors drawn on their own (not from the launches' structs): per-tensor
    E4M3 ``w_kc`` [32, 128, 512] and ``w_vc`` [32, 512, 128] at a scalar ``w_scale``, and
    a rotary ``cos_sin_cache`` [positions, 64] built as SGLang's rotary embedding builds
    it (angles pos * theta^(-2i/64), cos then sin)."""
    g = torch.Generator().manual_seed(seed)
    codes = lambda *shape: torch.randint(0, 0x7E, shape, generator=g, dtype=torch.uint8) | (
        torch.randint(0, 2, shape, generator=g, dtype=torch.uint8) << 7)
    w_kc = codes(DSV32.heads, DSV32.nope_dim, DSV32.kv_lora).view(FP8)
    w_vc = codes(DSV32.heads, DSV32.kv_lora, DSV32.v_dim).view(FP8)
    inv = 10000.0 ** (-torch.arange(0, 64, 2, dtype=torch.float64) / 64)
    ang = torch.arange(positions, dtype=torch.float64)[:, None] * inv[None]
    cache = torch.cat([ang.cos(), ang.sin()], 1).float()
    return NS(w_kc=w_kc, w_vc=w_vc, w_scale=torch.tensor(SCALE),
              rotary_emb=NS(cos_sin_cache=cache))


@pytest.mark.parametrize("layout", [layouts.ROWMAJOR, layouts.AITER16])
def test_packed_absorb_matrices_apply_sglangs_products(layout):
    """SGLang absorbs with q_lat[h] = q_nope[h] @ w_kc[h], maps the latent back with
    o[h] = o_lat[h] @ w_vc[h] (both times w_scale) and rotates with cos, sin =
    cos_sin_cache[pos].chunk(2, -1). The packed W_UK / W_UV rows, applied as the launches'
    GEMVs apply theirs (``oracle.dense.w8a16_gemv``: y = W x over row-major [out, in]),
    give exactly those products, and the bf16 table holds the two halves. A W packed
    without the transpose (the plain reshape of w_kc / w_vc) gives other products: the
    check tells a transpose slip from the right packing."""
    from oracle import dense as D
    from oracle import formats as F

    attn = _sglang_attn(11)
    copies = {}
    w_uk, s_uk = binding.pack_uk(attn, 2, copies, layout)
    w_uv, s_uv = binding.pack_uv(attn, 2, copies, layout)
    g = torch.Generator().manual_seed(12)
    q_nope = torch.randn(3, DSV32.heads, DSV32.nope_dim, generator=g).to(torch.bfloat16).double()
    o_lat = torch.randn(3, DSV32.heads, DSV32.kv_lora, generator=g).to(torch.bfloat16).double()
    kc = torch.from_numpy(F.e4m3_to_f32(attn.w_kc.view(torch.uint8).numpy())).double() * SCALE
    vc = torch.from_numpy(F.e4m3_to_f32(attn.w_vc.view(torch.uint8).numpy())).double() * SCALE
    for h in (0, 17, 31):
        uk = _rowmajor(w_uk[h], layout).view(torch.uint8).numpy()
        uv = _rowmajor(w_uv[h], layout).view(torch.uint8).numpy()
        got_lat = D.w8a16_gemv(q_nope[:, h], uk, s_uk[h].numpy())
        got_o = D.w8a16_gemv(o_lat[:, h], uv, s_uv[h].numpy())
        np.testing.assert_allclose(got_lat, (q_nope[:, h] @ kc[h]).numpy(), rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(got_o, (o_lat[:, h] @ vc[h]).numpy(), rtol=1e-12, atol=1e-12)
        # the negative control: the same bytes read without the transpose
        wrong = attn.w_kc[h].view(torch.uint8).reshape(DSV32.kv_lora, DSV32.nope_dim).numpy()
        bad = D.w8a16_gemv(q_nope[:, h], wrong, s_uk[h].numpy())
        assert not np.allclose(bad, (q_nope[:, h] @ kc[h]).numpy(), rtol=1e-3, atol=1e-3)
    cos, sin = binding.rope_table({2: NS(self_attn=attn)}, copies)
    cache = attn.rotary_emb.cos_sin_cache
    pos = torch.tensor([0, 5, 95])
    want_cos, want_sin = cache[pos].chunk(2, -1)
    assert torch.equal(cos[pos], want_cos.to(torch.bfloat16))
    assert torch.equal(sin[pos], want_sin.to(torch.bfloat16))
    assert {k[2] for k in copies} == {"w_uk", "s_uk", "w_uv", "s_uv", "cos", "sin"}


def test_one_rope_table_serves_every_layer_and_the_indexers_must_agree():
    """The covered layers share one bf16 table (logged once); a layer's indexer whose
    rotary holds another cache (a different base) refuses the model."""
    a, b = _sglang_attn(1), _sglang_attn(2)
    b.rotary_emb = a.rotary_emb  # SGLang shares the rotary module between layers
    a.indexer = NS(rotary_emb=NS(cos_sin_cache=a.rotary_emb.cos_sin_cache.clone()))
    copies = {}
    cos, sin = binding.rope_table({4: NS(self_attn=b), 3: NS(self_attn=a)}, copies)
    assert list(copies) == [("RoPE table bf16", 3, "cos"), ("RoPE table bf16", 3, "sin")]
    other = _sglang_attn(3, positions=96)
    other.rotary_emb.cos_sin_cache[:, :32] *= 0.5
    a.indexer = NS(rotary_emb=other.rotary_emb)
    with pytest.raises(ValueError, match="indexer"):
        binding.rope_table({3: NS(self_attn=a), 4: NS(self_attn=b)}, {})
