"""Seeded synthetic inputs of the benchmark configs (no checkpoints here).

Distributions follow the reference's kernel tests: router ~N(0,1)*2/sqrt(H) and bias
0.1*N(0,1) (``test/kernels/glm53/check_layer.py:96-99``), expert weights ``randn`` cast
to E4M3 (``check_layer.py:56-59``), norm weights 1 + 0.1*N(0,1) (``:67-68``); block
scales ~U(0.5, 2)/448; MXFP4 codes random bytes with E8M0 scales in [119, 122]
(``test/kernels/test_minimax_m31_ffn.py:44-51``). Each tensor family draws from its own
``torch.Generator`` seeded from (seed, family) in a fixed order.
"""

from __future__ import annotations

import torch

from .. import _lib, layouts
from .config import DSV32, MXFP4_MOE, LayerConfig, Mxfp4MoeConfig
from .moe import MoeFp8Weights, MoeMxfp4LayerWeights, MoeMxfp4Weights
from .post import PostWeights
from .front import FrontCaches, FrontWeights

FP8 = torch.float8_e4m3fn


def _gen(device, seed: int, family: int) -> torch.Generator:
    return torch.Generator(device=device).manual_seed(1_000_003 * seed + 7919 * family + 17)


def _router(dev, seed: int, cfg: LayerConfig):
    """The router w_r bf16 [E, H], its bias f32 [E] and the post-attention norm bf16 [H]."""
    h, e = cfg.hidden, cfg.experts
    g = _gen(dev, seed, 1)
    w_r = (torch.randn(e, h, generator=g, device=dev) * (2.0 / h ** 0.5)).to(torch.bfloat16)
    bias = torch.randn(e, generator=_gen(dev, seed, 2), device=dev) * 0.1
    g_post = (1 + 0.1 * torch.randn(h, generator=_gen(dev, seed, 3), device=dev)).to(torch.bfloat16)
    return w_r, bias, g_post


def moe_fp8_weights(device, seed: int = 0, cfg: LayerConfig = DSV32,
                    experts: int | None = None, layout: str = layouts.ROWMAJOR) -> MoeFp8Weights:
    """Config 2 weights; ``experts`` limits how many expert slots get random values
    (the rest stay zero) to keep CPU-side fixtures small; ``layout`` "aiter16" stores the
    same values in AITER's (16, 16) shuffle."""
    dev = torch.device(device)
    h, i, e = cfg.hidden, cfg.inter, cfg.experts
    n = e + 1
    w_r, bias, g_post = _router(dev, seed, cfg)
    w13 = torch.zeros(n, 2 * i, h, dtype=FP8, device=dev)
    w2 = torch.zeros(n, h, i, dtype=FP8, device=dev)
    gw = _gen(dev, seed, 4)
    live = range(n) if experts is None else sorted(set(range(min(experts, n))) | {n - 1})
    for x in live:
        w13[x] = torch.randn(2 * i, h, generator=gw, device=dev).to(FP8)
        w2[x] = torch.randn(h, i, generator=gw, device=dev).to(FP8)
    gs = _gen(dev, seed, 5)
    s13 = (0.5 + 1.5 * torch.rand(n, 2 * i // 128, h // 128, generator=gs, device=dev)) / 448.0
    s2 = (0.5 + 1.5 * torch.rand(n, h // 128, i // 128, generator=gs, device=dev)) / 448.0
    if layout == layouts.AITER16:
        for x in range(n):  # expert by expert: no 2x peak copy of ~3 GB
            w13[x] = layouts.shuffle_16x16(w13[x].view(torch.uint8)).view(FP8)
            w2[x] = layouts.shuffle_16x16(w2[x].view(torch.uint8)).view(FP8)
    return MoeFp8Weights(g_post=g_post, w_r=w_r, bias=bias, w13=w13, s13=s13, w2=w2, s2=s2,
                         layout=layout)


def rowmajor_expert(w: MoeFp8Weights, e: int):
    """Expert e's (w13, s13, w2, s2) on the host as numpy, row-major (for the oracle)."""
    w13, w2 = w.w13[e].view(torch.uint8), w.w2[e].view(torch.uint8)
    if w.layout == layouts.AITER16:
        w13, w2 = layouts.unshuffle_16x16(w13), layouts.unshuffle_16x16(w2)
    return (w13.cpu().numpy(), w.s13[e].cpu().numpy(), w2.cpu().numpy(), w.s2[e].cpu().numpy())


def rows_bf16(rows: int, hidden: int, device, seed: int = 0) -> torch.Tensor:
    """Activation rows ~N(0,1), bf16."""
    g = _gen(torch.device(device), seed, 100 + rows)
    return torch.randn(rows, hidden, generator=g, device=device).to(torch.bfloat16)


def mxfp4_moe_weights(device, seed: int = 0, cfg: Mxfp4MoeConfig = MXFP4_MOE,
                      layout: str = layouts.ROWMAJOR, e13=(119, 122),
                      e2=(119, 122)) -> MoeMxfp4Weights:
    """Config 4: E2M1 codes (random bytes, even index in the low nibble) with E8M0
    scales per 32 in [119, 122]; w13 [E+1, 2I, H/2] + [E+1, 2I, H/32], w2 [E+1, H, I/2] +
    [E+1, H, I/32]; router bias f32 0.01*N(0,1). ``layout`` "aiter16" stores the same
    values in the (16, 16) code shuffle and the e8m0 scale shuffle."""
    dev = torch.device(device)
    h, i, n = cfg.hidden, cfg.inter, cfg.experts + 1
    g = _gen(dev, seed, 11)
    u8 = dict(dtype=torch.uint8, device=dev, generator=g)
    w13 = torch.randint(0, 256, (n, 2 * i, h // 2), **u8)
    s13 = torch.randint(e13[0], e13[1] + 1, (n, 2 * i, h // 32), **u8)
    w2 = torch.randint(0, 256, (n, h, i // 2), **u8)
    s2 = torch.randint(e2[0], e2[1] + 1, (n, h, i // 32), **u8)
    bias = torch.randn(cfg.experts, generator=_gen(dev, seed, 12), device=dev) * 0.01
    if layout == layouts.AITER16:
        w13, w2 = layouts.shuffle_16x16(w13), layouts.shuffle_16x16(w2)
        s13, s2 = layouts.shuffle_e8m0(s13), layouts.shuffle_e8m0(s2)
    return MoeMxfp4Weights(bias=bias, w13=w13, s13=s13, w2=w2, s2=s2, layout=layout)


# MXFP4 experts at the layer's geometry (hidden 7168, expert intermediate 512)
MXFP4_LAYER_MOE = Mxfp4MoeConfig(hidden=DSV32.hidden, inter=DSV32.inter)


def moe_mxfp4_layer_weights(device, seed: int = 0, cfg: LayerConfig = DSV32,
                            layout: str = layouts.ROWMAJOR) -> MoeMxfp4LayerWeights:
    """The layer's FFN with MXFP4 experts: the router and norm as ``moe_fp8_weights``
    draws them, the experts as ``mxfp4_moe_weights`` at the layer's geometry with E8M0
    exponents around the variance-preserving scale (weight rms ~ 1/sqrt(K); random E2M1
    codes have rms 2.93): 2^(e - 127) 2.93 sqrt(7168) ~ 1 at e = 119 for w13 and
    2.93 sqrt(512) ~ 2^6 at e = 121 for w2, each +-1, so the rows' MoE sum is O(1)."""
    dev = torch.device(device)
    w_r, bias, g_post = _router(dev, seed, cfg)
    x = mxfp4_moe_weights(dev, seed, Mxfp4MoeConfig(hidden=cfg.hidden, inter=cfg.inter,
                                                    experts=cfg.experts), layout=layout,
                          e13=(118, 120), e2=(120, 122))
    return MoeMxfp4LayerWeights(g_post=g_post, w_r=w_r, bias=bias, w13=x.w13, s13=x.s13,
                                w2=x.w2, s2=x.s2, layout=layout)


def rowmajor_mxfp4_expert(w, e: int, cfg: Mxfp4MoeConfig = MXFP4_MOE):
    """Expert e's (w13, s13, w2, s2) bytes on the host as numpy, row-major."""
    w13, s13, w2, s2 = w.w13[e], w.s13[e], w.w2[e], w.s2[e]
    if w.layout == layouts.AITER16:
        w13, w2 = layouts.unshuffle_16x16(w13), layouts.unshuffle_16x16(w2)
        s13 = layouts.unshuffle_e8m0(s13, cfg.hidden // 32)
        s2 = layouts.unshuffle_e8m0(s2, cfg.inter // 32)
    return tuple(t.cpu().numpy() for t in (w13, s13, w2, s2))


def logits_f32(rows: int, experts: int, device, seed: int = 0) -> torch.Tensor:
    g = _gen(torch.device(device), seed, 200 + rows)
    return torch.randn(rows, experts, generator=g, device=device)


def dsa_pages(pages: int, device, seed: int = 0) -> torch.Tensor:
    """DSA index pages uint8 [pages, 8448] with random contents: E4M3 values (no NaN
    codes), then per-token power-of-two f32 scales 2^-10 .. 2^-6."""
    dev = torch.device(device)
    g = _gen(dev, seed, 24)
    vals = torch.randint(0, 256, (pages, 8192), generator=g, device=dev, dtype=torch.uint8)
    vals[(vals & 0x7F) == 0x7F] ^= 1
    sc = torch.exp2(torch.randint(-10, -5, (pages, 64), generator=g, device=dev).float())
    return torch.cat([vals, sc.view(torch.uint8).view(pages, 256)], 1).contiguous()


def attention_inputs(rows: int, ctx: int, device, seed: int = 0, positions=None,
                     extra_pages: int = 3, index_format: int = _lib.INDEX_FP4_PLANE):
    """Config 3: each row its own request seeing ``ctx`` keys (position ctx - 1 unless
    ``positions`` is given), its pages a random permutation of the plane (as
    ``test/kernels/test_deepseek_v41_k2i.py:109-119``). Index plane: random E2M1 bytes,
    E8M0 scales in [123, 129]; index query likewise; head weights 0.05 N(0, 1); q bf16
    N(0, 1); KV rows E4M3 of N(0, 1) with per-token scales U(0.5, 1.5). With a DSA
    ``index_format``: DSA pages (``dsa_pages``) and a bf16 N(0, 1) index query."""
    from .attn import AttnInputs

    dev = torch.device(device)
    ppr = -(-ctx // 64)
    pages = rows * ppr + extra_pages
    g = _gen(dev, seed, 21)
    u8 = dict(dtype=torch.uint8, device=dev, generator=g)
    plane = torch.randint(0, 256, (pages, 4, 64, 16), **u8)
    plane_scale = torch.randint(123, 130, (pages, 4, 64), **u8)
    perm = torch.randperm(pages, generator=g, device=dev).to(torch.int32)
    page_table = perm[: rows * ppr].view(rows, ppr).contiguous()
    iq = torch.randint(0, 256, (rows, 64, 64), **u8)
    iqs = torch.randint(123, 130, (rows, 4, 16, 4), **u8)
    if index_format != _lib.INDEX_FP4_PLANE:
        plane, plane_scale, iqs = dsa_pages(pages, dev, seed), None, None
        iq = torch.randn(rows, 64, 128, generator=_gen(dev, seed, 25), device=dev).to(torch.bfloat16)
    gq = _gen(dev, seed, 22)
    iw = torch.randn(rows, 64, generator=gq, device=dev) * 0.05
    q = torch.randn(rows, 32, 576, generator=gq, device=dev).to(torch.bfloat16)
    gk = _gen(dev, seed, 23)
    kv = torch.empty(pages * 64, 576, dtype=torch.uint8, device=dev)
    for i in range(0, pages * 64, 1 << 16):  # in pieces: no f32 copy of the whole cache
        n = min(1 << 16, pages * 64 - i)
        kv[i : i + n] = torch.randn(n, 576, generator=gk, device=dev).to(FP8).view(torch.uint8)
    kv_scale = 0.5 + torch.rand(pages * 64, generator=gk, device=dev)
    if positions is None:
        positions = torch.full((rows,), ctx - 1, dtype=torch.int64, device=dev)
    else:
        positions = torch.as_tensor(positions, dtype=torch.int64, device=dev)
    req_ids = torch.arange(rows, dtype=torch.int32, device=dev)
    return AttnInputs(q=q, iq=iq, iqs=iqs, iw=iw, plane=plane, plane_scale=plane_scale, kv=kv,
                      kv_scale=kv_scale, positions=positions, req_ids=req_ids,
                      page_table=page_table, index_format=index_format)


def post_weights(device, seed: int = 0, cfg: LayerConfig = DSV32,
                 layout: str = layouts.ROWMAJOR) -> PostWeights:
    """W_UV [32, 128, 512] and o_proj [7168, 4096]: ``randn`` cast to E4M3 with block
    scales ~U(0.5, 2)/448 (as the expert weights); ``layout`` "aiter16" shuffles each
    [N, K] matrix."""
    dev = torch.device(device)
    hh, v, c, hid = cfg.heads, cfg.v_dim, cfg.kv_lora, cfg.hidden
    g = _gen(dev, seed, 40)
    w_uv = torch.randn(hh, v, c, generator=g, device=dev).to(FP8)
    w_o = torch.randn(hid, hh * v, generator=g, device=dev).to(FP8)
    gs = _gen(dev, seed, 41)
    s_uv = (0.5 + 1.5 * torch.rand(hh, v // 128, c // 128, generator=gs, device=dev)) / 448.0
    s_o = (0.5 + 1.5 * torch.rand(hid // 128, hh * v // 128, generator=gs, device=dev)) / 448.0
    if layout == layouts.AITER16:
        for i in range(hh):
            w_uv[i] = layouts.shuffle_16x16(w_uv[i].view(torch.uint8)).view(FP8)
        w_o = layouts.shuffle_16x16(w_o.view(torch.uint8)).view(FP8)
    return PostWeights(w_uv=w_uv, s_uv=s_uv, w_o=w_o, s_o=s_o, layout=layout)


def rowmajor_post(w: PostWeights):
    """(w_uv, s_uv, w_o, s_o) on the host as numpy, row-major (for the oracle)."""
    w_uv, w_o = w.w_uv.view(torch.uint8), w.w_o.view(torch.uint8)
    if w.layout == layouts.AITER16:
        w_uv = torch.stack([layouts.unshuffle_16x16(x) for x in w_uv])
        w_o = layouts.unshuffle_16x16(w_o)
    return (w_uv.cpu().numpy(), w.s_uv.cpu().numpy(), w_o.cpu().numpy(), w.s_o.cpu().numpy())


def rope_tables(rows: int, device, dim: int = 64, base: float = 10000.0):
    """bf16 cos / sin [rows, dim / 2] of position p and pair i: angle p base^(-2i / dim)."""
    i = torch.arange(dim // 2, dtype=torch.float64)
    ang = torch.arange(rows, dtype=torch.float64)[:, None] * base ** (-2.0 * i / dim)[None]
    return (ang.cos().to(torch.bfloat16).to(device), ang.sin().to(torch.bfloat16).to(device))


def front_weights(device, seed: int = 0, cfg: LayerConfig = DSV32, layout: str = layouts.ROWMAJOR,
                  rope_rows: int = 32768) -> FrontWeights:
    """The attention front of one layer: FP8 matrices ``randn`` cast to E4M3 with block
    scales ~U(0.5, 2)/448, norm weights 1 + 0.1 N(0, 1) (``check_layer.py:67-68``), the
    head weights bf16 N(0, 1) / sqrt(7168), the index-key LayerNorm bias 0.1 N(0, 1)."""
    dev = torch.device(device)
    H, QL, KL, PE = cfg.hidden, cfg.q_lora, cfg.kv_lora, cfg.rope_dim
    qkv = QL + KL + PE
    g = _gen(dev, seed, 60)
    norm = lambda n: (1 + 0.1 * torch.randn(n, generator=g, device=dev)).to(torch.bfloat16)
    g_in, g_q, g_kv = norm(H), norm(QL), norm(KL)
    gw = _gen(dev, seed, 61)
    fp8 = lambda *shape: torch.randn(*shape, generator=gw, device=dev).to(FP8)
    w_qkv_a, w_k = fp8(qkv, H), fp8(cfg.index_dim, H)
    w_qb = fp8(cfg.heads * cfg.qk_dim, QL)
    w_iq = fp8(cfg.index_heads * cfg.index_dim, QL)
    w_uk = fp8(cfg.heads, KL, cfg.nope_dim)
    gs = _gen(dev, seed, 62)
    sc = lambda *shape: (0.5 + 1.5 * torch.rand(*shape, generator=gs, device=dev)) / 448.0
    cb = lambda n: (n + 127) // 128
    s_qkv_a, s_k = sc(cb(qkv), H // 128), sc(1, H // 128)
    s_qb, s_iq = sc(w_qb.shape[0] // 128, QL // 128), sc(w_iq.shape[0] // 128, QL // 128)
    s_uk = sc(cfg.heads, KL // 128, 1)
    gx = _gen(dev, seed, 63)
    w_w = (torch.randn(cfg.index_heads, H, generator=gx, device=dev) / H ** 0.5).to(torch.bfloat16)
    g_k = 1 + 0.1 * torch.randn(cfg.index_dim, generator=gx, device=dev)
    b_k = 0.1 * torch.randn(cfg.index_dim, generator=gx, device=dev)
    if layout == layouts.AITER16:
        sh = lambda t: layouts.shuffle_16x16(t.view(torch.uint8)).view(FP8)
        w_qkv_a, w_k, w_qb, w_iq = sh(w_qkv_a), sh(w_k), sh(w_qb), sh(w_iq)
        w_uk = torch.stack([sh(w_uk[i]) for i in range(cfg.heads)])
    cos, sin = rope_tables(rope_rows, dev, PE)
    return FrontWeights(g_in=g_in, g_q=g_q, g_kv=g_kv, w_qkv_a=w_qkv_a, s_qkv_a=s_qkv_a, w_k=w_k,
                        s_k=s_k, w_w=w_w, g_k=g_k, b_k=b_k, w_qb=w_qb, s_qb=s_qb, w_iq=w_iq,
                        s_iq=s_iq, w_uk=w_uk, s_uk=s_uk, cos=cos, sin=sin, layout=layout)


def rowmajor_front(w: FrontWeights) -> dict:
    """The oracle's arguments (numpy, row-major) of ``oracle.front.front``."""
    u8 = lambda t: t.view(torch.uint8)
    un = (lambda t: layouts.unshuffle_16x16(u8(t))) if w.layout == layouts.AITER16 else u8
    w_uk = torch.stack([un(w.w_uk[i]) for i in range(w.w_uk.shape[0])])
    np_ = lambda t: t.cpu().numpy()
    return dict(g_in=w.g_in.cpu(), g_q=w.g_q.cpu(), g_kv=w.g_kv.cpu(), w_qkv_a=np_(un(w.w_qkv_a)),
                s_qkv_a=np_(w.s_qkv_a), w_k=np_(un(w.w_k)), s_k=np_(w.s_k), w_w=w.w_w.cpu(),
                g_k=np_(w.g_k), b_k=np_(w.b_k), w_qb=np_(un(w.w_qb)), s_qb=np_(w.s_qb),
                w_iq=np_(un(w.w_iq)), s_iq=np_(w.s_iq), w_uk=np_(w_uk), s_uk=np_(w.s_uk),
                cos=w.cos.cpu(), sin=w.sin.cpu())


def front_caches(device, slots: int, pages: int, seed: int = 0,
                 index_format: int = _lib.INDEX_FP4_PLANE) -> FrontCaches:
    """Caches with random prior contents (so untouched slots can be checked)."""
    dev = torch.device(device)
    g = _gen(dev, seed, 64)
    kv = torch.randint(0, 256, (slots, 576), generator=g, device=dev, dtype=torch.uint8)
    kv[(kv & 0x7F) == 0x7F] = 0  # no NaN codes
    kv_scale = torch.rand(slots, generator=g, device=dev)
    if index_format != _lib.INDEX_FP4_PLANE:
        return FrontCaches(kv=kv, kv_scale=kv_scale, plane=dsa_pages(pages, dev, seed),
                           plane_scale=None, index_format=index_format)
    plane = torch.randint(0, 256, (pages, 4, 64, 16), generator=g, device=dev, dtype=torch.uint8)
    plane_scale = torch.randint(120, 130, (pages, 4, 64), generator=g, device=dev, dtype=torch.uint8)
    return FrontCaches(kv=kv, kv_scale=kv_scale, plane=plane, plane_scale=plane_scale)


def layer(rows: int, ctx: int, device, seed: int = 0, layout: str = layouts.AITER16,
          index_format: int = _lib.INDEX_FP4_PLANE, experts: str = "fp8"):
    """Config 5, one layer: its weights (front, output block, MoE with ``experts`` "fp8" or
    "mxfp4"), caches as config 3
    (each row its own request at position ctx - 1 over shuffled pages; the index keys in
    ``index_format``), the step's tables (each row's slot the page-table entry of its
    position) and the input rows h. Returns (LayerWeights, FrontCaches, LayerStep, h)."""
    from .layer import LayerStep, LayerWeights

    dev = torch.device(device)
    w = LayerWeights(front=front_weights(dev, seed, layout=layout, rope_rows=max(ctx, 1)),
                     post=post_weights(dev, seed, layout=layout),
                     moe=moe_fp8_weights(dev, seed, layout=layout) if experts == "fp8" else
                     moe_mxfp4_layer_weights(dev, seed, layout=layout))
    if experts not in ("fp8", "mxfp4"):
        raise ValueError(f"experts {experts!r}: 'fp8' or 'mxfp4'")
    a = attention_inputs(rows, ctx, dev, seed=seed, index_format=index_format)
    caches = FrontCaches(kv=a.kv, kv_scale=a.kv_scale, plane=a.plane, plane_scale=a.plane_scale,
                         index_format=index_format)
    pos = a.positions
    page = a.page_table.gather(1, (pos // 64).to(torch.int64)[:, None])[:, 0].to(torch.int64)
    step = LayerStep(positions=pos, slots=page * 64 + pos % 64, req_ids=a.req_ids,
                     page_table=a.page_table)
    return w, caches, step, rows_bf16(rows, DSV32.hidden, dev, seed=seed)
