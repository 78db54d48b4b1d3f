"""One GPU's TP=4 share of a DeepSeek-V3.2 DSA decoder layer on gfx950: the front (norms,
projections, RoPE, KV and index-key cache writes), the attention phase (FP4 indexer,
exact top-2048, sparse MLA), the output block (W_UV, o_proj, residual) and the MoE
(post-norm, router, top-8 + shared experts, residual) over FP8 or, in the one launch,
MXFP4 (A16W4) experts.

``FusedLayerOp.launch(h, caches, step) -> x_out`` runs the layer as ONE persistent launch
(``mono_layer_launch``); ``LayerOp`` runs the same four phases as four launches on one
stream (each phase's own entry point: bit-equal results, and the per-phase timings).
Both mirror the reference's per-layer entry ``Glm53LayerOp.launch(h, caches, cos, sin,
step)`` (``sgl_amd_mono/glm53/gfx950/runner.py:240-321``): shapes and dtypes are checked
before anything launches (``ValueError``), launches go on the current stream with no
host synchronisation, and the result is runtime-owned (two parity output buffers, so a
launch never writes the tensor the previous one returned). The W == 1 reduces are the
local residual adds of the output block and the MoE (``kernel.py:1665-1669``).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Union

import torch

import ctypes

from .. import _lib, layouts
from ..runtime import MonoRuntime, shared_or_new
from .attn import MAX_CTX, AttnInputs, AttnOp
from .config import DSV32, LayerConfig
from .front import FrontCaches, FrontOp, FrontWeights
from .moe import MoeFp8Op, MoeFp8Weights, MoeMxfp4LayerWeights, _need
from .post import PostOp, PostWeights


@dataclass
class LayerWeights:
    front: FrontWeights
    post: PostWeights
    moe: Union[MoeFp8Weights, MoeMxfp4LayerWeights]


@dataclass
class LayerStep:
    """A decode step's tables (rows [R]): positions i64, cache slots i64 (page * 64 +
    offset; -1 for a pad row), request ids i32, the page table i32 [requests, pages]."""

    positions: torch.Tensor
    slots: torch.Tensor
    req_ids: torch.Tensor
    page_table: torch.Tensor


class LayerRuntimes:
    """The scratch and guard blocks of the four launch kinds, shareable by every layer
    on a device (the layers' launches are ordered on one stream, and each launch's tag
    comes from its runtime's epoch, so one set serves all of them)."""

    def __init__(self, device, cfg: LayerConfig = DSV32, max_rows: int = 8,
                 ctx_max: int = 32768, deadline_s: float = 10.0):
        lib = _lib.lib()
        self.device = torch.device(device)
        self.max_rows, self.ctx_max = max_rows, ctx_max
        self.front = MonoRuntime(lib.mono_front_scratch_bytes(), self.device, deadline_s)
        self.attn = MonoRuntime(lib.mono_attn_scratch_bytes(max_rows), self.device, deadline_s)
        self.post = MonoRuntime(lib.mono_post_scratch_bytes(), self.device, deadline_s)
        self.moe = MonoRuntime(lib.mono_moe_fp8_scratch_bytes(cfg.hidden, cfg.inter, cfg.experts),
                               self.device, deadline_s)

    def all(self):
        return (self.front, self.attn, self.post, self.moe)


class LayerOp:
    """The four launches of one layer for up to ``max_rows`` rows, on a device (with
    runtimes of its own) or on shared ``LayerRuntimes``."""

    def __init__(self, weights: LayerWeights, device_or_rts, cfg: LayerConfig = DSV32,
                 max_rows: int = 8, ctx_max: int = 32768, deadline_s: float = 10.0,
                 sm_scale: Optional[float] = None):
        rts = device_or_rts
        if isinstance(weights.moe, MoeMxfp4LayerWeights):
            raise ValueError("MXFP4 experts run in the one-launch layer (FusedLayerOp) only")
        if not isinstance(rts, LayerRuntimes):
            rts = LayerRuntimes(rts, cfg, max_rows, ctx_max, deadline_s)
        device, max_rows, ctx_max = rts.device, rts.max_rows, rts.ctx_max
        self.cfg, self.device, self.rts = cfg, device, rts
        self.front = FrontOp(weights.front, device, cfg, max_rows, deadline_s, rt=rts.front)
        self.attn = AttnOp(device, cfg, max_rows, ctx_max, sm_scale=sm_scale,
                           deadline_s=deadline_s, rt=rts.attn)
        self.post = PostOp(weights.post, device, cfg, max_rows, deadline_s, rt=rts.post)
        self.moe = MoeFp8Op(weights.moe, device, cfg, max_rows=max_rows, deadline_s=deadline_s,
                            rt=rts.moe)
        self.max_rows = max_rows

    def runtimes(self):
        return self.rts.all()

    def check(self) -> None:
        for rt in self.runtimes():
            rt.check()

    def launch(self, h: torch.Tensor, caches: FrontCaches, step: LayerStep,
               out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
        f = self.front.launch(h, caches, step.positions, step.slots, stream=stream)
        inp = AttnInputs(q=f.q, iq=f.iq, iqs=f.iqs, iw=f.iw, plane=caches.plane,
                         plane_scale=caches.plane_scale, kv=caches.kv, kv_scale=caches.kv_scale,
                         positions=step.positions, req_ids=step.req_ids,
                         page_table=step.page_table, index_format=caches.index_format)
        o_lat = self.attn.launch(inp, stream=stream)
        a = self.post.launch(o_lat, h, stream=stream)
        return self.moe.launch(a, out=out, stream=stream)


@dataclass
class LayerDebug:
    """Optional views into a layer launch (each None or a tensor of the named shape, rows
    [R]): the phases' hand-offs q bf16 [R, 32, 576], iq u8 [R, 64, 64] (a DSA index
    page's: bf16 [R, 64, 128]), iqs u8 [R, 4, 16, 4] (FP4 plane only), iw f32 [R, 64], o_lat bf16 [R, 32, 512], a bf16 [R, 7168]; and outputs scores f32
    [R, ctx_max], topk i32 [R, 2048], y f32 [R, 7168], moe_scores f32 [R, 256], ids i32
    [R, 9], weights f32 [R, 9]."""

    q: Optional[torch.Tensor] = None
    iq: Optional[torch.Tensor] = None
    iqs: Optional[torch.Tensor] = None
    iw: Optional[torch.Tensor] = None
    o_lat: Optional[torch.Tensor] = None
    a: Optional[torch.Tensor] = None
    scores: Optional[torch.Tensor] = None
    topk: Optional[torch.Tensor] = None
    y: Optional[torch.Tensor] = None
    moe_scores: Optional[torch.Tensor] = None
    ids: Optional[torch.Tensor] = None
    weights: Optional[torch.Tensor] = None

    def check(self, r: int, ctx_max: int, cfg: LayerConfig, device,
              index_format: int = _lib.INDEX_FP4_PLANE) -> None:
        fp4 = index_format == _lib.INDEX_FP4_PLANE
        if not fp4 and self.iqs is not None:
            raise ValueError("iqs: a DSA index page's query has no E8M0 scales")
        shapes = dict(q=(torch.bfloat16, (r, cfg.heads, cfg.kv_row)),
                      iq=(torch.uint8, (r, cfg.index_heads, cfg.index_dim // 2)) if fp4 else
                      (torch.bfloat16, (r, cfg.index_heads, cfg.index_dim)),
                      iqs=(torch.uint8, (r, 4, 16, 4)),
                      iw=(torch.float32, (r, cfg.index_heads)),
                      o_lat=(torch.bfloat16, (r, cfg.heads, cfg.kv_lora)),
                      a=(torch.bfloat16, (r, cfg.hidden)),
                      scores=(torch.float32, (r, ctx_max)),
                      topk=(torch.int32, (r, cfg.index_topk)),
                      y=(torch.float32, (r, cfg.hidden)),
                      moe_scores=(torch.float32, (r, cfg.experts)),
                      ids=(torch.int32, (r, cfg.top_k + 1)),
                      weights=(torch.float32, (r, cfg.top_k + 1)))
        for name, (dtype, shape) in shapes.items():
            t = getattr(self, name)
            if t is not None:
                _need(t, name, dtype, shape, device)


def layer_runtime(device, max_rows: int = 8, deadline_s: float = 10.0) -> MonoRuntime:
    """The scratch and guard of the one-launch layer for up to ``max_rows`` rows: one per
    device can serve every layer (their launches are ordered on one stream)."""
    nbytes = _lib.lib().mono_layer_scratch_bytes(max_rows)
    if nbytes == 0:
        raise ValueError(f"no layer launch for {max_rows} rows (1..8)")
    return MonoRuntime(nbytes, device, deadline_s)


class FusedLayerOp:
    """The layer as one persistent launch for up to ``max_rows`` rows (<= 8) seeing at most
    ``ctx_max`` keys, with a runtime of its own or a shared one (``rt``; FP8- and
    MXFP4-expert layers can share one). ``weights.moe`` is ``MoeFp8Weights`` (W8A8) or
    ``MoeMxfp4LayerWeights`` (A16W4)."""

    def __init__(self, weights: LayerWeights, device, cfg: LayerConfig = DSV32,
                 max_rows: int = 8, ctx_max: int = 32768, deadline_s: float = 10.0,
                 sm_scale: Optional[float] = None, fault=(0, 0),
                 rt: Optional[MonoRuntime] = None):
        self.cfg, self.device = cfg, torch.device(device)
        if not 1 <= max_rows <= 8:
            raise ValueError("max_rows must be 1..8")
        if not 1 <= ctx_max <= MAX_CTX:
            raise ValueError(f"ctx_max must be 1..{MAX_CTX}")
        self.mx = isinstance(weights.moe, MoeMxfp4LayerWeights)
        if self.mx:
            weights = LayerWeights(weights.front, weights.post, weights.moe.bytes_view())
        weights.front.validate(cfg, self.device)
        weights.post.validate(cfg, self.device)
        weights.moe.validate(cfg, self.device)
        lays = {weights.front.layout, weights.post.layout, weights.moe.layout}
        if len(lays) != 1:
            raise ValueError(f"one weight layout for the whole layer, got {sorted(lays)}")
        self.w, self.layout = weights, lays.pop()
        nbytes = _lib.lib().mono_layer_scratch_bytes(max_rows)
        self.rt = shared_or_new(rt, nbytes, self.device, deadline_s)
        self.max_rows, self.ctx_max, self.fault = max_rows, ctx_max, fault
        self.sm_scale = sm_scale if sm_scale is not None else cfg.softmax_scale
        self.outs = [torch.empty(max_rows, cfg.hidden, dtype=torch.bfloat16, device=self.device)
                     for _ in range(2)]
        self.parity = 0

    def check(self) -> None:
        self.rt.check()

    def launch(self, h: torch.Tensor, caches: FrontCaches, step: LayerStep,
               out: Optional[torch.Tensor] = None, stream=None,
               debug: Optional[LayerDebug] = None,
               timeline: Optional[torch.Tensor] = None,
               phase_timeline: Optional[torch.Tensor] = None) -> torch.Tensor:
        """``timeline`` i64 [grid, 8] takes the launch's marks (start, each phase done,
        exit); ``phase_timeline`` i64 [4, grid, 8] each phase's own stamps."""
        cfg, dev, w = self.cfg, self.device, self.w
        r = h.shape[0] if h.dim() == 2 else -1
        if not 1 <= r <= self.max_rows:
            raise ValueError(f"h: needs [1..{self.max_rows}, {cfg.hidden}]")
        _need(h, "h", torch.bfloat16, (r, cfg.hidden), dev)
        _need(step.positions, "positions", torch.int64, (r,), dev)
        _need(step.slots, "slots", torch.int64, (r,), dev)
        _need(step.req_ids, "req_ids", torch.int32, (r,), dev)
        pt = step.page_table
        if pt.dtype != torch.int32 or pt.dim() != 2 or pt.device != dev or pt.stride(1) != 1:
            raise ValueError("page_table: needs int32 [requests, pages] with contiguous rows")
        if pt.shape[1] * cfg.page < self.ctx_max:
            raise ValueError(f"page_table: {pt.shape[1]} pages a request cannot hold "
                             f"ctx_max {self.ctx_max}")
        kv = caches.kv if caches.kv.dtype == torch.uint8 else caches.kv.view(torch.uint8)
        _need(kv, "kv", torch.uint8, (kv.shape[0], cfg.kv_row), dev)
        if caches.kv_scale is not None:
            _need(caches.kv_scale, "kv_scale", torch.float32, (kv.shape[0],), dev)
        pages = caches.plane.shape[0]
        fmt = caches.index_format
        if fmt == _lib.INDEX_FP4_PLANE:
            _need(caches.plane, "plane", torch.uint8, (pages, 4, cfg.page, 16), dev)
            _need(caches.plane_scale, "plane_scale", torch.uint8, (pages, 4, cfg.page), dev)
        elif fmt in (_lib.INDEX_FP8_PAGE, _lib.INDEX_FP8_ROWS):
            _need(caches.plane, "plane", torch.uint8, (pages, _lib.DSA_PAGE_BYTES), dev)
        else:
            raise ValueError(f"index_format {fmt}: not one of _lib.INDEX_*")
        if out is None:
            out = self.outs[self.parity][:r]
            self.parity ^= 1
        _need(out, "out", torch.bfloat16, (r, cfg.hidden), dev)
        d = debug or LayerDebug()
        d.check(r, self.ctx_max, cfg, dev, fmt)
        if timeline is not None:
            _need(timeline, "timeline", torch.int64, (self.rt.grid, _lib.TL_COLS), dev)
        if phase_timeline is not None:
            _need(phase_timeline, "phase_timeline", torch.int64, (4, self.rt.grid, _lib.TL_COLS),
                  dev)
        self.rt.before_launch()
        ptr = lambda t: t.data_ptr() if t is not None else None
        f, po, m = w.front, w.post, w.moe
        args = _lib.MonoLayerArgs(
            rows=r, rows_max=self.max_rows, hidden=cfg.hidden, heads=cfg.heads, inter=cfg.inter,
            experts=cfg.experts,
            layout=_lib.LAYOUT_AITER16 if self.layout == layouts.AITER16 else _lib.LAYOUT_ROWMAJOR,
            ctx_max=self.ctx_max, pt_stride=pt.stride(0), pt_rows=pt.shape[0],
            rope_rows=f.cos.shape[0], kv_slots=kv.shape[0], plane_pages=pages, eps=cfg.rms_eps,
            sm_scale=self.sm_scale, route_scale=cfg.route_scale, n_group=cfg.n_group,
            topk_group=cfg.topk_group, h=h.data_ptr(),
            out=out.data_ptr(), positions=step.positions.data_ptr(), slots=step.slots.data_ptr(),
            req_ids=step.req_ids.data_ptr(), page_table=pt.data_ptr(), kv=kv.data_ptr(),
            kv_scale=ptr(caches.kv_scale), plane=caches.plane.data_ptr(),
            plane_scale=ptr(caches.plane_scale), g_in=f.g_in.data_ptr(),
            g_q=f.g_q.data_ptr(), g_kv=f.g_kv.data_ptr(), w_qkv_a=f.w_qkv_a.data_ptr(),
            s_qkv_a=f.s_qkv_a.data_ptr(), w_k=f.w_k.data_ptr(), s_k=f.s_k.data_ptr(),
            w_w=f.w_w.data_ptr(), g_k=f.g_k.data_ptr(), b_k=f.b_k.data_ptr(),
            w_qb=f.w_qb.data_ptr(), s_qb=f.s_qb.data_ptr(), w_iq=f.w_iq.data_ptr(),
            s_iq=f.s_iq.data_ptr(), w_uk=f.w_uk.data_ptr(), s_uk=f.s_uk.data_ptr(),
            cos=f.cos.data_ptr(), sin=f.sin.data_ptr(), w_uv=po.w_uv.data_ptr(),
            s_uv=po.s_uv.data_ptr(), w_o=po.w_o.data_ptr(), s_o=po.s_o.data_ptr(),
            g_post=m.g_post.data_ptr(), w_r=m.w_r.data_ptr(), bias=m.bias.data_ptr(),
            w13=m.w13.data_ptr(), w2=m.w2.data_ptr(),
            s13=None if self.mx else m.s13.data_ptr(), s2=None if self.mx else m.s2.data_ptr(),
            expert_format=_lib.EXPERTS_MXFP4 if self.mx else _lib.EXPERTS_FP8,
            e13=m.s13.data_ptr() if self.mx else None, e2=m.s2.data_ptr() if self.mx else None,
            q=ptr(d.q), iq=ptr(d.iq), iqs=ptr(d.iqs), iw=ptr(d.iw), o_lat=ptr(d.o_lat),
            a=ptr(d.a), scores=ptr(d.scores), topk_pos=ptr(d.topk), y=ptr(d.y),
            moe_scores=ptr(d.moe_scores), ids=ptr(d.ids), weights=ptr(d.weights),
            scratch=self.rt.scratch.data_ptr(), guard=self.rt.guard.data_ptr(),
            host_error=self.rt.host_error.data_ptr(), fault_site=int(self.fault[0]),
            fault_after=int(self.fault[1]), timeline=ptr(timeline),
            phase_timeline=ptr(phase_timeline), index_format=int(fmt))
        with torch.cuda.device(dev):
            _lib.check(_lib.lib().mono_layer_launch(ctypes.byref(args), _lib.stream_handle(stream)),
                       "mono_layer_launch")
        return out
