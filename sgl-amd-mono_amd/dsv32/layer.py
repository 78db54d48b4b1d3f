"""One GPU's TP=4 share of a DeepSeek-V3.2 DSA decoder layer, as four persistent gfx950
launches on one stream: the front (norms, projections, RoPE, KV and index-key cache
writes), the attention phase (FP4 indexer, exact top-2048, sparse MLA), the output block
(W_UV, o_proj, residual) and the FP8 MoE (post-norm, router, top-8 + shared experts,
residual).

``LayerOp.launch(h, caches, step) -> x_out`` mirrors the reference's per-layer entry
``Glm53LayerOp.launch(h, caches, cos, sin, step)`` (``sgl_amd_mono/glm53/gfx950/
runner.py:240-321``): shapes and dtypes are checked before anything launches
(``ValueError``), every launch goes on the current stream with no host synchronisation,
and the result is runtime-owned (parity buffers of the MoE op). The W == 1 reduces are the
local residual adds of the output block and the MoE (``kernel.py:1665-1669``).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from .. import _lib
from ..runtime import MonoRuntime
from .attn import AttnInputs, AttnOp
from .config import DSV32, LayerConfig
from .front import FrontCaches, FrontOp, FrontWeights
from .moe import MoeFp8Op, MoeFp8Weights
from .post import PostOp, PostWeights


@dataclass
class LayerWeights:
    front: FrontWeights
    post: PostWeights
    moe: MoeFp8Weights


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
                         page_table=step.page_table)
        o_lat = self.attn.launch(inp, stream=stream)
        a = self.post.launch(o_lat, h, stream=stream)
        return self.moe.launch(a, out=out, stream=stream)
