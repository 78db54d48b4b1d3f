"""Host op of the attention phase: FP4 indexer scores, exact top-2048 and sparse MLA
decode over the FP8 paged KV cache, as one persistent gfx950 launch.

``AttnOp.launch(inp) -> out`` takes one GPU's rows of a decode step (absorbed queries
[R, 32, 576], index queries and head weights, the request's page table and positions)
with the layer's caches read in place, and returns the latent attention output
[R, 32, 512] (bf16, before W_UV). It replaces the index-score, top-k, split and merge
stages of the reference layer kernel (``sgl_amd_mono/glm53/gfx950/kernel.py:2684-4123``;
FP4 index plane ``sgl_amd_mono/deepseek_v41/gfx950/indexer/score_fp4.py:1-20``).
Validation and ownership as the MoE ops: shapes and dtypes checked before the launch
(``ValueError``), no host synchronisation, two parity output buffers.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from .. import _lib
from ..runtime import MonoRuntime, shared_or_new
from .config import DSV32, LayerConfig
from .moe import _need

ATTN_MAX_ROWS = 48
MAX_CTX = 163840  # DeepSeek-V3.2's context: five 32768-key top-k blocks a row
U8 = torch.uint8


@dataclass
class AttnInputs:
    """One step's attention inputs (rows [R]); caches are read in place.

    q bf16 [R, 32, 576]: absorbed latent query then rope; iq uint8 [R, 64, 64] E2M1 index
    query; iqs uint8 [R, 4, 16, 4] E8M0 (chunk, head % 16, head // 16); iw f32 [R, 64];
    plane uint8 [pages, 4, 64, 16] and plane_scale uint8 [pages, 4, 64] (SGLang's FP4 index
    plane); kv uint8/E4M3 [slots, 576] with kv_scale f32 [slots] (None: raw E4M3 rows at
    scale 1, SGLang's FP8 MLA pool); positions i64 [R]; req_ids i32 [R]; page_table i32
    [requests, pages_per_request]. With ``index_format`` a DSA page (``_lib.INDEX_FP8_PAGE``
    or ``INDEX_FP8_ROWS``): plane uint8 [pages, 8448] (SGLang's DSA index pages), iq bf16
    [R, 64, 128], plane_scale and iqs None."""

    q: torch.Tensor
    iq: torch.Tensor
    iqs: Optional[torch.Tensor]
    iw: torch.Tensor
    plane: torch.Tensor
    plane_scale: Optional[torch.Tensor]
    kv: torch.Tensor
    kv_scale: Optional[torch.Tensor]
    positions: torch.Tensor
    req_ids: torch.Tensor
    page_table: torch.Tensor
    index_format: int = _lib.INDEX_FP4_PLANE

    @property
    def rows(self) -> int:
        return self.q.shape[0]


def check_index_inputs(cfg: LayerConfig, dev, r: int, fmt: int, iq, iqs, plane, plane_scale):
    """The index query and key cache for ``fmt`` (``_lib.INDEX_*``): the FP4 plane with
    E2M1 queries, or DSA pages with bf16 queries (``ValueError`` otherwise)."""
    if fmt == _lib.INDEX_FP4_PLANE:
        _need(iq, "iq", U8, (r, cfg.index_heads, cfg.index_dim // 2), dev)
        _need(iqs, "iqs", U8, (r, 4, 16, 4), dev)
        pages = plane.shape[0]
        _need(plane, "plane", U8, (pages, 4, cfg.page, 16), dev)
        _need(plane_scale, "plane_scale", U8, (pages, 4, cfg.page), dev)
    elif fmt in (_lib.INDEX_FP8_PAGE, _lib.INDEX_FP8_ROWS):
        _need(iq, "iq", torch.bfloat16, (r, cfg.index_heads, cfg.index_dim), dev)
        _need(plane, "plane", U8, (plane.shape[0], _lib.DSA_PAGE_BYTES), dev)
    else:
        raise ValueError(f"index_format {fmt}: not one of _lib.INDEX_*")


class AttnOp:
    """The attention-phase launch on one device for up to ``max_rows`` rows seeing at
    most ``ctx_max`` keys each."""

    def __init__(self, device, cfg: LayerConfig = DSV32, max_rows: int = 8,
                 ctx_max: int = 32768, sm_scale: Optional[float] = None,
                 deadline_s: float = 10.0, fault=(0, 0), rt: Optional[MonoRuntime] = None):
        self.cfg, self.device = cfg, torch.device(device)
        if not 1 <= max_rows <= ATTN_MAX_ROWS:
            raise ValueError(f"max_rows must be 1..{ATTN_MAX_ROWS}")
        if not 1 <= ctx_max <= MAX_CTX:
            raise ValueError(f"ctx_max must be 1..{MAX_CTX}")
        nbytes = _lib.lib().mono_attn_scratch_bytes(max_rows)
        if nbytes == 0:
            raise ValueError("no attention kernel for this many rows")
        self.rt = shared_or_new(rt, nbytes, self.device, deadline_s)
        self.max_rows, self.ctx_max = max_rows, ctx_max
        self.sm_scale = sm_scale if sm_scale is not None else (cfg.nope_dim + cfg.rope_dim) ** -0.5
        self.fault = fault
        self.outs = [torch.empty(max_rows, cfg.heads, cfg.kv_lora, dtype=torch.bfloat16,
                                 device=self.device) for _ in range(2)]
        self.parity = 0

    def _validate(self, x: AttnInputs) -> None:
        cfg, dev, r = self.cfg, self.device, x.rows
        if not 1 <= r <= self.max_rows:
            raise ValueError(f"rows {r}: needs 1..{self.max_rows}")
        kvd = cfg.kv_lora + cfg.rope_dim
        _need(x.q, "q", torch.bfloat16, (r, cfg.heads, kvd), dev)
        _need(x.iw, "iw", torch.float32, (r, cfg.index_heads), dev)
        check_index_inputs(cfg, dev, r, x.index_format, x.iq, x.iqs, x.plane, x.plane_scale)
        kv = x.kv if x.kv.dtype == U8 else x.kv.view(U8)
        _need(kv, "kv", U8, (kv.shape[0], kvd), dev)
        if x.kv_scale is not None:
            _need(x.kv_scale, "kv_scale", torch.float32, (kv.shape[0],), dev)
        _need(x.positions, "positions", torch.int64, (r,), dev)
        _need(x.req_ids, "req_ids", torch.int32, (r,), dev)
        if x.page_table.dtype != torch.int32 or x.page_table.dim() != 2 or x.page_table.device != dev:
            raise ValueError("page_table: needs int32 [requests, pages] on the device")
        if x.page_table.stride(1) != 1:
            raise ValueError("page_table: rows must be contiguous")
        if x.page_table.shape[1] * cfg.page < self.ctx_max:
            raise ValueError(f"page_table: {x.page_table.shape[1]} pages a request cannot hold "
                             f"ctx_max {self.ctx_max}")

    def launch(self, x: AttnInputs, out: Optional[torch.Tensor] = None,
               scores: Optional[torch.Tensor] = None, topk: Optional[torch.Tensor] = None,
               stream=None, timeline: Optional[torch.Tensor] = None) -> torch.Tensor:
        cfg = self.cfg
        self._validate(x)
        r = x.rows
        if out is None:
            out = self.outs[self.parity][:r]
            self.parity ^= 1
        _need(out, "out", torch.bfloat16, (r, cfg.heads, cfg.kv_lora), self.device)
        if scores is not None:
            _need(scores, "scores", torch.float32, (r, self.ctx_max), self.device)
        if topk is not None:
            _need(topk, "topk", torch.int32, (r, cfg.index_topk), self.device)
        if timeline is not None:
            _need(timeline, "timeline", torch.int64, (self.rt.grid, _lib.TL_COLS), self.device)
        self.rt.before_launch()
        kv = x.kv if x.kv.dtype == U8 else x.kv.view(U8)
        ptr = lambda t: t.data_ptr() if t is not None else None
        args = _lib.MonoAttnArgs(
            rows=r, rows_max=self.max_rows, heads=cfg.heads, index_heads=cfg.index_heads, topk=cfg.index_topk,
            page=cfg.page, ctx_max=self.ctx_max, pt_stride=x.page_table.stride(0),
            pt_rows=x.page_table.shape[0], plane_pages=x.plane.shape[0], kv_slots=kv.shape[0],
            sm_scale=self.sm_scale, positions=x.positions.data_ptr(),
            req_ids=x.req_ids.data_ptr(), page_table=x.page_table.data_ptr(),
            q=x.q.data_ptr(), iq=x.iq.data_ptr(), iqs=ptr(x.iqs), iw=x.iw.data_ptr(),
            plane=x.plane.data_ptr(), plane_scale=ptr(x.plane_scale), kv=kv.data_ptr(),
            kv_scale=ptr(x.kv_scale), out=out.data_ptr(), scores=ptr(scores),
            topk_pos=ptr(topk), scratch=self.rt.scratch.data_ptr(),
            guard=self.rt.guard.data_ptr(), host_error=self.rt.host_error.data_ptr(),
            fault_site=int(self.fault[0]), fault_after=int(self.fault[1]),
            timeline=ptr(timeline), index_format=int(x.index_format))
        with torch.cuda.device(self.device):
            _lib.check(_lib.lib().mono_attn_launch(ctypes.byref(args), _lib.stream_handle(stream)),
                       "mono_attn_launch")
        return out
