"""Host op of the attention output block: W_UV per head, o_proj and the residual add,
as one persistent gfx950 launch.

``PostOp.launch(o_lat, h) -> a`` takes the merged latent attention output [R, 32, 512]
(bf16) and the residual stream h [R, 7168], and returns a = bf16(h + W_o (W_UV o_lat))
(the handed-over o in bf16), replacing the W_UV, o_proj and W == 1 reduce stages of the
reference layer kernel (``sgl_amd_mono/glm53/gfx950/kernel.py:3975-4197``,
``:1665-1669``). Validation and ownership as the MoE ops: shapes and dtypes checked before
the launch (``ValueError``), no host synchronisation, two parity output buffers.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from .. import _lib, layouts
from ..runtime import MonoRuntime, shared_or_new
from .config import DSV32, LayerConfig
from .moe import FP8, _need

POST_MAX_ROWS = 16


@dataclass
class PostWeights:
    """The attention output weights of one layer's TP shard, read in place.

    w_uv E4M3 [32, 128, 512] (the value half of ``kv_b_proj`` per local head) with
    s_uv f32 [32, 1, 4]; w_o E4M3 [7168, 4096] (``o_proj``) with s_o f32 [56, 32]. Each
    [N, K] matrix row-major or in AITER's (16, 16) shuffle (``layout``)."""

    w_uv: torch.Tensor
    s_uv: torch.Tensor
    w_o: torch.Tensor
    s_o: torch.Tensor
    layout: str = layouts.ROWMAJOR

    def validate(self, cfg: LayerConfig, device) -> None:
        hh, v, c, hid = cfg.heads, cfg.v_dim, cfg.kv_lora, cfg.hidden
        _need(self.w_uv, "w_uv", FP8, (hh, v, c), device)
        _need(self.s_uv, "s_uv", torch.float32, (hh, v // 128, c // 128), device)
        _need(self.w_o, "w_o", FP8, (hid, hh * v), device)
        _need(self.s_o, "s_o", torch.float32, (hid // 128, hh * v // 128), device)
        if self.layout not in layouts.LAYOUTS:
            raise ValueError(f"layout {self.layout!r}: needs one of {layouts.LAYOUTS}")


class PostOp:
    """The attention output launch on one device for up to ``max_rows`` rows."""

    def __init__(self, weights: PostWeights, device, cfg: LayerConfig = DSV32,
                 max_rows: int = 8, deadline_s: float = 10.0, fault=(0, 0),
                 rt: Optional[MonoRuntime] = None):
        self.cfg, self.device = cfg, torch.device(device)
        if not 1 <= max_rows <= POST_MAX_ROWS:
            raise ValueError(f"max_rows must be 1..{POST_MAX_ROWS}")
        weights.validate(cfg, self.device)
        self.w = weights
        self.rt = shared_or_new(rt, _lib.lib().mono_post_scratch_bytes(), self.device,
                                deadline_s)
        self.max_rows, self.fault = max_rows, fault
        self.outs = [torch.empty(max_rows, cfg.hidden, dtype=torch.bfloat16, device=self.device)
                     for _ in range(2)]
        self.parity = 0

    def launch(self, o_lat: torch.Tensor, h: torch.Tensor, out: Optional[torch.Tensor] = None,
               o: Optional[torch.Tensor] = None, stream=None,
               timeline: Optional[torch.Tensor] = None) -> torch.Tensor:
        cfg, dev = self.cfg, self.device
        r = o_lat.shape[0] if o_lat.dim() == 3 else -1
        if not 1 <= r <= self.max_rows:
            raise ValueError(f"o_lat: needs [1..{self.max_rows}, {cfg.heads}, {cfg.kv_lora}]")
        _need(o_lat, "o_lat", torch.bfloat16, (r, cfg.heads, cfg.kv_lora), dev)
        _need(h, "h", torch.bfloat16, (r, cfg.hidden), dev)
        if out is None:
            out = self.outs[self.parity][:r]
            self.parity ^= 1
        _need(out, "out", torch.bfloat16, (r, cfg.hidden), dev)
        if o is not None:
            _need(o, "o", torch.bfloat16, (r, cfg.heads * cfg.v_dim), dev)
        if timeline is not None:
            _need(timeline, "timeline", torch.int64, (self.rt.grid, _lib.TL_COLS), dev)
        self.rt.before_launch()
        ptr = lambda t: t.data_ptr() if t is not None else None
        w = self.w
        args = _lib.MonoPostArgs(
            rows=r, heads=cfg.heads, hidden=cfg.hidden, layout=_lib.LAYOUT_AITER16 if w.layout == layouts.AITER16 else _lib.LAYOUT_ROWMAJOR,
            o_lat=o_lat.data_ptr(), h=h.data_ptr(), w_uv=w.w_uv.data_ptr(),
            s_uv=w.s_uv.data_ptr(), w_o=w.w_o.data_ptr(), s_o=w.s_o.data_ptr(),
            out=out.data_ptr(), o=ptr(o), scratch=self.rt.scratch.data_ptr(),
            guard=self.rt.guard.data_ptr(), host_error=self.rt.host_error.data_ptr(),
            fault_site=int(self.fault[0]), fault_after=int(self.fault[1]),
            timeline=ptr(timeline))
        with torch.cuda.device(dev):
            _lib.check(_lib.lib().mono_post_launch(ctypes.byref(args), _lib.stream_handle(stream)),
                       "mono_post_launch")
        return out
