"""Host op of the front of the layer: from the layer input h to the attention launch's
inputs, with the rows' KV and index-key cache writes, as one persistent gfx950 launch.

``FrontOp.launch(h, caches, positions, slots) -> FrontOut`` takes one GPU's rows of a
decode step and returns the absorbed queries q [R, 32, 576] (bf16: q_lat | q_pe), the
FP4 index query (iq [R, 64, 64] + iqs [R, 4, 16, 4]) and the head weights iw [R, 64], and
writes each row's KV row (E4M3 + a per-token scale) and FP4 index key at its slot. It
replaces the qkv_a, q_norm, cache, q_b, index_q and uk stages of the reference layer
kernel (``sgl_amd_mono/glm53/gfx950/kernel.py:1781-2443``) and the FP4 index paths of
``sgl_amd_mono/deepseek_v4/gfx950/kernels/stages/indexer.py:143-151,311-408``.
Validation and ownership as the other ops: shapes and dtypes checked before the launch
(``ValueError``), no host synchronisation, two parity output bundles.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from .. import _lib, layouts
from ..runtime import MonoRuntime, shared_or_new
from .config import DSV32, LayerConfig
from .attn import check_index_inputs
from .moe import FP8, _need

FRONT_MAX_ROWS = 8
U8 = torch.uint8
BF16 = torch.bfloat16


@dataclass
class FrontWeights:
    """One layer's attention-front weights (one TP shard), read in place.

    g_in / g_q / g_kv bf16 RMSNorm weights [7168] / [1536] / [512]; w_qkv_a E4M3 [2112,
    7168] (q_a rows, then kv_a) + s_qkv_a f32 [17, 56]; the index key w_k E4M3 [128, 7168]
    + s_k [1, 56] with its LayerNorm g_k / b_k f32 [128]; the head weights w_w bf16 [64,
    7168]; w_qb E4M3 [6144, 1536] + s_qb [48, 12]; the index query w_iq E4M3 [8192, 1536] +
    s_iq [64, 12]; W_UK E4M3 [32, 512, 128] + s_uk [32, 4, 1]; RoPE tables cos / sin bf16
    [positions, 32]. FP8 matrices row-major or in AITER's (16, 16) shuffle (``layout``)."""

    g_in: torch.Tensor
    g_q: torch.Tensor
    g_kv: torch.Tensor
    w_qkv_a: torch.Tensor
    s_qkv_a: torch.Tensor
    w_k: torch.Tensor
    s_k: torch.Tensor
    w_w: torch.Tensor
    g_k: torch.Tensor
    b_k: torch.Tensor
    w_qb: torch.Tensor
    s_qb: torch.Tensor
    w_iq: torch.Tensor
    s_iq: torch.Tensor
    w_uk: torch.Tensor
    s_uk: torch.Tensor
    cos: torch.Tensor
    sin: torch.Tensor
    layout: str = layouts.ROWMAJOR

    def validate(self, cfg: LayerConfig, device) -> None:
        H, QL, KL, PE = cfg.hidden, cfg.q_lora, cfg.kv_lora, cfg.rope_dim
        qkv = QL + KL + PE
        cb = lambda n: (n + 127) // 128
        _need(self.g_in, "g_in", BF16, (H,), device)
        _need(self.g_q, "g_q", BF16, (QL,), device)
        _need(self.g_kv, "g_kv", BF16, (KL,), device)
        _need(self.w_qkv_a, "w_qkv_a", FP8, (qkv, H), device)
        _need(self.s_qkv_a, "s_qkv_a", torch.float32, (cb(qkv), H // 128), device)
        _need(self.w_k, "w_k", FP8, (cfg.index_dim, H), device)
        _need(self.s_k, "s_k", torch.float32, (cb(cfg.index_dim), H // 128), device)
        _need(self.w_w, "w_w", BF16, (cfg.index_heads, H), device)
        _need(self.g_k, "g_k", torch.float32, (cfg.index_dim,), device)
        _need(self.b_k, "b_k", torch.float32, (cfg.index_dim,), device)
        qb = cfg.heads * cfg.qk_dim
        _need(self.w_qb, "w_qb", FP8, (qb, QL), device)
        _need(self.s_qb, "s_qb", torch.float32, (qb // 128, QL // 128), device)
        iq = cfg.index_heads * cfg.index_dim
        _need(self.w_iq, "w_iq", FP8, (iq, QL), device)
        _need(self.s_iq, "s_iq", torch.float32, (iq // 128, QL // 128), device)
        _need(self.w_uk, "w_uk", FP8, (cfg.heads, KL, cfg.nope_dim), device)
        _need(self.s_uk, "s_uk", torch.float32, (cfg.heads, KL // 128, cb(cfg.nope_dim)), device)
        n = self.cos.shape[0] if self.cos.dim() == 2 else -1
        _need(self.cos, "cos", BF16, (n, PE // 2), device)
        _need(self.sin, "sin", BF16, (n, PE // 2), device)
        if self.layout not in layouts.LAYOUTS:
            raise ValueError(f"layout {self.layout!r}: needs one of {layouts.LAYOUTS}")


@dataclass
class FrontCaches:
    """The layer's caches the front writes: kv E4M3 (uint8) [slots, 576] + kv_scale f32
    [slots] (None: raw E4M3 rows at scale 1, SGLang's FP8 MLA pool layout); the FP4 index
    plane [pages, 4, 64, 16] + its scales [pages, 4, 64], or with ``index_format`` a DSA
    page format (``_lib.INDEX_FP8_PAGE`` / ``INDEX_FP8_ROWS``) SGLang's DSA index pages
    uint8 [pages, 8448] as ``plane`` and no ``plane_scale``."""

    kv: torch.Tensor
    kv_scale: Optional[torch.Tensor]
    plane: torch.Tensor
    plane_scale: Optional[torch.Tensor]
    index_format: int = _lib.INDEX_FP4_PLANE


@dataclass
class FrontOut:
    q: torch.Tensor    # bf16 [R, 32, 576]
    iq: torch.Tensor   # uint8 [R, 64, 64] (DSA pages: bf16 [R, 64, 128])
    iqs: Optional[torch.Tensor]  # uint8 [R, 4, 16, 4] (DSA pages: None)
    iw: torch.Tensor   # f32 [R, 64]


class FrontOp:
    """The front launch on one device for up to ``max_rows`` rows."""

    def __init__(self, weights: FrontWeights, device, cfg: LayerConfig = DSV32,
                 max_rows: int = 8, deadline_s: float = 10.0, fault=(0, 0),
                 rt: Optional[MonoRuntime] = None):
        self.cfg, self.device = cfg, torch.device(device)
        if not 1 <= max_rows <= FRONT_MAX_ROWS:
            raise ValueError(f"max_rows must be 1..{FRONT_MAX_ROWS}")
        weights.validate(cfg, self.device)
        self.w = weights
        self.rt = shared_or_new(rt, _lib.lib().mono_front_scratch_bytes(), self.device,
                                deadline_s)
        self.max_rows, self.fault = max_rows, fault
        d = self.device
        self.outs = [FrontOut(
            q=torch.empty(max_rows, cfg.heads, cfg.kv_row, dtype=BF16, device=d),
            iq=torch.empty(max_rows, cfg.index_heads, cfg.index_dim // 2, dtype=U8, device=d),
            iqs=torch.empty(max_rows, 4, 16, 4, dtype=U8, device=d),
            iw=torch.empty(max_rows, cfg.index_heads, dtype=torch.float32, device=d))
            for _ in range(2)]
        # a DSA page's bf16 query, by parity
        self.iq16 = [torch.empty(max_rows, cfg.index_heads, cfg.index_dim, dtype=BF16, device=d)
                     for _ in range(2)]
        self.parity = 0

    def launch(self, h: torch.Tensor, caches: FrontCaches, positions: torch.Tensor,
               slots: torch.Tensor, out: Optional[FrontOut] = None, stream=None,
               timeline: Optional[torch.Tensor] = None, ik_raw: Optional[torch.Tensor] = None,
               iq_raw: Optional[torch.Tensor] = None) -> FrontOut:
        """One launch; ``ik_raw`` f32 [R, 128] / ``iq_raw`` bf16 [R, 64, 128], if given,
        receive the index key's and query's projections before their LayerNorm / RoPE."""
        cfg, dev, w = self.cfg, self.device, self.w
        r = h.shape[0] if h.dim() == 2 else -1
        if not 1 <= r <= self.max_rows:
            raise ValueError(f"h: needs [1..{self.max_rows}, {cfg.hidden}]")
        _need(h, "h", BF16, (r, cfg.hidden), dev)
        _need(positions, "positions", torch.int64, (r,), dev)
        _need(slots, "slots", torch.int64, (r,), dev)
        kv = caches.kv if caches.kv.dtype == U8 else caches.kv.view(U8)
        _need(kv, "kv", U8, (kv.shape[0], cfg.kv_row), dev)
        if caches.kv_scale is not None:
            _need(caches.kv_scale, "kv_scale", torch.float32, (kv.shape[0],), dev)
        fmt = caches.index_format
        pages = caches.plane.shape[0]
        if out is None:
            o = self.outs[self.parity]
            out = (FrontOut(q=o.q[:r], iq=o.iq[:r], iqs=o.iqs[:r], iw=o.iw[:r])
                   if fmt == _lib.INDEX_FP4_PLANE else
                   FrontOut(q=o.q[:r], iq=self.iq16[self.parity][:r], iqs=None, iw=o.iw[:r]))
            self.parity ^= 1
        check_index_inputs(cfg, dev, r, fmt, out.iq, out.iqs, caches.plane, caches.plane_scale)
        _need(out.q, "q", BF16, (r, cfg.heads, cfg.kv_row), dev)
        _need(out.iw, "iw", torch.float32, (r, cfg.index_heads), dev)
        if timeline is not None:
            _need(timeline, "timeline", torch.int64, (self.rt.grid, _lib.TL_COLS), dev)
        if ik_raw is not None:
            _need(ik_raw, "ik_raw", torch.float32, (r, cfg.index_dim), dev)
        if iq_raw is not None:
            _need(iq_raw, "iq_raw", BF16, (r, cfg.index_heads, cfg.index_dim), dev)
        self.rt.before_launch()
        ptr = lambda t: t.data_ptr() if t is not None else None
        args = _lib.MonoFrontArgs(
            rows=r, hidden=cfg.hidden, heads=cfg.heads,
            layout=_lib.LAYOUT_AITER16 if w.layout == layouts.AITER16 else _lib.LAYOUT_ROWMAJOR,
            rope_rows=w.cos.shape[0], kv_slots=kv.shape[0], plane_pages=pages, eps=cfg.rms_eps,
            h=h.data_ptr(), g_in=w.g_in.data_ptr(), g_q=w.g_q.data_ptr(), g_kv=w.g_kv.data_ptr(),
            w_qkv_a=w.w_qkv_a.data_ptr(), s_qkv_a=w.s_qkv_a.data_ptr(), w_k=w.w_k.data_ptr(),
            s_k=w.s_k.data_ptr(), w_w=w.w_w.data_ptr(), g_k=w.g_k.data_ptr(), b_k=w.b_k.data_ptr(),
            w_qb=w.w_qb.data_ptr(), s_qb=w.s_qb.data_ptr(), w_iq=w.w_iq.data_ptr(),
            s_iq=w.s_iq.data_ptr(), w_uk=w.w_uk.data_ptr(), s_uk=w.s_uk.data_ptr(),
            cos=w.cos.data_ptr(), sin=w.sin.data_ptr(), positions=positions.data_ptr(),
            slots=slots.data_ptr(), kv=kv.data_ptr(), kv_scale=ptr(caches.kv_scale),
            plane=caches.plane.data_ptr(), plane_scale=ptr(caches.plane_scale),
            q=out.q.data_ptr(), iq=out.iq.data_ptr(), iqs=ptr(out.iqs), iw=out.iw.data_ptr(),
            scratch=self.rt.scratch.data_ptr(), guard=self.rt.guard.data_ptr(),
            host_error=self.rt.host_error.data_ptr(), fault_site=int(self.fault[0]),
            fault_after=int(self.fault[1]), timeline=ptr(timeline), ik_raw=ptr(ik_raw),
            iq_raw=ptr(iq_raw), index_format=int(fmt))
        with torch.cuda.device(dev):
            _lib.check(_lib.lib().mono_front_launch(ctypes.byref(args), _lib.stream_handle(stream)),
                       "mono_front_launch")
        return out
