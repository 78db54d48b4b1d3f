"""Host ops of the MoE half of the layer: the weight bundle and the launch.

``MoeFp8Op.launch(a) -> out`` runs the FFN half of the DSA layer as one persistent
gfx950 launch: post-attention RMSNorm, router GEMV and sigmoid, top-8 + shared expert,
W8A8 expert SwiGLU, down projection with route weights, and the residual add of the
W == 1 reduce (``sgl_amd_mono/glm53/gfx950/kernel.py:4199-5187``, ``:1665-1669``).
Like ``Glm53LayerOp.launch`` (``glm53/gfx950/runner.py:240-321``) it validates shapes,
dtypes and contiguity before the launch (``ValueError``), launches on the current
stream without a host synchronisation, and returns a runtime-owned output valid until
the launch after next (two parity buffers, so a launch never writes what the previous
one returned: ``runner.py:190-195``).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from .. import _lib, layouts
from ..runtime import MonoRuntime, shared_or_new
from .config import DSV32, MAX_ROWS, MXFP4_MOE, LayerConfig, Mxfp4MoeConfig

FP8 = torch.float8_e4m3fn


def _need(t: torch.Tensor, name: str, dtype, shape, device) -> None:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name}: expected a tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name}: dtype {t.dtype}, needs {dtype}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: shape {tuple(t.shape)}, needs {tuple(shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: needs a contiguous tensor")
    if t.device != device:
        raise ValueError(f"{name}: on {t.device}, needs {device}")


@dataclass
class MoeFp8Weights:
    """One layer's FFN weights in SGLang's loaded layout, read in place.

    w13 E4M3 [E + 1, 2 I, H] (gate rows, then up rows; the shared expert is id E),
    row-major or in AITER's (16, 16) shuffle (``layout``; ``layouts.py``),
    s13 f32 [E + 1, 2 I / 128, H / 128] (``w13_weight_scale_inv``), w2 E4M3 [E + 1, H, I],
    s2 f32 [E + 1, H / 128, I / 128]; router w_r bf16 [E, H], bias f32 [E]
    (``e_score_correction_bias``), post-attention norm g_post bf16 [H]."""

    g_post: torch.Tensor
    w_r: torch.Tensor
    bias: torch.Tensor
    w13: torch.Tensor
    s13: torch.Tensor
    w2: torch.Tensor
    s2: torch.Tensor
    layout: str = layouts.ROWMAJOR  # of w13 and w2: "rowmajor" or "aiter16"

    def validate(self, cfg: LayerConfig, device) -> None:
        h, i, e = cfg.hidden, cfg.inter, cfg.experts
        if self.layout not in layouts.LAYOUTS:
            raise ValueError(f"layout {self.layout!r}: one of {layouts.LAYOUTS}")
        _need(self.g_post, "g_post", torch.bfloat16, (h,), device)
        _need(self.w_r, "w_r", torch.bfloat16, (e, h), device)
        _need(self.bias, "bias", torch.float32, (e,), device)
        _need(self.w13, "w13", FP8, (e + 1, 2 * i, h), device)
        _need(self.s13, "s13", torch.float32, (e + 1, 2 * i // 128, h // 128), device)
        _need(self.w2, "w2", FP8, (e + 1, h, i), device)
        _need(self.s2, "s2", torch.float32, (e + 1, h // 128, i // 128), device)


@dataclass
class MoeRouting:
    """Optional routing outputs of a launch (rows [R]): sigmoid scores [R, E], slot
    ids [R, 9] (slot 0 the shared expert 256) and weights [R, 9]."""

    scores: torch.Tensor
    ids: torch.Tensor
    weights: torch.Tensor


class MoeFp8Op:
    """The FP8 routed-MoE launch on one device for up to ``max_rows`` rows."""

    def __init__(self, weights: MoeFp8Weights, device, cfg: LayerConfig = DSV32,
                 max_rows: int = MAX_ROWS, deadline_s: float = 10.0, fault=(0, 0),
                 rt: Optional[MonoRuntime] = None):
        self.cfg, self.device = cfg, torch.device(device)
        if not 1 <= max_rows <= MAX_ROWS:
            raise ValueError(f"max_rows must be 1..{MAX_ROWS}")
        weights.validate(cfg, self.device)
        self.w = weights
        nbytes = _lib.lib().mono_moe_fp8_scratch_bytes(cfg.hidden, cfg.inter, cfg.experts)
        if nbytes == 0:
            raise ValueError(f"no FP8 MoE kernel for hidden {cfg.hidden}, inter {cfg.inter}")
        self.rt = shared_or_new(rt, nbytes, self.device, deadline_s)
        self.max_rows = max_rows
        self.fault = fault
        # two parity outputs: a launch never writes the tensor the previous one returned
        self.outs = [torch.empty(max_rows, cfg.hidden, dtype=torch.bfloat16, device=self.device)
                     for _ in range(2)]
        self.parity = 0

    def launch(self, a: torch.Tensor, y: Optional[torch.Tensor] = None,
               routing: Optional[MoeRouting] = None, out: Optional[torch.Tensor] = None,
               stream=None, timeline: Optional[torch.Tensor] = None) -> torch.Tensor:
        """a bf16 [R, H] -> a + MoE(a), bf16 [R, H] (``out`` or a runtime buffer)."""
        cfg = self.cfg
        if a.dim() != 2 or not 1 <= a.shape[0] <= self.max_rows:
            raise ValueError(f"a: needs [rows <= {self.max_rows}, {cfg.hidden}], got {tuple(a.shape)}")
        r = a.shape[0]
        _need(a, "a", torch.bfloat16, (r, cfg.hidden), self.device)
        if out is None:
            out = self.outs[self.parity][:r]
            self.parity ^= 1
        _need(out, "out", torch.bfloat16, (r, cfg.hidden), self.device)
        if y is not None:
            _need(y, "y", torch.float32, (r, cfg.hidden), self.device)
        if routing is not None:
            _need(routing.scores, "scores", torch.float32, (r, cfg.experts), self.device)
            _need(routing.ids, "ids", torch.int32, (r, cfg.top_k + 1), self.device)
            _need(routing.weights, "weights", torch.float32, (r, cfg.top_k + 1), self.device)
        if timeline is not None:
            _need(timeline, "timeline", torch.int64, (self.rt.grid, _lib.TL_COLS), self.device)
        self.rt.before_launch()
        w = self.w
        args = _lib.MonoMoeFp8Args(
            rows=r, hidden=cfg.hidden, inter=cfg.inter, experts=cfg.experts,
            layout=_lib.LAYOUT_AITER16 if w.layout == layouts.AITER16 else _lib.LAYOUT_ROWMAJOR,
            eps=cfg.rms_eps, route_scale=cfg.route_scale, n_group=cfg.n_group,
            topk_group=cfg.topk_group,
            a=a.data_ptr(), out=out.data_ptr(), g_post=w.g_post.data_ptr(),
            w_r=w.w_r.data_ptr(), bias=w.bias.data_ptr(), w13=w.w13.data_ptr(),
            s13=w.s13.data_ptr(), w2=w.w2.data_ptr(), s2=w.s2.data_ptr(),
            y=y.data_ptr() if y is not None else None,
            scores=routing.scores.data_ptr() if routing else None,
            ids=routing.ids.data_ptr() if routing else None,
            weights=routing.weights.data_ptr() if routing else None,
            scratch=self.rt.scratch.data_ptr(), guard=self.rt.guard.data_ptr(),
            host_error=self.rt.host_error.data_ptr(),
            fault_site=int(self.fault[0]), fault_after=int(self.fault[1]),
            timeline=timeline.data_ptr() if timeline is not None else None,
        )
        with torch.cuda.device(self.device):
            _lib.check(_lib.lib().mono_moe_fp8_launch(ctypes.byref(args),
                                                       _lib.stream_handle(stream)),
                       "mono_moe_fp8_launch")
        return out


U8 = torch.uint8


@dataclass
class MoeMxfp4Weights:
    """MXFP4 (A16W4) expert weights, read in place.

    w13 E2M1 codes uint8 [E + 1, 2 I, H / 2] (two a byte, the even K index in the low
    nibble; gate rows then up rows; the shared expert is id E), s13 E8M0 uint8
    [E + 1, 2 I, H / 32]; w2 [E + 1, H, I / 2], s2 [E + 1, H, I / 32]; bias f32 [E].
    ``aiter16``: codes in AITER's (16, 16) byte shuffle and scales in the e8m0 shuffle,
    [E + 1, N, C8] with C8 the scale columns rounded up to 8 (``layouts.py``). A
    float4_e2m1fn_x2 / float8_e8m0fnu tensor is taken as its bytes."""

    bias: torch.Tensor
    w13: torch.Tensor
    s13: torch.Tensor
    w2: torch.Tensor
    s2: torch.Tensor
    layout: str = layouts.ROWMAJOR

    def bytes_view(self) -> "MoeMxfp4Weights":
        v = lambda t: t if t.dtype == U8 else t.view(U8)
        return MoeMxfp4Weights(self.bias, v(self.w13), v(self.s13), v(self.w2), v(self.s2),
                               self.layout)

    def validate(self, cfg: Mxfp4MoeConfig, device) -> None:
        h, i, e = cfg.hidden, cfg.inter, cfg.experts
        if self.layout not in layouts.LAYOUTS:
            raise ValueError(f"layout {self.layout!r}: one of {layouts.LAYOUTS}")
        cols = (lambda c: layouts.e8m0_cols(c)) if self.layout == layouts.AITER16 else (lambda c: c)
        _need(self.bias, "bias", torch.float32, (e,), device)
        _need(self.w13, "w13", U8, (e + 1, 2 * i, h // 2), device)
        _need(self.s13, "s13", U8, (e + 1, 2 * i, cols(h // 32)), device)
        _need(self.w2, "w2", U8, (e + 1, h, i // 2), device)
        _need(self.s2, "s2", U8, (e + 1, h, cols(i // 32)), device)


@dataclass
class MoeMxfp4LayerWeights:
    """One layer's FFN with MXFP4 (A16W4) experts, for the one-launch layer: the router and
    norm as ``MoeFp8Weights`` (g_post bf16 [H], w_r bf16 [E, H], bias f32 [E]) and the
    experts as ``MoeMxfp4Weights`` at the layer's geometry: w13 E2M1 codes uint8
    [E + 1, 2 I, H / 2], s13 E8M0 uint8 [E + 1, 2 I, H / 32], w2 [E + 1, H, I / 2], s2
    [E + 1, H, I / 32] (``aiter16``: the (16, 16) code shuffle and the e8m0 scale shuffle,
    what aiter's MXFP4 MoE method leaves in place). The reference's A16W4 mode
    (``sgl_amd_mono/glm53/gfx950/config.py:15-21,88-93``)."""

    g_post: torch.Tensor
    w_r: torch.Tensor
    bias: torch.Tensor
    w13: torch.Tensor
    s13: torch.Tensor
    w2: torch.Tensor
    s2: torch.Tensor
    layout: str = layouts.ROWMAJOR

    def bytes_view(self) -> "MoeMxfp4LayerWeights":
        v = lambda t: t if t.dtype == U8 else t.view(U8)
        return MoeMxfp4LayerWeights(self.g_post, self.w_r, self.bias, v(self.w13), v(self.s13),
                                    v(self.w2), v(self.s2), self.layout)

    def validate(self, cfg: LayerConfig, device) -> None:
        h, i, e = cfg.hidden, cfg.inter, cfg.experts
        if self.layout not in layouts.LAYOUTS:
            raise ValueError(f"layout {self.layout!r}: one of {layouts.LAYOUTS}")
        cols = (lambda c: layouts.e8m0_cols(c)) if self.layout == layouts.AITER16 else (lambda c: c)
        _need(self.g_post, "g_post", torch.bfloat16, (h,), device)
        _need(self.w_r, "w_r", torch.bfloat16, (e, h), device)
        _need(self.bias, "bias", torch.float32, (e,), device)
        _need(self.w13, "w13", U8, (e + 1, 2 * i, h // 2), device)
        _need(self.s13, "s13", U8, (e + 1, 2 * i, cols(h // 32)), device)
        _need(self.w2, "w2", U8, (e + 1, h, i // 2), device)
        _need(self.s2, "s2", U8, (e + 1, h, cols(i // 32)), device)


class MoeMxfp4Op:
    """The MXFP4 (A16W4) routed-MoE launch on one device for up to ``max_rows`` rows:
    x bf16 [R, H] and gate logits f32 [R, E] -> bf16(res + y) (``bf16(y)`` without a
    residual). Validation, stream and output ownership as ``MoeFp8Op``."""

    def __init__(self, weights: MoeMxfp4Weights, device, cfg: Mxfp4MoeConfig = MXFP4_MOE,
                 max_rows: int = MAX_ROWS, deadline_s: float = 10.0, fault=(0, 0)):
        self.cfg, self.device = cfg, torch.device(device)
        if not 1 <= max_rows <= MAX_ROWS:
            raise ValueError(f"max_rows must be 1..{MAX_ROWS}")
        weights = weights.bytes_view()
        weights.validate(cfg, self.device)
        self.w = weights
        nbytes = _lib.lib().mono_moe_mxfp4_scratch_bytes(cfg.hidden, cfg.inter, cfg.experts)
        if nbytes == 0:
            raise ValueError(f"no MXFP4 MoE kernel for hidden {cfg.hidden}, inter {cfg.inter}")
        self.rt = MonoRuntime(nbytes, self.device, deadline_s)
        self.max_rows = max_rows
        self.fault = fault
        self.outs = [torch.empty(max_rows, cfg.hidden, dtype=torch.bfloat16, device=self.device)
                     for _ in range(2)]
        self.parity = 0

    def launch(self, x: torch.Tensor, logits: torch.Tensor, res: Optional[torch.Tensor] = None,
               y: Optional[torch.Tensor] = None, routing: Optional[MoeRouting] = None,
               out: Optional[torch.Tensor] = None, stream=None,
               timeline: Optional[torch.Tensor] = None) -> torch.Tensor:
        cfg = self.cfg
        if x.dim() != 2 or not 1 <= x.shape[0] <= self.max_rows:
            raise ValueError(f"x: needs [rows <= {self.max_rows}, {cfg.hidden}], got {tuple(x.shape)}")
        r = x.shape[0]
        _need(x, "x", torch.bfloat16, (r, cfg.hidden), self.device)
        _need(logits, "logits", torch.float32, (r, cfg.experts), self.device)
        if res is not None:
            _need(res, "res", torch.bfloat16, (r, cfg.hidden), self.device)
        if out is None:
            out = self.outs[self.parity][:r]
            self.parity ^= 1
        _need(out, "out", torch.bfloat16, (r, cfg.hidden), self.device)
        if y is not None:
            _need(y, "y", torch.float32, (r, cfg.hidden), self.device)
        if routing is not None:
            _need(routing.scores, "scores", torch.float32, (r, cfg.experts), self.device)
            _need(routing.ids, "ids", torch.int32, (r, cfg.top_k + 1), self.device)
            _need(routing.weights, "weights", torch.float32, (r, cfg.top_k + 1), self.device)
        if timeline is not None:
            _need(timeline, "timeline", torch.int64, (self.rt.grid, _lib.TL_COLS), self.device)
        self.rt.before_launch()
        w = self.w
        ptr = lambda t: t.data_ptr() if t is not None else None
        args = _lib.MonoMoeMxfp4Args(
            rows=r, hidden=cfg.hidden, inter=cfg.inter, experts=cfg.experts,
            layout=_lib.LAYOUT_AITER16 if w.layout == layouts.AITER16 else _lib.LAYOUT_ROWMAJOR,
            route_scale=cfg.route_scale, n_group=cfg.n_group, topk_group=cfg.topk_group,
            x=x.data_ptr(), res=ptr(res), out=out.data_ptr(),
            logits=logits.data_ptr(), bias=w.bias.data_ptr(), w13=w.w13.data_ptr(),
            s13=w.s13.data_ptr(), w2=w.w2.data_ptr(), s2=w.s2.data_ptr(), y=ptr(y),
            scores=ptr(routing.scores) if routing else None,
            ids=ptr(routing.ids) if routing else None,
            weights=ptr(routing.weights) if routing else None,
            scratch=self.rt.scratch.data_ptr(), guard=self.rt.guard.data_ptr(),
            host_error=self.rt.host_error.data_ptr(),
            fault_site=int(self.fault[0]), fault_after=int(self.fault[1]),
            timeline=ptr(timeline),
        )
        with torch.cuda.device(self.device):
            _lib.check(_lib.lib().mono_moe_mxfp4_launch(ctypes.byref(args),
                                                         _lib.stream_handle(stream)),
                       "mono_moe_mxfp4_launch")
        return out
