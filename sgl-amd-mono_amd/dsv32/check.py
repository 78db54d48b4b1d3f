"""Check mode (``SGLANG_AMD_MONO_CHECK=1``, eager steps only).

Before each covered layer's launch, SGLang's own decoder layer runs on a copy of the
launch's input rows and on the caches as they stand. What it writes to the caches is
kept aside and the caches are put back, so the launch meets them exactly as SGLang's
layer did. The launch is then scored against SGLang's layer:

- ``layer.out.rel`` / ``layer.out.max_abs``: the hidden stream the launch hands on (the
  error in norm relative to SGLang's, and the largest difference beyond 1e-2 of it);
- ``router.ids.mismatch``: the share of rows whose 8 routed experts differ. SGLang's
  fused top-k adds the correction bias in bf16, so while its layer runs, its top-k module
  is swapped for one that routes in f32, the way the launch routes;
- ``indexer.topk.mismatch``: the largest share of a row's KV slots SGLang's indexer picks
  that the launch's selection leaves out;
- ``layer.topk_exact.max_abs``: per row, how many keys of the exact top-2048 of the
  launch's own index scores (score descending, then position) its selection misses;
- ``layer.kv.cosine``: the MLA cache rows the launch wrote at the step's slots against the
  rows SGLang's layer wrote there, both read back from E4M3;
- ``layer.index.cosine``: the same for the index keys the step adds, decoded from the
  pool's index cache (DSA pages: E4M3 times the token's scale; the FP4 plane: E2M1 times
  the 32-value group's E8M0).

Every value is logged at INFO and every bound missed at ERROR; a bound named
``*.cosine`` is a floor, any other a ceiling. The metrics and their floors follow the
reference's check (``sgl_amd_mono/glm53/check.py:1-11``, bounds ``glm53/spec.py:154-165``);
the SGLang names used are its layer interface: ``TopK.forward(hidden_states,
router_logits, ...)`` returning a ``TopKOutput`` named tuple, the decoder layer's call,
and the residual-stream helpers ``set_written`` / ``fold`` / ``take_output``.
"""

from __future__ import annotations

import logging
import os
from dataclasses import dataclass
from typing import Optional

import torch

logger = logging.getLogger(__name__)

SHARED_EXPERT = 256  # the id SGLang gives the fused shared expert
PAGE = 64  # tokens a cache page holds
DSA_VALUES = PAGE * 128  # a DSA index page's E4M3 bytes; the tokens' f32 scales follow


def enabled() -> bool:
    return os.environ.get("SGLANG_AMD_MONO_CHECK") == "1"


# ------------------------------------------------------------------ f32 routing
def _radix(x: torch.Tensor) -> torch.Tensor:
    """Order-preserving int64 image of f32 values (the launch ranks these bits)."""
    b = x.contiguous().view(torch.int32).to(torch.int64)
    return torch.where(b >= 0, b + (1 << 31), (~b) & 0xFFFFFFFF)


def route_f32(x: torch.Tensor, gate_w: torch.Tensor, bias: torch.Tensor, cfg):
    """The launch's routing of rows ``x`` [S, hidden]: scores = sigmoid of the f32 router
    logits; a row's candidates are scores + bias in f32, limited to the topk_group best of
    n_group expert groups when n_group > 1 (a group's value is the sum of its two largest
    candidates; ties to the lower group); the top_k largest candidates win, ties to the
    lower id. Weights: each pick's score over the picks' sum, times route_scale.
    Returns (ids int64 [S, k], weights f32 [S, k])."""
    scores = torch.sigmoid(x.float() @ gate_w.float().t())
    cand = scores + bias.float()
    S, E = cand.shape
    rank = _radix(cand)
    if cfg.n_group > 1:
        per = E // cfg.n_group
        two = cand.view(S, cfg.n_group, per).topk(2, dim=-1).values
        gval = _radix(two[..., 0] + two[..., 1])
        # descending value, lower group first: a lexicographic key (value, -group)
        gkey = gval * cfg.n_group + (cfg.n_group - 1 - torch.arange(cfg.n_group))
        kept = gkey.topk(cfg.topk_group, dim=-1).indices
        live = torch.zeros(S, cfg.n_group, dtype=torch.bool).scatter_(1, kept, True)
        rank = torch.where(live.repeat_interleave(per, 1), rank, torch.full_like(rank, -1))
    # descending rank, lower id first, as one key
    key = rank * E + (E - 1 - torch.arange(E))
    ids = key.topk(cfg.top_k, dim=-1).indices
    raw = torch.gather(scores, 1, ids)
    return ids, raw / raw.sum(-1, keepdim=True) * cfg.route_scale


class _F32TopK(torch.nn.Module):
    """SGLang's top-k module with its routed picks replaced by ``route_f32``'s. The
    original still runs, so the output keeps SGLang's form (a fused shared expert's
    column, dtypes, padding); ``picked`` keeps the f32 ids of the last call."""

    def __init__(self, inner, mlp, cfg):
        super().__init__()
        self.inner, self.mlp, self.cfg = inner, mlp, cfg
        self.picked = None

    def forward(self, hidden_states, router_logits, *args, **kwargs):
        out = self.inner(hidden_states, router_logits, *args, **kwargs)
        gate = self.mlp.gate
        ids, w = route_f32(hidden_states.cpu(), gate.weight.cpu(),
                           gate.e_score_correction_bias.cpu(), self.cfg)
        self.picked = ids
        sg_ids, sg_w = out.topk_ids, out.topk_weights
        routed = (sg_ids != SHARED_EXPERT).cpu()
        # the routed columns of each row, in order, take the f32 picks
        col = torch.cumsum(routed.to(torch.int64), 1) - 1
        src = col.clamp(0, self.cfg.top_k - 1)
        new_ids = torch.where(routed, torch.gather(ids, 1, src), sg_ids.cpu().to(torch.int64))
        new_w = torch.where(routed, torch.gather(w, 1, src), sg_w.cpu().float())
        return out._replace(topk_ids=new_ids.to(sg_ids.dtype).to(sg_ids.device),
                            topk_weights=new_w.to(sg_w.dtype).to(sg_w.device))


class f32_routing:
    """``with f32_routing(mlp, cfg) as r:`` swaps ``mlp.topk`` for ``_F32TopK`` and puts
    the original back on exit; ``r.picked`` holds the ids of the last routed call."""

    def __init__(self, mlp, cfg):
        self.mlp, self.cfg, self.inner, self.topk = mlp, cfg, mlp.topk, None

    def __enter__(self):
        self.topk = _F32TopK(self.inner, self.mlp, self.cfg)
        self.mlp.topk = self.topk
        return self.topk

    def __exit__(self, *exc):
        self.mlp.topk = self.inner
        return False


# ------------------------------------------------------------------ cache entries
@dataclass
class StepEntries:
    """The cache entries a step of a layer writes: the KV rows at its live slots and the
    index keys of the same tokens (the page-granular index tensors are kept whole per page
    touched, so they can be put back)."""

    slots: torch.Tensor  # i64 [n] live slots of the step
    kv: torch.Tensor  # [slots, 576] byte view of the pool's MLA rows
    index: list  # the pool's index tensors, page-major
    pages: torch.Tensor  # i64 pages the step touches

    @classmethod
    def of(cls, pool, layer: int, out_cache_loc: torch.Tensor, S: int) -> "StepEntries":
        from .binding import index_buffers

        loc = out_cache_loc[:S].to(torch.int64)
        slots = loc[loc > 0]  # slot 0 is SGLang's padding slot
        kv = pool.get_key_buffer(layer)
        return cls(slots=slots, kv=kv.view(torch.uint8).view(kv.shape[0], -1),
                   index=index_buffers(pool, layer), pages=torch.unique(slots // PAGE))

    def save(self) -> dict:
        return {"kv": self.kv[self.slots].clone(),
                "index": [t[self.pages].clone() for t in self.index]}

    def restore(self, saved: dict) -> None:
        self.kv[self.slots] = saved["kv"]
        for t, s in zip(self.index, saved["index"]):
            t[self.pages] = s

    def kv_values(self, saved: Optional[dict] = None) -> torch.Tensor:
        """The KV rows (the saved ones, or the pool's now) as f32 from E4M3."""
        rows = saved["kv"] if saved is not None else self.kv[self.slots]
        return rows.contiguous().view(torch.float8_e4m3fn).float()

    def index_keys(self, saved: Optional[dict] = None) -> torch.Tensor:
        """The step's index keys [n, 128] in f32, decoded from the pool's format."""
        pages = saved["index"] if saved is not None else [t[self.pages] for t in self.index]
        at = torch.searchsorted(self.pages, self.slots // PAGE)  # each slot's page row
        tok = self.slots % PAGE
        if len(pages) == 1:
            return _dsa_keys(pages[0].reshape(pages[0].shape[0], -1), at, tok)
        return _fp4_keys(pages[0], pages[1], at, tok)


def _dsa_keys(pages: torch.Tensor, at: torch.Tensor, tok: torch.Tensor) -> torch.Tensor:
    """Keys of tokens ``tok`` on page rows ``at`` of DSA index pages [n, 8448]: value d of
    token t sits in the 16-token x 16-byte tiles at (t / 16) 2048 + (d / 16) 256 +
    (t % 16) 16 + d % 16; the token's f32 scale at 8192 + 4 t."""
    d = torch.arange(128)
    off = (tok[:, None] // 16) * 2048 + (d // 16) * 256 + (tok[:, None] % 16) * 16 + d % 16
    codes = pages.cpu()[at.cpu()[:, None], off.cpu()]
    vals = codes.contiguous().view(torch.float8_e4m3fn).float()
    sc_bytes = pages.cpu()[at.cpu()][:, DSA_VALUES:].contiguous().view(torch.float32)
    return vals * torch.gather(sc_bytes, 1, tok.cpu()[:, None])


_E2M1 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                      -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])


def _fp4_keys(pay: torch.Tensor, sc: torch.Tensor, at: torch.Tensor,
              tok: torch.Tensor) -> torch.Tensor:
    """Keys from the FP4 index plane: payload [n, 1, 4, 64, 16] (32-value group c, slot s,
    E2M1 pairs low nibble first) and E8M0 [n, 1, 4, 64] with slot s's byte of group c at
    (s % 16) 4 + s / 16 of the group's 64."""
    p = pay.cpu().reshape(pay.shape[0], 4, PAGE, 16)[at.cpu(), :, tok.cpu()]  # [n, 4, 16]
    nib = torch.stack([p & 15, p >> 4], -1).reshape(-1, 4, 32).long()
    s = sc.cpu().reshape(sc.shape[0], 4, PAGE)[at.cpu()]  # [n, 4, 64]
    byte = (tok.cpu() % 16) * 4 + tok.cpu() // 16
    e8 = torch.gather(s, 2, byte[:, None, None].expand(-1, 4, 1))[..., 0].float()
    return (_E2M1[nib] * torch.exp2(e8 - 127.0)[..., None]).reshape(-1, 128)


# ------------------------------------------------------------------ SGLang's layer
@torch.no_grad()
def reference(L, positions, h_rows: torch.Tensor, forward_batch, S: int, cfg, pool) -> dict:
    """SGLang's decoder layer ``L.module`` on a copy of ``h_rows`` [S, hidden], routed in
    f32. Returns its output stream, its routed ids, its indexer's selection and the cache
    entries it wrote; the caches are then as they were before it ran."""
    from sglang.srt.layers.layer_boundary.residual.batch import fold, set_written, take_output
    from sglang.srt.utils.common import BumpAllocator

    entries = StepEntries.of(pool, L.i, forward_batch.out_cache_loc, S)
    before = entries.save()
    # one layer's share of the zero buffers the model's forward hands its layers
    zeros = BumpAllocator(buffer_size=2, dtype=torch.float32, device=h_rows.device)
    try:
        with f32_routing(L.module.mlp, cfg) as router:
            stream = set_written(h_rows.clone(), forward_batch)
            res, selection = L.module(positions[:S], stream, forward_batch, zeros, None, None,
                                      prev_topk_indices=None)
            out = take_output(fold(res, forward_batch), forward_batch).clone()
        written = entries.save()
    finally:
        entries.restore(before)
    return {"out": out, "ids": router.picked, "topk": selection, "written": written,
            "entries": entries}


# ------------------------------------------------------------------ the comparison
def _cosine(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double().flatten(), b.double().flatten()
    den = float(a.norm() * b.norm())
    return float(a @ b) / den if den > 0 else (1.0 if float(a.norm() + b.norm()) == 0 else 0.0)


def exact_topk_misses(scores: torch.Tensor, selected: torch.Tensor, counts, k: int) -> int:
    """The most keys, over the rows, of the exact top-``k`` of ``scores`` [S, >= n] (f32,
    the launch's own; score descending, then lower position) that the row's ``selected``
    positions (-1 padded) leave out. ``counts[s]``: the keys row s sees."""
    worst = 0
    for s, n in enumerate(counts):
        n = int(n)
        if n <= 0:
            continue
        key = _radix(scores[s, :n].float().cpu()) * n + (n - 1 - torch.arange(n))
        want = set(key.topk(min(k, n)).indices.tolist())
        have = set(int(p) for p in selected[s].tolist() if p >= 0)
        worst = max(worst, len(want - have))
    return worst


def compare(L, got: torch.Tensor, ref: dict, S: int, *, ids=None, topk_slots=None,
            scores=None, topk_pos=None, counts=None, numerics=None) -> dict:
    """Score the launch against ``reference``'s result and log it. ``got`` [S, hidden]:
    the launch's stream; ``ids`` [S, 8] its routed experts; ``topk_slots`` [S, 2048] its
    selection as KV slots (-1 padded); ``scores`` [S, ctx] and ``topk_pos`` [S, 2048] its
    index scores and selection as positions, with ``counts`` the keys each row sees.
    Returns {metric: value}."""
    values = {}
    a, b = got[:S].float(), ref["out"].float()
    values["layer.out.rel"] = float((a - b).norm() / b.norm().clamp_min(1e-30))
    values["layer.out.max_abs"] = float(((a - b).abs() - 1e-2 * b.abs()).max())
    if ids is not None and ref.get("ids") is not None:
        mine = torch.sort(ids[:S].cpu().to(torch.int64), -1).values
        want = torch.sort(ref["ids"][:S].to(torch.int64), -1).values
        values["router.ids.mismatch"] = float((mine != want).any(-1).double().mean())
    if topk_slots is not None and ref.get("topk") is not None:
        share = 0.0
        for s in range(S):
            want = set(k for k in ref["topk"][s].tolist() if k >= 0)
            if want:
                have = set(k for k in topk_slots[s].tolist() if k >= 0)
                share = max(share, len(want - have) / len(want))
        values["indexer.topk.mismatch"] = share
    if scores is not None and topk_pos is not None and counts is not None:
        k = topk_pos.shape[-1]
        values["layer.topk_exact.max_abs"] = float(exact_topk_misses(scores, topk_pos, counts, k))
    entries, written = ref.get("entries"), ref.get("written")
    if entries is not None and written is not None and entries.slots.numel():
        values["layer.kv.cosine"] = _cosine(entries.kv_values(), entries.kv_values(written))
        values["layer.index.cosine"] = _cosine(entries.index_keys(),
                                               entries.index_keys(written))
    logger.info("monokernel check layer %d (%d rows): %s", L.i, S,
                " ".join(f"{k}={v:.6g}" for k, v in values.items()))
    for name, bound in (numerics or {}).items():
        v = values.get(name)
        if v is None:
            continue
        if (v < bound) if name.endswith(".cosine") else (v > bound):
            logger.error("monokernel check violation: layer %d %s = %.6g, bound %g", L.i, name,
                         v, bound)
    return values
