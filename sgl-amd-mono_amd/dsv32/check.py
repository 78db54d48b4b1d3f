"""Check mode (``SGLANG_AMD_MONO_CHECK=1``, eager steps only): every covered layer also
runs SGLang's own layer module on the same input rows, before its launch, and the
launch is held to the spec's ``NUMERICS`` bounds against it:

- ``layer.out``: the hidden stream the launch hands on against SGLang's (relative error
  in norm, and the largest difference beyond 1e-2 of the reference value);
- ``router.ids``: the share of rows whose 8 routed experts differ from SGLang's, SGLang
  routed in f32 as the launch routes (its fused top-k adds the correction bias in bf16);
- ``indexer.topk``: the largest share of a row's selected KV slots SGLang picks that the
  launch does not.

Every comparison is logged at INFO, a bound missed at ERROR. The cache rows SGLang's
layer writes are put back before the launch writes its own. Follows the reference's
check (``sgl_amd_mono/glm53/check.py:159-278``) and its call around the launch
(``glm53/spec.py:394-411``); the SGLang names read here are its layer interface.
"""

from __future__ import annotations

import logging
import os

import torch

from .binding import index_buffers

logger = logging.getLogger(__name__)

SHARED_EXPERT = 256  # SGLang's id of the fused shared expert


def enabled() -> bool:
    return os.environ.get("SGLANG_AMD_MONO_CHECK") == "1"


@torch.no_grad()
def _f32_topk(x, mlp, top_k: int, n_group: int, topk_group: int, route_scale: float):
    """The routed experts of rows ``x`` as the launch picks them: sigmoid of the f32 router
    logits, plus the correction bias in f32, group-limited when n_group > 1 (each group's
    two largest summed, the topk_group best groups kept, ties to the lower group), top-k
    with ties to the lower id; weights = score / sum of the k scores * route_scale."""
    scores = torch.sigmoid(x.float() @ mlp.gate.weight.float().t())
    choice = scores + mlp.gate.e_score_correction_bias.float()
    n = choice.shape[-1]
    if n_group > 1:
        g = choice.view(-1, n_group, n // n_group)
        gs = g.topk(2, dim=-1).values.sum(-1)
        # ties to the lower group: a stable descending sort
        keep = torch.sort(gs, dim=-1, descending=True, stable=True).indices[:, :topk_group]
        mask = torch.zeros_like(gs, dtype=torch.bool).scatter_(1, keep, True)
        choice = choice.masked_fill(~mask.repeat_interleave(n // n_group, 1), float("-inf"))
    ids = torch.sort(choice, dim=-1, descending=True, stable=True).indices[:, :top_k]
    raw = scores.gather(1, ids)
    return ids, raw / raw.sum(-1, keepdim=True) * route_scale


def _route_in_f32(mlp, cfg):
    """Hooks making SGLang's top-k route in f32 (its output keeps SGLang's form: the
    shared expert's column stays as SGLang put it)."""
    seen = {}

    def gate_in(mod, args):
        seen["x"] = args[0]

    def route(mod, args, out):
        ids, w = _f32_topk(seen.pop("x"), mlp, cfg.top_k, cfg.n_group, cfg.topk_group,
                           cfg.route_scale)
        routed = out.topk_ids != SHARED_EXPERT
        new_ids, new_w = out.topk_ids.clone(), out.topk_weights.clone()
        new_ids[routed] = ids.to(new_ids.dtype).reshape(-1)
        new_w[routed] = w.to(new_w.dtype).reshape(-1)
        seen["ids"] = ids
        return out._replace(topk_ids=new_ids, topk_weights=new_w)

    return seen, (mlp.register_forward_pre_hook(gate_in), mlp.topk.register_forward_hook(route))


@torch.no_grad()
def reference(L, positions, h_rows: torch.Tensor, forward_batch, S: int, cfg, pool) -> dict:
    """SGLang's layer on a copy of ``h_rows`` [S, hidden]: its output stream, its routed
    expert ids and its top-k; the KV rows and index pages it wrote are put back."""
    from sglang.srt.layers.layer_boundary.residual.batch import fold, set_written, take_output
    from sglang.srt.utils.common import BumpAllocator

    loc = forward_batch.out_cache_loc[:S].long()
    slots = loc[loc >= 0]
    kv = pool.get_key_buffer(L.i)
    kv_rows = kv.view(kv.shape[0], -1)
    saved_kv = kv_rows[slots].clone()
    index = index_buffers(pool, L.i)
    pages = (slots // 64).unique()
    saved_index = [t[pages].clone() for t in index]
    seen, hooks = _route_in_f32(L.module.mlp, cfg)
    try:
        hidden = set_written(h_rows.clone(), forward_batch)
        zero = BumpAllocator(buffer_size=4, dtype=torch.float32, device=h_rows.device)
        out, topk = L.module(positions[:S], hidden, forward_batch, zero, None, None,
                             prev_topk_indices=None)
        stream = take_output(fold(out, forward_batch), forward_batch).clone()
    finally:
        for hk in hooks:
            hk.remove()
        kv_rows[slots] = saved_kv
        for t, saved in zip(index, saved_index):
            t[pages] = saved
    return {"out": stream, "ids": seen.get("ids"), "topk": topk}


def compare(L, got: torch.Tensor, ref: dict, S: int, *, ids=None, topk_slots=None,
            numerics=None) -> dict:
    """The launch's ``got`` [S, hidden] (and, when given, its routed ids [S, 8] and its
    selected slots [S, 2048], -1 padded) against ``reference``'s; logs every value and
    each bound missed. Returns {name: value}."""
    values = {}
    a, b = got.float(), ref["out"].float()
    d = (a - b).abs()
    values["layer.out.rel"] = float((a - b).norm() / b.norm().clamp_min(1e-30))
    values["layer.out.max_abs"] = float((d - 1e-2 * b.abs()).max())
    if ids is not None and ref.get("ids") is not None:
        mine = torch.sort(ids[:S].long().cpu(), -1).values
        want = torch.sort(ref["ids"][:S].long().cpu(), -1).values
        values["router.ids.mismatch"] = float((mine != want).any(-1).float().mean())
    if topk_slots is not None and ref.get("topk") is not None:
        worst = 0.0
        for s in range(S):
            want = {int(k) for k in ref["topk"][s].tolist() if k >= 0}
            if want:
                have = {int(k) for k in topk_slots[s].tolist() if k >= 0}
                worst = max(worst, len(want - have) / len(want))
        values["indexer.topk.mismatch"] = worst
    logger.info("monokernel check layer %d (%d rows): %s", L.i, S,
                " ".join(f"{k}={v:.6g}" for k, v in values.items()))
    for name, bound in (numerics or {}).items():
        v = values.get(name)
        if v is not None and v > bound:
            logger.error("monokernel check violation: layer %d %s = %.6g, bound %g", L.i, name,
                         v, bound)
    return values
