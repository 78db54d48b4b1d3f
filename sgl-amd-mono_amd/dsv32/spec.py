"""DeepSeek-V3.2 (DSA) on gfx950: the monokernel spec SGLang routes decode steps to.

The plugin surface of ``sgl_amd_mono/glm53/spec.py:584-616``: a ``MonoSpec`` registered
under backend ``amd`` for the architecture, with device limits, requirements, numerics
bounds, config and model refusal reasons (lists of reasons, never exceptions), and
``build(model, hf_config, ctx)`` returning an object whose ``forward(plan, input_ids,
positions, forward_batch, ...)`` SGLang calls for a routed step. The forward decides by
the graph key alone (``plan.key.rows`` against the widths built), so every rank and every
graph replay makes the same choice; a wider step runs the model's own forward.

Every covered layer (the MoE layers) runs as the layer launch over SGLang's weights in
place (the few copies logged by ``binding``) and its KV / FP4 index pages in place. The
dense layers before them run on SGLang's path; the residual stream crosses between the
two through SGLang's layer-boundary API, as the reference's backbone does
(``glm53/spec.py:319-352``, ``:354-417``): the first covered layer folds the pending
residual add of the layer before it into its input, the last marks its output as a
written stream for the final norm.

The kernels carry one GPU's TP=4 share of a layer (32 heads, expert intermediate 512)
and the two TP exchanges are not built, so the spec serves a model whose shapes at TP 1
are that share, and refuses any other with the reason.
"""

from __future__ import annotations

import dataclasses
import math

import torch

try:
    from sglang.kernels.plugin_kernels.amd.spec import (
        DeviceLimits,
        Feature,
        MonoSpec,
        Numerics,
        NumericsKind,
        Requirements,
    )
except ModuleNotFoundError:  # SGLang before sgl-project/sglang#45389
    from sglang.srt.monokernels.spec import (
        DeviceLimits,
        Feature,
        MonoSpec,
        Numerics,
        NumericsKind,
        Requirements,
    )

from .config import DSV32
from .runner import StepRows

MAX_ROWS = 8  # the front builds x of at most 8 rows in LDS
WIDTHS = tuple(range(1, MAX_ROWS + 1))  # one build serves every row count up to 8
TP_SIZES = (1,)
BLOCKS = 256  # one CTA per MI355X CU
PAGE_SIZE = DSV32.page
MAX_CONTEXT = 163840  # keys a row's exact top-k ranks (five 32768-key blocks)

# the bounds a check-mode step is held to (the north star's parity bar)
NUMERICS = Numerics(
    NumericsKind.TOLERANCE,
    {
        "layer.out.max_abs": 2e-2,
        "layer.out.rel": 1e-2,
        "router.ids.mismatch": 0.0,
        "indexer.topk.mismatch": 0.0,
        # the cache rows the launch writes against SGLang's (floors)
        "layer.kv.cosine": 0.995,
        "layer.index.cosine": 0.999,
        # the selection is exactly the top-k of the launch's own scores
        "layer.topk_exact.max_abs": 0.0,
    },
)

# the shapes, routing and rotary layout the kernels build in (a layer's share at TP 1)
HF_CONFIG = dict(
    hidden_size=DSV32.hidden,
    num_attention_heads=DSV32.heads,
    q_lora_rank=DSV32.q_lora,
    kv_lora_rank=DSV32.kv_lora,
    qk_rope_head_dim=DSV32.rope_dim,
    qk_nope_head_dim=DSV32.nope_dim,
    v_head_dim=DSV32.v_dim,
    n_routed_experts=DSV32.experts,
    num_experts_per_tok=DSV32.top_k,
    n_shared_experts=1,
    moe_intermediate_size=DSV32.inter,
    routed_scaling_factor=DSV32.route_scale,
    scoring_func="sigmoid",
    topk_method="noaux_tc",
    norm_topk_prob=True,
    hidden_act="silu",
    rms_norm_eps=DSV32.rms_eps,
    index_n_heads=DSV32.index_heads,
    index_head_dim=DSV32.index_dim,
    index_topk=DSV32.index_topk,
    indexer_rope_interleave=True,
)


def _width(rows: int) -> int:
    return next(w for w in WIDTHS if w >= rows)


def covered_layers(hf_config) -> list:
    """The MoE layers the forward covers (the dense layers run SGLang's path)."""
    first = getattr(hf_config, "first_k_dense_replace", 3)
    return list(range(first, hf_config.num_hidden_layers))


def _rope(hf_config) -> dict:
    return dict(getattr(hf_config, "rope_parameters", None)
                or getattr(hf_config, "rope_scaling", None) or {})


def softmax_scale(hf_config) -> float:
    """(nope + rope)^-1/2, times YaRN's mscale^2 when the rotary embedding is YaRN (the
    scale SGLang's MLA attention applies: 0.1 mscale_all_dim ln(factor) + 1 per factor
    above 1); the launch's scale is a plain argument, so it follows the model."""
    scale = (DSV32.nope_dim + DSV32.rope_dim) ** -0.5
    rope = _rope(hf_config)
    if rope.get("rope_type", rope.get("type", "default")) == "yarn":
        factor = float(rope.get("factor", 1.0))
        m_all = float(rope.get("mscale_all_dim", 0.0) or 0.0)
        if factor > 1.0 and m_all:
            m = 0.1 * m_all * math.log(factor) + 1.0
            scale *= m * m
    return scale


def _groups(hf_config):
    """The model's group-limited routing (n_group, topk_group); 1, 1 when it has none."""
    return (int(getattr(hf_config, "n_group", 1) or 1),
            int(getattr(hf_config, "topk_group", 1) or 1))


def _groups_ok(n_group: int, topk_group: int) -> bool:
    """What the launches route (route_groups_ok in csrc/moe_common.h)."""
    if n_group == 1:
        return True
    experts = DSV32.experts
    return (2 <= n_group <= 16 and experts % n_group == 0 and 1 <= topk_group <= n_group
            and topk_group * (experts // n_group) >= DSV32.top_k)


def _same(have, want) -> bool:
    if isinstance(want, float):
        return have is not None and abs(float(have) - want) <= 1e-9 * max(1.0, abs(want))
    return have == want


def _config_disable_reasons(cfg, hf_config) -> list:
    """Why this spec cannot serve a model config (an empty list: it can)."""
    reasons = [f"needs {key} = {want!r}, got {getattr(hf_config, key, None)!r}"
               for key, want in HF_CONFIG.items() if not _same(getattr(hf_config, key, None), want)]
    if getattr(hf_config, "rope_interleave", True) is not True:
        reasons.append("the MLA rotary embedding must rotate interleaved pairs "
                       "(rope_interleave = True)")
    rope_type = (lambda r: r.get("rope_type", r.get("type", "default")))(_rope(hf_config))
    if rope_type not in ("default", "yarn"):
        reasons.append(f"RoPE {rope_type!r}: the launches read SGLang's cos / sin table "
                       "and scale the softmax for default or YaRN RoPE only")
    if getattr(hf_config, "moe_layer_freq", 1) != 1:
        reasons.append("needs every layer after the dense ones to be MoE")
    n_group, topk_group = _groups(hf_config)
    if not _groups_ok(n_group, topk_group):
        reasons.append(f"n_group {n_group} / topk_group {topk_group}: the router keeps "
                       "1..16 groups dividing the 256 experts, holding at least 8 of them")
    tp = int(getattr(cfg, "tp_size", 1) or 1)
    if tp not in TP_SIZES:
        reasons.append(f"TP {tp}: the launches compute one GPU's share and the TP "
                       "exchanges are not built")
    page = getattr(cfg, "page_size", None)
    if page not in (None, PAGE_SIZE):
        reasons.append(f"--page-size {page}: the DSA caches need {PAGE_SIZE}")
    context = getattr(cfg, "context_length", None) or getattr(
        hf_config, "max_position_embeddings", None)
    if context is not None and int(context) > MAX_CONTEXT:
        reasons.append(f"context {context}: the exact top-k ranks at most {MAX_CONTEXT} "
                       "keys a row (--context-length to serve within it)")
    if getattr(cfg, "speculative_algorithm", None) is not None:
        reasons.append("speculative verify rows are not built: plain decode rows only")
    q = getattr(hf_config, "quantization_config", None) or {}
    if q.get("quant_method") != "fp8" or list(q.get("weight_block_size") or ()) != [128, 128]:
        reasons.append("needs the FP8 checkpoint with 128 x 128 block scales, got "
                       f"{q.get('quant_method')!r} {q.get('weight_block_size')!r}")
    return reasons


def _model_disable_reasons(model, hf_config, copies) -> list:
    """Why the loaded model cannot be read in place (an empty list: it can)."""
    from .binding import layer_disable_reason, rope_table

    reasons = []
    layers = {i: model.model.layers[i] for i in covered_layers(hf_config)}
    for i, layer in layers.items():
        why = layer_disable_reason(layer, i)
        if why is not None:
            reasons.append(why)
    if layers and not reasons:
        try:
            rope_table(layers, {})
        except (ValueError, AttributeError) as e:
            reasons.append(str(e))
    return reasons


class _Layer:
    """A covered layer: its index, SGLang module and launch; its caches bind at its
    first launch and rebind when SGLang's pool moves."""

    def __init__(self, i: int, module, op):
        self.i, self.module, self.op = i, module, op
        self.caches = None


class _Built:
    """One rank's layer launches, the step's row tables per width, and the forward."""

    def __init__(self, lm, layers: dict, device, context_len: int, cfg=DSV32):
        from . import check

        self.lm, self.layers, self.cfg = lm, layers, cfg
        self.check = check.enabled()  # SGLANG_AMD_MONO_CHECK=1: eager steps checked
        self.first = min(layers) if layers else None
        self.last = max(layers) if layers else None
        self.max_rows = MAX_ROWS
        self.max_position = context_len - 1
        self.steps = {w: StepRows.empty(w, device, context_len) for w in WIDTHS}
        self.pad_h = {w: torch.zeros(w, DSV32.hidden, dtype=torch.bfloat16, device=device)
                      for w in WIDTHS}

    def forward(self, plan, input_ids, positions, forward_batch, input_embeds=None,
                pp_proxy_tensors=None):
        """``DeepseekV2ForCausalLM.forward`` for a routed decode step; a step wider than
        the built widths runs the model's own forward (decided by the graph key)."""
        lm = self.lm
        if plan.key.rows > self.max_rows:
            return type(lm).forward(lm, input_ids, positions, forward_batch, input_embeds,
                                    pp_proxy_tensors)
        from sglang.srt.layers.layer_boundary import get_attn_tp_context

        with get_attn_tp_context().maybe_input_scattered(forward_batch):
            hidden = self._backbone(plan, input_ids, positions, forward_batch, input_embeds)
        return lm.logits_processor(input_ids, hidden, lm.lm_head, forward_batch, None)

    def _backbone(self, plan, input_ids, positions, forward_batch, input_embeds):
        """``DeepseekV2Model.forward``: the embedding and the dense layers on SGLang's
        path (each returns its stream and its top-k), the covered layers as launches,
        then the final norm."""
        from sglang.srt.layers.layer_boundary.residual.batch import (
            complete_output,
            final_norm,
            start,
        )
        from sglang.srt.utils.common import BumpAllocator

        m = self.lm.model
        hidden = m.embed_tokens(input_ids) if input_embeds is None else input_embeds
        start(forward_batch)
        zeros = BumpAllocator(buffer_size=(m.end_layer - m.start_layer) * 2,
                              dtype=torch.float32, device=hidden.device)
        gemm_zeros = None
        if getattr(m, "gemm_output_zero_allocator_size", 0) > 0:
            gemm_zeros = BumpAllocator(buffer_size=m.gemm_output_zero_allocator_size,
                                       dtype=torch.float32, device=hidden.device)
        topk = None
        for i in range(m.start_layer, m.end_layer):
            L = self.layers.get(i)
            if L is None:
                hidden, topk = m.layers[i](
                    positions, hidden, forward_batch, zeros, gemm_zeros, None,
                    prev_topk_indices=topk,
                    next_full_attention_layer_id=m.next_full_attention_layer_id.get(i))
            else:
                hidden = self._layer(L, plan, positions, hidden, forward_batch)
                topk = None
        hidden = complete_output(hidden, forward_batch)
        if not forward_batch.forward_mode.is_idle():
            hidden = final_norm(hidden, forward_batch, m.norm)
        return hidden

    def _layer(self, L: _Layer, plan, positions, hidden, forward_batch):
        """One covered layer: the first takes the full stream (the previous layer's output
        with its pending residual add folded in), padded to the width; later ones take
        the previous launch's output. The last hands its rows back as a written stream."""
        from sglang.srt.layers.layer_boundary.residual.batch import fold, set_written, take_output

        S = plan.key.rows
        W = _width(S)
        st = self.step(plan, positions, forward_batch)
        if L.i == self.first:
            h = take_output(fold(hidden, forward_batch), forward_batch)
            if S < W:
                pad = self.pad_h[W]
                pad[:S].copy_(h)
                pad[S:].zero_()
                h = pad
        else:
            h = hidden
        caches, lstep = self._caches(L, forward_batch), st.as_layer_step(W)
        capturing = torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()
        if self.check and not capturing:
            out = self._checked(L, positions, h, caches, lstep, forward_batch, S)
        else:
            out = L.op.launch(h, caches, lstep)
        if L.i != self.last:
            return out
        return set_written(out[:S], forward_batch)

    def _checked(self, L: _Layer, positions, h, caches, lstep, forward_batch, S: int):
        """The launch, with SGLang's layer run first on the same rows (check mode). The
        one launch also hands out its routed ids, index scores and selection, which
        ``check.compare`` scores against SGLang's and against the exact top-k."""
        from . import check
        from .layer import FusedLayerOp, LayerDebug

        ref = check.reference(L, positions, h[:S], forward_batch, S, self.cfg,
                              forward_batch.token_to_kv_pool)
        extra = {}
        if isinstance(L.op, FusedLayerOp):
            W, dev, cfg = h.shape[0], h.device, self.cfg
            dbg = LayerDebug(
                ids=torch.empty(W, cfg.top_k + 1, dtype=torch.int32, device=dev),
                topk=torch.empty(W, cfg.index_topk, dtype=torch.int32, device=dev),
                scores=torch.empty(W, L.op.ctx_max, dtype=torch.float32, device=dev))
            out = L.op.launch(h, caches, lstep, debug=dbg)
            pos = dbg.topk[:S].long()
            pages = lstep.page_table[lstep.req_ids[:S].long()[:, None],
                                     pos.clamp_min(0) // cfg.page].long()
            counts = torch.where(lstep.slots[:S] >= 0, lstep.positions[:S] + 1, 0)
            extra = dict(ids=dbg.ids[:, 1:],
                         topk_slots=torch.where(pos >= 0, pages * cfg.page + pos % cfg.page, -1),
                         scores=dbg.scores[:S], topk_pos=pos, counts=counts.tolist())
        else:
            out = L.op.launch(h, caches, lstep)
        check.compare(L, out[:S], ref, S, numerics=NUMERICS.bounds, **extra)
        return out

    def step(self, plan, positions, forward_batch):
        """The step's row tables, written once a step (in the graph when captured). The
        page table is the attention backend's ``real_page_table`` in place when it covers
        the served context (the launches read a row's pages up to ``ctx_max``); the DSA
        backend sizes that table by the batch's longest sequence, so a narrower one is
        replaced by the step's own full-width table, filled from ``req_to_token``."""
        if "step" not in plan.state:
            S = plan.key.rows
            st = self.steps[_width(S)]
            md = getattr(getattr(forward_batch, "attn_backend", None), "forward_metadata", None)
            pt = getattr(md, "real_page_table", None)
            if not self.page_table_covers(pt):
                pt = st.fill_pages(forward_batch.req_to_token_pool.req_to_token,
                                   forward_batch.req_pool_indices, S)
            st.write(positions, forward_batch.out_cache_loc, S, self.max_position,
                     page_table=pt)
            plan.state["step"] = _Step(st)
        return plan.state["step"]

    def page_table_covers(self, pt) -> bool:
        """Whether a backend page table can be read in place: int32 [requests, pages]
        with contiguous rows and pages for every key up to the served context."""
        return (pt is not None and pt.dtype == torch.int32 and pt.dim() == 2
                and pt.stride(1) == 1 and pt.shape[1] * PAGE_SIZE >= self.max_position + 1)

    @staticmethod
    def _caches(L: _Layer, forward_batch):
        """The layer's caches in SGLang's pool, bound once (rebound if the pool moved)."""
        from .binding import caches

        pool = forward_batch.token_to_kv_pool
        kv = pool.get_key_buffer(L.i)
        if L.caches is None or L.caches.kv.data_ptr() != kv.data_ptr():
            L.caches = caches(pool, L.i)
        return L.caches


class _Step:
    """A step's tables as the launches take them."""

    def __init__(self, st: StepRows):
        self.st = st

    def as_layer_step(self, width: int):
        from .layer import LayerStep

        st = self.st
        return LayerStep(positions=st.positions[:width], slots=st.slots[:width],
                         req_ids=st.req_ids[:width], page_table=st.page_table)


def _build(model, hf_config, ctx):
    """The launch of every covered layer, over SGLang's loaded weights in place: one
    persistent launch a layer. Layers share one runtime (scratch and guard block): their
    launches are stream ordered, and a failure raises the block's abort word, which every
    later launch of the step sees, so each of them ends with NaN outputs too. A layer whose
    projections SGLang left in mixed FP8 layouts runs as the four launches instead.
    ``SGLANG_AMD_MONO_FAULT_INJECT`` (``rank:site[:after]``) arms a test stall."""
    from ..guard import fault_injection, watchdog_deadline
    from .binding import layer_weights, rope_table
    from .layer import FusedLayerOp, LayerOp, LayerRuntimes, layer_runtime

    deadline = watchdog_deadline(getattr(ctx, "deadline_s", 120.0) * 2)
    context_len = min(int(getattr(ctx, "context_len", None) or MAX_CONTEXT), MAX_CONTEXT)
    copies = getattr(ctx, "copies", None)
    copies = {} if copies is None else copies
    sm_scale = softmax_scale(hf_config)
    n_group, topk_group = _groups(hf_config)
    cfg = dataclasses.replace(DSV32, n_group=n_group, topk_group=topk_group)
    fault = fault_injection(int(getattr(ctx, "tp_rank", 0) or 0)) or (0, 0)
    layers, rt, chained, device = {}, None, None, None
    modules = {i: model.model.layers[i] for i in covered_layers(hf_config)}
    rope = rope_table(modules, copies) if modules else None  # one table for every layer
    for i, mod in modules.items():
        w = layer_weights(mod, i, copies, rope=rope)
        device = w.moe.w13.device
        if rt is None:
            rt = layer_runtime(device, MAX_ROWS, deadline)
        try:
            op = FusedLayerOp(w, device, cfg=cfg, max_rows=MAX_ROWS, ctx_max=context_len,
                              sm_scale=sm_scale, fault=fault, rt=rt)
        except ValueError:  # mixed layouts: the four launches read each struct's own
            if chained is None:
                chained = LayerRuntimes(device, cfg, max_rows=MAX_ROWS, ctx_max=context_len,
                                        deadline_s=deadline)
            op = LayerOp(w, chained, cfg=cfg, sm_scale=sm_scale)
        layers[i] = _Layer(i, mod, op)
    return _Built(model, layers, device or torch.device("cpu"), context_len=context_len, cfg=cfg)


SPEC = MonoSpec(
    name="dsv32_hip",
    devices={"gfx950": DeviceLimits(widths=WIDTHS, tp_sizes=TP_SIZES, resident_blocks=BLOCKS)},
    features=frozenset(),
    requires=Requirements(
        dtypes=frozenset({"bfloat16"}),
        attention_backends=frozenset({"dsa"}),
        server_args={
            "moe_runner_backend": frozenset({"auto", "aiter"}),
            "speculative_algorithm": frozenset({None}),
            "expert_distribution_recorder_mode": frozenset({None}),
        },
        env={
            "SGLANG_SIMULATE_UNIFORM_EXPERTS": False,
            "SGLANG_SIMULATE_ROUND_ROBIN_EXPERTS": False,
        },
    ),
    numerics=NUMERICS,
    model_disable_reasons=_model_disable_reasons,
    build=_build,
    api_version=1,
    config_disable_reasons=_config_disable_reasons,
)
