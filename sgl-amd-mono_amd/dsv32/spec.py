"""DeepSeek-V3.2 (DSA) on gfx950: the monokernel spec SGLang routes decode steps to.

The plugin surface of ``sgl_amd_mono/glm53/spec.py:584-616``: a ``MonoSpec`` registered
under backend ``amd`` for the architecture, with device limits, requirements, numerics
bounds, config and model refusal reasons, and ``build(model, hf_config, ctx)``
returning an object whose ``forward(plan, input_ids, positions, forward_batch, ...)``
SGLang calls for a routed step. The forward decides by the graph key alone
(``plan.key.rows`` against the widths built), so every rank and every graph replay makes
the same choice; a wider step runs the model's own forward.

A covered layer whose attention half binds (``binding.layer_disable_reason`` is None)
runs as the four launches of ``LayerOp``: front, attention, output block and MoE, over
SGLang's weights in place (the few copies logged by ``binding``) and its KV / FP4
index pages in place. Any other covered layer runs its FFN half as one persistent launch
(``MoeFp8Op``: post-attention RMSNorm, router, top-8 + shared expert, W8A8 experts and
the residual add, experts, router and norm read in place) after SGLang's attention.

One GPU's TP=4 share is what the kernels compute; the two TP exchanges of the layer are
not built, so ``build`` refuses a TP size above 1 with that reason rather than serve
unreduced partial sums.
"""

from __future__ import annotations

import os

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

from .config import DSV32, MAX_ROWS
from .runner import alloc_step, fill_step, page_table

# one build takes any row count up to 16 (the kernels read the count at run time)
WIDTHS = tuple(range(1, MAX_ROWS + 1))
TP_SIZES = (1, 4)
BLOCKS = 256  # one CTA per MI355X CU

# the bounds a check-mode step is held to (the north star's parity bar)
NUMERICS = Numerics(
    NumericsKind.TOLERANCE,
    {
        "moe.out.max_abs": 2e-2,
        "moe.out.rel": 1e-2,
        "router.ids.mismatch": 0.0,
        "indexer.topk.mismatch": 0.0,
    },
)

HF_CONFIG = dict(
    hidden_size=DSV32.hidden,
    n_routed_experts=DSV32.experts,
    num_experts_per_tok=DSV32.top_k,
    n_shared_experts=1,
    q_lora_rank=DSV32.q_lora,
    kv_lora_rank=DSV32.kv_lora,
    qk_rope_head_dim=DSV32.rope_dim,
    qk_nope_head_dim=DSV32.nope_dim,
    v_head_dim=DSV32.v_dim,
    routed_scaling_factor=DSV32.route_scale,
    scoring_func="sigmoid",
    topk_method="noaux_tc",
    rms_norm_eps=DSV32.rms_eps,
)


def _width(rows: int) -> int:
    return next(w for w in WIDTHS if w >= rows)


def covered_layers(hf_config) -> list:
    """The MoE layers the forward covers (the dense layers run SGLang's path)."""
    first = getattr(hf_config, "first_k_dense_replace", 3)
    return list(range(first, hf_config.num_hidden_layers))


def _config_disable_reasons(cfg, hf_config) -> list:
    """Why this spec cannot serve a model config (an empty list: it can)."""
    reasons = []
    for key, want in HF_CONFIG.items():
        have = getattr(hf_config, key, None)
        if have is None or (isinstance(want, float) and abs(float(have) - want) > 1e-9) or (
            not isinstance(want, float) and have != want
        ):
            reasons.append(f"{key} is {have!r}, the kernels are built for {want!r}")
    q = getattr(hf_config, "quantization_config", None) or {}
    if q.get("quant_method") != "fp8" or list(q.get("weight_block_size", [])) != [128, 128]:
        reasons.append("the experts must be FP8 with 128 x 128 block scales")
    if getattr(cfg, "speculative_algorithm", None) not in (None,):
        reasons.append("speculative verify rows are not built: plain decode rows only")
    return reasons


def _model_disable_reasons(model, hf_config, copies) -> list:
    """Why the loaded model cannot be read in place (an empty list: it can)."""
    reasons = []
    for i in covered_layers(hf_config):
        mlp = model.model.layers[i].mlp
        experts = getattr(mlp, "experts", None)
        if experts is None:
            reasons.append(f"layer {i}: no fused experts module")
            continue
        if experts.w13_weight.dtype != torch.float8_e4m3fn:
            reasons.append(f"layer {i}: experts are {experts.w13_weight.dtype}, need E4M3")
    return reasons


class _Layer:
    """A covered layer: its SGLang module and its launch (``LayerOp`` for the whole
    layer, or ``MoeFp8Op`` for its FFN half, ``full`` saying which)."""

    def __init__(self, i: int, module, op, full: bool = False, kv_scale=None):
        self.i, self.module, self.op, self.full = i, module, op, full
        self.kv_scale = kv_scale  # f32 [slots]: the per-token scales of the layer's KV rows
        self.caches = None


def plan_layers(model, hf_config) -> dict:
    """Layer -> None (the whole layer binds) or the reason its attention half does not
    (it then runs its FFN half only)."""
    from .binding import layer_disable_reason

    return {i: layer_disable_reason(model.model.layers[i], i) for i in covered_layers(hf_config)}


class _Built:
    """One rank's launches and the forward SGLang calls for a routed step."""

    def __init__(self, lm, layers: dict, device, context_len: int, max_rows: int = MAX_ROWS):
        self.lm, self.layers = lm, layers
        self.max_rows = max_rows
        self.max_position = context_len - 1
        self.steps = {w: alloc_step(w, device) for w in WIDTHS}
        self.check_layers = os.environ.get("SGLANG_AMD_MONO_CHECK") == "1"

    def forward(self, plan, input_ids, positions, forward_batch, input_embeds=None,
                pp_proxy_tensors=None):
        """``DeepseekV2ForCausalLM.forward`` for a routed decode step; a step wider than
        the built widths runs the model's own forward (decided by the graph key)."""
        lm = self.lm
        if plan.key.rows > self.max_rows:
            return type(lm).forward(lm, input_ids, positions, forward_batch, input_embeds,
                                    pp_proxy_tensors)
        hidden = self._backbone(plan, input_ids, positions, forward_batch, input_embeds)
        return lm.logits_processor(input_ids, hidden, lm.lm_head, forward_batch, None)

    def step(self, plan, positions, forward_batch):
        """The step's row tables, built once a step (in the graph when captured)."""
        if "step" not in plan.state:
            S = plan.key.rows
            st = self.steps[_width(S)]
            pt = None
            if any(L.full for L in self.layers.values()):
                pt = page_table(forward_batch.req_to_token_pool.req_to_token,
                                forward_batch.req_pool_indices, S, self.max_position + 1)
            plan.state["step"] = fill_step(st, positions, forward_batch.out_cache_loc, S,
                                           self.max_position, page_table=pt)
        return plan.state["step"]

    def _backbone(self, plan, input_ids, positions, forward_batch, input_embeds):
        """The embedding and dense layers on SGLang's path; a fully bound layer as its
        four launches; any other covered layer's attention half on its module and its
        FFN half as one launch."""
        m = self.lm.model
        hidden = m.embed_tokens(input_ids) if input_embeds is None else input_embeds
        st = self.step(plan, positions, forward_batch)
        for i, layer in enumerate(m.layers):
            L = self.layers.get(i)
            if L is None:
                hidden = layer(positions, hidden, forward_batch)
            elif L.full:
                hidden = L.op.launch(hidden.contiguous(), self._caches(L, forward_batch),
                                     self._layer_step(st, forward_batch, plan.key.rows))
            else:
                a = layer.attention_half(positions, hidden, forward_batch)
                hidden = L.op.launch(a.contiguous())
        return m.norm(hidden)

    @staticmethod
    def _caches(L, forward_batch):
        """The layer's caches in SGLang's pool, bound once (rebound if the pool moved)."""
        from .binding import caches

        pool = forward_batch.token_to_kv_pool
        if getattr(pool, "page_size", 64) != 64:
            raise RuntimeError(f"KV pool page size {pool.page_size}: the launches' pages hold 64")
        kv = pool.get_key_buffer(L.i)
        if L.caches is None or L.caches.kv.data_ptr() != kv.data_ptr():
            if L.kv_scale is None or L.kv_scale.numel() * kv.shape[-1] != kv.numel():
                L.kv_scale = torch.ones(kv.numel() // kv.shape[-1], dtype=torch.float32,
                                        device=kv.device)
            L.caches = caches(pool, L.i, L.kv_scale)
        return L.caches

    @staticmethod
    def _layer_step(st, forward_batch, rows: int):
        """The launches' row tables from the step's: a row's page table is its request's
        slots at every 64th position, as page ids."""
        from .layer import LayerStep

        if st.page_table.shape[0] < rows:
            raise RuntimeError("the step has no page table: fill_step(page_table=...) first")
        return LayerStep(positions=st.positions[:rows], slots=st.slots[:rows],
                         req_ids=st.req_ids[:rows], page_table=st.page_table)


def _build(model, hf_config, ctx):
    """The launches of every covered layer, over SGLang's loaded weights in place."""
    from sglang.srt.runtime_context import get_parallel

    from ..guard import watchdog_deadline
    from .attn import MAX_CTX
    from .binding import layer_weights, moe_weights
    from .front import FRONT_MAX_ROWS
    from .layer import LayerOp
    from .moe import MoeFp8Op

    p = get_parallel()
    if p.tp_size > 1:
        raise ValueError(
            f"the DSA monokernel computes one GPU's TP share, but its TP exchanges are "
            f"not built: TP {p.tp_size} would serve unreduced partials")
    deadline = watchdog_deadline(getattr(ctx, "deadline_s", 120.0) * 2)
    context_len = getattr(ctx, "context_len", 163840)
    copies = getattr(ctx, "copies", None)
    copies = {} if copies is None else copies
    layers = {}
    plans = plan_layers(model, hf_config)
    if context_len > MAX_CTX:  # the attention launch's score rows end at MAX_CTX keys
        plans = {i: f"context {context_len} > {MAX_CTX}" for i in plans}
    for i, why in plans.items():
        mod = model.model.layers[i]
        if why is None:
            w = layer_weights(mod, i, copies)
            op = LayerOp(w, w.moe.w13.device, max_rows=FRONT_MAX_ROWS, ctx_max=context_len,
                         deadline_s=deadline)
            layers[i] = _Layer(i, mod, op, full=True)
        else:
            w = moe_weights(mod)
            op = MoeFp8Op(w, w.w13.device, max_rows=MAX_ROWS, deadline_s=deadline)
            layers[i] = _Layer(i, mod, op)
    device = next(iter(layers.values())).op.device
    full = any(L.full for L in layers.values())
    return _Built(model, layers, device, context_len=context_len,
                  max_rows=FRONT_MAX_ROWS if full else MAX_ROWS)


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
