"""DeepSeek-V3.2 (DSA) on gfx950: the monokernel spec SGLang routes decode steps to.

The plugin surface of ``sgl_amd_mono/glm53/spec.py:584-616``: a ``MonoSpec`` registered
under backend ``amd`` for the architecture, with device limits, requirements, numerics
bounds, config and model refusal reasons, and ``build(model, hf_config, ctx)``
returning an object whose ``forward(plan, input_ids, positions, forward_batch, ...)``
SGLang calls for a routed step. The forward decides by the graph key alone
(``plan.key.rows`` against the widths built), so every rank and every graph replay makes
the same choice; a wider step runs the model's own forward.

Each covered MoE layer runs its FFN half as one persistent launch (``MoeFp8Op``): the
post-attention RMSNorm, router, top-8 + shared expert, W8A8 experts and the residual
add, reading SGLang's loaded weights in place (no copy is made of the experts, the
router or the norm). The attention half still runs SGLang's module.

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
from .runner import alloc_step, fill_step

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
    """A covered layer: its SGLang module and its launch."""

    def __init__(self, i: int, module, op):
        self.i, self.module, self.op = i, module, op


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
            plan.state["step"] = fill_step(st, positions, forward_batch.out_cache_loc, S,
                                           self.max_position)
        return plan.state["step"]

    def _backbone(self, plan, input_ids, positions, forward_batch, input_embeds):
        """The embedding and dense layers on SGLang's path; each covered layer's
        attention half on its module, its FFN half as one launch."""
        m = self.lm.model
        hidden = m.embed_tokens(input_ids) if input_embeds is None else input_embeds
        self.step(plan, positions, forward_batch)
        for i, layer in enumerate(m.layers):
            L = self.layers.get(i)
            if L is None:
                hidden = layer(positions, hidden, forward_batch)
                continue
            a = layer.attention_half(positions, hidden, forward_batch)
            hidden = L.op.launch(a.contiguous())
        return m.norm(hidden)


def _build(model, hf_config, ctx):
    """The launches of every covered layer, over SGLang's loaded weights in place."""
    from sglang.srt.runtime_context import get_parallel

    from ..guard import watchdog_deadline
    from .moe import MoeFp8Op, MoeFp8Weights

    p = get_parallel()
    if p.tp_size > 1:
        raise ValueError(
            f"the DSA monokernel computes one GPU's TP share, but its TP exchanges are "
            f"not built: TP {p.tp_size} would serve unreduced partials")
    layers = {}
    for i in covered_layers(hf_config):
        mod = model.model.layers[i]
        ex = mod.mlp.experts
        w = MoeFp8Weights(
            g_post=mod.post_attention_layernorm.weight,
            w_r=mod.mlp.gate.weight,
            bias=mod.mlp.gate.e_score_correction_bias,
            w13=ex.w13_weight, s13=ex.w13_weight_scale_inv,
            w2=ex.w2_weight, s2=ex.w2_weight_scale_inv,
            layout="aiter16" if getattr(ex.w13_weight, "is_shuffled", False) else "rowmajor",
        )
        op = MoeFp8Op(w, w.w13.device, max_rows=MAX_ROWS,
                      deadline_s=watchdog_deadline(getattr(ctx, "deadline_s", 120.0) * 2))
        layers[i] = _Layer(i, mod, op)
    device = next(iter(layers.values())).op.device
    return _Built(model, layers, device, context_len=getattr(ctx, "context_len", 163840))


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
