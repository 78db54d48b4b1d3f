"""The plugin surface on CPU: registration under backend "amd", refusal reasons, the
step tables against the reference's known answers, routing by the graph key, and the
backbone's residual hand-over through SGLang's layer-boundary API (SGLang-shaped fakes)."""

import json
import math
from pathlib import Path
from types import SimpleNamespace as NS

import pytest
import torch

from tests import fake_sglang

registry = fake_sglang.install()

import sgl_amd_mono_amd  # noqa: E402
from sgl_amd_mono_amd.dsv32 import spec as dsv32  # noqa: E402
from sgl_amd_mono_amd.dsv32.runner import StepRows  # noqa: E402

GOLDEN = json.loads((Path(__file__).parent / "golden" / "step_tables.json").read_text())
# a model whose TP-1 shapes are one GPU's TP=4 share of DeepSeek-V3.2
MODEL = NS(
    **dsv32.HF_CONFIG,
    num_hidden_layers=61,
    first_k_dense_replace=3,
    max_position_embeddings=32768,
    quantization_config={"quant_method": "fp8", "weight_block_size": [128, 128]},
    architectures=["DeepseekV32ForCausalLM"],
)
SERVER = NS(speculative_algorithm=None, tp_size=1, page_size=64, context_length=None)


def _with(obj, **kw):
    return NS(**{**vars(obj), **kw})


def test_the_plugin_registers_the_spec_under_amd():
    sgl_amd_mono_amd.register_specs()
    found, why = registry.find_spec(backend=sgl_amd_mono_amd.BACKEND,
                                    architectures=["DeepseekV32ForCausalLM"], isa="gfx950")
    assert found is dsv32.SPEC, why
    found, why = registry.find_spec(backend="amd", architectures=["DeepseekV32ForCausalLM"],
                                    isa="gfx942")
    assert found is None and "gfx942" in why
    limits = dsv32.SPEC.devices["gfx950"]
    assert limits.resident_blocks == 256 and limits.tp_sizes == (1,)
    assert limits.widths == tuple(range(1, 9))
    assert dsv32.SPEC.numerics.bound("layer.out.max_abs") == 2e-2


def test_the_forward_covers_the_moe_layers():
    assert dsv32.covered_layers(MODEL) == list(range(3, 61))


def test_a_served_config_has_no_reasons():
    assert dsv32._config_disable_reasons(SERVER, MODEL) == []


@pytest.mark.parametrize("change, words", [
    (dict(hidden_size=6144), "hidden_size"),
    (dict(num_attention_heads=128), "num_attention_heads"),
    (dict(n_group=3, topk_group=1), "n_group 3"),
    (dict(n_group=8, topk_group=9), "n_group 8"),
    (dict(n_group=32, topk_group=4), "n_group 32"),
    (dict(indexer_rope_interleave=False), "indexer_rope_interleave"),
    (dict(rope_interleave=False), "interleaved pairs"),
    (dict(rope_scaling={"rope_type": "linear", "factor": 4.0}), "RoPE 'linear'"),
    (dict(quantization_config=None), "FP8 checkpoint"),
    (dict(max_position_embeddings=262144), "context 262144"),
])
def test_config_reasons_name_each_mismatch(change, words):
    reasons = dsv32._config_disable_reasons(SERVER, _with(MODEL, **change))
    assert any(words in r for r in reasons), reasons


@pytest.mark.parametrize("change, words", [
    (dict(tp_size=4), "TP 4"),
    (dict(page_size=16), "--page-size 16"),
    (dict(speculative_algorithm="EAGLE"), "decode rows only"),
    (dict(context_length=200000), "context 200000"),
])
def test_server_reasons_are_reasons_not_exceptions(change, words):
    reasons = dsv32._config_disable_reasons(_with(SERVER, **change), MODEL)
    assert any(words in r for r in reasons), reasons


def test_a_shorter_served_context_is_accepted():
    long = _with(MODEL, max_position_embeddings=262144)
    assert dsv32._config_disable_reasons(_with(SERVER, context_length=163840), long) == []


def test_yarn_scales_the_softmax_by_mscale_squared():
    """DeepSeek-V3.2's YaRN (factor 40, mscale_all_dim 1): SGLang's MLA scales the
    softmax by (0.1 ln 40 + 1)^2 = 1.8738 on top of 192^-1/2; plain RoPE keeps 192^-1/2."""
    yarn = _with(MODEL, rope_scaling={"type": "yarn", "factor": 40, "mscale": 1.0,
                                      "mscale_all_dim": 1.0,
                                      "original_max_position_embeddings": 4096})
    assert dsv32._config_disable_reasons(SERVER, yarn) == []
    base = 192 ** -0.5
    assert dsv32.softmax_scale(MODEL) == pytest.approx(base, rel=1e-15)
    m = 0.1 * math.log(40.0) + 1.0
    assert dsv32.softmax_scale(yarn) == pytest.approx(base * m * m, rel=1e-12)
    assert dsv32.softmax_scale(yarn) / base == pytest.approx(1.8738, abs=1e-4)


@pytest.mark.parametrize("case", GOLDEN["cases"], ids=[c["name"] for c in GOLDEN["cases"]])
def test_each_row_attends_the_keys_up_to_its_position(case):
    st = StepRows.empty(4, "cpu")
    st.write(torch.tensor(case["positions"]), torch.tensor(case["slots"]), 4,
             case["context_len"] - 1)
    assert st.positions.tolist() == case["want_positions"]
    assert st.indptr().tolist() == case["want_indptr"]
    assert st.slots.tolist() == [s if s != 0 else -1 for s in case["slots"]]


def test_a_short_step_pads_the_width():
    st = StepRows.empty(4, "cpu")
    st.write(torch.tensor([5, 9]), torch.tensor([40, 41]), 2, 100)
    assert st.indptr().tolist() == [0, 6, 16, 16, 16]
    assert st.slots.tolist() == [40, 41, -1, -1]
    assert st.req_ids.tolist() == [0, 1, 0, 0]
    # a narrower step after a wider one leaves nothing of the wider one behind
    st.write(torch.tensor([3, 4, 5, 6]), torch.tensor([1, 2, 3, 4]), 4, 100)
    st.write(torch.tensor([7]), torch.tensor([9]), 1, 100)
    assert st.positions.tolist() == [7, 0, 0, 0] and st.slots.tolist() == [9, -1, -1, -1]
    assert st.indptr().tolist() == [0, 8, 8, 8, 8]
    with pytest.raises(ValueError):
        st.write(torch.tensor([1] * 5), torch.tensor([1] * 5), 5, 100)


class _Lm:
    """A model whose own forward records that it ran."""

    def __init__(self):
        self.model, self.ran = NS(), []

    def forward(self, *args):
        self.ran.append(args)
        return "the model's forward"


def test_a_step_wider_than_the_built_rows_runs_the_model():
    lm = _Lm()
    built = dsv32._Built(lm, {}, "cpu", context_len=4096)
    key = registry.ShapeKey(forward_mode="decode", batch_size=9, tokens_per_request=1)
    assert built.forward(registry.Plan(key=key), "ids", "positions", "batch") == "the model's forward"
    assert lm.ran == [("ids", "positions", "batch", None, None)]
    assert [dsv32._width(r) for r in (1, 5, 8)] == [1, 5, 8]


class _DenseLayer:
    """SGLang's decoder layer as the backbone calls it: (positions, hidden, batch, zero
    allocators, ...) -> (output, top-k), with the residual add left pending."""

    def __init__(self, k):
        self.k, self.calls = k, []

    def __call__(self, positions, hidden, fb, zeros, gemm_zeros, _, prev_topk_indices=None,
                 next_full_attention_layer_id=None):
        assert isinstance(zeros, fake_sglang.BumpAllocator)
        x = fake_sglang.fold(hidden, fb)
        self.calls.append(x.clone())
        fb.pending = x
        return x * self.k, "topk"


class _Op:
    """A layer launch stand-in: records its input and returns h * k + 1."""

    def __init__(self, k):
        self.k, self.seen = k, []

    def launch(self, h, caches, step):
        self.seen.append((h.clone(), caches, step))
        return h * self.k + 1


def _model(dense, covered, width_rows=8):
    layers = [_DenseLayer(k) for k in dense] + [NS() for _ in covered]
    m = NS(embed_tokens=lambda ids: ids.to(torch.bfloat16)[:, None].expand(-1, 7168).clone(),
           start_layer=0, end_layer=len(layers), layers=layers,
           next_full_attention_layer_id={}, norm=lambda x: x * 0.5,
           gemm_output_zero_allocator_size=0)
    lm = NS(model=m, lm_head="head",
            logits_processor=lambda ids, hidden, head, fb, aux: hidden)
    ops = {len(dense) + j: _Op(k) for j, k in enumerate(covered)}
    built = dsv32._Built(lm, {i: dsv32._Layer(i, layers[i], op) for i, op in ops.items()}, "cpu",
                         context_len=4096)
    return built, lm, ops


def _batch(rows, table_pages=64):
    """A decode batch: request r at pool row 2 r, its KV slots r * 4096 + position (64
    pages of 64), the attention backend's page table ``table_pages`` wide (the served
    context of ``_model`` is 4096 keys: 64 pages)."""
    pool = NS(get_key_buffer=lambda i: torch.zeros(64, 1, 576, dtype=torch.uint8))
    req_to_token = torch.zeros(2 * rows, 4096, dtype=torch.int32)
    for r in range(rows):
        req_to_token[2 * r] = r * 4096 + torch.arange(4096, dtype=torch.int32)
    real = (torch.arange(rows, dtype=torch.int32)[:, None] * 64
            + torch.arange(table_pages, dtype=torch.int32)[None])
    md = NS(real_page_table=real)
    return NS(out_cache_loc=torch.arange(1, rows + 1) * 3, token_to_kv_pool=pool,
              attn_backend=NS(forward_metadata=md), forward_mode=NS(is_idle=lambda: False),
              req_to_token_pool=NS(req_to_token=req_to_token),
              req_pool_indices=torch.arange(rows) * 2)


def test_the_backbone_hands_the_full_stream_to_the_first_launch(monkeypatch):
    """Dense layers x2 and x3 (each leaving its residual add pending), then launches
    h*5+1 and h*7+1: the first launch gets the folded stream (layer 0: 2x, pending x;
    layer 1 folds 3x, outputs 9x, pending 3x: 12x), the next one the previous launch's
    output, and the last hands back a written stream that the final norm halves with no
    residual added again."""
    from sgl_amd_mono_amd.dsv32 import binding

    monkeypatch.setattr(binding, "caches", lambda pool, i: ("caches", i))
    built, lm, ops = _model([2, 3], [5, 7])
    rows = 3
    ids = torch.tensor([1, 2, 3])
    fb = _batch(rows)
    plan = registry.Plan(key=registry.ShapeKey("decode", rows, 1))
    out = built.forward(plan, ids, torch.tensor([10, 20, 30]), fb)
    x = ids.float()[:, None]
    # layer 0: out 2x, pending x; layer 1 folds: x1 = 2x + x = 3x, out 9x, pending 3x
    full = 9 * x + 3 * x  # the stream the first launch must see
    h0, caches0, step0 = ops[2].seen[0]
    assert h0.shape == (3, 7168)  # width 3: no pad rows
    assert torch.equal(h0.float(), full.expand(-1, 7168))
    assert caches0 == ("caches", 2)
    assert step0.positions.tolist() == [10, 20, 30] and step0.slots.tolist() == [3, 6, 9]
    assert step0.page_table.shape == (3, 64)
    assert step0.page_table.data_ptr() == fb.attn_backend.forward_metadata.real_page_table.data_ptr()
    h1, _, _ = ops[3].seen[0]
    first = full.to(torch.bfloat16) * 5 + 1  # the launches' bf16 arithmetic
    assert torch.equal(h1, first.expand(-1, 7168))
    want = (first * 7 + 1) * 0.5
    assert torch.equal(out, want.expand(-1, 7168))
    assert fb.written


def test_a_narrow_step_runs_at_the_next_width_with_pad_rows(monkeypatch):
    from sgl_amd_mono_amd.dsv32 import binding

    monkeypatch.setattr(binding, "caches", lambda pool, i: None)
    monkeypatch.setattr(dsv32, "WIDTHS", (1, 2, 4, 8))
    built, _, ops = _model([2], [5])
    built.steps = {w: StepRows.empty(w, "cpu") for w in (1, 2, 4, 8)}
    built.pad_h = {w: torch.full((w, 7168), 9.0, dtype=torch.bfloat16) for w in (1, 2, 4, 8)}
    fb = _batch(3)
    plan = registry.Plan(key=registry.ShapeKey("decode", 3, 1))
    out = built.forward(plan, torch.tensor([1, 2, 3]), torch.tensor([4, 5, 6]), fb)
    h, _, step = ops[1].seen[0]
    assert h.shape == (4, 7168) and torch.all(h[3] == 0)  # the pad row is zeroed
    assert step.slots.tolist() == [3, 6, 9, -1]
    assert out.shape == (3, 7168)


def _fake_build(monkeypatch, mixed=()):
    """``_build`` with the binding and launches replaced by stand-ins (CPU): records the
    runtimes made and the ops' arguments; layers in ``mixed`` refuse the one launch."""
    from sgl_amd_mono_amd.dsv32 import binding, layer

    made = []

    class _Rt:
        def __init__(self, device, max_rows, deadline_s):
            self.device = torch.device("cpu")
            made.append(("layer", max_rows))

    class _Rts:
        def __init__(self, device, cfg, max_rows, ctx_max, deadline_s):
            self.device = torch.device("cpu")
            made.append(("chain", max_rows, ctx_max))

    class _Fused:
        def __init__(self, w, device, cfg, max_rows, ctx_max, sm_scale, fault, rt):
            if w.i in mixed:
                raise ValueError("one FP8 layout for the whole layer")
            self.w, self.rt, self.sm_scale, self.fault = w, rt, sm_scale, fault
            self.ctx_max, self.cfg = ctx_max, cfg

    class _LayerOp:
        def __init__(self, w, rts, cfg, sm_scale):
            self.w, self.rts, self.sm_scale, self.cfg = w, rts, sm_scale, cfg

    monkeypatch.setattr(binding, "layer_weights",
                        lambda mod, i, copies, rope=None: NS(moe=NS(w13=NS(device="cpu")), i=i,
                                                             rope=rope))
    monkeypatch.setattr(binding, "rope_table", lambda layers, copies: ("cos", "sin"))
    monkeypatch.setattr(layer, "layer_runtime", _Rt)
    monkeypatch.setattr(layer, "LayerRuntimes", _Rts)
    monkeypatch.setattr(layer, "FusedLayerOp", _Fused)
    monkeypatch.setattr(layer, "LayerOp", _LayerOp)
    return made, _Fused, _LayerOp


def test_build_reads_each_layer_and_scales_the_softmax(monkeypatch):
    """``_build`` binds every covered layer as one launch, all on one shared runtime, with
    the model's softmax scale and the served context bound."""
    made, fused, _ = _fake_build(monkeypatch)
    cfg = _with(MODEL, num_hidden_layers=6, rope_scaling={"type": "yarn", "factor": 40,
                                                           "mscale_all_dim": 1.0})
    model = NS(model=NS(layers=[NS() for _ in range(6)]))
    built = dsv32._build(model, cfg, NS(context_len=8192, deadline_s=30.0))
    assert sorted(built.layers) == [3, 4, 5] and made == [("layer", 8)]
    ops = [built.layers[i].op for i in (3, 4, 5)]
    assert all(isinstance(op, fused) for op in ops)
    assert ops[0].rt is ops[1].rt is ops[2].rt
    assert all(op.sm_scale == dsv32.softmax_scale(cfg) for op in ops)
    assert all(op.ctx_max == 8192 and op.fault == (0, 0) for op in ops)
    assert built.max_position == 8191


def test_build_falls_back_to_four_launches_for_mixed_layouts(monkeypatch):
    """A layer whose FP8 projections SGLang left in two layouts runs as the four
    launches (each reads its own struct's layout) on one shared set of their runtimes."""
    made, fused, chain = _fake_build(monkeypatch, mixed=(4, 5))
    model = NS(model=NS(layers=[NS() for _ in range(6)]))
    cfg = _with(MODEL, num_hidden_layers=6)
    built = dsv32._build(model, cfg, NS(context_len=4096, deadline_s=30.0))
    assert isinstance(built.layers[3].op, fused)
    assert isinstance(built.layers[4].op, chain) and isinstance(built.layers[5].op, chain)
    assert built.layers[4].op.rts is built.layers[5].op.rts
    assert made == [("layer", 8), ("chain", 8, 4096)]


def test_build_arms_the_fault_injection_of_its_rank(monkeypatch):
    """SGLANG_AMD_MONO_FAULT_INJECT=rank:site:after reaches the launches of that rank."""
    _, _, _ = _fake_build(monkeypatch)
    monkeypatch.setenv("SGLANG_AMD_MONO_FAULT_INJECT", "0:5:3")
    model = NS(model=NS(layers=[NS() for _ in range(6)]))
    built = dsv32._build(model, _with(MODEL, num_hidden_layers=6),
                         NS(context_len=4096, deadline_s=30.0))
    assert all(built.layers[i].op.fault == (5, 3) for i in (3, 4, 5))
    monkeypatch.setenv("SGLANG_AMD_MONO_FAULT_INJECT", "1:5:3")
    built = dsv32._build(model, _with(MODEL, num_hidden_layers=6),
                         NS(context_len=4096, deadline_s=30.0))
    assert all(built.layers[i].op.fault == (0, 0) for i in (3, 4, 5))


def test_group_limited_routing_is_served_and_reaches_the_launches(monkeypatch):
    """DeepSeek-V3.2's own router (n_group 8, topk_group 4) is accepted, and every covered
    layer's launch routes with it."""
    _, _, _ = _fake_build(monkeypatch)
    real = _with(MODEL, n_group=8, topk_group=4, num_hidden_layers=6)
    assert dsv32._config_disable_reasons(SERVER, real) == []
    model = NS(model=NS(layers=[NS() for _ in range(6)]))
    built = dsv32._build(model, real, NS(context_len=4096, deadline_s=30.0))
    assert all((built.layers[i].op.cfg.n_group, built.layers[i].op.cfg.topk_group) == (8, 4)
               for i in (3, 4, 5))


def test_check_mode_runs_sglang_first_and_compares(monkeypatch):
    """SGLANG_AMD_MONO_CHECK=1: each covered launch of an eager step is preceded by
    SGLang's layer on the same rows (``check.reference``) and compared with it."""
    from sgl_amd_mono_amd.dsv32 import binding, check

    monkeypatch.setattr(binding, "caches", lambda pool, i: ("caches", i))
    monkeypatch.setenv("SGLANG_AMD_MONO_CHECK", "1")
    calls = []

    def reference(L, positions, h_rows, fb, S, cfg, pool):
        calls.append(("ref", L.i, tuple(h_rows.shape)))
        return {"out": h_rows * 5 + 1, "ids": None, "topk": None}

    def compare(L, got, ref, S, *, ids=None, topk_slots=None, numerics=None):
        calls.append(("cmp", L.i, float((got.float() - ref["out"].float()).abs().max())))
        assert set(numerics) == set(dsv32.NUMERICS.bounds)
        return {}

    monkeypatch.setattr(check, "reference", reference)
    monkeypatch.setattr(check, "compare", compare)
    built, lm, ops = _model([2], [5, 7])
    assert built.check
    fb = _batch(3)
    plan = registry.Plan(key=registry.ShapeKey("decode", 3, 1))
    built.forward(plan, torch.tensor([1, 2, 3]), torch.tensor([10, 20, 30]), fb)
    # layer 1's launch is h*5+1: its comparison finds no difference; layer 2's is h*7+1
    assert [c[:2] for c in calls] == [("ref", 1), ("cmp", 1), ("ref", 2), ("cmp", 2)]
    assert calls[1][2] == 0.0 and calls[3][2] > 0.0


def test_a_page_table_narrower_than_the_context_is_rebuilt_full_width(monkeypatch):
    """The DSA backend sizes ``real_page_table`` by the batch's longest sequence. One
    narrower than the served context (4096 keys: 64 pages) is not read in place: the step
    fills its own full-width table from ``req_to_token`` (request r's page p is
    r * 64 + p), and the launch's page-table checks see every page of the context."""
    from sgl_amd_mono_amd.dsv32 import binding
    from sgl_amd_mono_amd.dsv32.layer import FusedLayerOp

    monkeypatch.setattr(binding, "caches", lambda pool, i: ("caches", i))
    built, _, ops = _model([2], [5])
    fb = _batch(3, table_pages=2)
    plan = registry.Plan(key=registry.ShapeKey("decode", 3, 1))
    built.forward(plan, torch.tensor([1, 2, 3]), torch.tensor([10, 20, 30]), fb)
    _, _, step = ops[1].seen[0]
    pt = step.page_table
    assert pt.shape == (3, 64) and pt.dtype == torch.int32 and pt.stride(1) == 1
    want = torch.arange(3, dtype=torch.int32)[:, None] * 64 + torch.arange(64, dtype=torch.int32)
    assert torch.equal(pt, want)
    assert pt.data_ptr() != fb.attn_backend.forward_metadata.real_page_table.data_ptr()
    # the one launch's argument check: a table of 2 pages a request is refused, the
    # rebuilt one passes the width check (it stops at the device, this is the CPU)
    op = FusedLayerOp.__new__(FusedLayerOp)
    op.cfg, op.device, op.max_rows, op.ctx_max = dsv32.DSV32, torch.device("cpu"), 8, 4096
    op.w = None
    h = torch.zeros(3, 7168, dtype=torch.bfloat16)
    from sgl_amd_mono_amd.dsv32.layer import LayerStep
    narrow = LayerStep(positions=step.positions[:3], slots=step.slots[:3],
                       req_ids=step.req_ids[:3],
                       page_table=fb.attn_backend.forward_metadata.real_page_table)
    with pytest.raises(ValueError, match="cannot hold"):
        op.launch(h, None, narrow)
    wide = LayerStep(positions=step.positions[:3], slots=step.slots[:3],
                     req_ids=step.req_ids[:3], page_table=pt)
    with pytest.raises(AttributeError):  # past the page-table check: the caches (None)
        op.launch(h, None, wide)
