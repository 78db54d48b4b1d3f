"""The plugin surface on CPU: registration under backend "amd", refusal reasons, the
step tables against the reference's known answers, and routing by the graph key."""

import json
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

from tests import fake_sglang

registry = fake_sglang.install()

import sgl_amd_mono_amd  # noqa: E402
from sgl_amd_mono_amd.dsv32 import spec as dsv32  # noqa: E402
from sgl_amd_mono_amd.dsv32.runner import TOPK, alloc_step, fill_step, take_topk  # noqa: E402

GOLDEN = json.loads((Path(__file__).parent / "golden" / "step_tables.json").read_text())
V32 = SimpleNamespace(
    **dsv32.HF_CONFIG,
    num_hidden_layers=61,
    first_k_dense_replace=3,
    quantization_config={"quant_method": "fp8", "weight_block_size": [128, 128]},
    architectures=["DeepseekV32ForCausalLM"],
)
CFG = SimpleNamespace(speculative_algorithm=None)


def test_the_plugin_registers_the_spec_under_amd():
    sgl_amd_mono_amd.register_specs()
    found, why = registry.find_spec(backend=sgl_amd_mono_amd.BACKEND,
                                    architectures=["DeepseekV32ForCausalLM"], isa="gfx950")
    assert found is dsv32.SPEC, why
    found, why = registry.find_spec(backend="amd", architectures=["DeepseekV32ForCausalLM"],
                                    isa="gfx942")
    assert found is None and "gfx942" in why
    assert dsv32.SPEC.devices["gfx950"].resident_blocks == 256
    assert dsv32.SPEC.numerics.bound("moe.out.max_abs") == 2e-2


def test_the_forward_covers_the_moe_layers():
    assert dsv32.covered_layers(V32) == list(range(3, 61))


def test_config_reasons_name_each_mismatch():
    assert dsv32._config_disable_reasons(CFG, V32) == []
    other = SimpleNamespace(**{**vars(V32), "hidden_size": 6144, "n_routed_experts": 160})
    reasons = dsv32._config_disable_reasons(CFG, other)
    assert any("hidden_size" in r for r in reasons) and any("n_routed_experts" in r for r in reasons)
    bf = SimpleNamespace(**{**vars(V32), "quantization_config": None})
    assert any("FP8" in r for r in dsv32._config_disable_reasons(CFG, bf))
    mtp = SimpleNamespace(speculative_algorithm="EAGLE")
    assert any("decode rows only" in r for r in dsv32._config_disable_reasons(mtp, V32))


@pytest.mark.parametrize("case", GOLDEN["cases"], ids=[c["name"] for c in GOLDEN["cases"]])
def test_each_row_attends_the_keys_up_to_its_position(case):
    st = alloc_step(4, "cpu")
    fill_step(st, torch.tensor(case["positions"]), torch.tensor(case["slots"]), 4,
              case["context_len"] - 1)
    assert st.positions.tolist() == case["want_positions"]
    assert st.indptr.tolist() == case["want_indptr"]
    want_slots = [s if s != 0 else -1 for s in case["slots"]]
    assert st.slots.tolist() == want_slots


def test_a_short_step_pads_the_width():
    st = alloc_step(4, "cpu")
    fill_step(st, torch.tensor([5, 9]), torch.tensor([40, 41]), 2, 100)
    assert st.indptr.tolist() == [0, 6, 16, 16, 16]
    assert st.slots.tolist() == [40, 41, -1, -1]
    with pytest.raises(ValueError):
        fill_step(st, torch.tensor([1] * 5), torch.tensor([1] * 5), 5, 100)


def test_take_topk_packs_rows_at_their_indptr():
    st = alloc_step(2, "cpu")
    fill_step(st, torch.tensor([2, 3000]), torch.tensor([7, 8]), 2, 10**6)
    src = torch.full((2, TOPK), -1, dtype=torch.int64)
    src[0, :3] = torch.tensor([11, 12, 13])
    src[1] = torch.arange(TOPK) + 100
    take_topk(st, src, 2)
    assert st.topk[:3].tolist() == [11, 12, 13]
    assert st.topk[3:3 + TOPK].tolist() == list(range(100, 100 + TOPK))


class _Lm:
    """A model whose own forward records that it ran."""

    def __init__(self):
        self.model, self.ran = SimpleNamespace(), []

    def forward(self, *args):
        self.ran.append(args)
        return "the model's forward"


def test_a_step_wider_than_the_built_rows_runs_the_model():
    lm = _Lm()
    built = dsv32._Built(lm, {}, "cpu", context_len=4096)
    key = registry.ShapeKey(forward_mode="decode", batch_size=17, tokens_per_request=1)
    assert built.forward(registry.Plan(key=key), "ids", "positions", "batch") == "the model's forward"
    assert lm.ran == [("ids", "positions", "batch", None, None)]
    assert [dsv32._width(r) for r in (1, 5, 16)] == [1, 5, 16]


def test_build_refuses_tp_above_one(monkeypatch):
    monkeypatch.setattr(fake_sglang, "PARALLEL", SimpleNamespace(tp_size=4, tp_rank=0))
    import sys
    sys.modules["sglang.srt.runtime_context"].get_parallel = lambda: fake_sglang.PARALLEL
    with pytest.raises(ValueError, match="TP exchanges are not built"):
        dsv32._build(SimpleNamespace(), V32, SimpleNamespace())
