"""Check mode (SGLANG_AMD_MONO_CHECK=1) on the CPU with SGLang-shaped stand-ins: SGLang's
layer runs on a copy of the rows, its top-k is re-routed in f32 as the launch routes
(plain and group-limited, against the oracle's router), the cache rows it wrote are put
back, and the comparison logs each value and every bound missed."""

import logging
from collections import namedtuple
from types import SimpleNamespace as NS

import numpy as np
import torch

from oracle import moe as om
from tests import fake_sglang

fake_sglang.install()

from sgl_amd_mono_amd.dsv32 import check  # noqa: E402
from sgl_amd_mono_amd.dsv32.config import DSV32  # noqa: E402

TopK = namedtuple("TopK", "topk_weights topk_ids")


class _TopK(torch.nn.Module):
    """SGLang's fused top-k as a stand-in: routes in bf16 (a different answer than f32 on
    near ties), with the shared expert appended as id 256."""

    def forward(self, x, logits, bias):
        s = torch.sigmoid(logits.float())
        choice = (s.bfloat16() + bias.bfloat16()).float()
        ids = choice.topk(8, -1).indices
        w = s.gather(1, ids)
        ids = torch.cat([ids, torch.full_like(ids[:, :1], 256)], 1)
        w = torch.cat([w, torch.ones_like(w[:, :1])], 1)
        return TopK(topk_weights=w, topk_ids=ids)


class _Mlp(torch.nn.Module):
    def __init__(self, g):
        super().__init__()
        self.gate = torch.nn.Module()
        self.gate.weight = torch.nn.Parameter(torch.randn(256, 64, generator=g))
        self.gate.e_score_correction_bias = torch.nn.Parameter(0.1 * torch.randn(256, generator=g))
        self.topk = _TopK()
        self.routed = None

    def forward(self, x):
        out = self.topk(x, x.float() @ self.gate.weight.float().t(), self.gate.e_score_correction_bias)
        self.routed = out.topk_ids
        return x * 2.0


class _Layer(torch.nn.Module):
    """A decoder layer stand-in: writes its KV row and index page at the step's slots,
    runs its MLP, returns (stream, top-k slots)."""

    def __init__(self, g, pool, i):
        super().__init__()
        self.mlp, self.pool, self.i = _Mlp(g), pool, i

    def forward(self, positions, hidden, fb, zeros, gemm_zeros, residual, prev_topk_indices=None):
        loc = fb.out_cache_loc.long()
        self.pool.get_key_buffer(self.i).view(-1, 4)[loc] = 7
        self.pool.get_index_k_fp4_payload_buffer(self.i)[loc // 64] = 9
        y = self.mlp(hidden)
        return y + 1.0, torch.arange(4)[None].repeat(hidden.shape[0], 1)


class _Pool:
    def __init__(self):
        self.kv = torch.zeros(256, 1, 4, dtype=torch.uint8)
        self.pay = torch.zeros(4, 1, 4, 64, 16, dtype=torch.uint8)
        self.sc = torch.zeros(4, 1, 4, 64, dtype=torch.uint8)

    def get_key_buffer(self, i):
        return self.kv

    def get_index_k_fp4_payload_buffer(self, i):
        return self.pay

    def get_index_k_fp4_scale_buffer(self, i):
        return self.sc


def test_f32_router_matches_the_oracle_plain_and_grouped():
    g = torch.Generator().manual_seed(3)
    mlp = _Mlp(g)
    x = torch.randn(6, 64, generator=g)
    for n_group, topk_group in ((1, 1), (8, 4), (4, 1)):
        ids, w = check._f32_topk(x, mlp, 8, n_group, topk_group, 2.5)
        scores = torch.sigmoid(x.float() @ mlp.gate.weight.detach().float().t())
        want, want_w = om.route_topk(scores, mlp.gate.e_score_correction_bias.detach(),
                                     n_group=n_group, topk_group=topk_group)
        assert np.array_equal(ids.numpy(), want), (n_group, topk_group)
        np.testing.assert_allclose(w.detach().numpy(), want_w, rtol=1e-6)


def test_reference_runs_the_layer_routes_in_f32_and_restores_the_caches():
    g = torch.Generator().manual_seed(4)
    pool = _Pool()
    pool.kv.view(-1, 4)[:] = 1
    layer = _Layer(g, pool, 5)
    fb = NS(out_cache_loc=torch.tensor([3, 70, 130]), pending=None, written=False)
    h = torch.randn(3, 64, generator=g)
    cfg = DSV32
    ref = check.reference(NS(i=5, module=layer), torch.arange(3), h, fb, 3, cfg, pool)
    assert torch.equal(ref["out"], h * 2.0 + 1.0)
    ids, _ = check._f32_topk(h, layer.mlp, 8, 1, 1, 2.5)
    assert torch.equal(ref["ids"], ids)
    # SGLang's routing was replaced by the f32 one (the shared column kept)
    assert torch.equal(layer.mlp.routed[:, :8], ids) and torch.all(layer.mlp.routed[:, 8] == 256)
    # the KV rows and index pages it wrote are back as they were
    assert torch.all(pool.kv == 1) and torch.all(pool.pay == 0)


def test_compare_logs_values_and_violations(caplog):
    L = NS(i=7)
    b = torch.randn(4, 32)
    ref = {"out": b, "ids": torch.arange(32).view(4, 8), "topk": torch.tensor([[1, 2, -1]] * 4)}
    bounds = {"layer.out.max_abs": 2e-2, "layer.out.rel": 1e-2, "router.ids.mismatch": 0.0,
              "indexer.topk.mismatch": 0.0}
    with caplog.at_level(logging.INFO, logger=check.__name__):
        v = check.compare(L, b + 1e-4, ref, 4, ids=torch.arange(32).view(4, 8),
                          topk_slots=torch.tensor([[2, 1, -1]] * 4), numerics=bounds)
    assert v["router.ids.mismatch"] == 0.0 and v["indexer.topk.mismatch"] == 0.0
    assert v["layer.out.rel"] < 1e-3
    assert not [r for r in caplog.records if r.levelno >= logging.ERROR]
    caplog.clear()
    bad_ids = torch.arange(32).view(4, 8).clone()
    bad_ids[1, 0] = 99
    with caplog.at_level(logging.INFO, logger=check.__name__):
        v = check.compare(L, b + 0.5, ref, 4, ids=bad_ids,
                          topk_slots=torch.tensor([[1, 5, -1]] * 4), numerics=bounds)
    assert v["router.ids.mismatch"] == 0.25 and v["indexer.topk.mismatch"] == 0.5
    errors = " ".join(r.getMessage() for r in caplog.records if r.levelno >= logging.ERROR)
    for name in bounds:
        assert name in errors, name


def test_check_mode_reads_its_variable(monkeypatch):
    monkeypatch.delenv("SGLANG_AMD_MONO_CHECK", raising=False)
    assert not check.enabled()
    monkeypatch.setenv("SGLANG_AMD_MONO_CHECK", "1")
    assert check.enabled()
