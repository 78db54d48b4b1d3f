"""Check mode (SGLANG_AMD_MONO_CHECK=1) on the CPU with SGLang-shaped stand-ins: SGLang's
layer runs on a copy of the rows, its top-k is re-routed in f32 as the launch routes
(plain and group-limited, against the oracle's router), the cache rows it wrote are put
back, and the comparison logs each value and every bound missed."""

import logging
from collections import namedtuple
from dataclasses import replace
from types import SimpleNamespace as NS

import numpy as np
import pytest
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
        cfg = replace(DSV32, n_group=n_group, topk_group=topk_group)
        ids, w = check.route_f32(x, mlp.gate.weight.detach(),
                                 mlp.gate.e_score_correction_bias.detach(), cfg)
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
    ids, _ = check.route_f32(h, layer.mlp.gate.weight.detach(),
                             layer.mlp.gate.e_score_correction_bias.detach(), cfg)
    assert torch.equal(ref["ids"], ids)
    # SGLang's routing was replaced by the f32 one (the shared column kept), and its own
    # top-k module is back in place
    assert torch.equal(layer.mlp.routed[:, :8], ids) and torch.all(layer.mlp.routed[:, 8] == 256)
    assert isinstance(layer.mlp.topk, _TopK)
    # the KV rows and index pages it wrote are back as they were, and kept aside
    assert torch.all(pool.kv == 1) and torch.all(pool.pay == 0)
    assert torch.all(ref["written"]["kv"] == 7) and torch.all(ref["written"]["index"][0] == 9)


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


def test_f32_router_ties_go_to_the_lower_id_and_the_lower_group():
    """Equal candidates: the lower expert id wins; equal group values: the lower group."""
    cfg = replace(DSV32, n_group=8, topk_group=4)
    x = torch.zeros(1, 4)
    w = torch.zeros(256, 4)  # every score sigmoid(0) = 0.5
    bias = torch.zeros(256)
    ids, wt = check.route_f32(x, w, bias, replace(DSV32))
    assert ids.tolist() == [list(range(8))]
    assert torch.allclose(wt, torch.full((1, 8), 2.5 / 8))
    # groups 5 and 6 lifted equally: they stay, then the lowest two of the rest (0, 1)
    bias[5 * 32 + 3] = 0.25
    bias[6 * 32 + 7] = 0.25
    ids, _ = check.route_f32(x, w, bias, cfg)
    want = om.route_topk(torch.full((1, 256), 0.5), bias, n_group=8, topk_group=4)[0]
    assert ids.tolist() == want.tolist()
    assert set(ids[0].tolist()) >= {5 * 32 + 3, 6 * 32 + 7}


def _fp4_pool(seed):
    g = torch.Generator().manual_seed(seed)
    pay = torch.randint(0, 256, (3, 1, 4, 64, 16), generator=g, dtype=torch.uint8)
    sc = torch.randint(118, 136, (3, 1, 4, 64), generator=g, dtype=torch.uint8)
    kv = torch.randint(0, 126, (256, 1, 576), generator=g, dtype=torch.uint8)
    return NS(get_key_buffer=lambda i: kv, get_index_k_fp4_payload_buffer=lambda i: pay,
              get_index_k_fp4_scale_buffer=lambda i: sc), kv, pay, sc


def test_step_entries_decode_the_fp4_plane_and_kv_rows_as_the_oracle_does():
    from oracle import attn as A
    from oracle import formats as F

    pool, kv, pay, sc = _fp4_pool(7)
    loc = torch.tensor([3, 0, 130, 77])  # slot 0: a pad row
    e = check.StepEntries.of(pool, 2, loc, 4)
    assert e.slots.tolist() == [3, 130, 77] and e.pages.tolist() == [0, 1, 2]
    got = e.index_keys()
    vals, ex = A.index_keys(pay[:, 0].numpy(), sc[:, 0].numpy(), np.arange(3), 192,
                            cols=[3, 130, 77])
    want = vals * np.exp2(ex.astype(np.float64))[..., None]
    np.testing.assert_array_equal(got.numpy(), want.reshape(3, 128))
    kvv = e.kv_values()
    np.testing.assert_array_equal(kvv.numpy(), F.e4m3_to_f32(kv[[3, 130, 77], 0].numpy()))


def test_step_entries_decode_dsa_pages_as_the_oracle_does():
    from oracle import attn as A

    g = torch.Generator().manual_seed(8)
    pages = torch.randint(0, 126, (3, 8448), generator=g, dtype=torch.uint8)
    scales = torch.exp2(torch.randint(-8, 4, (3, 64), generator=g).float())
    pages[:, 8192:] = scales.view(torch.uint8).view(3, 256)
    kv = torch.zeros(256, 1, 576, dtype=torch.uint8)
    pool = NS(get_key_buffer=lambda i: kv, get_index_k_with_scale_buffer=lambda i: pages)
    e = check.StepEntries.of(pool, 2, torch.tensor([65, 191, 7]), 3)
    want = A.dsa_keys(pages.numpy(), np.arange(3), 192, cols=[65, 191, 7])
    np.testing.assert_array_equal(e.index_keys().double().numpy(), want)


def test_compare_scores_the_cache_rows_the_launch_wrote():
    """SGLang wrote its rows (``reference``'s ``written``); the launch's rows now in the
    pool give the cosines; rows far from SGLang's miss the floors."""
    pool, kv, pay, sc = _fp4_pool(9)
    e = check.StepEntries.of(pool, 2, torch.tensor([3, 130]), 2)
    written = e.save()  # SGLang's rows
    b = torch.randn(2, 32)
    ref = {"out": b, "ids": None, "topk": None, "entries": e, "written": written}
    bounds = {"layer.kv.cosine": 0.995, "layer.index.cosine": 0.999}
    v = check.compare(NS(i=1), b, ref, 2, numerics=bounds)
    assert v["layer.kv.cosine"] == pytest.approx(1.0) and v["layer.index.cosine"] == pytest.approx(1.0)
    kv[3, 0, :] = torch.randint(0, 126, (576,), dtype=torch.uint8)  # the launch's rows
    pay[0, 0, :, 3, :] ^= 0x77
    v = check.compare(NS(i=1), b, ref, 2, numerics=bounds)
    assert v["layer.kv.cosine"] < 0.995 and v["layer.index.cosine"] < 0.999


def test_exact_topk_misses_counts_keys_of_the_own_scores_left_out():
    scores = torch.tensor([[0.5, 2.0, 2.0, -1.0, 3.0, 0.0],
                           [1.0, 1.0, 1.0, 1.0, 1.0, 1.0]])
    # row 0, k 3: 4, then the tie 1 and 2; row 1 (4 keys seen): the lowest positions
    assert check.exact_topk_misses(scores, torch.tensor([[4, 1, 2], [0, 1, 2]]), [6, 4], 3) == 0
    assert check.exact_topk_misses(scores, torch.tensor([[4, 1, 0], [0, 1, 3]]), [6, 4], 3) == 1
    assert check.exact_topk_misses(scores, torch.tensor([[5, 3, -1], [-1, -1, -1]]), [6, 4], 3) == 3
    # fewer keys than k: every key is selected
    assert check.exact_topk_misses(scores, torch.tensor([[0, 1, -1]]), [2], 3) == 0
