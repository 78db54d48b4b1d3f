"""FP8 routed MoE launch (config 2) against the CPU oracle on the same seeded inputs.

Bars: router top-8 ids bit-exact given the launch's own sigmoid scores (lowest-id
ties); scores within f32 accumulation-order error of the oracle's; the MoE sum y within
1e-2 relative (norm) and cos >= 0.9999 of the oracle run on the launch's routing; the
layer output a + y within 2e-2 max-abs + 1e-2 relative (bf16, fp32 accumulation)."""

import numpy as np
import pytest
import torch

from oracle import moe as omoe
from sgl_amd_mono_amd.dsv32 import synthetic
from sgl_amd_mono_amd.dsv32.config import DSV32
from sgl_amd_mono_amd.dsv32.moe import MoeFp8Op, MoeRouting

pytestmark = pytest.mark.gpu
H, E = DSV32.hidden, DSV32.experts


@pytest.fixture(scope="module")
def layer(gpu):
    return synthetic.moe_fp8_weights(gpu, seed=0)


@pytest.fixture(scope="module")
def layer_aiter(gpu):
    return synthetic.moe_fp8_weights(gpu, seed=0, layout="aiter16")


def _routing(rows, dev):
    return MoeRouting(scores=torch.empty(rows, E, dtype=torch.float32, device=dev),
                      ids=torch.empty(rows, 9, dtype=torch.int32, device=dev),
                      weights=torch.empty(rows, 9, dtype=torch.float32, device=dev))


def _cpu_experts(w, ids):
    return {int(e): synthetic.rowmajor_expert(w, int(e)) for e in np.unique(ids)}


def _run(op, a):
    rows = a.shape[0]
    y = torch.full((rows, H), float("nan"), dtype=torch.float32, device=a.device)
    rt = _routing(rows, a.device)
    out = op.launch(a, y=y, routing=rt)
    op.rt.check()
    return out, y, rt


@pytest.mark.parametrize("rows,layout", [(1, "rowmajor"), (4, "rowmajor"), (8, "rowmajor"),
                                         (16, "rowmajor"), (1, "aiter16"), (8, "aiter16"),
                                         (16, "aiter16")])
def test_moe_fp8_matches_oracle(request, gpu, rows, layout):
    print(f"case rows={rows} layout={layout}", flush=True)
    layer = request.getfixturevalue("layer" if layout == "rowmajor" else "layer_aiter")
    op = MoeFp8Op(layer, gpu, max_rows=16)
    a = synthetic.rows_bf16(rows, H, gpu, seed=rows)
    out, y, rt = _run(op, a)
    ids, wts = rt.ids.cpu().numpy(), rt.weights.cpu().numpy()
    scores = rt.scores.cpu()
    bias = layer.bias.cpu()
    # selection: bit-exact against the oracle's top-8 of the launch's own scores
    sel, sel_w = omoe.route_topk(scores, bias)
    assert np.array_equal(ids[:, 1:], sel), "router ids differ"
    assert np.all(ids[:, 0] == 256) and np.all(wts[:, 0] == 1.0)
    np.testing.assert_allclose(wts[:, 1:], sel_w, rtol=2e-6, atol=1e-7)
    # the oracle end to end
    ref = omoe.moe_fp8(a.cpu(), layer.g_post.cpu(), layer.w_r.cpu(), bias, None, None, None,
                       None, experts=_cpu_experts(layer, np.concatenate([ids, ref_ids(a, layer)])),
                       routing=(ids, wts))
    # the router stages the normalised rows as bf16 (as the reference does): a 1-ulp
    # difference in rstd flips the bf16 rounding of a few of the 7168 inputs, ~1e-4 of
    # logit each, on top of the f32 accumulation order (the oracle sums in f64)
    np.testing.assert_allclose(scores.numpy(), ref["scores"].numpy(), rtol=1e-3, atol=5e-4)
    got, want = y.cpu().double(), ref["y"].double()
    rel = float((got - want).norm() / want.norm())
    cos = float(torch.nn.functional.cosine_similarity(got.flatten(), want.flatten(), dim=0))
    print(f"rows={rows} y rel={rel:.3e} cos={cos:.6f}", flush=True)
    assert rel <= 1e-2 and cos >= 0.9999, (rel, cos)
    o = out.cpu().float()
    assert torch.all((o - ref["out"]).abs() <= 2e-2 + 1e-2 * ref["out"].abs())
    # the oracle's own routing agrees wherever the 8th/9th keys are clearly apart
    own, _ = omoe.route_topk(ref["scores"], bias)
    key = (ref["scores"] + bias).numpy()
    srt = -np.sort(-key, 1)
    clear = (srt[:, 7] - srt[:, 8]) > 2e-3
    assert np.array_equal(np.sort(own[clear], 1), np.sort(ids[clear, 1:], 1))


def ref_ids(a, layer):
    """The oracle's own routing ids (its experts are needed for the comparison too)."""
    xn = omoe.rmsnorm(a.cpu(), layer.g_post.cpu())
    s = omoe.sigmoid(omoe.router_logits(xn, layer.w_r.cpu()))
    return omoe.slots_with_shared(*omoe.route_topk(s, layer.bias.cpu()))[0]


def test_moe_fp8_is_deterministic_and_writes_only_its_rows(layer, gpu):
    print("case determinism rows=8", flush=True)
    op = MoeFp8Op(layer, gpu, max_rows=16)
    a = synthetic.rows_bf16(8, H, gpu, seed=42)
    full = torch.full((16, H), 7.0, dtype=torch.bfloat16, device=gpu)
    r1 = op.launch(a, out=full[:8]).clone()
    r2 = op.launch(a).clone()
    r3 = op.launch(a).clone()
    op.rt.check()
    assert torch.equal(r1, r2) and torch.equal(r2, r3)
    assert torch.all(full[8:] == 7.0), "wrote past its rows"


def test_moe_fp8_back_to_back_launches_match_fresh_runtimes(layer, gpu):
    """Launches on one runtime alternate between two scratch hand-off buffers, each
    cleared by the launch before: with new inputs and row counts every launch, each
    result equals that of a runtime that never launched (nothing stale is read)."""
    print("case back-to-back rows=8,3,8,16,5", flush=True)
    op = MoeFp8Op(layer, gpu, max_rows=16)
    for i, rows in enumerate((8, 3, 8, 16, 5)):
        a = synthetic.rows_bf16(rows, H, gpu, seed=300 + i)
        got = op.launch(a).clone()
        want = MoeFp8Op(layer, gpu, max_rows=16).launch(a)
        torch.cuda.synchronize()
        op.rt.check()
        assert torch.equal(got, want), f"launch {i} rows={rows}"


def test_moe_fp8_graph_replay_matches_eager(layer, gpu):
    print("case graph replay rows=4", flush=True)
    op = MoeFp8Op(layer, gpu, max_rows=16)
    a = synthetic.rows_bf16(4, H, gpu, seed=7)
    out = torch.empty(4, H, dtype=torch.bfloat16, device=gpu)
    eager = op.launch(a).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        op.launch(a, out=out)  # warm up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        op.launch(a, out=out)
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        op.launch(a)  # eager work between replays
        torch.cuda.synchronize()
    op.rt.check()


def test_moe_fp8_deadline_stops_and_reports(layer, gpu):
    """Fault injection from the host: the mid-quant wait never completes, so it times
    out after a 5 ms deadline; every CTA still exits, the output is all NaN, the host
    raises, and a reset runtime launches cleanly again."""
    print("case fault injection site=mid", flush=True)
    a = synthetic.rows_bf16(2, H, gpu, seed=3)
    op = MoeFp8Op(layer, gpu, max_rows=16, deadline_s=0.005, fault=(2, 0))
    bad = op.launch(a)
    torch.cuda.synchronize()
    assert torch.isnan(bad.float()).all()
    with pytest.raises(RuntimeError, match="mid"):
        op.rt.check()
    with pytest.raises(RuntimeError):
        op.launch(a)  # refused after a failure
    words = op.rt.guard.cpu().tolist()
    assert words[3] == 3 and words[5] == 1  # 1 + site, fault-injected
    op.fault = (0, 0)
    op.rt.reset()
    op.rt.set_deadline(10.0)
    clean = op.launch(a).clone()
    op.rt.check()
    ref = MoeFp8Op(layer, gpu, max_rows=16).launch(a)
    torch.cuda.synchronize()
    assert torch.equal(clean, ref)


@pytest.mark.parametrize("n_group,topk_group", [(8, 4), (4, 1)])
def test_moe_fp8_group_limited_routing(gpu, layer_aiter, n_group, topk_group):
    """DeepSeek-V3.2's router (8 groups of 32 experts, 4 kept) and a narrow one (4 groups,
    1 kept: all 8 picks from one group of 64): ids bit-exact against the oracle's
    group-limited top-8 of the launch's own scores, every pick in a kept group, weights
    and y against the oracle on that routing."""
    import dataclasses

    print(f"case fp8 grouped routing n_group={n_group} topk_group={topk_group}", flush=True)
    cfg = dataclasses.replace(DSV32, n_group=n_group, topk_group=topk_group)
    op = MoeFp8Op(layer_aiter, gpu, cfg=cfg, max_rows=16)
    a = synthetic.rows_bf16(8, H, gpu, seed=80 + n_group)
    out, y, rt = _run(op, a)
    ids, wts = rt.ids.cpu().numpy(), rt.weights.cpu().numpy()
    scores, bias = rt.scores.cpu(), layer_aiter.bias.cpu()
    sel, sel_w = omoe.route_topk(scores, bias, n_group=n_group, topk_group=topk_group)
    assert np.array_equal(ids[:, 1:], sel), "grouped router ids differ"
    np.testing.assert_allclose(wts[:, 1:], sel_w, rtol=2e-6, atol=1e-7)
    keep = omoe.group_mask((scores.numpy() + bias.numpy()).astype(np.float32), n_group,
                           topk_group)
    assert np.all(np.take_along_axis(keep, ids[:, 1:].astype(np.int64), 1))
    if topk_group == 1:
        assert np.all(ids[:, 1:] // (256 // n_group) == ids[:, 1:2] // (256 // n_group))
    experts = {int(e): synthetic.rowmajor_expert(layer_aiter, int(e)) for e in np.unique(ids)}
    ref = omoe.moe_fp8(a.cpu(), layer_aiter.g_post.cpu(), layer_aiter.w_r.cpu(), bias, None,
                       None, None, None, experts=experts, routing=(ids, wts))
    got, want = y.cpu().double(), ref["y"].double()
    rel = float((got - want).norm() / want.norm())
    assert rel <= 1e-2, rel
