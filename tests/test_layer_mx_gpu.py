"""The one-launch layer with MXFP4 (A16W4) experts (``expert_format`` MONO_EXPERTS_MXFP4),
checked against the CPU oracle on its own routing.

Everything before the MoE is the FP8 layer's code, so the launch's hand-offs (q, the
index query and weights, scores, top-k, o_lat, a) must be bit-equal to the front,
attention and output-block launches run on the same inputs. The MoE: the router's scores
within f32 accumulation-order error of the oracle's (bf16(rmsnorm(a) g) against W_r in
f64: 1e-3 relative + 5e-4, the FP8 MoE test's bar), its top-8 bit-exact
against the exact top-8 of the launch's own scores (lowest-id ties), and y and the layer
output to the bf16 bars (2e-2 max-abs + 1e-2 relative, 1e-2 relative in norm) against
``oracle.moe.moe_mxfp4`` on x = bf16(rmsnorm(a) g) with the launch's ids and weights."""

import numpy as np
import pytest
import torch

from oracle import moe as M
from sgl_amd_mono_amd.dsv32 import synthetic
from sgl_amd_mono_amd.dsv32.attn import AttnInputs, AttnOp
from sgl_amd_mono_amd.dsv32.front import FrontOp
from sgl_amd_mono_amd.dsv32.layer import FusedLayerOp, LayerDebug, LayerStep, layer_runtime
from sgl_amd_mono_amd.dsv32.post import PostOp

pytestmark = pytest.mark.gpu
TOPK = 2048


def _close(got, want, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel <= 1e-2, (what, rel)
    bad = np.abs(got - want) > 2e-2 + 1e-2 * np.abs(want)
    assert not bad.any(), (what, int(bad.sum()), np.argwhere(bad)[:4])


def _debug(rows, ctx, gpu):
    bf, f32, i32 = torch.bfloat16, torch.float32, torch.int32
    return LayerDebug(q=torch.empty(rows, 32, 576, dtype=bf, device=gpu),
                      iq=torch.empty(rows, 64, 64, dtype=torch.uint8, device=gpu),
                      iqs=torch.empty(rows, 4, 16, 4, dtype=torch.uint8, device=gpu),
                      iw=torch.empty(rows, 64, dtype=f32, device=gpu),
                      o_lat=torch.empty(rows, 32, 512, dtype=bf, device=gpu),
                      a=torch.empty(rows, 7168, dtype=bf, device=gpu),
                      scores=torch.full((rows, ctx), float("nan"), device=gpu),
                      topk=torch.full((rows, TOPK), -7, dtype=i32, device=gpu),
                      y=torch.empty(rows, 7168, dtype=f32, device=gpu),
                      moe_scores=torch.empty(rows, 256, dtype=f32, device=gpu),
                      ids=torch.empty(rows, 9, dtype=i32, device=gpu),
                      weights=torch.empty(rows, 9, dtype=f32, device=gpu))


def _ragged(step: LayerStep, positions) -> LayerStep:
    pos = torch.as_tensor(positions, dtype=torch.int64, device=step.positions.device)
    page = step.page_table.gather(1, (pos // 64)[:, None])[:, 0].to(torch.int64)
    return LayerStep(positions=pos, slots=page * 64 + pos % 64, req_ids=step.req_ids,
                     page_table=step.page_table)


@pytest.mark.parametrize("layout", ["aiter16", "rowmajor"])
@pytest.mark.parametrize("rows", [1, 8])
def test_layer_mxfp4_experts_match_the_oracle(gpu, rows, layout):
    print(f"case MXFP4-expert layer rows={rows} layout={layout}", flush=True)
    ctx = 4096
    w, caches, step, h = synthetic.layer(rows, ctx, gpu, seed=70 + rows, layout=layout,
                                         experts="mxfp4")
    if rows == 8:
        step = _ragged(step, [4095, 3000, 2048, 2047, 100, 1, 4000, 0])
    # the phases before the MoE as launches of their own, on copies of the caches (the
    # front writes this step's keys: the same bytes at the same slots either way)
    kv0, plane0, ps0 = caches.kv.clone(), caches.plane.clone(), caches.plane_scale.clone()
    front = FrontOp(w.front, gpu, max_rows=rows)
    attn = AttnOp(gpu, max_rows=rows, ctx_max=ctx)
    post = PostOp(w.post, gpu, max_rows=rows)
    f = front.launch(h, caches, step.positions, step.slots)
    inp = AttnInputs(q=f.q, iq=f.iq, iqs=f.iqs, iw=f.iw, plane=caches.plane,
                     plane_scale=caches.plane_scale, kv=caches.kv, kv_scale=caches.kv_scale,
                     positions=step.positions, req_ids=step.req_ids, page_table=step.page_table)
    topk = torch.full((rows, TOPK), -7, dtype=torch.int32, device=gpu)
    o_lat = attn.launch(inp, topk=topk)
    a = post.launch(o_lat, h)
    for op in (front, attn, post):
        op.check() if hasattr(op, "check") else op.rt.check()
    written = (caches.kv.clone(), caches.plane.clone(), caches.plane_scale.clone())
    caches.kv.copy_(kv0)
    caches.plane.copy_(plane0)
    caches.plane_scale.copy_(ps0)

    fused = FusedLayerOp(w, gpu, max_rows=rows, ctx_max=ctx)
    dbg = _debug(rows, ctx, gpu)
    out = fused.launch(h, caches, step, debug=dbg)
    fused.check()
    for name, got, want in (("kv", caches.kv, written[0]), ("plane", caches.plane, written[1]),
                            ("plane scale", caches.plane_scale, written[2]), ("q", dbg.q, f.q),
                            ("iq", dbg.iq, f.iq), ("iqs", dbg.iqs, f.iqs), ("iw", dbg.iw, f.iw),
                            ("topk", dbg.topk, topk), ("o_lat", dbg.o_lat, o_lat),
                            ("a", dbg.a, a)):
        assert torch.equal(got, want), f"MXFP4-expert layer vs the phase launches: {name}"

    m = w.moe
    a_cpu = a.cpu()
    xn = M.rmsnorm(a_cpu.float(), m.g_post.cpu())
    x = xn.to(torch.bfloat16)
    want_sc = M.sigmoid(M.router_logits(xn, m.w_r.cpu())).numpy()
    sc = dbg.moe_scores.cpu().numpy()
    np.testing.assert_allclose(sc, want_sc, rtol=1e-3, atol=5e-4)
    ids, wts = dbg.ids.cpu().numpy(), dbg.weights.cpu().numpy()
    sel8, w8 = M.route_topk(dbg.moe_scores.cpu(), m.bias.cpu())
    assert np.array_equal(ids[:, 1:], sel8), "router top-8 (selection order)"
    assert np.all(ids[:, 0] == 256) and np.all(wts[:, 0] == 1.0)
    np.testing.assert_allclose(wts[:, 1:], w8, rtol=1e-6, atol=0)
    cfg = synthetic.MXFP4_LAYER_MOE
    ex = {int(e): synthetic.rowmajor_mxfp4_expert(m, int(e), cfg) for e in np.unique(ids)}
    pick = lambda k: {e: v[k] for e, v in ex.items()}  # noqa: E731
    # the routing is the launch's: the oracle's logits are not used
    ref = M.moe_mxfp4(x, torch.zeros(rows, 256), m.bias.cpu(), pick(0), pick(1), pick(2),
                      pick(3), residual=a_cpu, routing=(ids, wts))
    _close(dbg.y.cpu(), ref["y"], "moe y")
    _close(out.float().cpu(), ref["out"], "layer out")


def test_mxfp4_and_fp8_layers_share_one_runtime(gpu):
    """An FP8-expert layer and an MXFP4-expert layer alternating on one runtime (one
    scratch layout): every MXFP4 launch bit-equal to the same layer on a fresh runtime of
    its own, every FP8 launch bit-equal to its first; graph replay of the pair equal too."""
    print("case FP8 and MXFP4 layers on one runtime rows=4", flush=True)
    rows, ctx = 4, 2048
    wm, cm, sm, hm = synthetic.layer(rows, ctx, gpu, seed=81, experts="mxfp4")
    wf, cf, sf, hf = synthetic.layer(rows, ctx, gpu, seed=82)
    alone = FusedLayerOp(wm, gpu, max_rows=rows, ctx_max=ctx)
    want_m = alone.launch(hm, cm, sm).clone()
    alone.check()
    rt = layer_runtime(gpu, max_rows=rows)
    om = FusedLayerOp(wm, gpu, max_rows=rows, ctx_max=ctx, rt=rt)
    of = FusedLayerOp(wf, gpu, max_rows=rows, ctx_max=ctx, rt=rt)
    want_f = of.launch(hf, cf, sf).clone()
    for i in range(3):
        got_m = om.launch(hm, cm, sm).clone()
        got_f = of.launch(hf, cf, sf).clone()
        torch.cuda.synchronize()
        assert torch.equal(got_m, want_m), f"MXFP4 layer, round {i}"
        assert torch.equal(got_f, want_f), f"FP8 layer, round {i}"
    rt.check()
    outs = (torch.empty_like(want_m), torch.empty_like(want_f))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        om.launch(hm, cm, sm, out=outs[0])
        of.launch(hf, cf, sf, out=outs[1])
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        om.launch(hm, cm, sm, out=outs[0])
        of.launch(hf, cf, sf, out=outs[1])
    for i in range(3):
        outs[0].zero_()
        outs[1].zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(outs[0], want_m) and torch.equal(outs[1], want_f), f"replay {i}"
        om.launch(hm, cm, sm)
        torch.cuda.synchronize()
    rt.check()
