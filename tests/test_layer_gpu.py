"""One decoder layer (config 5): the four launches chained on one stream, every phase
checked against the CPU oracle on the inputs that phase received from the one before,
and the one-launch layer (``mono_layer_launch``) bit-equal to the chain at every hand-off
(q, the index query and weights, scores, top-k, o_lat, a, routing, y) and at its output.

Bars as the per-phase tests: q and the output block within 2e-2 max-abs + 1e-2 relative
and 1e-2 relative in norm of the oracle's f64; indexer scores within 1e-5 of the row's
largest; the selection bit-exact against the exact top-2048 of the launch's own scores;
the router's top-8 bit-exact against the oracle's over the launch's own scores; the
MoE's y and the layer output to the same bf16 bars."""

import numpy as np
import pytest
import torch

from oracle import attn as A
from oracle import dense as D
from oracle import front as Fr
from oracle import moe as M
from oracle.topk import topk_sort
from sgl_amd_mono_amd import _lib
from sgl_amd_mono_amd.dsv32 import synthetic
from sgl_amd_mono_amd.dsv32.attn import AttnInputs
from sgl_amd_mono_amd.dsv32.layer import FusedLayerOp, LayerDebug, LayerOp, LayerStep
from sgl_amd_mono_amd.dsv32.moe import MoeRouting

pytestmark = pytest.mark.gpu
TOPK = 2048


def _close(got, want, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel <= 1e-2, (what, rel)
    bad = np.abs(got - want) > 2e-2 + 1e-2 * np.abs(want)
    assert not bad.any(), (what, int(bad.sum()), np.argwhere(bad)[:4])


def _ragged(step: LayerStep, positions) -> LayerStep:
    """The same requests at other positions: each row's slot is its page-table entry."""
    pos = torch.as_tensor(positions, dtype=torch.int64, device=step.positions.device)
    page = step.page_table.gather(1, (pos // 64)[:, None])[:, 0].to(torch.int64)
    return LayerStep(positions=pos, slots=page * 64 + pos % 64, req_ids=step.req_ids,
                     page_table=step.page_table)


def test_layer_eight_rows_ragged_contexts(gpu):
    """8 rows seeing 8192, 5001, 2049, 2048, 101, 7001, 3000 and 1 keys."""
    print("case layer rows=8 ctx<=8192 ragged", flush=True)
    _layer_case(gpu, 8, 8192, [8191, 5000, 2048, 2047, 100, 7000, 2999, 0], seed=3)


def test_layer_eight_rows_at_32k(gpu):
    """Config 5's step: 8 rows each at position 32767 (the bench's workload)."""
    print("case layer rows=8 ctx=32768", flush=True)
    _layer_case(gpu, 8, 32768, None, seed=32)


def test_layer_dsa_index_pages(gpu):
    """The layer over SGLang's DSA index pages (E4M3 keys at per-token scales, bf16 index
    query): 8 ragged rows, the chain against the oracle and the one launch bit-equal."""
    print("case layer DSA pages rows=8 ctx<=8192 ragged", flush=True)
    _layer_case(gpu, 8, 8192, [8191, 5000, 2048, 2047, 100, 7000, 2999, 0], seed=5,
                index_format=_lib.INDEX_FP8_PAGE)


def _layer_case(gpu, rows, ctx, positions, seed, index_format=0):
    w, caches, step, h = synthetic.layer(rows, ctx, gpu, seed=seed, index_format=index_format)
    fp4 = index_format == _lib.INDEX_FP4_PLANE
    if positions is not None:
        step = _ragged(step, positions)
    op = LayerOp(w, gpu, max_rows=rows, ctx_max=ctx)
    f = op.front.launch(h, caches, step.positions, step.slots)
    inp = AttnInputs(q=f.q, iq=f.iq, iqs=f.iqs, iw=f.iw, plane=caches.plane,
                     plane_scale=caches.plane_scale, kv=caches.kv, kv_scale=caches.kv_scale,
                     positions=step.positions, req_ids=step.req_ids, page_table=step.page_table,
                     index_format=index_format)
    scores = torch.full((rows, ctx), float("nan"), device=gpu)
    topk = torch.full((rows, TOPK), -7, dtype=torch.int32, device=gpu)
    o_lat = op.attn.launch(inp, scores=scores, topk=topk)
    a = op.post.launch(o_lat, h)
    y = torch.empty(rows, 7168, dtype=torch.float32, device=gpu)
    rt = MoeRouting(torch.empty(rows, 256, device=gpu), torch.empty(rows, 9, dtype=torch.int32,
                    device=gpu), torch.empty(rows, 9, device=gpu))
    out = op.moe.launch(a, y=y, routing=rt)
    op.check()

    # the same layer as one launch, on the same caches (its cache writes are the same
    # bytes at the same slots): bit-equal at every hand-off and at its output
    fused = FusedLayerOp(w, gpu, max_rows=rows, ctx_max=ctx)
    dbg = LayerDebug(q=torch.empty_like(f.q), iq=torch.empty_like(f.iq),
                     iqs=torch.empty_like(f.iqs) if fp4 else None, iw=torch.empty_like(f.iw),
                     o_lat=torch.empty_like(o_lat), a=torch.empty_like(a),
                     scores=torch.full_like(scores, float("nan")),
                     topk=torch.full_like(topk, -7), y=torch.empty_like(y),
                     moe_scores=torch.empty_like(rt.scores), ids=torch.empty_like(rt.ids),
                     weights=torch.empty_like(rt.weights))
    fout = fused.launch(h, caches, step, debug=dbg)
    fused.check()
    for name, got, want in (("q", dbg.q, f.q), ("iq", dbg.iq, f.iq),
                            ("iqs", dbg.iqs if fp4 else f.iq, f.iqs if fp4 else f.iq),
                            ("iw", dbg.iw, f.iw), ("topk", dbg.topk, topk),
                            ("o_lat", dbg.o_lat, o_lat), ("a", dbg.a, a), ("y", dbg.y, y),
                            ("moe scores", dbg.moe_scores, rt.scores), ("ids", dbg.ids, rt.ids),
                            ("weights", dbg.weights, rt.weights), ("out", fout, out)):
        assert torch.equal(got, want), f"one launch vs four: {name}"
    assert torch.equal(dbg.scores.isnan(), scores.isnan())
    assert torch.equal(dbg.scores.nan_to_num(0.0), scores.nan_to_num(0.0))

    pos = step.positions.cpu().numpy()
    fr = Fr.front(h.cpu(), positions=pos, **synthetic.rowmajor_front(w.front))
    _close(f.q.float().cpu(), fr["q"], "front q")

    sc, tk = scores.cpu().numpy(), topk.cpu().numpy()
    iw = f.iw.cpu().numpy()
    plane = caches.plane.cpu().numpy()
    if fp4:
        iq, iqs, psc = f.iq.cpu().numpy(), f.iqs.cpu().numpy(), caches.plane_scale.cpu().numpy()
    else:
        iq = f.iq.float().cpu().numpy().astype(np.float64)
    kv, ksc = caches.kv.cpu().numpy(), caches.kv_scale.cpu().numpy()
    pt = step.page_table.cpu().numpy()
    rng = np.random.default_rng(seed)
    for r in range(rows):
        n = int(pos[r]) + 1
        pages = pt[r]
        cols = np.arange(n) if n <= 3000 else np.sort(rng.choice(n, 3000, replace=False))
        want = (A.index_scores(iq[r], iqs[r], iw[r], plane, psc, pages, n, cols=cols) if fp4
                else A.index_scores_fp8(iq[r], iw[r], plane, pages, n, cols=cols))
        err = np.abs(sc[r, cols] - want).max() / max(np.abs(want).max(), 1e-30)
        assert err <= 1e-5, (r, err)
        k = min(n, TOPK)
        want_sel = np.arange(n, dtype=np.int32) if n <= TOPK else topk_sort(sc[r, :n], TOPK)
        assert np.array_equal(tk[r, :k], want_sel), (r, n)
        assert np.all(tk[r, k:] == -1), r
        slots = pages[tk[r, :k] // 64].astype(np.int64) * 64 + tk[r, :k] % 64
        o, _ = A.sparse_mla(f.q[r].cpu(), kv, ksc, slots, op.attn.sm_scale)
        _close(o_lat[r].float().cpu(), o, f"o_lat row {r}")

    pr = D.attn_out(o_lat.cpu(), h.cpu(), *synthetic.rowmajor_post(w.post))
    _close(a.float().cpu(), pr["a"], "post a")

    ids = rt.ids.cpu().numpy()
    sel8, _ = M.route_topk(rt.scores.cpu(), w.moe.bias.cpu())
    assert np.array_equal(np.sort(ids[:, 1:], 1), np.sort(sel8, 1)), "router top-8"
    experts = {int(e): synthetic.rowmajor_expert(w.moe, int(e)) for e in np.unique(ids)}
    ref = M.moe_fp8(a.cpu(), w.moe.g_post.cpu(), w.moe.w_r.cpu(), w.moe.bias.cpu(), None, None,
                    None, None, experts=experts, routing=(ids, rt.weights.cpu().numpy()))
    _close(y.cpu(), ref["y"], "moe y")
    _close(out.float().cpu(), ref["out"], "layer out")


def test_layer_graph_replay_matches_eager(gpu):
    """The layer captured in one graph: three replays, with eager layers between them,
    each bit-equal to the eager result."""
    print("case layer graph replay rows=8 ctx=4096", flush=True)
    rows = 8
    w, caches, step, h = synthetic.layer(rows, 4096, gpu, seed=4)
    op = LayerOp(w, gpu, max_rows=rows, ctx_max=4096)
    want = op.launch(h, caches, step).clone()
    again = op.launch(h, caches, step).clone()
    op.check()
    assert torch.equal(want, again)
    out = torch.empty_like(want)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        op.launch(h, caches, step, out=out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        op.launch(h, caches, step, out=out)
    for i in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"
        op.launch(h, caches, step)
        torch.cuda.synchronize()
    op.check()


def test_layer_bound_from_sglang_modules_matches_the_oracle(gpu):
    """A layer as SGLang loads it, bound by ``binding`` and run as the one launch, against
    the oracle under SGLang's own statement of its tensors. W_UK / W_UV are drawn as
    SGLang holds them (per-tensor E4M3 ``w_kc`` [32, 128, 512], ``w_vc`` [32, 512, 128] at a
    scalar ``w_scale``) and the oracle applies SGLang's products, q_lat = q_nope @ w_kc and
    o = o_lat @ w_vc; the rotary is SGLang's f32 ``cos_sin_cache`` read as
    ``cos, sin = cache.chunk(2, -1)`` (the tables the front reads are bf16). Nothing of
    the expected values goes through the binding's packing, so a misread layout fails:
    q, the cache rows, o_lat, a and the layer output to the bf16 bars; the top-k and the
    router bit-exact on the launch's own scores."""
    from types import SimpleNamespace as NS

    from oracle import formats as F
    from sgl_amd_mono_amd import layouts
    from sgl_amd_mono_amd.dsv32 import binding
    from sgl_amd_mono_amd.dsv32.moe import FP8

    print("case layer bound from SGLang modules vs the oracle", flush=True)
    rows, ctx, scale = 4, 2048, 0.0078125
    w, caches, step, h = synthetic.layer(rows, ctx, gpu, seed=6)
    g = torch.Generator().manual_seed(61)
    codes = lambda *shape: (torch.randint(0, 0x78, shape, generator=g, dtype=torch.uint8)
                            | (torch.randint(0, 2, shape, generator=g, dtype=torch.uint8) << 7))
    w_kc = codes(32, 128, 512).view(FP8).to(gpu)
    w_vc = codes(32, 512, 128).view(FP8).to(gpu)
    inv = 10000.0 ** (-torch.arange(0, 64, 2, dtype=torch.float64) / 64)
    ang = torch.arange(ctx, dtype=torch.float64)[:, None] * inv[None]
    cache = torch.cat([ang.cos(), ang.sin()], 1).float().to(gpu)
    lin = lambda wt, s: NS(weight=wt, weight_scale_inv=s, aiter_bpreshuffled=True)
    f, po, m = w.front, w.post, w.moe
    m.w13.is_shuffled = True
    attn = NS(fused_qkv_a_proj_with_mqa=lin(f.w_qkv_a, f.s_qkv_a), q_b_proj=lin(f.w_qb, f.s_qb),
              o_proj=lin(po.w_o, po.s_o), q_a_layernorm=NS(weight=f.g_q),
              kv_a_layernorm=NS(weight=f.g_kv), w_kc=w_kc, w_vc=w_vc,
              w_scale=torch.tensor(scale, device=gpu), rotary_emb=NS(cos_sin_cache=cache),
              indexer=NS(wk=lin(f.w_k, f.s_k), wq_b=lin(f.w_iq, f.s_iq),
                         weights_proj=NS(weight=f.w_w), rotary_emb=NS(cos_sin_cache=cache),
                         k_norm=NS(weight=f.g_k.clone(), bias=f.b_k.clone())))
    module = NS(self_attn=attn, input_layernorm=NS(weight=f.g_in),
                post_attention_layernorm=NS(weight=m.g_post),
                mlp=NS(gate=NS(weight=m.w_r, e_score_correction_bias=m.bias),
                       experts=NS(w13_weight=m.w13, w13_weight_scale_inv=m.s13,
                                  w2_weight=m.w2, w2_weight_scale_inv=m.s2)))
    copies = {}
    bound = binding.layer_weights(module, 9, copies)
    assert bound.front.w_qkv_a is f.w_qkv_a and bound.moe.w13 is m.w13 and len(copies) == 8
    fused = FusedLayerOp(bound, gpu, max_rows=rows, ctx_max=ctx)
    dbg = LayerDebug(q=torch.empty(rows, 32, 576, dtype=torch.bfloat16, device=gpu),
                     o_lat=torch.empty(rows, 32, 512, dtype=torch.bfloat16, device=gpu),
                     a=torch.empty(rows, 7168, dtype=torch.bfloat16, device=gpu),
                     scores=torch.full((rows, ctx), float("nan"), device=gpu),
                     topk=torch.full((rows, TOPK), -7, dtype=torch.int32, device=gpu),
                     y=torch.empty(rows, 7168, device=gpu),
                     moe_scores=torch.empty(rows, 256, device=gpu),
                     ids=torch.empty(rows, 9, dtype=torch.int32, device=gpu),
                     weights=torch.empty(rows, 9, device=gpu))
    out = fused.launch(h, caches, step, debug=dbg)
    fused.check()

    # SGLang's statement of the absorbed products and of the rotary halves
    kc = torch.from_numpy(F.e4m3_to_f32(w_kc.view(torch.uint8).cpu().numpy())).double() * scale
    vc = torch.from_numpy(F.e4m3_to_f32(w_vc.view(torch.uint8).cpu().numpy())).double() * scale
    cos_h, sin_h = cache.cpu().chunk(2, -1)
    args = synthetic.rowmajor_front(f)
    args.update(w_uk=None, s_uk=None, cos=cos_h.to(torch.bfloat16), sin=sin_h.to(torch.bfloat16))
    pos = step.positions.cpu().numpy()
    fr = Fr.front(h.cpu(), positions=pos, kv_scaled=caches.kv_scale is not None,
                  absorb=lambda qn, hh: (torch.from_numpy(np.asarray(qn, np.float64)) @ kc[hh]).numpy(),
                  **args)
    _close(dbg.q.float().cpu(), fr["q"], "q under SGLang's w_kc")
    # the cache rows the front wrote (latent + rotated key), read back: within an E4M3
    # step of the oracle's bf16 row, plus 2^-7 of the row's rms for one-ulp upstream
    # differences (hardware rsqrt in the norm)
    slots = step.slots.cpu().numpy()
    kv_ks = None if caches.kv_scale is None else caches.kv_scale.cpu().numpy()
    got_rows = A.kv_rows(caches.kv.cpu().numpy(), kv_ks, slots)
    for r in range(rows):
        orow = fr["kv_rows"][r]
        ks = 1.0 if kv_ks is None else float(kv_ks[slots[r]])
        stepv = np.maximum(2.0 ** (np.floor(np.log2(np.maximum(np.abs(orow), 1e-30))) - 3),
                           2.0 ** -9 * ks)
        err = np.abs(got_rows[r] - orow) - (stepv + 2.0 ** -7 * np.sqrt(np.mean(orow ** 2)))
        assert np.all(err <= 0), ("cache row under SGLang's rotary", r, int(np.argmax(err)))
    # the attention on the launch's own q and scores
    sc, tk = dbg.scores.cpu().numpy(), dbg.topk.cpu().numpy()
    pt = step.page_table.cpu().numpy()
    kv = caches.kv.cpu().numpy()
    for r in range(rows):
        n = int(pos[r]) + 1
        want_sel = np.arange(n, dtype=np.int32) if n <= TOPK else topk_sort(sc[r, :n], TOPK)
        k = min(n, TOPK)
        assert np.array_equal(tk[r, :k], want_sel), r
        sl = pt[r][tk[r, :k] // 64].astype(np.int64) * 64 + tk[r, :k] % 64
        o, _ = A.sparse_mla(dbg.q[r].cpu(), kv, kv_ks, sl, fused.sm_scale)
        _close(dbg.o_lat[r].float().cpu(), o, f"o_lat row {r}")
    _, _, w_o, s_o = synthetic.rowmajor_post(po)
    pr = D.attn_out(dbg.o_lat.cpu(), h.cpu(), None, None, w_o, s_o,
                    uv=lambda x, hh: (torch.from_numpy(np.asarray(x, np.float64)) @ vc[hh]).numpy())
    _close(dbg.a.float().cpu(), pr["a"], "a under SGLang's w_vc")
    ids = dbg.ids.cpu().numpy()
    sel8, _ = M.route_topk(dbg.moe_scores.cpu(), m.bias.cpu())
    assert np.array_equal(np.sort(ids[:, 1:], 1), np.sort(sel8, 1)), "router top-8"
    experts = {int(e): synthetic.rowmajor_expert(m, int(e)) for e in np.unique(ids)}
    ref = M.moe_fp8(dbg.a.cpu(), m.g_post.cpu(), m.w_r.cpu(), m.bias.cpu(), None, None, None,
                    None, experts=experts, routing=(ids, dbg.weights.cpu().numpy()))
    _close(dbg.y.cpu(), ref["y"], "moe y")
    _close(out.float().cpu(), ref["out"], "layer out")


def test_one_launch_layer_graph_replay_matches_eager(gpu):
    """The one-launch layer captured in a graph: three replays, eager launches between
    them, every replay bit-equal to the eager result; 3 rows, one of them a pad row."""
    print("case one-launch layer graph replay rows=3 ctx=4096", flush=True)
    rows = 3
    w, caches, step, h = synthetic.layer(rows, 4096, gpu, seed=41)
    step = LayerStep(positions=step.positions, slots=step.slots.clone(), req_ids=step.req_ids,
                     page_table=step.page_table)
    step.slots[2] = -1  # a pad row: writes no cache entry
    op = FusedLayerOp(w, gpu, max_rows=8, ctx_max=4096)
    want = op.launch(h, caches, step).clone()
    again = op.launch(h, caches, step).clone()
    op.check()
    assert torch.equal(want, again)
    out = torch.empty_like(want)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        op.launch(h, caches, step, out=out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        op.launch(h, caches, step, out=out)
    for i in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"
        op.launch(h, caches, step)
        torch.cuda.synchronize()
    op.check()


@pytest.mark.parametrize("site", [11, 13, 5, 2])
def test_one_launch_layer_deadline_stops_and_reports(gpu, site):
    """A wait forced to stall from the host (the phase barrier, the stage-A wait for x, a
    split's top-k wait, a mid quant's wait): it times out after 5 ms, every CTA runs to the end of the launch, the
    output is all NaN, the host raises naming the site, and a reset runtime launches
    cleanly."""
    from sgl_amd_mono_amd import _lib

    print(f"case one-launch layer fault injection site={site}", flush=True)
    rows = 2
    w, caches, step, h = synthetic.layer(rows, 4096, gpu, seed=43)
    op = FusedLayerOp(w, gpu, max_rows=rows, ctx_max=4096, deadline_s=0.005, fault=(site, 0))
    bad = op.launch(h, caches, step)
    torch.cuda.synchronize()
    assert torch.isnan(bad.float()).all()
    with pytest.raises(RuntimeError, match=f"timed out at {_lib.SITES[site]} "):
        op.check()
    words = op.rt.guard.cpu().tolist()
    assert words[3] == site + 1 and words[5] == 1
    op.fault = (0, 0)
    op.rt.reset()
    op.rt.set_deadline(10.0)
    clean = op.launch(h, caches, step).clone()
    op.check()
    ref = FusedLayerOp(w, gpu, max_rows=rows, ctx_max=4096).launch(h, caches, step)
    torch.cuda.synchronize()
    assert torch.equal(clean, ref)


def test_one_launch_layer_fail_stop_inside_graph_replay(gpu):
    """Fail-stop with no host code between launches: the one-launch layer captured in a
    graph whose wait for the top-k is armed, through fault injection set from the host, to
    stall from the launch that starts at epoch 4 on. Replays 1-3 equal the eager output;
    replay 4 times out after 5 ms, its output is all NaN and the pinned error word names
    the site; replay 5 is all NaN again (the abort word stays set); after a reset the same
    graph replays cleanly."""
    from sgl_amd_mono_amd import _lib

    print("case one-launch layer fail-stop in graph replay rows=2 ctx=4096", flush=True)
    rows = 2
    w, caches, step, h = synthetic.layer(rows, 4096, gpu, seed=44)
    ref = FusedLayerOp(w, gpu, max_rows=rows, ctx_max=4096).launch(h, caches, step).clone()
    site = next(k for k, v in _lib.SITES.items() if v == "topk")
    op = FusedLayerOp(w, gpu, max_rows=rows, ctx_max=4096, deadline_s=0.005, fault=(site, 4))
    out = torch.empty_like(ref)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        op.launch(h, caches, step, out=out)  # epoch 0 -> 1
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        op.launch(h, caches, step, out=out)
    for i in range(5):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        if i < 3:
            assert torch.equal(out, ref), f"replay {i}"
            assert int(op.rt.host_error[0]) == 0
        else:
            assert torch.isnan(out.float()).all(), f"replay {i}"
            assert int(op.rt.host_error[0]) == site + 1
    words = op.rt.guard.cpu().tolist()
    assert words[3] == site + 1 and words[7] == 1
    op.rt.reset()
    out.zero_()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    op.check()


def test_one_launch_layer_across_the_tag_wrap(gpu):
    """Launch tags run 1 .. 2^32 - 2 and start again at 1. With the epoch set just short of
    the end of the cycle (on a cleared scratch, as the scrub leaves a pair that old), four
    launches cross the wrap, each bit-equal to a fresh runtime's output, and the epoch ends
    at 3. After each launch the 16 KiB chunk of scratch its last CTA cleared (tag mod the
    number of chunks) reads zero."""
    from sgl_amd_mono_amd import _lib

    print("case one-launch layer tag wrap rows=2 ctx=4096", flush=True)
    rows = 2
    w, caches, step, h = synthetic.layer(rows, 4096, gpu, seed=45)
    ref = FusedLayerOp(w, gpu, max_rows=rows, ctx_max=4096).launch(h, caches, step).clone()
    op = FusedLayerOp(w, gpu, max_rows=rows, ctx_max=4096)
    op.rt.reset()
    op.rt.guard[0] = 0xFFFFFFFD - (1 << 32)  # epoch 2^32 - 3 as an int32 word
    nchunk = -(-_lib.lib().mono_layer_scratch_bytes(rows) // 16384)
    for want_tag in (0xFFFFFFFE, 1, 2, 3):
        got = op.launch(h, caches, step).clone()
        torch.cuda.synchronize()
        assert torch.equal(got, ref), hex(want_tag)
        assert int(op.rt.guard[0]) & 0xFFFFFFFF == want_tag
        c = want_tag % nchunk
        chunk = op.rt.scratch[c * 16384:(c + 1) * 16384]
        assert int(chunk.count_nonzero()) == 0, (hex(want_tag), c)
    op.check()


def test_layer_rows_longer_than_one_block(gpu):
    """The layer at 131072 keys (four top-k blocks) and 70001 keys (a short third block):
    the four launches against the oracle and the one launch bit-equal to them."""
    print("case layer rows=2 ctx=131072", flush=True)
    _layer_case(gpu, 2, 131072, [131071, 70000], seed=1310)


def test_one_launch_layer_group_limited_routing(gpu):
    """The one launch with DeepSeek-V3.2's router (8 groups, 4 kept): the routing ids
    bit-exact against the oracle's group-limited top-8 of the launch's own scores, and
    the same bits as the four launches with that router."""
    import dataclasses

    from oracle import moe as om
    from sgl_amd_mono_amd.dsv32.config import DSV32

    print("case one-launch layer grouped routing rows=4 ctx=4096", flush=True)
    cfg = dataclasses.replace(DSV32, n_group=8, topk_group=4)
    rows = 4
    w, caches, step, h = synthetic.layer(rows, 4096, gpu, seed=84)
    kv0, plane0 = caches.kv.clone(), caches.plane.clone()
    want = LayerOp(w, gpu, cfg=cfg, max_rows=rows, ctx_max=4096).launch(h, caches, step).clone()
    caches.kv.copy_(kv0)
    caches.plane.copy_(plane0)
    dbg = LayerDebug(moe_scores=torch.empty(rows, 256, device=gpu),
                     ids=torch.empty(rows, 9, dtype=torch.int32, device=gpu),
                     weights=torch.empty(rows, 9, device=gpu))
    op = FusedLayerOp(w, gpu, cfg=cfg, max_rows=rows, ctx_max=4096)
    got = op.launch(h, caches, step, debug=dbg)
    op.check()
    assert torch.equal(got, want)
    sel, _ = om.route_topk(dbg.moe_scores.cpu(), w.moe.bias.cpu(), n_group=8, topk_group=4)
    assert np.array_equal(dbg.ids.cpu().numpy()[:, 1:], sel)
