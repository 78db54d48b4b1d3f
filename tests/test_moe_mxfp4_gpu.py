"""MXFP4 (A16W4) routed MoE launch (config 4) against the CPU oracle.

Bars: router top-8 ids bit-exact given the launch's own sigmoid scores (lowest-id
ties) and equal to the oracle's wherever the 8th/9th keys are apart by more than the
1-ulp sigmoid difference; scores within 1e-6 relative of torch's f32 sigmoid; the MoE sum y
within 1e-2 relative (norm) and cos >= 0.9999 of the oracle on the launch's routing;
out = bf16(res + y) within 2e-2 max-abs + 1e-2 relative (bf16, fp32 accumulation)."""

import numpy as np
import pytest
import torch

from oracle import moe as omoe
from sgl_amd_mono_amd.dsv32 import synthetic
from sgl_amd_mono_amd.dsv32.config import MXFP4_MOE
from sgl_amd_mono_amd.dsv32.moe import MoeMxfp4Op, MoeRouting

pytestmark = pytest.mark.gpu
H, E = MXFP4_MOE.hidden, MXFP4_MOE.experts


@pytest.fixture(scope="module")
def mx_rowmajor(gpu):
    return synthetic.mxfp4_moe_weights(gpu, seed=0)


@pytest.fixture(scope="module")
def mx_aiter(gpu):
    return synthetic.mxfp4_moe_weights(gpu, seed=0, layout="aiter16")


class _Experts:
    """Row-major expert bytes on the host, fetched per expert id as the oracle asks."""

    def __init__(self, w, part):
        self.w, self.part, self.cache = w, part, {}

    def __getitem__(self, e):
        e = int(e)
        if e not in self.cache:
            self.cache[e] = synthetic.rowmajor_mxfp4_expert(self.w, e)
        return self.cache[e][self.part]


def _oracle(w, x, logits, res, routing=None):
    shared = {}
    parts = [_Experts(w, k) for k in range(4)]
    for p in parts:
        p.cache = shared
    return omoe.moe_mxfp4(x.cpu(), logits.cpu(), w.bias.cpu(), *parts,
                          route_scale=MXFP4_MOE.route_scale, residual=res, routing=routing)


def _routing(rows, dev):
    return MoeRouting(scores=torch.empty(rows, E, dtype=torch.float32, device=dev),
                      ids=torch.empty(rows, 9, dtype=torch.int32, device=dev),
                      weights=torch.empty(rows, 9, dtype=torch.float32, device=dev))


@pytest.mark.parametrize("rows,layout,with_res", [(1, "rowmajor", False), (8, "rowmajor", True),
                                                  (16, "rowmajor", False), (1, "aiter16", True),
                                                  (8, "aiter16", False), (16, "aiter16", True)])
def test_moe_mxfp4_matches_oracle(request, gpu, rows, layout, with_res):
    print(f"case rows={rows} layout={layout} res={with_res}", flush=True)
    w = request.getfixturevalue("mx_rowmajor" if layout == "rowmajor" else "mx_aiter")
    op = MoeMxfp4Op(w, gpu, max_rows=16)
    x = synthetic.rows_bf16(rows, H, gpu, seed=rows)
    logits = synthetic.logits_f32(rows, E, gpu, seed=rows)
    res = synthetic.rows_bf16(rows, H, gpu, seed=100 + rows) if with_res else None
    y = torch.full((rows, H), float("nan"), dtype=torch.float32, device=gpu)
    rt = _routing(rows, gpu)
    out = op.launch(x, logits, res=res, y=y, routing=rt)
    op.rt.check()
    ids, wts = rt.ids.cpu().numpy(), rt.weights.cpu().numpy()
    scores = rt.scores.cpu()
    bias = w.bias.cpu()
    sel, sel_w = omoe.route_topk(scores, bias)
    assert np.array_equal(ids[:, 1:], sel), "router ids differ"
    assert np.all(ids[:, 0] == 256) and np.all(wts[:, 0] == 1.0)
    np.testing.assert_allclose(wts[:, 1:], sel_w, rtol=2e-6, atol=1e-7)
    ref = _oracle(w, x, logits, res.cpu() if res is not None else None, routing=(ids, wts))
    np.testing.assert_allclose(scores.numpy(), ref["scores"].numpy(), rtol=1e-6, atol=0)
    got, want = y.cpu().double(), ref["y"].double()
    rel = float((got - want).norm() / want.norm())
    cos = float(torch.nn.functional.cosine_similarity(got.flatten(), want.flatten(), dim=0))
    print(f"rows={rows} y rel={rel:.3e} cos={cos:.6f}", flush=True)
    assert rel <= 1e-2 and cos >= 0.9999, (rel, cos)
    o = out.cpu().float()
    assert torch.all((o - ref["out"]).abs() <= 2e-2 + 1e-2 * ref["out"].abs())
    # the oracle's own routing on torch's sigmoid agrees wherever the keys are apart
    own, _ = omoe.route_topk(ref["scores"], bias)
    key = (ref["scores"] + bias).numpy()
    srt = -np.sort(-key, 1)
    clear = (srt[:, 7] - srt[:, 8]) > 1e-6
    assert clear.mean() > 0.5
    assert np.array_equal(np.sort(own[clear], 1), np.sort(ids[clear, 1:], 1))


def test_moe_mxfp4_is_deterministic_and_writes_only_its_rows(mx_aiter, gpu):
    print("case mxfp4 determinism rows=8", flush=True)
    op = MoeMxfp4Op(mx_aiter, gpu, max_rows=16)
    x = synthetic.rows_bf16(8, H, gpu, seed=42)
    logits = synthetic.logits_f32(8, E, gpu, seed=42)
    full = torch.full((16, H), 7.0, dtype=torch.bfloat16, device=gpu)
    r1 = op.launch(x, logits, res=x, out=full[:8]).clone()
    r2 = op.launch(x, logits, res=x).clone()
    r3 = op.launch(x, logits, res=x).clone()
    op.rt.check()
    assert torch.equal(r1, r2) and torch.equal(r2, r3)
    assert torch.all(full[8:] == 7.0), "wrote past its rows"


def test_moe_mxfp4_graph_replay_matches_eager(mx_aiter, gpu):
    print("case mxfp4 graph replay rows=4", flush=True)
    op = MoeMxfp4Op(mx_aiter, gpu, max_rows=16)
    x = synthetic.rows_bf16(4, H, gpu, seed=7)
    logits = synthetic.logits_f32(4, E, gpu, seed=7)
    out = torch.empty(4, H, dtype=torch.bfloat16, device=gpu)
    eager = op.launch(x, logits).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        op.launch(x, logits, out=out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        op.launch(x, logits, out=out)
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        op.launch(x, logits)
        torch.cuda.synchronize()
    op.rt.check()


def test_moe_mxfp4_deadline_stops_and_reports(mx_rowmajor, gpu):
    """The down stage's wait for the mid tiles is forced to stall from the host; it
    times out after 5 ms, every CTA exits, the output is all NaN, the host raises, and a
    reset runtime launches cleanly again."""
    print("case mxfp4 fault injection site=mid", flush=True)
    x = synthetic.rows_bf16(2, H, gpu, seed=3)
    logits = synthetic.logits_f32(2, E, gpu, seed=3)
    op = MoeMxfp4Op(mx_rowmajor, gpu, max_rows=16, deadline_s=0.005, fault=(2, 0))
    bad = op.launch(x, logits)
    torch.cuda.synchronize()
    assert torch.isnan(bad.float()).all()
    with pytest.raises(RuntimeError, match="mid"):
        op.rt.check()
    words = op.rt.guard.cpu().tolist()
    assert words[3] == 3 and words[5] == 1
    op.fault = (0, 0)
    op.rt.reset()
    op.rt.set_deadline(10.0)
    clean = op.launch(x, logits).clone()
    op.rt.check()
    ref = MoeMxfp4Op(mx_rowmajor, gpu, max_rows=16).launch(x, logits)
    torch.cuda.synchronize()
    assert torch.equal(clean, ref)
