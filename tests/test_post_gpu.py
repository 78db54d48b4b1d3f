"""The attention output launch (W_UV, o_proj, residual) against the CPU oracle on the
same seeded inputs.

Bars: the handed-over o within one bf16 ulp of the oracle's bf16(f64 W_UV o_lat) (the
launch sums in f32, the oracle in f64; both round once); the output within one bf16 ulp
of bf16(h + W_o o) taken over the launch's own o, and within 2e-2 max-abs + 1e-2
relative and 1e-2 relative in norm of the oracle end to end."""

import numpy as np
import pytest
import torch

from oracle import dense as D
from sgl_amd_mono_amd import layouts
from sgl_amd_mono_amd.dsv32 import synthetic
from sgl_amd_mono_amd.dsv32.post import PostOp

pytestmark = pytest.mark.gpu
ULP = 2.0 ** -7  # a bf16 ulp relative to the value, at most


@pytest.fixture(scope="module", params=[layouts.ROWMAJOR, layouts.AITER16])
def post_w(request, gpu):
    w = synthetic.post_weights(gpu, seed=3, layout=request.param)
    return w, synthetic.rowmajor_post(w)


def _inputs(rows, gpu, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    o_lat = torch.randn(rows, 32, 512, generator=g, device=gpu).to(torch.bfloat16)
    # a small residual keeps W_o o visible above h's rounding
    h = (0.01 * torch.randn(rows, 7168, generator=g, device=gpu)).to(torch.bfloat16)
    return o_lat, h


@pytest.mark.parametrize("rows", [1, 8, 16])
def test_post_matches_oracle(gpu, post_w, rows):
    w, (w_uv, s_uv, w_o, s_o) = post_w
    print(f"case post rows={rows} layout={w.layout}", flush=True)
    o_lat, h = _inputs(rows, gpu, seed=rows)
    op = PostOp(w, gpu, max_rows=16)
    o = torch.full((rows, 4096), float("nan"), dtype=torch.bfloat16, device=gpu)
    a = op.launch(o_lat, h, o=o)
    op.rt.check()
    a, o = a.float().cpu().numpy(), o.float().cpu().numpy()
    ref = D.attn_out(o_lat.cpu(), h.cpu(), w_uv, s_uv, w_o, s_o)
    assert np.all(np.abs(o - ref["o"]) <= ULP * np.abs(ref["o"]) + 1e-30)
    y_own = D.w8a16_gemv(torch.from_numpy(o).to(torch.bfloat16), w_o, s_o)
    a_own = D.bf16(h.float().cpu().numpy() + y_own)
    assert np.all(np.abs(a - a_own) <= ULP * np.abs(a_own) + 1e-30)
    want = ref["a"].astype(np.float64)
    assert np.linalg.norm(a - want) <= 1e-2 * np.linalg.norm(want)
    assert np.all(np.abs(a - want) <= 2e-2 + 1e-2 * np.abs(want))


def test_post_deterministic_and_graph_replay(gpu, post_w):
    w, _ = post_w
    print(f"case post determinism + graph layout={w.layout}", flush=True)
    o_lat, h = _inputs(8, gpu, seed=21)
    op = PostOp(w, gpu, max_rows=8)
    a = op.launch(o_lat, h).clone()
    b = op.launch(o_lat, h).clone()
    op.rt.check()
    assert torch.equal(a, b)
    out = torch.empty_like(a)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        op.launch(o_lat, h, out=out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        op.launch(o_lat, h, out=out)
    for i in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, a), f"replay {i}"
        op.launch(o_lat, h)
        torch.cuda.synchronize()
    op.rt.check()


def test_post_deadline_stops_and_reports(gpu, post_w):
    """o_proj's wait for the W_UV outputs is forced to stall from the host: it times out
    after 5 ms, every CTA exits, the output is all NaN, the host raises, and a reset
    launches cleanly."""
    w, _ = post_w
    print(f"case post fault injection site=o layout={w.layout}", flush=True)
    o_lat, h = _inputs(2, gpu, seed=9)
    op = PostOp(w, gpu, max_rows=2, deadline_s=0.005, fault=(7, 0))
    bad = op.launch(o_lat, h)
    torch.cuda.synchronize()
    assert torch.isnan(bad.float()).all()
    with pytest.raises(RuntimeError, match="timed out at o "):
        op.rt.check()
    words = op.rt.guard.cpu().tolist()
    assert words[3] == 8 and words[5] == 1
    op.fault = (0, 0)
    op.rt.reset()
    op.rt.set_deadline(10.0)
    clean = op.launch(o_lat, h).clone()
    op.rt.check()
    ref = PostOp(w, gpu, max_rows=2).launch(o_lat, h)
    torch.cuda.synchronize()
    assert torch.equal(clean, ref)
