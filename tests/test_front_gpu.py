"""The front launch against the CPU oracle (``oracle/front.py``) on the same seeded inputs.

Bars (the launch computes in f32 with hardware rsqrt, the oracle in f64, each rounding
once where the reference rounds):
* q (bf16): within 2e-2 max-abs + 1e-2 relative and 1e-2 relative in norm of the oracle;
* the head weights: within two bf16 ulps (2^-7 relative) of the oracle;
* the KV rows written at the rows' slots: the per-token scale equal to the oracle's, each
  dequantised value within one E4M3 step plus 2^-7 of the row's RMS of the oracle's bf16
  value (x may round one bf16 ulp apart under the hardware rsqrt, moving every GEMV
  output by ~2^-8 of the row's magnitude; a value near a rounding boundary then lands one
  step over);
* the FP4 index key and query, from the launch's own projections (``ik_raw`` = W_k x,
  ``iq_raw`` = W_iq q_an, checked against the oracle's to the bf16 bars above) through the
  oracle's chains (``index_key`` / ``index_query``: bf16 after the norm, after RoPE and
  after the FWHT, then FP4): the E8M0 scales equal and the codes equal, except that a
  value whose f32 rotation or transform lands within f32 rounding of a bf16 tie may take
  the other bf16 and so the adjacent E2M1 value: at most max(2, 0.05%) of the codes;
* end to end from h (q_an and the projections may round one bf16 ulp apart between the
  f32 and f64 paths; through the FWHT that moves every value of a head by ~2^-8 of the
  block's magnitude, ~0.01 in units of the scale, and with bf16 inputs an FP4 tie is
  exactly representable, so such a value can land on either side of it): codes differing
  only where the oracle's scaled value sits within 0.02 of the midpoint of two adjacent
  grid values, then only to the adjacent value, for at most 2% of the query's codes and
  4% of the keys' (a few hundred codes: a one-row case sees a handful of such ties);
* every cache slot the rows do not own unchanged, a pad row (slot -1) writes nothing."""

import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import front as Fr
from sgl_amd_mono_amd import _lib, layouts
from sgl_amd_mono_amd.dsv32 import synthetic
from sgl_amd_mono_amd.dsv32.front import FrontOp

pytestmark = pytest.mark.gpu
SLOTS, PAGES = 4096, 64


@pytest.fixture(scope="module", params=[layouts.ROWMAJOR, layouts.AITER16])
def front_w(request, gpu):
    w = synthetic.front_weights(gpu, seed=7, layout=request.param, rope_rows=SLOTS)
    return w, synthetic.rowmajor_front(w)


def _fp4_close(codes_dev, e8_dev, pre, codes_ora, e8_ora, what, max_frac=0.02):
    """Device FP4 (codes [.., n], e8 [.., n/32]) against the oracle's, as in the header."""
    assert np.array_equal(e8_dev, e8_ora), what
    sc = np.repeat(2.0 ** (e8_ora.astype(np.float64) - 127), 32, -1)
    v = np.clip(pre / sc, -6, 6)
    dv = F.E2M1[codes_dev].astype(np.float64)
    ov = F.E2M1[codes_ora].astype(np.float64)
    diff = dv != ov
    if diff.any():
        a, b = dv[diff], ov[diff]
        mid = (a + b) / 2
        assert np.all(np.abs(v[diff] - mid) <= 0.02), what
        grid = Fr.E2M1_GRID
        ia = np.searchsorted(grid, np.abs(a))
        ib = np.searchsorted(grid, np.abs(b))
        assert np.all((np.abs(ia - ib) <= 1) & (np.sign(a) * np.sign(b) >= 0)), what
        assert diff.sum() <= max_frac * diff.size, (what, int(diff.sum()))
    print(f"{what}: {int(diff.sum())} of {diff.size} codes one step apart", flush=True)
    return int(diff.sum())


def _fp4_tight(codes_dev, e8_dev, codes_ora, e8_ora, what):
    """Device FP4 against the oracle's chain over the device's own projections: scales
    equal, codes equal but for max(2, 0.05%) adjacent values (f32 vs f64 rounding at a
    bf16 tie)."""
    assert np.array_equal(e8_dev, e8_ora), what
    dv = F.E2M1[codes_dev].astype(np.float64)
    ov = F.E2M1[codes_ora].astype(np.float64)
    diff = dv != ov
    if diff.any():
        grid = Fr.E2M1_GRID
        ia = np.searchsorted(grid, np.abs(dv[diff]))
        ib = np.searchsorted(grid, np.abs(ov[diff]))
        assert np.all((np.abs(ia - ib) <= 1) & (np.sign(dv[diff]) * np.sign(ov[diff]) >= 0)), what
    assert diff.sum() <= max(2, 5e-4 * diff.size), (what, int(diff.sum()))
    if diff.any():
        print(f"{what}: {int(diff.sum())} of {diff.size} codes one step apart", flush=True)
    return int(diff.sum())


def _nibbles(b):
    b = np.asarray(b, np.uint8)
    out = np.empty(b.shape[:-1] + (b.shape[-1] * 2,), np.uint8)
    out[..., 0::2] = b & 15
    out[..., 1::2] = b >> 4
    return out


def _run_case(gpu, front_w, rows, positions, slots, seed, scaled=True):
    w, ws = front_w
    print(f"case front rows={rows} layout={w.layout} positions={positions} slots={slots} "
          f"kv_scaled={scaled}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(seed)
    h = torch.randn(rows, 7168, generator=g, device=gpu).to(torch.bfloat16)
    caches = synthetic.front_caches(gpu, SLOTS, PAGES, seed=seed)
    if not scaled:  # SGLang's pool: raw E4M3 rows, no scale array
        caches.kv_scale = None
    before = {k: getattr(caches, k).clone() for k in ("kv", "plane", "plane_scale")}
    before["kv_scale"] = caches.kv_scale.clone() if scaled else torch.ones(SLOTS, device=gpu)
    pos = torch.tensor(positions, dtype=torch.int64, device=gpu)
    sl = torch.tensor(slots, dtype=torch.int64, device=gpu)
    op = FrontOp(w, gpu, max_rows=8)
    ik_raw = torch.full((rows, 128), float("nan"), device=gpu)
    iq_raw = torch.full((rows, 64, 128), float("nan"), dtype=torch.bfloat16, device=gpu)
    out = op.launch(h, caches, pos, sl, ik_raw=ik_raw, iq_raw=iq_raw)
    op.rt.check()
    ref = Fr.front(h.cpu(), positions=np.array(positions), kv_scaled=scaled, **ws)
    # the index projections, then the key / query chains from them
    ikr = ik_raw.cpu().numpy().astype(np.float64)
    iqr = iq_raw.float().cpu().numpy().astype(np.float64)
    for got, want, name in ((ikr, ref["k"], "ik_raw"), (iqr, ref["iq_raw"], "iq_raw")):
        assert np.linalg.norm(got - want) <= 1e-2 * np.linalg.norm(want), name
        assert np.all(np.abs(got - want) <= 2e-2 + 1e-2 * np.abs(want)), name
    cs = ws["cos"].float().numpy().astype(np.float64)[np.array(positions)]
    sn = ws["sin"].float().numpy().astype(np.float64)[np.array(positions)]
    qd = Fr.index_query(iqr, cs, sn)
    kd = Fr.index_key(ikr, ws["g_k"], ws["b_k"], cs, sn)
    # q
    q = out.q.float().cpu().numpy().astype(np.float64)
    want = ref["q"]
    assert np.linalg.norm(q - want) <= 1e-2 * np.linalg.norm(want)
    assert np.all(np.abs(q - want) <= 2e-2 + 1e-2 * np.abs(want))
    # head weights
    iw = out.iw.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(iw - ref["iw"]) <= 2.0 ** -7 * np.abs(ref["iw"]) + 1e-30)
    # index query
    iq, iqs = out.iq.cpu().numpy(), out.iqs.cpu().numpy()
    e8 = np.stack([iqs[:, c, np.arange(64) % 16, np.arange(64) // 16] for c in range(4)], -1)
    _fp4_close(_nibbles(iq), e8, ref["iq_pre"], ref["iq_codes"], ref["iq_e8"], "index query")
    _fp4_tight(_nibbles(iq), e8, qd["codes"], qd["e8"], "index query from iq_raw")
    # caches
    # a reader of the unscaled pool ignores scales: every row reads at scale 1
    kv = caches.kv.cpu().numpy()
    ksc = caches.kv_scale.cpu().numpy() if scaled else np.ones(SLOTS, np.float32)
    plane, psc = caches.plane.cpu().numpy(), caches.plane_scale.cpu().numpy()
    exp_kv, exp_ksc = before["kv"].cpu().numpy().copy(), before["kv_scale"].cpu().numpy().copy()
    exp_plane, exp_psc = before["plane"].cpu().numpy().copy(), before["plane_scale"].cpu().numpy().copy()
    key_dev, key_ora = [], []
    for r, s in enumerate(slots):
        if s < 0:
            continue
        assert ksc[s] == ref["kv_scale"][r], (r, ksc[s], ref["kv_scale"][r])
        got = F.e4m3_to_f32(kv[s]).astype(np.float64) * ksc[s]
        orow = ref["kv_rows"][r]
        # E4M3's step at a value: 2^(exponent - 3), and scale 2^-9 among the subnormals
        step = np.maximum(2.0 ** (np.floor(np.log2(np.maximum(np.abs(orow), 1e-30))) - 3),
                          2.0 ** -9 * ksc[s])
        # plus upstream noise: x = bf16(rmsnorm(h) g_in) may round one ulp apart (hardware
        # rsqrt), which moves every GEMV output by ~2^-8 of the row's magnitude
        rms = np.sqrt(np.mean(orow ** 2))
        err = np.abs(got - orow) - (step + 2.0 ** -7 * rms)
        assert np.all(err <= 0), (r, int(np.argmax(err)), got[np.argmax(err)], orow[np.argmax(err)])
        page, sl_ = divmod(s, 64)
        codes = _nibbles(plane[page, :, sl_, :].reshape(-1))
        e8k = psc[page, :, (sl_ % 16) * 4 + sl_ // 16]
        key_dev.append((codes, e8k))
        key_ora.append((ref["ik"][r], ref["ik_codes"][r], ref["ik_e8"][r]))
        _fp4_tight(codes, e8k, kd["codes"][r], kd["e8"][r], f"index key {r} from ik_raw")
        exp_kv[s], exp_ksc[s] = kv[s], ksc[s]
        exp_plane[page, :, sl_, :] = plane[page, :, sl_, :]
        exp_psc[page, :, (sl_ % 16) * 4 + sl_ // 16] = e8k
    if key_dev:
        _fp4_close(np.stack([c for c, _ in key_dev]), np.stack([e for _, e in key_dev]),
                   np.stack([p for p, _, _ in key_ora]), np.stack([c for _, c, _ in key_ora]),
                   np.stack([e for _, _, e in key_ora]), "index keys", max_frac=0.04)
    assert np.array_equal(kv, exp_kv) and np.array_equal(ksc, exp_ksc)
    assert np.array_equal(plane, exp_plane) and np.array_equal(psc, exp_psc)
    return op, out


def test_front_one_row(gpu, front_w):
    _run_case(gpu, front_w, 1, [32767 % SLOTS], [123], seed=1)


def test_front_eight_rows_with_a_pad_row(gpu, front_w):
    _run_case(gpu, front_w, 8, [0, 1, 63, 64, 100, 2047, 4000, 5],
              [0, 1, 63, 64, 1000, 2047, -1, 4095], seed=8)


def test_front_unscaled_rows_read_back_without_scales(gpu, front_w):
    """Without a scale array the KV rows go into the cache as raw E4M3 (SGLang's MLA
    pool): read back as plain E4M3 values, with no scale, they match the oracle's rows."""
    _run_case(gpu, front_w, 3, [5, 700, 4095], [17, 700, 4000], seed=12, scaled=False)


def _e4m3_near(dev_codes, ora_codes, what, max_frac=0.01):
    """E4M3 codes equal, but for at most ``max_frac`` of them one step apart (the f32
    chain against the f64 one at a rounding boundary)."""
    dv = F.e4m3_to_f32(dev_codes).astype(np.float64)
    ov = F.e4m3_to_f32(ora_codes).astype(np.float64)
    diff = dv != ov
    mag = np.maximum(np.abs(dv), np.abs(ov))
    step = np.maximum(2.0 ** (np.floor(np.log2(np.maximum(mag, 1e-30))) - 3), 2.0 ** -9)
    assert np.all(np.abs(dv - ov)[diff] <= step[diff]), what
    print(f"{what}: {int(diff.sum())} of {diff.size} codes one step apart", flush=True)
    assert diff.sum() <= max(2, max_frac * diff.size), (what, int(diff.sum()))


@pytest.mark.parametrize("fmt", [_lib.INDEX_FP8_PAGE, _lib.INDEX_FP8_ROWS])
def test_front_dsa_index_pages(gpu, front_w, fmt):
    """SGLang's DSA index page instead of the FP4 plane: each row's key as E4M3 at a
    power-of-two per-token scale in its page (tiled or token-major) and the bf16 index
    query, from the launch's own projections through the oracle's DSA chains
    (``index_key_fp8`` / ``index_query_bf16``): scales equal, codes equal but for at most
    1% one step apart, the query's bf16 values equal but for at most 0.1% one ulp apart;
    every other byte of the pages unchanged, a pad row writing nothing."""
    w, ws = front_w
    rows, positions = 8, [0, 1, 63, 64, 100, 2047, 4000, 5]
    slots = [0, 1, 63, 64, 1000, 2047, -1, 4095]
    print(f"case front DSA pages fmt={fmt} layout={w.layout}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(21)
    h = torch.randn(rows, 7168, generator=g, device=gpu).to(torch.bfloat16)
    caches = synthetic.front_caches(gpu, SLOTS, PAGES, seed=21, index_format=fmt)
    before = caches.plane.cpu().numpy().copy()
    pos = torch.tensor(positions, dtype=torch.int64, device=gpu)
    sl = torch.tensor(slots, dtype=torch.int64, device=gpu)
    op = FrontOp(w, gpu, max_rows=8)
    ik_raw = torch.full((rows, 128), float("nan"), device=gpu)
    iq_raw = torch.full((rows, 64, 128), float("nan"), dtype=torch.bfloat16, device=gpu)
    out = op.launch(h, caches, pos, sl, ik_raw=ik_raw, iq_raw=iq_raw)
    op.rt.check()
    assert out.iqs is None and out.iq.dtype == torch.bfloat16
    ikr = ik_raw.cpu().numpy().astype(np.float64)
    iqr = iq_raw.float().cpu().numpy().astype(np.float64)
    cs = ws["cos"].float().numpy().astype(np.float64)[np.array(positions)]
    sn = ws["sin"].float().numpy().astype(np.float64)[np.array(positions)]
    # the query: one bf16 rounding after the rotation and the transform
    want = Fr.index_query_bf16(iqr, cs, sn)
    got = out.iq.float().cpu().numpy().astype(np.float64)
    diff = got != want
    assert np.all(np.abs(got - want)[diff] <= 2.0 ** -7 * np.abs(want)[diff]), "iq ulp"
    assert diff.sum() <= max(2, 1e-3 * diff.size), int(diff.sum())
    # the keys
    kd = Fr.index_key_fp8(ikr, ws["g_k"], ws["b_k"], cs, sn)
    pages = caches.plane.cpu().numpy()
    expect = before.copy()
    tiled = fmt == _lib.INDEX_FP8_PAGE
    for r, s in enumerate(slots):
        if s < 0:
            continue
        page, off = divmod(s, 64)
        at = Fr.dsa_value_offset(off, np.arange(128), tiled)
        scale = pages[page, 8192 + 4 * off: 8192 + 4 * off + 4].copy().view(np.float32)[0]
        assert scale == kd["scale"][r], (r, scale, kd["scale"][r])
        _e4m3_near(pages[page, at], kd["codes"][r], f"DSA key {r}")
        expect[page, at] = pages[page, at]
        expect[page, 8192 + 4 * off: 8192 + 4 * off + 4] = pages[page, 8192 + 4 * off: 8192 + 4 * off + 4]
    assert np.array_equal(pages, expect), "bytes outside the rows' keys changed"


def test_front_deterministic_and_graph_replay(gpu, front_w):
    w, _ = front_w
    print(f"case front determinism + graph layout={w.layout}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(3)
    h = torch.randn(8, 7168, generator=g, device=gpu).to(torch.bfloat16)
    caches = synthetic.front_caches(gpu, SLOTS, PAGES, seed=3)
    pos = torch.arange(8, dtype=torch.int64, device=gpu) * 7
    sl = torch.arange(8, dtype=torch.int64, device=gpu) * 9
    op = FrontOp(w, gpu, max_rows=8)
    a = op.launch(h, caches, pos, sl)
    a = [t.clone() for t in (a.q, a.iq, a.iqs, a.iw)]
    b = op.launch(h, caches, pos, sl)
    op.rt.check()
    for x, y in zip(a, (b.q, b.iq, b.iqs, b.iw)):
        assert torch.equal(x, y)
    kv0 = caches.kv.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        out = op.launch(h, caches, pos, sl)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        op.launch(h, caches, pos, sl, out=out)
    for i in range(3):
        out.q.zero_()
        out.iw.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.q, a[0]) and torch.equal(out.iw, a[3]), f"replay {i}"
        assert torch.equal(caches.kv, kv0)
        op.launch(h, caches, pos, sl)
        torch.cuda.synchronize()
    op.rt.check()


def test_front_deadline_stops_and_reports(gpu, front_w):
    """A row task's wait for the stage-A outputs is forced to stall from the host: it
    times out after 5 ms, every CTA exits, q and the index head weights are all NaN, the
    host raises, and a reset launches cleanly."""
    w, _ = front_w
    print(f"case front fault injection site=front_a layout={w.layout}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(4)
    h = torch.randn(2, 7168, generator=g, device=gpu).to(torch.bfloat16)
    caches = synthetic.front_caches(gpu, SLOTS, PAGES, seed=4)
    pos = torch.tensor([10, 20], dtype=torch.int64, device=gpu)
    sl = torch.tensor([10, 20], dtype=torch.int64, device=gpu)
    op = FrontOp(w, gpu, max_rows=2, deadline_s=0.005, fault=(8, 0))
    bad = op.launch(h, caches, pos, sl)
    torch.cuda.synchronize()
    assert torch.isnan(bad.q.float()).all() and torch.isnan(bad.iw).all()
    with pytest.raises(RuntimeError, match="timed out at front_a "):
        op.rt.check()
    words = op.rt.guard.cpu().tolist()
    assert words[3] == 9 and words[5] == 1
    op.fault = (0, 0)
    op.rt.reset()
    op.rt.set_deadline(10.0)
    clean = op.launch(h, caches, pos, sl).q.clone()
    op.rt.check()
    ref = FrontOp(w, gpu, max_rows=2).launch(h, caches, pos, sl).q
    torch.cuda.synchronize()
    assert torch.equal(clean, ref)
