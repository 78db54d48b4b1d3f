"""The MoE oracle against brute force, closed forms and independent evaluations."""

import itertools

import numpy as np
import torch
import torch.nn.functional as tF

from oracle import formats as F
from oracle import moe as M


def _brute_topk(score, bias, k):
    """Sort the (key, id) pairs by hand: larger f32 (score + bias) first, ties by lower
    id, with -0 below +0 (the radix order of the f32 bits)."""
    v = (np.float32(score) + np.float32(bias)).astype(np.float32)
    def key(i):
        x = float(v[i])
        return (x, 1 if (x == 0 and not np.signbit(v[i])) else 0, -i)
    return sorted(range(len(v)), key=key, reverse=True)[:k]


def test_route_topk_brute_force_with_ties_and_signed_zero():
    rng = np.random.default_rng(0)
    for trial in range(200):
        n = 16
        # few distinct values: many exact ties, and zeros of both signs
        s = rng.choice(np.array([0.25, 0.5, 0.75, 0.0], np.float32), n)
        b = rng.choice(np.array([0.0, -0.0, 0.25, -0.25], np.float32), n)
        ids, w = M.route_topk(s[None], b, top_k=5, route_scale=2.5)
        want = _brute_topk(s, b, 5)
        assert ids[0].tolist() == want, (trial, s, b)


def test_route_weights_closed_form():
    s = np.array([[0.9, 0.1, 0.8, 0.3]], np.float32)
    ids, w = M.route_topk(s, np.zeros(4, np.float32), top_k=2, route_scale=2.5)
    assert ids.tolist() == [[0, 2]]
    np.testing.assert_allclose(w[0], [0.9 / 1.7 * 2.5, 0.8 / 1.7 * 2.5], rtol=1e-6)


def _brute_grouped(score, bias, k, n_group, topk_group):
    """Group-limited top-k by hand: each group's two largest choice values summed (the
    larger first), groups ranked by that sum (ties to the lower group), the kept groups'
    experts ranked as ``_brute_topk`` ranks them."""
    v = (np.float32(score) + np.float32(bias)).astype(np.float32)
    gs = len(v) // n_group
    sums = []
    for g in range(n_group):
        a, b2 = sorted(v[g * gs:(g + 1) * gs].tolist(), reverse=True)[:2]
        sums.append(float(np.float32(a) + np.float32(b2)))
    groups = sorted(range(n_group), key=lambda g: (sums[g], -g), reverse=True)[:topk_group]
    keep = [i for i in range(len(v)) if i // gs in groups]
    def key(i):
        x = float(v[i])
        return (x, 1 if (x == 0 and not np.signbit(v[i])) else 0, -i)
    return sorted(keep, key=key, reverse=True)[:k]


def test_grouped_route_against_brute_force_with_ties():
    rng = np.random.default_rng(7)
    for trial in range(300):
        n_group, topk_group = [(2, 1), (4, 2), (8, 4), (8, 2), (16, 8)][trial % 5]
        n = 64 if n_group <= 8 else 128
        s = rng.choice(np.array([0.25, 0.5, 0.75, 0.875, 0.0], np.float32), n)
        b = rng.choice(np.array([0.0, 0.125, -0.125], np.float32), n)
        k = min(8, topk_group * n // n_group)
        ids, _ = M.route_topk(s[None], b, top_k=k, n_group=n_group, topk_group=topk_group)
        assert ids[0].tolist() == _brute_grouped(s, b, k, n_group, topk_group), trial


def test_grouped_route_drops_the_best_expert_of_a_weak_group():
    """Expert 0 alone has the largest score, but its group's second best is tiny: with
    8 groups keeping 4, group 0 loses to four groups of two good experts each, so expert
    0 is not picked although plain routing picks it first."""
    s = np.full((1, 256), 0.01, np.float32)
    s[0, 0] = 0.99
    for g in (1, 2, 3, 4):
        s[0, 32 * g] = s[0, 32 * g + 1] = 0.6
    b = np.zeros(256, np.float32)
    plain, _ = M.route_topk(s, b)
    grouped, _ = M.route_topk(s, b, n_group=8, topk_group=4)
    assert plain[0, 0] == 0
    assert 0 not in grouped[0].tolist()
    assert sorted(grouped[0].tolist())[:8] == sorted([32, 33, 64, 65, 96, 97, 128, 129])
    # one group: the same as plain routing
    one, _ = M.route_topk(s, b, n_group=1, topk_group=1)
    assert np.array_equal(one, plain)


def test_w8a8_gemv_equals_dequantised_matmul():
    rng = np.random.default_rng(1)
    n, k = 256, 384
    w = F.f32_to_e4m3(np.clip(rng.normal(0, 1, (n, k)), -448, 448).astype(np.float32))
    sw = rng.uniform(0.5, 2, (n // 128, k // 128)).astype(np.float32) / 448
    x = rng.normal(0, 1, (3, k)).astype(np.float32)
    xq, xs = F.quant_scaled_128(x)
    got = M._w8a8_gemv(w, sw, xq, xs).numpy()
    # dequantise in f64: the block scales factor out of each 128-chunk exactly
    wd = F.e4m3_to_f32(w).astype(np.float64) * np.repeat(np.repeat(sw, 128, 0), 128, 1)
    xd = (F.e4m3_to_f32(xq).astype(np.float64).reshape(3, -1, 128) * xs[..., None]).reshape(3, k)
    np.testing.assert_allclose(got, xd @ wd.T, rtol=1e-9, atol=1e-15)


def _tiny_fp8_layer(h=256, inter=128, e=4, seed=0):
    g = torch.Generator().manual_seed(seed)
    w13 = torch.randn(e + 1, 2 * inter, h, generator=g).to(torch.float8_e4m3fn).view(torch.uint8)
    w2 = torch.randn(e + 1, h, inter, generator=g).to(torch.float8_e4m3fn).view(torch.uint8)
    s13 = (0.5 + 1.5 * torch.rand(e + 1, 2 * inter // 128, h // 128, generator=g)) / 448
    s2 = (0.5 + 1.5 * torch.rand(e + 1, h // 128, inter // 128, generator=g)) / 448
    return w13.numpy(), s13.numpy(), w2.numpy(), s2.numpy()


def test_moe_fp8_shared_only_is_a_dense_swiglu():
    """With every route weight 0, y is the shared expert's SwiGLU on the quantised rows."""
    h, inter = 256, 128
    w13, s13, w2, s2 = _tiny_fp8_layer(h, inter)
    x = torch.randn(3, h, generator=torch.Generator().manual_seed(5))
    g_post = torch.ones(h)
    ids = np.array([[4, 0], [4, 1], [4, 2]])  # slot 0 shared (id 4 in this tiny layer)
    wts = np.array([[1.0, 0.0]] * 3, np.float32)
    M_SHARED, M.SHARED = M.SHARED, 4
    try:
        ref = M.moe_fp8(x, g_post, None, None, w13, s13, w2, s2, routing=(ids, wts),
                        experts={i: (w13[i], s13[i], w2[i], s2[i]) for i in range(5)})
    finally:
        M.SHARED = M_SHARED
    xn = M.rmsnorm(x, g_post).numpy()
    xq, xs = F.quant_scaled_128(xn)
    xd = torch.from_numpy((F.e4m3_to_f32(xq).reshape(3, -1, 128) * xs[..., None]).reshape(3, h))
    wg = torch.from_numpy(F.dequant_fp8_block128(w13[4], s13[4]))
    hh = xd.double() @ wg.double().T
    mid = (tF.silu(hh[:, :inter]) * hh[:, inter:]).float().numpy()
    mq, ms = F.quant_scaled_128(mid)
    md = torch.from_numpy((F.e4m3_to_f32(mq).reshape(3, -1, 128) * ms[..., None]).reshape(3, inter))
    want = md.double() @ torch.from_numpy(F.dequant_fp8_block128(w2[4], s2[4])).double().T
    np.testing.assert_allclose(ref["y"].numpy(), want.numpy(), rtol=2e-5, atol=1e-7)


def test_moe_fp8_is_linear_in_the_route_weight():
    """The route weight folds into the mid scale: doubling it doubles that expert's term."""
    h, inter = 256, 128
    w13, s13, w2, s2 = _tiny_fp8_layer(h, inter, seed=3)
    x = torch.randn(2, h, generator=torch.Generator().manual_seed(9))
    experts = {i: (w13[i], s13[i], w2[i], s2[i]) for i in range(5)}
    M_SHARED, M.SHARED = M.SHARED, 4
    try:
        def y(w):
            ids = np.array([[4, 1], [4, 1]])
            wts = np.array([[0.0, w], [0.0, w]], np.float32)
            return M.moe_fp8(x, torch.ones(h), None, None, None, None, None, None,
                             experts=experts, routing=(ids, wts))["y"].numpy()
        np.testing.assert_allclose(y(0.5) * 2, y(1.0), rtol=1e-6, atol=1e-9)
        assert np.abs(y(1.0)).max() > 0
    finally:
        M.SHARED = M_SHARED


def test_config1_softmax_top2_block_against_dense_masked():
    """Config 1 (CPU plumbing): H 1024, 8 experts, top-2 softmax, inter 512, bf16
    weights ~N(0, 0.02), 4 rows ~N(0, 1), seed 0 -- against a dense evaluation of every
    expert masked by the routing."""
    g = torch.Generator().manual_seed(0)
    h, e, inter = 1024, 8, 512
    bf = torch.bfloat16
    w_r = (torch.randn(e, h, generator=g) * 0.02).to(bf)
    w1 = (torch.randn(e, inter, h, generator=g) * 0.02).to(bf)
    w3 = (torch.randn(e, inter, h, generator=g) * 0.02).to(bf)
    w2 = (torch.randn(e, h, inter, generator=g) * 0.02).to(bf)
    x = torch.randn(4, h, generator=g).to(bf)
    ids, wts, y = M.moe_softmax_bf16(x, w_r, w1, w3, w2, top_k=2)
    xf = x.float()
    p = torch.softmax(xf @ w_r.float().T, -1)
    dense = torch.stack([(tF.silu(xf @ w1[i].float().T) * (xf @ w3[i].float().T)) @ w2[i].float().T
                         for i in range(e)], 1)  # [R, E, H]
    top = torch.topk(p, 2, -1)
    mask = torch.zeros_like(p).scatter(1, top.indices, top.values)
    mask = mask / mask.sum(-1, keepdim=True)
    want = (dense * mask[..., None]).sum(1)
    assert sorted(map(tuple, np.sort(ids, 1))) == sorted(map(tuple, np.sort(top.indices.numpy(), 1)))
    torch.testing.assert_close(y, want, rtol=1e-4, atol=1e-6)


def _e2m1_bits(codes: torch.Tensor) -> torch.Tensor:
    """E2M1 values from the bit fields (sign, 2-bit exponent, 1-bit mantissa), low
    nibble first, computed independently of the oracle's table."""
    nib = torch.stack([codes & 15, codes >> 4], -1).reshape(*codes.shape[:-1], -1).long()
    s, e, m = (nib >> 3) & 1, (nib >> 1) & 3, nib & 1
    mag = torch.where(e == 0, 0.5 * m, torch.exp2(e.double() - 1) * (1 + 0.5 * m))
    return torch.where(s == 1, -mag, mag)


def _mx_dequant(codes, scales):
    c = torch.from_numpy(np.ascontiguousarray(codes))
    sc = torch.from_numpy(np.ascontiguousarray(scales)).view(torch.float8_e8m0fnu).double()
    return _e2m1_bits(c) * sc.repeat_interleave(32, -1)


def _tiny_mx_layer(h=256, inter=128, e=4, seed=0):
    g = torch.Generator().manual_seed(seed)
    u8 = dict(dtype=torch.uint8, generator=g)
    w13 = torch.randint(0, 256, (e + 1, 2 * inter, h // 2), **u8).numpy()
    s13 = torch.randint(119, 123, (e + 1, 2 * inter, h // 32), **u8).numpy()
    w2 = torch.randint(0, 256, (e + 1, h, inter // 2), **u8).numpy()
    s2 = torch.randint(119, 123, (e + 1, h, inter // 32), **u8).numpy()
    return w13, s13, w2, s2


def _with_shared(id_, fn):
    saved, M.SHARED = M.SHARED, id_
    try:
        return fn()
    finally:
        M.SHARED = saved


def test_moe_mxfp4_against_dense_masked_evaluation():
    """The A16W4 block with its own routing against every expert evaluated densely from
    bit-field dequantised weights (F.silu, bf16 mid) and masked by torch.topk routing."""
    h, inter, e = 256, 128, 8
    w13, s13, w2, s2 = _tiny_mx_layer(h, inter, e, seed=1)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(3, h, generator=g).to(torch.bfloat16)
    logits = torch.randn(3, e, generator=g)
    bias = torch.randn(e, generator=g) * 0.01
    ref = _with_shared(e, lambda: M.moe_mxfp4(x, logits, bias, w13, s13, w2, s2, top_k=3))
    xf = x.double()
    dense = []
    for i in range(e + 1):
        hh = (xf @ _mx_dequant(w13[i], s13[i]).T).float()
        mid = (tF.silu(hh[:, :inter]) * hh[:, inter:]).to(torch.bfloat16).double()
        dense.append(mid @ _mx_dequant(w2[i], s2[i]).T)
    dense = torch.stack(dense, 1)  # [R, E + 1, H]
    sc = torch.sigmoid(logits)
    top = torch.topk(sc + bias, 3, -1).indices
    raw = sc.gather(1, top).double()
    wts = raw / raw.sum(-1, keepdim=True) * 2.5
    mask = torch.zeros(3, e + 1, dtype=torch.float64).scatter(1, top, wts)
    mask[:, e] = 1.0
    want = (dense * mask[..., None]).sum(1)
    assert np.array_equal(np.sort(ref["ids"][:, 1:], 1), np.sort(top.numpy(), 1))
    np.testing.assert_allclose(ref["y"].numpy(), want.numpy(), rtol=1e-5, atol=1e-6)


def test_moe_mxfp4_power_of_two_scales_are_exact():
    """E8M0 codes + 1 on every down scale, or on every up-row scale, doubles y exactly
    (the bf16 mid of 2u is exactly twice that of u)."""
    h, inter, e = 256, 128, 4
    w13, s13, w2, s2 = _tiny_mx_layer(h, inter, e, seed=4)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(2, h, generator=g).to(torch.bfloat16)
    ids = np.array([[e, 1], [e, 2]])
    wts = np.array([[1.0, 0.75], [1.0, 1.25]], np.float32)
    run = lambda a, b, c, d: _with_shared(e, lambda: M.moe_mxfp4(
        x, torch.zeros(2, e), torch.zeros(e), a, b, c, d, routing=(ids, wts))["y"].numpy())
    base = run(w13, s13, w2, s2)
    s2b = s2 + 1
    s13b = s13.copy()
    s13b[:, inter:] += 1
    assert np.abs(base).max() > 0
    np.testing.assert_array_equal(run(w13, s13, w2, s2b), 2 * base)
    np.testing.assert_array_equal(run(w13, s13b, w2, s2), 2 * base)
