"""The MoE half of the layer, restated on the CPU (torch f32 / f64 on the host).

Follows the reference monokernel's stages:

* post-attention RMSNorm + router GEMV + sigmoid (``glm53/gfx950/kernel.py:4199-4330``)
* sigmoid + bias top-8 with lowest-id ties, route weights raw / sum * 2.5, slot 0 the
  shared expert with weight 1 (``kernel.py:1575-1629``, ``kernel.py:4332-4350``)
* FP8 W8A8 expert up/gate + SiLU (``kernel.py:4352-4999``, unit ``unit_f8f8`` ``:847-875``)
* mid per-128 quant, expert down, route weighting, residual (``kernel.py:5001-5187``)
* the MXFP4 A16W4 experts of config 4 (``minimax_m31/a16w4.py:1-92``; route as
  ``test/kernels/test_minimax_m31_ffn.py:146-151``; mid kept in bf16 as ``:139-141``)

Pinned by (``tests/test_oracle_moe.py``): route selection against a brute-force sort
on tiny inputs with ties and +-0; the W8A8 expert against an independent f64 matmul
of dequantised weights with the activations' quantise-dequantise (closed form: the
block scales factor out of each 128-chunk); linearity in the down weights; the shared
expert alone against ``torch.nn.functional.silu`` dense MLP; the bf16 softmax top-2
block (config 1) against a dense all-experts evaluation masked by the routing.
"""

from __future__ import annotations

import numpy as np
import torch

from . import formats as F

ROUTE_SCALE = 2.5  # DeepSeek-V3 routed_scaling_factor (glm53/check.py:39)
TOP_K = 8
N_EXPERTS = 256
SHARED = 256  # the fused shared expert's id (glm53/check.py:38)
RMS_EPS = 1e-6


def rmsnorm(x, gamma, eps=RMS_EPS):
    """f32 RMSNorm (``kernel.py:1367-1414``): x * rsqrt(mean(x^2) + eps) * gamma."""
    x = torch.as_tensor(x).float()
    g = torch.as_tensor(gamma).float()
    var = (x * x).mean(-1, keepdim=True)
    return x * torch.rsqrt(var + eps) * g


def router_logits(xn, w_r):
    """Router GEMV on bf16 activations and bf16 weights, f32 accumulation
    (``kernel.py:4207-4330``: the normalised rows are staged as bf16)."""
    xb = torch.as_tensor(xn).float().to(torch.bfloat16).double()
    return (xb @ torch.as_tensor(w_r).double().T).float()


def sigmoid(logits):
    """score = 1 / (1 + exp(-logit)) in f32 (``kernel.py:4326-4329``)."""
    return torch.sigmoid(torch.as_tensor(logits).float())


def group_mask(choice, n_group, topk_group):
    """Group-limited routing (DeepSeek-V3's noaux_tc, as SGLang's ``biased_grouped_topk``
    computes it): experts in n_group groups of consecutive ids; a group scores the f32 sum
    of its two largest choice values (larger first); the topk_group best groups stay, ties
    to the lower group. Returns a bool mask [R, E] of the experts left."""
    c = np.asarray(choice, dtype=np.float32)
    r, e = c.shape
    g = c.reshape(r, n_group, e // n_group)
    top2 = -np.sort(-g, axis=-1)[..., :2]
    gscore = (top2[..., 0] + top2[..., 1]).astype(np.float32)  # one f32 add, larger first
    order = np.lexsort((np.broadcast_to(np.arange(n_group), gscore.shape), -gscore), axis=-1)
    keep = np.zeros((r, n_group), bool)
    np.put_along_axis(keep, order[:, :topk_group], True, axis=-1)
    return np.repeat(keep, e // n_group, axis=-1)


def route_topk(scores, bias, top_k=TOP_K, route_scale=ROUTE_SCALE, n_group=1, topk_group=1):
    """Top-k of (score + bias) by the radix order key, lowest expert id among equal
    keys (``kernel.py:1575-1629``). Weights = score[pick] / sum(score[picks]) *
    route_scale, picks in selection order. With n_group > 1, only the experts of the
    groups ``group_mask`` keeps take part (the others rank below every real key).
    Returns (ids int32 [R, k], weights f32 [R, k])."""
    s = np.asarray(torch.as_tensor(scores).float(), dtype=np.float32)
    b = np.asarray(torch.as_tensor(bias).float(), dtype=np.float32)
    keys = F.radix_key((s + b).astype(np.float32)).astype(np.int64)
    if n_group > 1:
        keys = np.where(group_mask((s + b).astype(np.float32), n_group, topk_group), keys, -1)
    n = s.shape[-1]
    # descending key, then ascending id: sort by (-key, id)
    order = np.lexsort((np.broadcast_to(np.arange(n), keys.shape), -keys), axis=-1)
    ids = order[..., :top_k].astype(np.int32)
    raw = np.take_along_axis(s, ids, axis=-1).astype(np.float64)
    w = raw / raw.sum(-1, keepdims=True) * route_scale
    return ids, w.astype(np.float32)


def slots_with_shared(ids, weights):
    """[R, 1 + k] slot tables: slot 0 the shared expert (id 256, weight 1), then the
    picks (``kernel.py:4343-4350``)."""
    r = ids.shape[0]
    sid = np.concatenate([np.full((r, 1), SHARED, np.int32), ids], axis=1)
    sw = np.concatenate([np.ones((r, 1), np.float32), weights], axis=1)
    return sid, sw


def _w8a8_gemv(w_codes, w_scales, xq, xs):
    """y[n] = sum_kb (sum_{k in kb} W[n,k] q[k]) * sw[n//128, kb] * xs[kb], in f64.
    ``w_codes`` [N, K] E4M3, ``w_scales`` [N/128, K/128] f32, ``xq`` [M, K] E4M3,
    ``xs`` [M, K/128] -> [M, N] f64 (``kernel.py:847-875``)."""
    wv = torch.from_numpy(F.e4m3_to_f32(w_codes)).double()
    qv = torch.from_numpy(F.e4m3_to_f32(xq)).double()
    n, k = wv.shape
    kb = k // 128
    part = torch.einsum("nbk,mbk->mnb", wv.view(n, kb, 128), qv.view(-1, kb, 128))
    sw = torch.from_numpy(np.asarray(w_scales, np.float32)).double()
    sw = sw.repeat_interleave(128, 0)[:n]  # [N, KB]
    sx = torch.from_numpy(np.asarray(xs, np.float32)).double()  # [M, KB]
    return (part * sw[None] * sx[:, None, :]).sum(-1)


def silu_mul(gate, up):
    """SwiGLU: silu(g) * u = g * sigmoid(g) * u (``kernel.py:4398-4404``)."""
    g = torch.as_tensor(gate).float()
    return g * torch.sigmoid(g) * torch.as_tensor(up).float()


def expert_fp8(e, xq, xs, w13, s13, w2, s2, inter):
    """One FP8 expert on quantised rows: (mid f32 [M, inter]) and a callable giving
    the down projection of a quantised mid. Shapes: w13 [E, 2*inter, H] E4M3 codes,
    s13 [E, 2*inter/128, H/128], w2 [E, H, inter], s2 [E, H/128, inter/128]."""
    h = _w8a8_gemv(w13[e], s13[e], xq, xs).float()
    return silu_mul(h[:, :inter], h[:, inter:])


def moe_fp8(a, g_post, w_r, bias, w13, s13, w2, s2, eps=RMS_EPS, route_scale=ROUTE_SCALE,
            top_k=TOP_K, experts=None, routing=None):
    """The FFN half of the layer with FP8 128x128 block-scaled W8A8 experts.

    a: bf16/f32 [R, H] (the residual stream after attention). Returns a dict with
    ``logits``/``scores`` f32 [R, 256], ``ids``/``weights`` [R, 9] (slot 0 shared),
    ``y`` f32 [R, H] (the MoE sum), ``out`` bf16-rounded f32 [R, H] = a + y.
    ``experts`` optionally maps id -> (w13, s13, w2, s2) views when only the routed
    experts are resident (the CPU baseline's on-the-fly dequant). ``routing`` = (ids
    [R, 9], weights [R, 9]) replaces the oracle's own routing, to compare the expert
    arithmetic of a launch on its own routing."""
    a = torch.as_tensor(a).float()
    xn = rmsnorm(a, g_post, eps)
    logits = router_logits(xn, w_r) if w_r is not None else None
    scores = sigmoid(logits) if logits is not None else None
    if routing is None:
        ids, wts = route_topk(scores, bias, top_k, route_scale)
        sid, sw = slots_with_shared(ids, wts)
    else:
        sid = np.asarray(routing[0], dtype=np.int64)
        sw = np.asarray(routing[1], dtype=np.float32)
    xq, xs = F.quant_scaled_128(xn.numpy())
    r, hdim = a.shape
    inter = (w2[0].shape[-1]) if experts is None else experts[SHARED][2].shape[-1]
    y = torch.zeros(r, hdim, dtype=torch.float64)
    for e in np.unique(sid):
        rows, slots = np.nonzero(sid == e)
        if experts is None:
            ew13, es13, ew2, es2 = w13[e], s13[e], w2[e], s2[e]
        else:
            ew13, es13, ew2, es2 = experts[int(e)]
        hh = _w8a8_gemv(ew13, es13, xq[rows], xs[rows]).float()
        mid = silu_mul(hh[:, :inter], hh[:, inter:]).numpy()
        mq, ms = F.quant_scaled_128(mid)
        coef = ms * sw[rows, slots][:, None]  # route weight folded into the mid scale
        y[rows] += _w8a8_gemv(ew2, es2, mq, coef)
    y = y.float()
    out = (a + y).to(torch.bfloat16).float()
    return dict(xn=xn, logits=logits, scores=scores, ids=sid, weights=sw, y=y, out=out,
                xq=xq, xs=xs)


def moe_mxfp4(x, logits, bias, w13, s13, w2, s2, route_scale=ROUTE_SCALE, top_k=TOP_K,
              residual=None, routing=None):
    """Config 4: MXFP4 (E2M1 + E8M0 per 32) A16W4 experts on bf16 rows.

    x bf16 [R, H]; logits f32 [R, 256] given; route sigmoid + bias top-k as
    ``test_minimax_m31_ffn.py:146-151`` (lowest-id ties). Expert: h = x @ W13^T
    (f32), mid = bf16(silu(gate) * up) (the A16W4 launch keeps mid in bf16,
    ``test_minimax_m31_ffn.py:132-141``), y_e = mid @ W2^T, y = sum_slots w * y_e
    (shared expert slot 0, weight 1). w13 [E, 2*inter, H/2] uint8 + s13 [E, 2*inter,
    H/32] E8M0; w2 [E, H, inter/2] + s2 [E, H, inter/32] (anything indexable by expert
    id). ``routing`` = (ids [R, 9], weights [R, 9]) replaces the oracle's own routing."""
    xf = torch.as_tensor(x).float().double()
    scores = sigmoid(logits)
    if routing is None:
        ids, wts = route_topk(scores, bias, top_k, route_scale)
        sid, sw = slots_with_shared(ids, wts)
    else:
        sid = np.asarray(routing[0], dtype=np.int64)
        sw = np.asarray(routing[1], dtype=np.float32)
    r, hdim = xf.shape
    inter = w2[SHARED].shape[-1] * 2
    y = torch.zeros(r, hdim, dtype=torch.float64)
    for e in np.unique(sid):
        rows, slots = np.nonzero(sid == e)
        wg = torch.from_numpy(F.dequant_mxfp4(w13[e], s13[e])).double()
        h = (xf[rows] @ wg.T).float()
        mid = silu_mul(h[:, :inter], h[:, inter:]).to(torch.bfloat16).double()
        wd = torch.from_numpy(F.dequant_mxfp4(w2[e], s2[e])).double()
        y[rows] += (mid @ wd.T) * torch.from_numpy(sw[rows, slots]).double()[:, None]
    y = y.float()
    out = y if residual is None else torch.as_tensor(residual).float() + y
    return dict(scores=scores, ids=sid, weights=sw, y=y,
                out=out.to(torch.bfloat16).float())


def moe_softmax_bf16(x, w_r, w1, w3, w2, top_k=2):
    """Config 1 (CPU plumbing): bf16 weights, softmax router, top-2 renormalised,
    SwiGLU experts. x [R, H]; w_r [E, H]; w1, w3 [E, I, H]; w2 [E, H, I].
    Softmax over all experts, top-k by probability with lowest-id ties, weights
    renormalised to sum 1 (SGLang's ``fused_topk(renormalize=True)``). Returns
    (ids [R, k], weights [R, k], y f32 [R, H])."""
    xf = torch.as_tensor(x).float()
    logits = xf @ torch.as_tensor(w_r).float().T
    p = torch.softmax(logits, -1)
    ids, _ = route_topk(p, torch.zeros(p.shape[-1]), top_k, 1.0)
    raw = np.take_along_axis(p.numpy(), ids, axis=-1).astype(np.float64)
    wts = (raw / raw.sum(-1, keepdims=True)).astype(np.float32)
    y = torch.zeros_like(xf)
    for e in np.unique(ids):
        rows, ks = np.nonzero(ids == e)
        g = xf[rows] @ torch.as_tensor(w1[e]).float().T
        u = xf[rows] @ torch.as_tensor(w3[e]).float().T
        ye = silu_mul(g, u) @ torch.as_tensor(w2[e]).float().T
        y[rows] += ye * torch.from_numpy(wts[rows, ks])[:, None]
    return ids, wts, y
