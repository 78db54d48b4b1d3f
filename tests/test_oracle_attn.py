"""The attention oracle against independent evaluations and closed forms."""

import numpy as np
import torch
import torch.nn.functional as tF

from oracle import attn as A
from oracle import formats as F
from oracle.topk import topk_sort


def _e2m1_value(nib):
    """One E2M1 code from its bit fields (sign, 2-bit exponent, 1-bit mantissa)."""
    s, e, m = (nib >> 3) & 1, (nib >> 1) & 3, nib & 1
    mag = 0.5 * m if e == 0 else 2.0 ** (e - 1) * (1 + 0.5 * m)
    return -mag if s else mag


def _tiny_plane(seed, pages=5, heads=8):
    rng = np.random.default_rng(seed)
    payload = rng.integers(0, 256, (pages, 4, 64, 16), dtype=np.uint8)
    kscale = rng.integers(123, 130, (pages, 4, 64), dtype=np.uint8)
    q = rng.integers(0, 256, (heads, 64), dtype=np.uint8)
    qs = rng.integers(123, 130, (4, 16, 4), dtype=np.uint8)
    w = (rng.normal(0, 0.05, heads)).astype(np.float32)
    table = rng.permutation(pages).astype(np.int32)
    return payload, kscale, q, qs, w, table


def test_index_scores_against_a_slot_by_slot_dequantisation():
    """Keys and queries dequantised element by element from the layout description
    (chunk c of slot s: 16 bytes at [page][c][s]; scale byte at s % 16 * 4 + s // 16;
    query scale at [c][h % 16][h // 16]), then relu(Q K^T) w as a plain matmul."""
    payload, kscale, q, qs, w, table = _tiny_plane(0)
    heads, n = q.shape[0], 4 * 64 - 9  # a ragged last page
    K = np.zeros((n, 128))
    for t in range(n):
        page, slot = table[t // 64], t % 64
        for c in range(4):
            sc = 2.0 ** (int(kscale[page, c, (slot % 16) * 4 + slot // 16]) - 127)
            for b in range(16):
                byte = int(payload[page, c, slot, b])
                K[t, 32 * c + 2 * b] = _e2m1_value(byte & 15) * sc
                K[t, 32 * c + 2 * b + 1] = _e2m1_value(byte >> 4) * sc
    Q = np.zeros((heads, 128))
    for h in range(heads):
        for c in range(4):
            sc = 2.0 ** (int(qs[c, h % 16, h // 16]) - 127)
            for b in range(16):
                byte = int(q[h, 16 * c + b])
                Q[h, 32 * c + 2 * b] = _e2m1_value(byte & 15) * sc
                Q[h, 32 * c + 2 * b + 1] = _e2m1_value(byte >> 4) * sc
    want = np.maximum(K @ Q.T, 0) @ w.astype(np.float64)
    got = A.index_scores(q, qs, w, payload, kscale, table, n)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-15)


def test_index_scores_scale_codes_are_exact_powers_of_two():
    payload, kscale, q, qs, w, table = _tiny_plane(1)
    n = 3 * 64
    base = A.index_scores(q, qs, w, payload, kscale, table, n)
    np.testing.assert_array_equal(A.index_scores(q, qs + 1, w, payload, kscale, table, n), 2 * base)
    np.testing.assert_array_equal(A.index_scores(q, qs, w, payload, kscale + 2, table, n), 4 * base)
    assert np.any(base != 0)


def test_sparse_mla_against_torch_sdpa():
    rng = np.random.default_rng(2)
    slots_total, heads = 300, 4
    kv = F.f32_to_e4m3(np.clip(rng.normal(0, 1, (slots_total, A.KV_DIM)), -448, 448).astype(np.float32))
    ks = rng.uniform(0.5, 1.5, slots_total).astype(np.float32)
    q = torch.randn(heads, A.KV_DIM, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    slots = rng.choice(slots_total, 77, replace=False)
    scale = 192 ** -0.5
    o, lse = A.sparse_mla(q, kv, ks, slots, scale)
    k = torch.from_numpy(F.e4m3_to_f32(kv[slots]).astype(np.float64) * ks[slots, None])
    want = tF.scaled_dot_product_attention(q.double()[None], k[None], k[None, :, : A.LATENT],
                                           scale=scale)[0]
    np.testing.assert_allclose(o, want.numpy(), rtol=1e-10, atol=1e-12)
    s = (q.double() @ k.T * scale).numpy()
    np.testing.assert_allclose(lse, np.log(np.exp(s).sum(-1)), rtol=1e-12)


def test_attention_row_selects_all_keys_up_to_topk_and_the_exact_topk_beyond():
    payload, kscale, q, qs, w, table = _tiny_plane(4, pages=6, heads=16)
    rng = np.random.default_rng(5)
    kv = F.f32_to_e4m3(np.clip(rng.normal(0, 1, (6 * 64, A.KV_DIM)), -448, 448).astype(np.float32))
    ks = rng.uniform(0.5, 1.5, 6 * 64).astype(np.float32)
    qa = torch.randn(4, A.KV_DIM, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    small = A.attention_row(qa, q, qs, w, payload, kscale, table, kv, ks, 40, 64, 0.1)
    assert np.array_equal(small["sel"], np.arange(41))
    big = A.attention_row(qa, q, qs, w, payload, kscale, table, kv, ks, 6 * 64 - 1, 64, 0.1)
    assert np.array_equal(big["sel"], topk_sort(big["scores"], 64))
    # the selection's slots go through the page table
    slots = table[big["sel"] // 64].astype(np.int64) * 64 + big["sel"] % 64
    o, _ = A.sparse_mla(qa, kv, ks, slots, 0.1)
    np.testing.assert_array_equal(o, big["o"])


def test_kv_rows_raw_e4m3_at_scale_one_and_scaled():
    """Without scales a row decodes as torch's float8_e4m3fn; with them each row is that
    times its token's scale."""
    rng = np.random.default_rng(9)
    kv = rng.integers(0, 256, (16, 576), dtype=np.uint8)
    kv[kv == 0x7F] = 0  # no NaN codes
    kv[kv == 0xFF] = 0
    slots = [3, 0, 15, 3]
    raw = A.kv_rows(kv, None, slots)
    want = torch.from_numpy(kv[slots]).view(torch.float8_e4m3fn).double().numpy()
    np.testing.assert_array_equal(raw, want)
    sc = np.linspace(0.5, 2.0, 16).astype(np.float32)
    np.testing.assert_array_equal(A.kv_rows(kv, sc, slots), want * sc[slots][:, None])
