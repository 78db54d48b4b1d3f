"""The front-of-layer oracle against library routines, closed forms and brute force."""

import numpy as np
import scipy.linalg
import torch

from oracle import attn as A
from oracle import formats as F
from oracle import front as Fr


def test_rmsnorm_and_layernorm_match_torch():
    rng = np.random.default_rng(0)
    x = rng.normal(0, 3, (5, 1536))
    g = rng.normal(1, 0.1, 1536)
    b = rng.normal(0, 0.1, 1536)
    want = torch.nn.functional.rms_norm(torch.from_numpy(x), (1536,), torch.from_numpy(g), 1e-6)
    np.testing.assert_allclose(Fr.rmsnorm(x, g, 1e-6), want.numpy(), rtol=1e-13, atol=0)
    want = torch.nn.functional.layer_norm(torch.from_numpy(x), (1536,), torch.from_numpy(g),
                                          torch.from_numpy(b), 1e-6)
    np.testing.assert_allclose(Fr.layernorm(x, g, b), want.numpy(), rtol=1e-12, atol=1e-13)


def test_rope_is_a_complex_rotation_and_inverts():
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, (3, 64))
    th = rng.uniform(-np.pi, np.pi, 32)
    got = Fr.rope(x, np.cos(th), np.sin(th))
    z = (x[:, 0::2] + 1j * x[:, 1::2]) * np.exp(1j * th)
    np.testing.assert_allclose(got[:, 0::2], z.real, atol=1e-14)
    np.testing.assert_allclose(got[:, 1::2], z.imag, atol=1e-14)
    np.testing.assert_allclose(Fr.rope(got, np.cos(th), -np.sin(th)), x, atol=1e-14)


def test_fwht_is_the_orthonormal_sylvester_hadamard():
    rng = np.random.default_rng(2)
    x = rng.normal(0, 1, (4, 128))
    h = scipy.linalg.hadamard(128) / np.sqrt(128.0)
    np.testing.assert_allclose(Fr.fwht128(x), x @ h.T, atol=1e-13)
    np.testing.assert_allclose(Fr.fwht128(Fr.fwht128(x)), x, atol=1e-13)
    e = np.zeros(128)
    e[0] = 1.0
    np.testing.assert_allclose(Fr.fwht128(e), np.full(128, 128 ** -0.5), atol=1e-15)


def test_pow2_ceil_against_log2():
    xs = np.array([1e-30, 0.1, 0.25, 0.26, 1.0, 1.5, 2.0, 3.0, 448.0, 1000.0, 2.0 ** -120])
    want = 2.0 ** np.ceil(np.log2(xs))
    np.testing.assert_array_equal(Fr.pow2_ceil(xs), want)


def test_fp4_codes_are_nearest_with_ties_to_even():
    vals = np.linspace(-7, 7, 2801)
    codes = Fr.fp4_codes(vals)
    deq = F.E2M1[codes].astype(np.float64)
    for v, d in zip(vals, deq):
        a = min(abs(v), 6.0)
        dist = np.abs(Fr.E2M1_GRID - a)
        best = np.flatnonzero(dist == dist.min())
        idx = best[0] if len(best) == 1 else best[best % 2 == 0][0]
        assert abs(d) == Fr.E2M1_GRID[idx], v
    # ties: 0.25 -> 0 (even), 0.75 -> 1.0, 1.25 -> 1.0, 1.75 -> 2.0, 2.5 -> 2, 3.5 -> 4, 5 -> 4
    got = F.E2M1[Fr.fp4_codes(np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]))]
    np.testing.assert_array_equal(got, [0.0, 1.0, 1.0, 2.0, 2.0, 4.0, 4.0])


def test_fp4_block_scale_rule_and_bound():
    rng = np.random.default_rng(3)
    v = rng.normal(0, 2, (6, 128))
    v[0, :32] = 0.0
    codes, e8, deq = Fr.fp4_block(v)
    blocks = v.reshape(6, 4, 32)
    amax = np.abs(blocks).max(-1)
    sc = 2.0 ** (e8.astype(np.float64) - 127)
    assert np.all(sc * 6.0 >= amax) and np.all(sc * 3.0 < np.maximum(amax, 6 * 2.0 ** -126))
    err = np.abs(deq - v).reshape(6, 4, 32)
    assert np.all(err <= sc[..., None] * 1.0 + 1e-12)  # half the widest step (2) of the grid


def test_kv_quant_scale_and_roundtrip():
    rng = np.random.default_rng(4)
    row = torch.from_numpy(rng.normal(0, 2, 576)).to(torch.bfloat16).double().numpy()
    codes, sc = Fr.kv_quant(row)
    assert sc == 2.0 ** np.ceil(np.log2(np.abs(row).max() / 448))
    back = F.e4m3_to_f32(codes).astype(np.float64) * sc
    want = torch.from_numpy(row / sc).to(torch.float8_e4m3fn).double().numpy() * sc
    np.testing.assert_array_equal(back, want)


def test_plane_and_query_bytes_read_back_through_the_attention_oracle():
    rng = np.random.default_rng(5)
    pages = 3
    plane = np.zeros((pages, 4, 64, 16), np.uint8)
    psc = np.zeros((pages, 4, 64), np.uint8)
    keys = rng.normal(0, 1, (130, 128))
    kc, ke, kd = Fr.fp4_block(keys)
    table = np.array([2, 0, 1])
    for t in range(130):
        Fr.plane_write(plane, psc, table[t // 64] * 64 + t % 64, kc[t], ke[t])
    vals, kexp = A.index_keys(plane, psc, table, 130)
    np.testing.assert_array_equal(vals.reshape(130, 128) * np.repeat(2.0 ** kexp, 32, -1), kd)
    q = rng.normal(0, 1, (2, 64, 128))
    qc, qe, qd = Fr.fp4_block(q)
    iq, iqs = Fr.iq_bytes(qc, qe)
    for r in range(2):
        v, e = A.index_query(iq[r], iqs[r])
        np.testing.assert_array_equal(v.reshape(64, 128) * np.repeat(2.0 ** e, 32, -1), qd[r])
