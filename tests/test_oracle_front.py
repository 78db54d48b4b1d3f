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


def test_kv_quant_unscaled_is_torchs_e4m3_cast_saturating_at_448():
    """SGLang's pool rows: raw E4M3 of the bf16 values at scale 1, beyond +-448 clipped
    (torch's cast would give NaN there)."""
    rng = np.random.default_rng(5)
    row = torch.from_numpy(rng.normal(0, 100, 576)).to(torch.bfloat16).double().numpy()
    row[:3] = [900.0, -1000.0, 448.0]
    codes, sc = Fr.kv_quant(row, scaled=False)
    assert sc == 1.0
    clipped = np.clip(row, -448.0, 448.0)
    want = torch.from_numpy(clipped).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(codes, want)
    assert F.e4m3_to_f32(codes[:3]).tolist() == [448.0, -448.0, 448.0]


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


# Known answers for the index key and query chains' bf16 rounding points. Each input is
# built so that one rounding decides an FP4 code; the expected codes are derived by hand
# in the docstrings (bf16 spacing 2^(e - 7) in [2^e, 2^(e + 1)); E2M1 grid 0, 0.5, 1, 1.5,
# 2, 3, 4, 6 with codes 0..7, ties to the even code), so dropping the rounding fails.
_IDENT = (np.ones((1, 32)), np.zeros((1, 32)))   # RoPE by angle 0: cos 1, sin 0


def _two_hot(a, b, lead=(1, 64)):
    v = np.zeros(lead + (128,))
    v[..., 0], v[..., 1] = a, b
    return v


def test_index_query_rounds_the_hadamard_output_to_bf16():
    """iq_raw = 39.5 e0 + 0.052734375 e1 in every head, RoPE by angle 0. The Hadamard
    output is (39.5 +- 0.052734375) / sqrt(128): 3.49600 at even dims, 3.48668 at odd
    ones, which bf16 makes 3.5 and 3.484375 (spacing 2^-6). amax 3.5 gives scale 1 (E8M0
    127); 3.5 is the tie of E2M1 3 and 4 and takes the even code 6; 3.484375 takes 3,
    code 5. Unrounded, 3.49600 would take code 5."""
    d = Fr.index_query(_two_hot(39.5, 0.052734375), *_IDENT)
    assert np.all(d["codes"][..., 0::2] == 6) and np.all(d["codes"][..., 1::2] == 5)
    assert np.all(d["e8"] == 127)


def test_index_query_rounds_the_rotated_half_to_bf16():
    """iq_raw dims (0, 1) = (38.5, 0.07470703125) rotated by the bf16 table pair (cos,
    sin) = (0.97265625, 0.234375): (37.429756, 9.096102), which bf16 makes (37.5, 9.125)
    (spacing 2^-2 and 2^-4). The Hadamard output: (37.5 + 9.125) / sqrt(128) = 4.12108
    at even dims (bf16 4.125, amax: scale 1) and (37.5 - 9.125) / sqrt(128) = 2.50802 at
    odd ones (bf16 2.515625, above the 2.5 tie of E2M1 2 and 3: code 5). Unrounded,
    (37.429756 - 9.096102) / sqrt(128) = 2.50436 would be bf16 2.5, the tie: code 4."""
    cs = (np.full((1, 32), 0.97265625), np.full((1, 32), 0.234375))
    d = Fr.index_query(_two_hot(38.5, 0.07470703125), *cs)
    assert np.all(d["codes"][..., 0::2] == 6) and np.all(d["codes"][..., 1::2] == 5)
    assert np.all(d["e8"] == 127)


def test_index_key_rounds_like_the_query():
    """With k = 0 and g = 0 the LayerNorm returns b exactly, so the key chain over b is the
    query chain over the same vector: both constructions above give the same codes."""
    zeros = np.zeros((1, 128))
    for a, b, cs in ((39.5, 0.052734375, _IDENT),
                     (38.5, 0.07470703125, (np.full((1, 32), 0.97265625),
                                            np.full((1, 32), 0.234375)))):
        d = Fr.index_key(zeros, np.zeros(128), _two_hot(a, b, (1,))[0], *cs)
        assert np.all(d["codes"][0, 0::2] == 6) and np.all(d["codes"][0, 1::2] == 5)
        assert np.all(d["e8"] == 127)


def test_index_key_rounds_the_norm_to_bf16():
    """k = 0.006 e0 - 0.006 e1, g = 0.515625 on dims 0 and 1, b = 0, RoPE by angle 0:
    mean 0, variance 0.006^2 / 64, so n0 = -n1 = 8 g 0.006 / sqrt(0.006^2 + 64e-6) = 2.475
    and the other dims 0; bf16 2.46875. The Hadamard output is 0 at even dims and
    2 n0 / sqrt(128) = 0.436420 at odd ones, bf16 0.435546875; scale pow2_ceil(0.4355 / 6)
    = 2^-3 (E8M0 124) and 3.484375 takes E2M1 3, code 5. Unrounded, n0 = 2.475 would give
    0.437521, bf16 0.4375, i.e. 3.5, the tie: code 6."""
    k = _two_hot(0.006, -0.006, (1,))
    g = np.ones(128)
    g[:2] = 0.515625
    d = Fr.index_key(k, g, np.zeros(128), *_IDENT)
    assert np.all(d["codes"][0, 0::2] == 0) and np.all(d["codes"][0, 1::2] == 5)
    assert np.all(d["e8"][0] == 124)
