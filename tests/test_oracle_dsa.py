"""The DSA (FP8) index-page oracle: the page layout against the reference's page decode,
the key and query chains against closed forms, the scores against constructed pages."""

import numpy as np

from oracle import attn as A
from oracle import formats as F
from oracle import front as Fr

S128 = np.array([[(-1) ** bin(i & j).count("1") for j in range(128)] for i in range(128)],
                np.float64)  # Sylvester order: S[i, j] = (-1)^popcount(i & j)


def _e4m3_bytes(rng, shape):
    """Random E4M3 codes without the two NaN encodings."""
    b = rng.integers(0, 256, shape, dtype=np.uint8)
    return np.where((b & 0x7F) == 0x7F, b ^ 1, b).astype(np.uint8)


def test_dsa_tiled_layout_is_the_reference_page_decode():
    """Every (token, dim) has its own byte of the 8192; the reference's decode
    (glm53/check.py:61-64: token = (b // 2048) * 16 + (b % 256) // 16) maps it back."""
    off, d = np.meshgrid(np.arange(64), np.arange(128), indexing="ij")
    b = Fr.dsa_value_offset(off, d, tiled=True)
    assert np.array_equal(np.sort(b.ravel()), np.arange(8192))
    assert np.array_equal((b // 2048) * 16 + (b % 256) // 16, off)
    assert np.array_equal(((b % 2048) // 256) * 16 + b % 16, d)
    b = Fr.dsa_value_offset(off, d, tiled=False)
    assert np.array_equal(b, off * 128 + d)


def test_dsa_keys_against_a_byte_by_byte_decode():
    rng = np.random.default_rng(5)
    pages = np.zeros((3, Fr.DSA_PAGE_BYTES), np.uint8)
    pages[:, :8192] = _e4m3_bytes(rng, (3, 8192))
    scales = np.exp2(rng.integers(-12, 4, (3, 64))).astype(np.float32)
    pages[:, 8192:] = scales.view(np.uint8).reshape(3, 256)
    table = [2, 0, 1]  # the request's pages
    for tiled in (True, False):
        want = np.zeros((192, 128))
        for p in range(3):
            for b in range(8192):
                tok, dim = ((b // 2048) * 16 + (b % 256) // 16, ((b % 2048) // 256) * 16 + b % 16) \
                    if tiled else (b // 128, b % 128)
                pos = table.index(p) * 64 + tok
                want[pos, dim] = F.e4m3_to_f32(pages[p, b]) * scales[p, tok]
        got = A.dsa_keys(pages, table, 192, tiled=tiled)
        assert np.array_equal(got, want), tiled
        cols = np.array([5, 130, 64, 191])
        assert np.array_equal(A.dsa_keys(pages, table, 192, cols=cols, tiled=tiled), want[cols])


def _one_hot_key(j, c):
    k = np.zeros((1, 128))
    k[0, j] = c
    return k


def test_index_key_fp8_of_a_one_hot_key_is_a_closed_form():
    """k = c e_j, LayerNorm weight 1 and bias 0, no rotation (cos 1, sin 0): the normalised
    key is c (e_j - 1/128) rstd and its transform rstd c (S[j] - e_0) / sqrt(128), so every
    value but the first has magnitude amax = rstd c / sqrt(128)."""
    c, j = 3.0, 77
    rstd = 1.0 / np.sqrt(c * c * 127.0 / 128.0 ** 2 + 1e-6)
    amax = rstd * c / np.sqrt(128.0)
    one, zero = np.ones((1, 32)), np.zeros((1, 32))
    got = Fr.index_key_fp8(_one_hot_key(j, c), np.ones(128), np.zeros(128), one, zero)
    want_t = amax * (S128[j] - np.eye(128)[0])
    np.testing.assert_allclose(got["pre"][0], want_t, rtol=1e-13, atol=1e-15)
    sc = float(got["scale"][0])
    m, e = np.frexp(np.float32(amax) / np.float32(448.0))
    assert sc == (2.0 ** (e - 1) if m == 0.5 else 2.0 ** e)
    mag = F.f32_to_e4m3(np.array([amax / sc]))[0]
    want = np.where(S128[j] > 0, mag, mag | 0x80).astype(np.uint8)
    assert np.array_equal(got["codes"][0, 1:], want[1:])
    assert got["codes"][0, 0] & 0x7F == 0  # a zero (its sign is the rounding noise's)


def test_index_key_fp8_scale_sees_the_unrounded_transform():
    """The LayerNorm weight puts amax at 448 2^-4 (1 + 2^-10): the scale is 2^-3; a chain
    that rounded the transform's output to bf16 first would see amax = 28 and pick 2^-4."""
    c, j = 3.0, 77
    rstd = 1.0 / np.sqrt(c * c * 127.0 / 128.0 ** 2 + 1e-6)
    target = 448.0 * 2.0 ** -4 * (1.0 + 2.0 ** -10)
    g = np.full(128, target / (rstd * c / np.sqrt(128.0)))
    got = Fr.index_key_fp8(_one_hot_key(j, c), g, np.zeros(128), np.ones((1, 32)), np.zeros((1, 32)))
    assert float(got["scale"][0]) == 2.0 ** -3
    assert float(Fr.pow2_ceil(Fr.bf16(np.abs(got["pre"]).max()) / 448.0)) == 2.0 ** -4


def test_index_key_fp8_rotates_the_leading_pairs():
    """A key whose centred values sit on dims 0, 1 only (k = (a, -a, 0 ..)): the rotation by
    theta takes the pair to a (cos + sin, sin - cos) before the transform."""
    a, th = 2.0, 0.7
    k = np.zeros((1, 128))
    k[0, 0], k[0, 1] = a, -a
    rstd = 1.0 / np.sqrt(2 * a * a / 128.0 + 1e-6)
    cs, sn = np.full((1, 32), np.cos(th)), np.full((1, 32), np.sin(th))
    got = Fr.index_key_fp8(k, np.ones(128), np.zeros(128), cs, sn)
    r0 = a * rstd * (np.cos(th) + np.sin(th))
    r1 = a * rstd * (np.sin(th) - np.cos(th))
    want = (r0 * S128[0] + r1 * S128[1]) / np.sqrt(128.0)
    np.testing.assert_allclose(got["pre"][0], want, rtol=1e-12, atol=1e-14)


def test_index_query_bf16_rounds_once_after_the_transform():
    """A two-hot query on dims 0, 1 rotated by theta: its transform is (r0 +- r1) / sqrt(128)
    (even / odd columns), rounded to bf16 once. The values are chosen so that rounding the
    rotated pair to bf16 first changes the result."""
    a, b = Fr.bf16(np.array([1.3671875, 0.59765625]))
    th = 0.3
    r0 = a * np.cos(th) - b * np.sin(th)
    r1 = a * np.sin(th) + b * np.cos(th)
    want = Fr.bf16(np.where(np.arange(128) % 2 == 0, r0 + r1, r0 - r1) / np.sqrt(128.0))
    early = Fr.bf16(np.where(np.arange(128) % 2 == 0, Fr.bf16(r0) + Fr.bf16(r1),
                             Fr.bf16(r0) - Fr.bf16(r1)) / np.sqrt(128.0))
    assert not np.array_equal(want, early)  # the case tells the two apart
    q = np.zeros((1, 64, 128))
    q[0, 9, 0], q[0, 9, 1] = a, b
    got = Fr.index_query_bf16(q, np.full((1, 32), np.cos(th)), np.full((1, 32), np.sin(th)))
    assert np.array_equal(got[0, 9], want)
    assert np.all(got[0, np.arange(64) != 9] == 0)


def test_dsa_scores_of_one_hot_queries_and_keys():
    """Token t's key: E4M3 value v_t on dim d_t, scale s_t; head h's query: a_h on dim e_h.
    s_t = sum_h w_h relu(a_h v_t s_t [e_h == d_t])."""
    rng = np.random.default_rng(7)
    for tiled in (True, False):
        pages = np.zeros((2, Fr.DSA_PAGE_BYTES), np.uint8)
        d = rng.integers(0, 8, 128)
        code = _e4m3_bytes(rng, 128)
        s = np.exp2(rng.integers(-6, 3, 128)).astype(np.float32)
        for t in range(128):
            codes = np.zeros(128, np.uint8)
            codes[d[t]] = code[t]
            Fr.dsa_page_write(pages, (1 - t // 64) * 64 + t % 64, codes, s[t], tiled)
        e = rng.integers(0, 8, 64)
        av = Fr.bf16(rng.normal(0, 1, 64))
        q = np.zeros((64, 128))
        q[np.arange(64), e] = av
        w = rng.normal(0, 1, 64)
        v = F.e4m3_to_f32(code).astype(np.float64)
        want = np.array([np.sum(w * np.maximum(av * v[t] * s[t] * (e == d[t]), 0.0))
                         for t in range(128)])
        got = A.index_scores_fp8(q, w, pages, [1, 0], 128, tiled=tiled)
        np.testing.assert_allclose(got, want, rtol=1e-14, atol=1e-300)
