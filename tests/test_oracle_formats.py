"""The oracle's number formats against torch's conversions and closed forms."""

import numpy as np
import pytest
import torch

from oracle import formats as F


def test_e4m3_decode_matches_torch_on_every_code():
    codes = torch.arange(256, dtype=torch.uint8)
    want = codes.view(torch.float8_e4m3fn).float().numpy()
    got = F.e4m3_to_f32(codes.numpy())
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))


def test_e4m3_encode_matches_torch_rne():
    rng = np.random.default_rng(0)
    # dense sweep over the range, exact midpoints, subnormals and signed zeros
    mids = (F.E4M3_VALUES[1:126].astype(np.float64) + F.E4M3_VALUES[2:127]) / 2
    x = np.concatenate([
        rng.uniform(-448, 448, 200_000),
        rng.normal(0, 1e-2, 50_000),
        mids, -mids,
        np.array([0.0, -0.0, 448.0, -448.0, 2.0**-9, 2.0**-10, 3 * 2.0**-11]),
    ]).astype(np.float32)
    got = F.f32_to_e4m3(x)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, want)


def test_e4m3_encode_refuses_unclamped():
    with pytest.raises(ValueError):
        F.f32_to_e4m3(np.array([449.0], np.float32))


def test_e8m0_matches_torch():
    codes = torch.arange(255, dtype=torch.uint8)
    want = codes.view(torch.float8_e8m0fnu).float().numpy()
    got = F.e8m0_to_f32(codes.numpy())
    assert np.array_equal(got, want)
    assert F.e8m0_to_f32(np.array([127]))[0] == 1.0


def test_e2m1_table_is_the_bit_fields():
    # e2m1: sign, 2 exponent bits (bias 1), 1 mantissa bit; exponent 0 is subnormal
    for n in range(16):
        s, e, m = n >> 3, (n >> 1) & 3, n & 1
        mag = m * 0.5 if e == 0 else (1 + m / 2) * 2.0 ** (e - 1)
        assert F.E2M1[n] == (-mag if s else mag)
        assert np.signbit(F.E2M1[n]) == bool(s)


def test_unpack_e2m1_low_nibble_first():
    got = F.unpack_e2m1(np.array([[0x21, 0xF7]], np.uint8))
    assert got.tolist() == [[0.5, 1.0, 6.0, -6.0]]


def test_dequant_mxfp4_closed_form():
    packed = np.full((2, 16), 0x22, np.uint8)  # every value 1.0
    scales = np.array([[127], [130]], np.uint8)  # 1, 8
    v = F.dequant_mxfp4(packed, scales)
    assert np.all(v[0] == 1.0) and np.all(v[1] == 8.0)


def test_quant_scaled_closed_forms():
    rng = np.random.default_rng(1)
    x = (rng.normal(0, 1, (7, 512)) * rng.uniform(0.01, 100, (7, 1))).astype(np.float32)
    x[3, :128] = 0.0  # an all-zero block: scale 1, codes 0
    q, s = F.quant_scaled_128(x)
    assert s.shape == (7, 4) and s[3, 0] == 1.0 and not q[3, :128].any()
    deq = F.e4m3_to_f32(q).reshape(7, 4, 128) * s[..., None]
    g = x.reshape(7, 4, 128)
    amax = np.abs(g).max(-1)
    # the block's amax element maps to +-448 exactly, dequantised back to itself
    i = np.abs(g).argmax(-1)
    top = np.take_along_axis(F.e4m3_to_f32(q).reshape(7, 4, 128), i[..., None], -1)[..., 0]
    nz = amax > 0
    assert np.all(np.abs(top[nz]) == 448.0)
    # every element within half an E4M3 ulp (relative 2^-4) of its block scale grid
    err = np.abs(deq - g)
    ulp = np.maximum(np.abs(g), s[..., None] * 2.0**-6) * 2.0**-4
    assert np.all(err <= ulp * 1.0001)


def test_radix_key_orders_like_floats():
    vals = np.array([-np.inf, -3.5, -1.0, -1e-30, -0.0, 0.0, 1e-30, 1.0, 2.5, np.inf],
                    np.float32)
    keys = F.radix_key(vals)
    assert np.all(np.diff(keys.astype(np.int64)) > 0)  # strictly increasing, -0 < +0
    rng = np.random.default_rng(2)
    x = rng.normal(0, 10, 10_000).astype(np.float32)
    order_k = np.argsort(F.radix_key(x), kind="stable")
    order_f = np.argsort(x, kind="stable")
    assert np.array_equal(x[order_k], x[order_f])
