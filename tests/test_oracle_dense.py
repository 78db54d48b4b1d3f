"""The dense-projection oracle against closed forms."""

import numpy as np
import torch

from oracle import dense as D
from oracle import formats as F


def _codes(x):
    return F.f32_to_e4m3(np.clip(np.asarray(x, np.float32), -448, 448))


def test_identity_weight_returns_the_activations():
    k = 256
    x = torch.randn(3, k, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    w = _codes(np.eye(k))
    s = np.ones((2, 2), np.float32)
    np.testing.assert_array_equal(D.w8a16_gemv(x, w, s), x.double().numpy())


def test_block_scale_scales_only_its_block():
    rng = np.random.default_rng(1)
    n, k = 256, 384
    w = _codes(rng.normal(0, 1, (n, k)))
    s = rng.uniform(0.5, 2, (2, 3)).astype(np.float32)
    x = torch.randn(2, k, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    base = D.w8a16_gemv(x, w, s)
    s2 = s.copy()
    s2[1, 2] *= 2
    got = D.w8a16_gemv(x, w, s2)
    xb = x.double().numpy()
    block = xb[:, 256:384] @ (F.e4m3_to_f32(w[128:, 256:384]).astype(np.float64) * s[1, 2]).T
    np.testing.assert_allclose(got[:, :128], base[:, :128], rtol=0, atol=0)
    np.testing.assert_allclose(got[:, 128:] - base[:, 128:], block, rtol=1e-12, atol=1e-12)


def test_attn_out_per_head_equals_block_diagonal():
    rng = np.random.default_rng(3)
    heads, hid = 2, 256
    o_lat = torch.randn(2, heads, 512, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    w_uv = np.stack([_codes(rng.normal(0, 1, (128, 512))) for _ in range(heads)])
    s_uv = rng.uniform(0.5, 2, (heads, 1, 4)).astype(np.float32)
    w_o = _codes(rng.normal(0, 1, (hid, heads * 128)))
    s_o = rng.uniform(0.5, 2, (hid // 128, heads)).astype(np.float32)
    h = torch.randn(2, hid, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    r = D.attn_out(o_lat, h, w_uv, s_uv, w_o, s_o)
    # block-diagonal W_UV over the concatenated latent
    big = np.zeros((heads * 128, heads * 512))
    for i in range(heads):
        big[i * 128:(i + 1) * 128, i * 512:(i + 1) * 512] = (
            F.e4m3_to_f32(w_uv[i]).astype(np.float64) * np.repeat(s_uv[i].astype(np.float64), 128, -1))
    o = o_lat.double().reshape(2, -1).numpy() @ big.T
    np.testing.assert_allclose(r["o"], D.bf16(o), rtol=0, atol=0)
    wo = F.e4m3_to_f32(w_o).astype(np.float64) * np.repeat(np.repeat(s_o.astype(np.float64), 128, 0), 128, 1)
    y = r["o"].astype(np.float64) @ wo.T
    np.testing.assert_allclose(r["y"], y, rtol=1e-12, atol=1e-10)
    np.testing.assert_array_equal(r["a"], D.bf16(h.float().numpy() + y))
