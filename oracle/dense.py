"""The dense projections of the layer, restated on the CPU (test infrastructure only).

W8A16 GEMV (``sgl_amd_mono/glm53/gfx950/kernel.py:823-875`` ``unit_fp8x2``, ``:1061-1213``):
FP8 E4M3 weights [N, K] with f32 block scales [N/128, K/128] (SGLang's
``weight_scale_inv``), bf16 activations; every product is exact and the sums are taken
in f64 here (the kernel sums in f32).

The attention output block (``kernel.py:3975-4197``): the merged latent o_lat [R, 32,
512] (bf16) goes through W_UV per head ([32, 128, 512]) to o [R, 4096], handed over in
bf16; o_proj ([7168, 4096]) and the residual add of the W == 1 reduce
(``kernel.py:1665-1669``): a = bf16(h + W_o o).

Pinned by ``tests/test_oracle_dense.py``: an identity weight returns the activations
exactly; one block's scale doubled changes exactly that block's share; per-head
grouping against a block-diagonal dense matrix.
"""

from __future__ import annotations

import numpy as np
import torch

from . import formats as F


def dequant_f64(w, s) -> np.ndarray:
    """[N, K] E4M3 codes + [N/128, K/128] f32 block scales -> f64 [N, K], exact (an E4M3
    value times an f32 scale fits a double)."""
    v = F.e4m3_to_f32(np.asarray(w)).astype(np.float64)
    sc = np.asarray(s, dtype=np.float64)
    return v * np.repeat(np.repeat(sc, 128, axis=-2), 128, axis=-1)[..., : v.shape[-2], : v.shape[-1]]


def w8a16_gemv(x, w, s) -> np.ndarray:
    """x [R, K] (bf16 values), w [N, K] E4M3 codes, s [N/128, K/128] f32 -> f64 [R, N]."""
    xf = torch.as_tensor(x).double()
    return (xf @ torch.from_numpy(dequant_f64(w, s)).T).numpy()


def bf16(x) -> np.ndarray:
    return torch.as_tensor(np.asarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def attn_out(o_lat, h, w_uv, s_uv, w_o, s_o, uv=None):
    """o_lat [R, H, 512] bf16 values; h [R, 7168]; w_uv [H, 128, 512] + s_uv [H, 1, 4];
    w_o [7168, H * 128] + s_o [56, H]. Returns dict(o bf16-rounded f32 [R, H * 128],
    y f64 [R, 7168] = W_o o, a bf16-rounded f32 = h + y). ``uv(o_lat_h [R, 512], h) ->
    [R, 128]`` replaces the W_UV GEMV (w_uv / s_uv may then be None)."""
    o_lat = np.asarray(torch.as_tensor(o_lat).float())
    heads = o_lat.shape[1]
    if uv is None:
        uv = lambda x, i: w8a16_gemv(x, w_uv[i], s_uv[i])  # noqa: E731
    o = np.concatenate([np.asarray(uv(o_lat[:, i], i), np.float64) for i in range(heads)], -1)
    o = bf16(o)
    y = w8a16_gemv(o, w_o, s_o)
    a = bf16(np.asarray(torch.as_tensor(h).float()) + y)
    return dict(o=o, y=y, a=a)
