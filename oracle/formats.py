"""Number formats of the hot path, restated on the CPU (numpy / torch).

Reference rules followed:

* E4M3 (``float8_e4m3fn``): the FP8 weights, KV cache and activation blocks.
  Values widen exactly (``common/ops.py:333-346``); the f32 -> E4M3 pack rounds to
  nearest even after the caller clamps to +-448 (``common/ops.py:259-262``,
  ``glm53/gfx950/kernel.py:1440-1450``).
* E8M0 scale = 2^(b - 127) (``common/mx.py:15-37``,
  ``test/kernels/deepseek_v41/check_ffn.py:107-114``).
* E2M1 nibbles, even index in the low nibble, the 16-entry table of
  ``test/kernels/deepseek_v41/check_ffn.py:22-39`` and ``:107-114``.
* Per-128 FP8 activation quant ``quant_scaled`` (``glm53/gfx950/kernel.py:1440-1450``).
* The radix order key of f32 bits (``glm53/gfx950/kernel.py:2698-2699``,
  ``glm53/check.py:94-97``).

Pinned by (``tests/test_oracle_formats.py``): torch's own ``float8_e4m3fn`` and
``float8_e8m0fnu`` conversions (library routines) over every code and a dense sweep
of f32 values; the reference's E2M1 table; closed forms for the quant (the block's
amax maps to +-448 exactly, dequant error within half an E4M3 ulp); the radix key's
order against ``sorted`` on f32 values including +-0 and +-inf.
"""

from __future__ import annotations

import numpy as np
import torch

FP8_MAX = 448.0
# f32 constant the reference multiplies amax by (``amax * (1.0 / FP8_MAX)``)
INV_FP8_MAX = np.float32(1.0 / 448.0)

# the reference's E2M1 value table (check_ffn.py:22-39): nibble -> value
E2M1 = np.array(
    [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
    dtype=np.float32,
)


def _e4m3_table() -> np.ndarray:
    """f32 value of each of the 256 E4M3 codes, from the bit fields (NaN at 0x7F/0xFF)."""
    b = np.arange(256, dtype=np.int64)
    sign = np.where(b >> 7, -1.0, 1.0)
    exp = (b >> 3) & 15
    man = b & 7
    mag = np.where(exp == 0, man * 2.0**-9, (1.0 + man / 8.0) * np.exp2(exp - 7.0))
    mag = np.where((exp == 15) & (man == 7), np.nan, mag)
    return (sign * mag).astype(np.float32)


E4M3_VALUES = _e4m3_table()
# non-negative finite codes 0..126 are increasing in value
_POS = E4M3_VALUES[:127].astype(np.float64)


def e4m3_to_f32(codes) -> np.ndarray:
    """Widen E4M3 codes (uint8 array) to f32 exactly."""
    return E4M3_VALUES[np.asarray(codes, dtype=np.uint8)]


def f32_to_e4m3(x) -> np.ndarray:
    """Round f32 values (already within +-448) to E4M3 codes, nearest even."""
    x = np.asarray(x, dtype=np.float32)
    if np.any(np.abs(x) > FP8_MAX) or np.any(np.isnan(x)):
        raise ValueError("f32_to_e4m3: clamp to +-448 first")
    a = np.abs(x).astype(np.float64)
    hi = np.searchsorted(_POS, a, side="left").clip(0, 126)
    lo = (hi - 1).clip(0, 126)
    dlo, dhi = a - _POS[lo], _POS[hi] - a
    take_hi = (dhi < dlo) | ((dhi == dlo) & (hi % 2 == 0))
    code = np.where(take_hi, hi, lo)
    code = np.where(a == _POS[hi], hi, code)
    sign = np.signbit(x).astype(np.int64) << 7
    # -0.0 keeps its sign bit, as the hardware pack does
    return (code | sign).astype(np.uint8)


def e8m0_to_f32(codes) -> np.ndarray:
    """E8M0 scale codes -> 2^(b - 127) (255 is NaN)."""
    b = np.asarray(codes, dtype=np.float64)
    v = np.exp2(b - 127.0)
    return np.where(b == 255, np.nan, v).astype(np.float32)


# byte -> (value of the low nibble, value of the high nibble)
_E2M1_PAIRS = np.stack([E2M1[np.arange(256) & 15], E2M1[np.arange(256) >> 4]], axis=-1)


def unpack_e2m1(packed) -> np.ndarray:
    """[..., K/2] uint8 (even index in the low nibble) -> [..., K] f32 values."""
    p = np.asarray(packed, dtype=np.uint8)
    return _E2M1_PAIRS[p].reshape(*p.shape[:-1], p.shape[-1] * 2)


def dequant_mxfp4(packed, scales) -> np.ndarray:
    """MXFP4 rows: [N, K/2] E2M1 + [N, K/32] E8M0 -> [N, K] f32
    (``check_ffn.py:107-114``)."""
    v = unpack_e2m1(packed)
    s = e8m0_to_f32(scales)
    return v * np.repeat(s, 32, axis=-1)


def dequant_fp8_block128(w, scales) -> np.ndarray:
    """FP8 weight with 128x128 f32 block scales: [N, K] E4M3 codes + [N/128, K/128] f32
    -> [N, K] f32 (the scale layout of SGLang's ``weight_scale_inv``, read by
    ``glm53/gfx950/kernel.py:847-875``)."""
    v = e4m3_to_f32(w)
    s = np.asarray(scales, dtype=np.float32)
    return v * np.repeat(np.repeat(s, 128, axis=-2), 128, axis=-1)[..., : v.shape[-2], : v.shape[-1]]


def quant_scaled_128(x):
    """Per-128 FP8 activation quant (``glm53/gfx950/kernel.py:1440-1450``).

    For each 128-block of the last axis: amax = max|x|; scale = amax * (1/448)
    (1 when amax == 0); q = E4M3(clamp(x * (448 / amax), +-448)). The reference
    forms 448/amax with ``v_rcp_f32``; this restatement and the HIP kernels use the
    IEEE f32 quotient, so they agree bit for bit with each other.
    Returns (codes uint8 [..., K], scales f32 [..., K/128])."""
    x = np.asarray(x, dtype=np.float32)
    k = x.shape[-1]
    if k % 128:
        raise ValueError("quant_scaled_128: K must be a multiple of 128")
    g = x.reshape(*x.shape[:-1], k // 128, 128)
    amax = np.abs(g).max(axis=-1)
    nz = amax > 0
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = np.where(nz, amax * INV_FP8_MAX, np.float32(1.0)).astype(np.float32)
        inv = np.where(nz, np.float32(FP8_MAX) / amax, np.float32(1.0)).astype(np.float32)
    q = np.clip(g * inv[..., None], -FP8_MAX, FP8_MAX).astype(np.float32)
    return f32_to_e4m3(q).reshape(x.shape), scale


def bf16_round(x) -> np.ndarray:
    """f32 -> bf16 -> f32, round to nearest even (torch's conversion)."""
    t = torch.as_tensor(np.asarray(x, dtype=np.float32))
    return t.to(torch.bfloat16).float().numpy()


def radix_key(x) -> np.ndarray:
    """The order key of f32 values (``glm53/gfx950/kernel.py:2698-2699``): bits >= 0
    (as int32) -> bits ^ 0x80000000, else ~bits. Larger key ranks first; +0 ranks
    above -0."""
    b = np.asarray(x, dtype=np.float32).view(np.int32).astype(np.int64)
    return np.where(b >= 0, b + (1 << 31), (~b) & 0xFFFFFFFF).astype(np.uint32)
