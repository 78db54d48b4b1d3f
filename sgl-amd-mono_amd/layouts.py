"""On-HBM weight layouts the kernels read in place.

``aiter16``: AITER's (16, 16) shuffle of an [.., N, K] byte matrix into
[.., N / 16, K / 32, 2, 16 rows, 16 bytes], the layout SGLang's gfx950 MoE load leaves
FP8 expert weights in (read by ``ld_fp8_chunk``, ``sgl_amd_mono/glm53/gfx950/kernel.py:787-808``).
Element (n, k) with n = 16 rg + r and k = 32 kk + 16 h + c sits at byte
((rg * K/32 + kk) * 2 + h) * 256 + r * 16 + c. MXFP4 codes (two E2M1 a byte) use the
same byte shuffle over [.., N, K / 2].

``e8m0 shuffle``: the order of MXFP4 E8M0 scales [.., N, C] (one per 32 K values) that
pairs with ``aiter16`` codes, byte index ((((r32 * CP/8 + c8) * 4 + e) * 16 + b) * 2 + d)
* 2 + a for row 32 r32 + 16 a + b and column 8 c8 + 4 d + e
(``sgl_amd_mono/common/mx.py:40-44``), over CP = C rounded up to a multiple of 8 columns
(the map groups columns by 8; the padding columns hold zeros).
"""

from __future__ import annotations

import torch

ROWMAJOR = "rowmajor"
AITER16 = "aiter16"
LAYOUTS = (ROWMAJOR, AITER16)


def shuffle_16x16(w: torch.Tensor) -> torch.Tensor:
    """Row-major [.., N, K] (1-byte elements) -> the (16, 16) shuffle, same shape."""
    *lead, n, k = w.shape
    if n % 16 or k % 32:
        raise ValueError(f"(16, 16) shuffle needs N % 16 == 0 and K % 32 == 0, got {n}, {k}")
    v = w.reshape(*lead, n // 16, 16, k // 32, 2, 16)
    nl = len(lead)
    perm = list(range(nl)) + [nl, nl + 2, nl + 3, nl + 1, nl + 4]
    return v.permute(*perm).contiguous().reshape(w.shape)


def unshuffle_16x16(w: torch.Tensor) -> torch.Tensor:
    """Inverse of ``shuffle_16x16``."""
    *lead, n, k = w.shape
    v = w.reshape(*lead, n // 16, k // 32, 2, 16, 16)
    nl = len(lead)
    perm = list(range(nl)) + [nl, nl + 3, nl + 1, nl + 2, nl + 4]
    return v.permute(*perm).contiguous().reshape(w.shape)


def e8m0_cols(c: int) -> int:
    """Columns of a shuffled E8M0 block holding ``c`` scale columns."""
    return (c + 7) // 8 * 8


def shuffle_e8m0(s: torch.Tensor) -> torch.Tensor:
    """Row-major E8M0 scales [.., N, C] (N % 32 == 0) -> the e8m0 shuffle [.., N, CP]."""
    *lead, n, c = s.shape
    if n % 32:
        raise ValueError(f"e8m0 shuffle needs N % 32 == 0, got {n}")
    cp = e8m0_cols(c)
    pad = torch.zeros(*lead, n, cp, dtype=s.dtype, device=s.device)
    pad[..., :c] = s
    v = pad.reshape(*lead, n // 32, 2, 16, cp // 8, 2, 4)  # r32, a, b, c8, d, e
    nl = len(lead)
    perm = list(range(nl)) + [nl, nl + 3, nl + 5, nl + 2, nl + 4, nl + 1]
    return v.permute(*perm).contiguous().reshape(*lead, n, cp)


def unshuffle_e8m0(s: torch.Tensor, c: int) -> torch.Tensor:
    """Inverse of ``shuffle_e8m0``: [.., N, CP] -> [.., N, c]."""
    *lead, n, cp = s.shape
    v = s.reshape(*lead, n // 32, cp // 8, 4, 16, 2, 2)  # r32, c8, e, b, d, a
    nl = len(lead)
    perm = list(range(nl)) + [nl, nl + 5, nl + 3, nl + 1, nl + 4, nl + 2]
    return v.permute(*perm).contiguous().reshape(*lead, n, cp)[..., :c].contiguous()
