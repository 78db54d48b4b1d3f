"""On-HBM weight layouts the kernels read in place.

``aiter16``: AITER's (16, 16) shuffle of an [.., N, K] byte matrix into
[.., N / 16, K / 32, 2, 16 rows, 16 bytes], the layout SGLang's gfx950 MoE load leaves
FP8 expert weights in (read by ``ld_fp8_chunk``, ``sgl_amd_mono/glm53/gfx950/kernel.py:787-808``).
Element (n, k) with n = 16 rg + r and k = 32 kk + 16 h + c sits at byte
((rg * K/32 + kk) * 2 + h) * 256 + r * 16 + c.
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
