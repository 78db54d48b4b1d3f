"""Exact top-k selection (test oracle): the C radix select of ``topk.c`` and a numpy
sort restatement of the same rule, which pin each other.

Rule (``sgl_amd_mono/glm53/gfx950/kernel.py:2698-2699``, ``:3002-3636``;
``glm53/check.py:94-117``): rank by the radix order key of the f32 score bits, larger
first, ties by lower position; output the selected positions in ascending order.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from .formats import radix_key

_LIB = Path(__file__).resolve().parent / "liboracle_topk.so"
_lib = None


def _c():
    global _lib
    if _lib is None:
        if not _LIB.exists():
            raise RuntimeError(f"{_LIB} missing: run `make -C oracle`")
        _lib = ctypes.CDLL(str(_LIB))
        _lib.oracle_topk.restype = ctypes.c_int
        _lib.oracle_topk.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        _lib.oracle_topk_rows.restype = None
        _lib.oracle_topk_rows.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    return _lib


def topk_sort(scores, k: int) -> np.ndarray:
    """Numpy restatement: stable sort by descending key, first k positions, ascending."""
    s = np.ascontiguousarray(scores, dtype=np.float32)
    keys = radix_key(s).astype(np.int64)
    order = np.argsort(-keys, kind="stable")[:k]
    return np.sort(order).astype(np.int32)


def topk_c(scores, k: int) -> np.ndarray:
    """The C radix select of ``topk.c`` on one row."""
    s = np.ascontiguousarray(scores, dtype=np.float32)
    out = np.empty(max(min(k, s.size), 0), dtype=np.int32)
    m = _c().oracle_topk(s.ctypes.data, s.size, k, out.ctypes.data)
    return out[:m]


def topk_rows(scores, lens, k: int) -> np.ndarray:
    """[rows, n] scores, each row over its first lens[r] entries -> [rows, k] ascending
    positions, -1 past a row's count (C radix select)."""
    s = np.ascontiguousarray(scores, dtype=np.float32)
    ln = np.ascontiguousarray(lens, dtype=np.int32)
    out = np.empty((s.shape[0], k), dtype=np.int32)
    _c().oracle_topk_rows(s.ctypes.data, s.shape[0], s.shape[1], ln.ctypes.data, k,
                          out.ctypes.data)
    return out
