"""ctypes binding of libmono_amd.so, the C ABI declared in ``include/mono_amd.h``.

The library is the only compute path: if it is missing or was built for another
target, ``lib()`` raises, and nothing falls back to a CPU or PyTorch implementation.
"""

from __future__ import annotations

import ctypes
import re
import threading
from ctypes import c_double, c_float, c_int32, c_size_t, c_uint32, c_void_p
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libmono_amd.so"
HEADER = PKG.parent / "include" / "mono_amd.h"

MONO_OK = 0
MONO_E_ARG = -1
MONO_E_DEVICE = -2
MONO_E_LAUNCH = -3
MONO_E_FAILED = -4

# guard block words (mono_amd.h MONO_GUARD_*)
GUARD_EPOCH = 0
GUARD_DEADLINE_LO = 1
GUARD_DEADLINE_HI = 2
GUARD_ERR_DEADLINE = 3
GUARD_ERR_PEER = 4
GUARD_ERR_FAULT = 5
GUARD_EXIT = 6
GUARD_ABORT = 7
GUARD_WORDS = 16

# index-key caches (MONO_INDEX_*): the FP4 plane, SGLang's DSA page (tiled or token-major)
INDEX_FP4_PLANE = 0
INDEX_FP8_PAGE = 1
INDEX_FP8_ROWS = 2
DSA_PAGE_BYTES = 64 * (128 + 4)

# on-HBM layouts of expert weights (MONO_LAYOUT_*)
LAYOUT_ROWMAJOR = 0
LAYOUT_AITER16 = 1

# expert weights of the layer launch (MONO_EXPERTS_*): FP8 W8A8 or MXFP4 A16W4
EXPERTS_FP8 = 0
EXPERTS_MXFP4 = 1

# timeline marks of the MoE launch (MONO_TL_*), u64 [grid, TL_COLS]
TL_MARKS = ("start", "staged", "routed", "upgate", "midq", "down", "end")
TL_COLS = 8

# wait sites (the deadline error word holds 1 + site)
SITES = {1: "logits", 2: "mid", 3: "mq", 4: "scores", 5: "topk", 6: "split", 7: "o",
         8: "front_a", 9: "q_an", 10: "q_b", 11: "phase", 12: "blocks", 13: "x"}
SITE_PHASE = 11
# timeline marks of the layer launch (same columns)
TL_LAYER_MARKS = ("start", "front", "attn", "post", "moe", "end")
SITE_MID, SITE_SCORES, SITE_TOPK, SITE_SPLIT, SITE_O = 2, 4, 5, 6, 7
SITE_FRONT_A, SITE_QAN, SITE_QB = 8, 9, 10
# timeline marks of the attention launch (same columns)
TL_ATTN_MARKS = ("start", "scores", "topk", "split", "merge", "exit", "end")


class MonoDeviceInfo(ctypes.Structure):
    _fields_ = [("cus", c_int32), ("lds_bytes", c_int32), ("is_gfx950", c_int32), ("grid", c_int32)]


class MonoMoeFp8Args(ctypes.Structure):
    """Mirror of ``MonoMoeFp8Args`` in mono_amd.h (same order and types)."""

    _fields_ = [
        ("rows", c_int32),
        ("hidden", c_int32),
        ("inter", c_int32),
        ("experts", c_int32),
        ("layout", c_int32),
        ("eps", c_float),
        ("route_scale", c_float),
        ("a", c_void_p),
        ("out", c_void_p),
        ("g_post", c_void_p),
        ("w_r", c_void_p),
        ("bias", c_void_p),
        ("w13", c_void_p),
        ("s13", c_void_p),
        ("w2", c_void_p),
        ("s2", c_void_p),
        ("y", c_void_p),
        ("scores", c_void_p),
        ("ids", c_void_p),
        ("weights", c_void_p),
        ("scratch", c_void_p),
        ("guard", c_void_p),
        ("host_error", c_void_p),
        ("fault_site", c_int32),
        ("fault_after", c_int32),
        ("timeline", c_void_p),
        ("n_group", c_int32),
        ("topk_group", c_int32),
    ]


class MonoMoeMxfp4Args(ctypes.Structure):
    """Mirror of ``MonoMoeMxfp4Args`` in mono_amd.h (same order and types)."""

    _fields_ = [
        ("rows", c_int32),
        ("hidden", c_int32),
        ("inter", c_int32),
        ("experts", c_int32),
        ("layout", c_int32),
        ("route_scale", c_float),
        ("x", c_void_p),
        ("res", c_void_p),
        ("out", c_void_p),
        ("logits", c_void_p),
        ("bias", c_void_p),
        ("w13", c_void_p),
        ("s13", c_void_p),
        ("w2", c_void_p),
        ("s2", c_void_p),
        ("y", c_void_p),
        ("scores", c_void_p),
        ("ids", c_void_p),
        ("weights", c_void_p),
        ("scratch", c_void_p),
        ("guard", c_void_p),
        ("host_error", c_void_p),
        ("fault_site", c_int32),
        ("fault_after", c_int32),
        ("timeline", c_void_p),
        ("n_group", c_int32),
        ("topk_group", c_int32),
    ]


class MonoAttnArgs(ctypes.Structure):
    """Mirror of ``MonoAttnArgs`` in mono_amd.h (same order and types)."""

    _fields_ = [
        ("rows", c_int32),
        ("rows_max", c_int32),
        ("heads", c_int32),
        ("index_heads", c_int32),
        ("topk", c_int32),
        ("page", c_int32),
        ("ctx_max", c_int32),
        ("pt_stride", c_int32),
        ("pt_rows", c_int32),
        ("plane_pages", c_uint32),
        ("kv_slots", c_uint32),
        ("sm_scale", c_float),
        ("positions", c_void_p),
        ("req_ids", c_void_p),
        ("page_table", c_void_p),
        ("q", c_void_p),
        ("iq", c_void_p),
        ("iqs", c_void_p),
        ("iw", c_void_p),
        ("plane", c_void_p),
        ("plane_scale", c_void_p),
        ("kv", c_void_p),
        ("kv_scale", c_void_p),
        ("out", c_void_p),
        ("scores", c_void_p),
        ("topk_pos", c_void_p),
        ("scratch", c_void_p),
        ("guard", c_void_p),
        ("host_error", c_void_p),
        ("fault_site", c_int32),
        ("fault_after", c_int32),
        ("timeline", c_void_p),
        ("index_format", c_int32),
    ]


class MonoPostArgs(ctypes.Structure):
    """Mirror of ``MonoPostArgs`` in mono_amd.h (same order and types)."""

    _fields_ = [
        ("rows", c_int32),
        ("heads", c_int32),
        ("hidden", c_int32),
        ("layout", c_int32),
        ("o_lat", c_void_p),
        ("h", c_void_p),
        ("w_uv", c_void_p),
        ("s_uv", c_void_p),
        ("w_o", c_void_p),
        ("s_o", c_void_p),
        ("out", c_void_p),
        ("o", c_void_p),
        ("scratch", c_void_p),
        ("guard", c_void_p),
        ("host_error", c_void_p),
        ("fault_site", c_int32),
        ("fault_after", c_int32),
        ("timeline", c_void_p),
    ]


class MonoFrontArgs(ctypes.Structure):
    """Mirror of ``MonoFrontArgs`` in mono_amd.h (same order and types)."""

    _fields_ = [
        ("rows", c_int32),
        ("hidden", c_int32),
        ("heads", c_int32),
        ("layout", c_int32),
        ("rope_rows", c_int32),
        ("kv_slots", c_uint32),
        ("plane_pages", c_uint32),
        ("eps", c_float),
        ("h", c_void_p),
        ("g_in", c_void_p),
        ("g_q", c_void_p),
        ("g_kv", c_void_p),
        ("w_qkv_a", c_void_p),
        ("s_qkv_a", c_void_p),
        ("w_k", c_void_p),
        ("s_k", c_void_p),
        ("w_w", c_void_p),
        ("g_k", c_void_p),
        ("b_k", c_void_p),
        ("w_qb", c_void_p),
        ("s_qb", c_void_p),
        ("w_iq", c_void_p),
        ("s_iq", c_void_p),
        ("w_uk", c_void_p),
        ("s_uk", c_void_p),
        ("cos", c_void_p),
        ("sin", c_void_p),
        ("positions", c_void_p),
        ("slots", c_void_p),
        ("kv", c_void_p),
        ("kv_scale", c_void_p),
        ("plane", c_void_p),
        ("plane_scale", c_void_p),
        ("q", c_void_p),
        ("iq", c_void_p),
        ("iqs", c_void_p),
        ("iw", c_void_p),
        ("scratch", c_void_p),
        ("guard", c_void_p),
        ("host_error", c_void_p),
        ("fault_site", c_int32),
        ("fault_after", c_int32),
        ("timeline", c_void_p),
        ("ik_raw", c_void_p),
        ("iq_raw", c_void_p),
        ("index_format", c_int32),
    ]


class MonoLayerArgs(ctypes.Structure):
    """Mirror of ``MonoLayerArgs`` in mono_amd.h (same order and types)."""

    _fields_ = [(n, c_int32) for n in ("rows", "rows_max", "hidden", "heads", "inter", "experts",
                                       "layout", "ctx_max", "pt_stride", "pt_rows", "rope_rows")]
    _fields_ += [("kv_slots", c_uint32), ("plane_pages", c_uint32), ("eps", c_float),
                 ("sm_scale", c_float), ("route_scale", c_float)]
    _fields_ += [(n, c_void_p) for n in (
        "h", "out", "positions", "slots", "req_ids", "page_table", "kv", "kv_scale", "plane",
        "plane_scale", "g_in", "g_q", "g_kv", "w_qkv_a", "s_qkv_a", "w_k", "s_k", "w_w", "g_k",
        "b_k", "w_qb", "s_qb", "w_iq", "s_iq", "w_uk", "s_uk", "cos", "sin", "w_uv", "s_uv",
        "w_o", "s_o", "g_post", "w_r", "bias", "w13", "s13", "w2", "s2", "q", "iq", "iqs", "iw",
        "o_lat", "a", "scores", "topk_pos", "y", "moe_scores", "ids", "weights", "scratch",
        "guard", "host_error")]
    _fields_ += [("fault_site", c_int32), ("fault_after", c_int32), ("timeline", c_void_p),
                 ("phase_timeline", c_void_p), ("n_group", c_int32), ("topk_group", c_int32),
                 ("index_format", c_int32), ("expert_format", c_int32), ("e13", c_void_p),
                 ("e2", c_void_p)]


# name -> (restype, argtypes)
SIGNATURES = {
    "mono_version": (c_int32, []),
    "mono_last_error": (ctypes.c_char_p, []),
    "mono_device_info": (c_int32, [c_int32, ctypes.POINTER(MonoDeviceInfo)]),
    "mono_set_deadline": (c_int32, [c_void_p, c_double, c_void_p]),
    "mono_reset": (c_int32, [c_void_p, c_size_t, c_void_p, c_void_p]),
    "mono_moe_fp8_scratch_bytes": (c_size_t, [c_int32, c_int32, c_int32]),
    "mono_moe_fp8_launch": (c_int32, [ctypes.POINTER(MonoMoeFp8Args), c_void_p]),
    "mono_moe_fp8_launch_static": (c_int32, [ctypes.POINTER(MonoMoeFp8Args), c_void_p]),
    "mono_moe_mxfp4_scratch_bytes": (c_size_t, [c_int32, c_int32, c_int32]),
    "mono_moe_mxfp4_launch": (c_int32, [ctypes.POINTER(MonoMoeMxfp4Args), c_void_p]),
    "mono_attn_scratch_bytes": (c_size_t, [c_int32]),
    "mono_attn_launch": (c_int32, [ctypes.POINTER(MonoAttnArgs), c_void_p]),
    "mono_post_scratch_bytes": (c_size_t, []),
    "mono_post_launch": (c_int32, [ctypes.POINTER(MonoPostArgs), c_void_p]),
    "mono_front_scratch_bytes": (c_size_t, []),
    "mono_front_launch": (c_int32, [ctypes.POINTER(MonoFrontArgs), c_void_p]),
    "mono_layer_scratch_bytes": (c_size_t, [c_int32]),
    "mono_layer_launch": (c_int32, [ctypes.POINTER(MonoLayerArgs), c_void_p]),
}

_lock = threading.Lock()
_lib = None


def header_functions() -> list[str]:
    """Every function the C header declares (``int name(`` / ``size_t name(`` ...)."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(mono_\w+)\s*\(", text, flags=re.M)


def lib() -> ctypes.CDLL:
    """The loaded library with typed entry points; raises if it is not built."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m sgl_amd_mono_amd.build` "
                    "(there is no fallback path)"
                )
            dll = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(dll, name)
                fn.restype, fn.argtypes = res, args
            _lib = dll
        return _lib


def last_error() -> str:
    msg = lib().mono_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    """Raise for a non-zero C ABI return code."""
    if rc == MONO_OK:
        return
    err = last_error()
    if rc == MONO_E_ARG:
        raise ValueError(f"{what}: {err}")
    raise RuntimeError(f"{what}: {err} (code {rc})")


def stream_handle(stream=None) -> int:
    """The hipStream_t of a torch stream (the current one by default)."""
    import torch

    s = torch.cuda.current_stream() if stream is None else stream
    return int(s.cuda_stream)
