"""The C ABI: the library loads, exports every function the header declares, and the
ctypes mirrors have the C layout (no GPU needed: no compute call is made)."""

import ctypes
import subprocess

import pytest

from sgl_amd_mono_amd import _lib, guard


def test_library_exports_every_header_function():
    dll = _lib.lib()
    names = _lib.header_functions()
    assert len(names) >= 7
    for n in names:
        assert hasattr(dll, n), n
    assert set(names) == set(_lib.SIGNATURES), "every declared function has a typed binding"
    assert dll.mono_version() == 1


def _c_layout(struct, fields, tmp_path):
    src = tmp_path / "layout.c"
    body = "".join(f'printf("%zu ", offsetof({struct}, {f}));' for f in fields)
    src.write_text(f'#include <stdio.h>\n#include <stddef.h>\n#include "mono_amd.h"\n'
                   f'int main(void) {{ {body} printf("%zu\\n", sizeof({struct})); return 0; }}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(_lib.HEADER.parent), str(src), "-o", str(exe)], check=True)
    return [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True,
                                            check=True).stdout.split()]


@pytest.mark.parametrize("cls,cname", [(_lib.MonoMoeFp8Args, "MonoMoeFp8Args"),
                                        (_lib.MonoMoeMxfp4Args, "MonoMoeMxfp4Args"),
                                        (_lib.MonoAttnArgs, "MonoAttnArgs"),
                                        (_lib.MonoPostArgs, "MonoPostArgs"),
                                        (_lib.MonoFrontArgs, "MonoFrontArgs"),
                                        (_lib.MonoLayerArgs, "MonoLayerArgs"),
                                        (_lib.MonoDeviceInfo, "MonoDeviceInfo")])
def test_ctypes_mirrors_match_the_c_layout(cls, cname, tmp_path):
    fields = [f for f, _ in cls._fields_]
    want = _c_layout(cname, fields, tmp_path)
    got = [getattr(cls, f).offset for f in fields] + [ctypes.sizeof(cls)]
    assert got == want


def test_null_args_are_refused_without_a_gpu():
    rc = _lib.lib().mono_moe_fp8_launch(None, None)
    assert rc == _lib.MONO_E_ARG and "null" in _lib.last_error()
    args = _lib.MonoMoeFp8Args(rows=0, experts=256)
    assert _lib.lib().mono_moe_fp8_launch(ctypes.byref(args), None) == _lib.MONO_E_ARG
    assert _lib.lib().mono_moe_mxfp4_launch(None, None) == _lib.MONO_E_ARG
    mx = _lib.MonoMoeMxfp4Args(rows=17, experts=256)
    assert _lib.lib().mono_moe_mxfp4_launch(ctypes.byref(mx), None) == _lib.MONO_E_ARG
    assert "rows" in _lib.last_error()
    at = _lib.MonoAttnArgs(rows=8, rows_max=8, heads=32, index_heads=64, topk=2048, page=64,
                           ctx_max=163841)
    assert _lib.lib().mono_attn_launch(ctypes.byref(at), None) == _lib.MONO_E_ARG
    assert "ctx_max" in _lib.last_error()
    at = _lib.MonoAttnArgs(rows=9, rows_max=8, heads=32, index_heads=64, topk=2048, page=64,
                           ctx_max=4096)
    assert _lib.lib().mono_attn_launch(ctypes.byref(at), None) == _lib.MONO_E_ARG
    assert "rows_max" in _lib.last_error()
    po = _lib.MonoPostArgs(rows=17, heads=32, hidden=7168)
    assert _lib.lib().mono_post_launch(ctypes.byref(po), None) == _lib.MONO_E_ARG
    assert "rows" in _lib.last_error()
    fr = _lib.MonoFrontArgs(rows=9, hidden=7168, heads=32)
    assert _lib.lib().mono_front_launch(ctypes.byref(fr), None) == _lib.MONO_E_ARG
    assert "rows" in _lib.last_error()
    po = _lib.MonoPostArgs(rows=4, heads=16, hidden=7168)
    assert _lib.lib().mono_post_launch(ctypes.byref(po), None) == _lib.MONO_E_ARG
    assert "32 heads" in _lib.last_error()
    ly = _lib.MonoLayerArgs(rows=9, rows_max=8, hidden=7168, heads=32, inter=512, experts=256)
    assert _lib.lib().mono_layer_launch(ctypes.byref(ly), None) == _lib.MONO_E_ARG
    assert "rows" in _lib.last_error()
    ly = _lib.MonoLayerArgs(rows=8, rows_max=8, hidden=7168, heads=32, inter=384, experts=256)
    assert _lib.lib().mono_layer_launch(ctypes.byref(ly), None) == _lib.MONO_E_ARG
    assert "intermediate 512" in _lib.last_error()
    ly = _lib.MonoLayerArgs(rows=8, rows_max=8, hidden=7168, heads=32, inter=512, experts=256,
                            ctx_max=4096, pt_stride=64, pt_rows=8, rope_rows=4096, kv_slots=64,
                            plane_pages=1)
    assert _lib.lib().mono_layer_launch(ctypes.byref(ly), None) == _lib.MONO_E_ARG
    assert "null tensor" in _lib.last_error()


def test_scratch_bytes_only_for_built_geometries():
    assert _lib.lib().mono_moe_fp8_scratch_bytes(7168, 512, 256) > 0
    assert _lib.lib().mono_moe_fp8_scratch_bytes(7168, 384, 256) == 0
    assert _lib.lib().mono_moe_mxfp4_scratch_bytes(3072, 384, 256) > 0
    assert _lib.lib().mono_moe_mxfp4_scratch_bytes(3072, 512, 256) == 0
    assert _lib.lib().mono_attn_scratch_bytes(48) > 0 and _lib.lib().mono_attn_scratch_bytes(49) == 0
    # sized by the rows it serves: 8 rows need about a sixth of 48 rows' scratch
    assert 5 * _lib.lib().mono_attn_scratch_bytes(8) < _lib.lib().mono_attn_scratch_bytes(48)
    assert _lib.lib().mono_post_scratch_bytes() >= 16 * 4096 * 2
    assert _lib.lib().mono_front_scratch_bytes() > 0
    assert _lib.lib().mono_layer_scratch_bytes(8) > _lib.lib().mono_attn_scratch_bytes(8)
    assert _lib.lib().mono_layer_scratch_bytes(9) == 0


def test_deadline_ticks_bounds():
    # the 100 MHz clock: a second is 10^8 ticks; deadlines lie in (0, 1 h]
    assert guard.deadline_ticks(1.0) == 100_000_000
    assert guard.deadline_ticks(3600) == 360_000_000_000
    for bad in (3600.5, 0, -1.0):
        with pytest.raises(ValueError, match="wait deadline"):
            guard.deadline_ticks(bad)
    assert guard.watchdog_deadline(300) == 60.0 and guard.watchdog_deadline(30) == 15.0


def test_fault_injection_env(monkeypatch):
    monkeypatch.setenv(guard.FAULT_ENV, "1:3:5")
    assert guard.fault_injection(1) == (3, 5)
    assert guard.fault_injection(0) is None
    monkeypatch.setenv(guard.FAULT_ENV, "0:2")
    assert guard.fault_injection(0) == (2, 0)
    for bad in ("0", "0:x", "1:2:3:4"):
        monkeypatch.setenv(guard.FAULT_ENV, bad)
        with pytest.raises(ValueError, match="rank:site"):
            guard.fault_injection(0)
    monkeypatch.delenv(guard.FAULT_ENV)
    assert guard.fault_injection(0) is None


def test_guard_words_describe():
    assert guard.describe([0] * 16) is None
    words = [0] * 16
    words[_lib.GUARD_ERR_DEADLINE] = 3  # site 2 = mid
    words[_lib.GUARD_ERR_FAULT] = 1
    msg = guard.describe(words)
    assert "mid" in msg and "fault-injected 1" in msg


def test_aiter16_shuffle_is_the_reference_index_map():
    """Element (n, k) of the (16, 16) shuffle sits at byte
    ((n // 16 * K // 32 + k // 32) * 2 + k % 32 // 16) * 256 + n % 16 * 16 + k % 16
    (ld_fp8_chunk, glm53/gfx950/kernel.py:787-808), and unshuffle inverts it."""
    import torch

    from sgl_amd_mono_amd import layouts

    n, k = 48, 96
    w = torch.arange(n * k, dtype=torch.int64).reshape(n, k)
    s = layouts.shuffle_16x16(w).reshape(-1)
    for nn, kk in [(0, 0), (5, 17), (16, 31), (47, 95), (33, 64)]:
        pos = ((nn // 16 * (k // 32) + kk // 32) * 2 + kk % 32 // 16) * 256 + nn % 16 * 16 + kk % 16
        assert int(s[pos]) == nn * k + kk
    assert torch.equal(layouts.unshuffle_16x16(layouts.shuffle_16x16(w)), w)
    e = torch.randint(0, 255, (3, 32, 64), dtype=torch.uint8)
    assert torch.equal(layouts.unshuffle_16x16(layouts.shuffle_16x16(e)), e)


def test_e8m0_shuffle_is_the_reference_index_map():
    """Scale (row, col) of the e8m0 shuffle sits at byte
    ((((r32 * CP/8 + c8) * 4 + e) * 16 + b) * 2 + d) * 2 + a, row = 32 r32 + 16 a + b,
    col = 8 c8 + 4 d + e (sgl_amd_mono/common/mx.py:40-44), with the columns padded to
    a multiple of 8; unshuffle inverts it."""
    import torch

    from sgl_amd_mono_amd import layouts

    for n, c in [(64, 12), (96, 96), (32, 8)]:
        s = torch.randint(0, 256, (n, c), dtype=torch.uint8)
        sh = layouts.shuffle_e8m0(s)
        cp = layouts.e8m0_cols(c)
        assert sh.shape == (n, cp)
        flat = sh.reshape(-1)
        for r in range(n):
            for k in range(c):
                r32, a, b = r // 32, (r // 16) % 2, r % 16
                c8, d, e = k // 8, (k // 4) % 2, k % 4
                pos = ((((r32 * (cp // 8) + c8) * 4 + e) * 16 + b) * 2 + d) * 2 + a
                assert int(flat[pos]) == int(s[r, k])
        assert torch.equal(layouts.unshuffle_e8m0(sh, c), s)
