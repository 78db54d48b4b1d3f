"""The allocation-free FP8 MoE launch (``mono_moe_fp8_launch_static``) against the
runtime launch it mirrors (``mono_moe_fp8_launch``), both through the C ABI: the same
kernels over the library's static block instead of a runtime's scratch, so every output
must be bit-equal. Two calls in a row, the second with fewer rows; sizes past the block's
maximum and caller scratch are refused with a clear error."""

import ctypes

import pytest
import torch

from sgl_amd_mono_amd import _lib, layouts
from sgl_amd_mono_amd.dsv32 import synthetic
from sgl_amd_mono_amd.dsv32.config import DSV32
from sgl_amd_mono_amd.dsv32.moe import MoeFp8Op, MoeRouting

pytestmark = pytest.mark.gpu


def _args(w, a, out, y, routing, host_error):
    return _lib.MonoMoeFp8Args(
        rows=a.shape[0], hidden=DSV32.hidden, inter=DSV32.inter, experts=DSV32.experts,
        layout=_lib.LAYOUT_AITER16 if w.layout == layouts.AITER16 else _lib.LAYOUT_ROWMAJOR,
        eps=DSV32.rms_eps, route_scale=DSV32.route_scale, a=a.data_ptr(), out=out.data_ptr(),
        g_post=w.g_post.data_ptr(), w_r=w.w_r.data_ptr(), bias=w.bias.data_ptr(),
        w13=w.w13.data_ptr(), s13=w.s13.data_ptr(), w2=w.w2.data_ptr(), s2=w.s2.data_ptr(),
        y=y.data_ptr(), scores=routing.scores.data_ptr(), ids=routing.ids.data_ptr(),
        weights=routing.weights.data_ptr(), scratch=None, guard=None,
        host_error=host_error.data_ptr(), fault_site=0, fault_after=0, timeline=None)


def _routing(rows, dev):
    return MoeRouting(torch.full((rows, DSV32.experts), float("nan"), device=dev),
                      torch.full((rows, 9), -1, dtype=torch.int32, device=dev),
                      torch.full((rows, 9), float("nan"), device=dev))


def test_static_launch_matches_the_runtime_launch(gpu):
    print("case moe_fp8 static block: rows 8 then 3", flush=True)
    w = synthetic.moe_fp8_weights(gpu, seed=71, layout=layouts.AITER16)
    op = MoeFp8Op(w, gpu, max_rows=16)
    host_error = torch.zeros(1, dtype=torch.int32, pin_memory=True)
    lib = _lib.lib()
    for rows, seed in ((8, 72), (3, 73)):
        a = synthetic.rows_bf16(rows, DSV32.hidden, gpu, seed=seed)
        y_ref = torch.empty(rows, DSV32.hidden, device=gpu)
        rt_ref = _routing(rows, gpu)
        want = op.launch(a, y=y_ref, routing=rt_ref).clone()
        op.rt.check()
        out = torch.full_like(want, float("nan"))
        y = torch.full_like(y_ref, float("nan"))
        rt = _routing(rows, gpu)
        args = _args(w, a, out, y, rt, host_error)
        rc = lib.mono_moe_fp8_launch_static(ctypes.byref(args), _lib.stream_handle())
        assert rc == _lib.MONO_OK, _lib.last_error()
        torch.cuda.synchronize()
        assert int(host_error[0]) == 0
        assert torch.equal(out, want), rows
        assert torch.equal(y, y_ref), rows
        for name in ("scores", "ids", "weights"):
            assert torch.equal(getattr(rt, name), getattr(rt_ref, name)), (rows, name)


def test_static_launch_refuses_what_its_block_cannot_hold(gpu):
    print("case moe_fp8 static block refusals", flush=True)
    w = synthetic.moe_fp8_weights(gpu, seed=74, experts=4)
    a = synthetic.rows_bf16(17, DSV32.hidden, gpu, seed=75)
    out = torch.empty_like(a)
    host_error = torch.zeros(1, dtype=torch.int32, pin_memory=True)
    args = _args(w, a, out, torch.empty(17, DSV32.hidden, device=gpu), _routing(17, gpu),
                 host_error)
    lib = _lib.lib()
    assert lib.mono_moe_fp8_launch_static(ctypes.byref(args), None) == _lib.MONO_E_ARG
    assert "rows must be 1..16" in _lib.last_error()
    args.rows = 4
    args.scratch = a.data_ptr()
    assert lib.mono_moe_fp8_launch_static(ctypes.byref(args), None) == _lib.MONO_E_ARG
    assert "must be null" in _lib.last_error()
    args.scratch = None
    args.inter = 384
    assert lib.mono_moe_fp8_launch_static(ctypes.byref(args), None) == _lib.MONO_E_ARG
    assert "sized for" in _lib.last_error()
