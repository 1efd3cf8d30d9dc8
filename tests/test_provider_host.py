"""Provider-level host logic without a GPU: segment text, per-node support answers and compile-time
rejection of what the provider cannot run (all decided before any device memory is touched)."""
import ctypes

import pytest

from sharplight_amd import native
from sharplight_amd.provider import GraphBuilder, HipExecutionProvider


def _supports(g: GraphBuilder, k: int):
    ok = ctypes.c_int(0)
    buf = ctypes.create_string_buffer(512)
    native.call("slhip_node_supports", g.to_ir().encode(), k, ctypes.byref(ok), buf, len(buf))
    return bool(ok.value), buf.value.decode()


def _compile_error(g: GraphBuilder):
    seg = ctypes.c_void_p(0)
    st = native.lib().slhip_segment_compile(g.to_ir().encode(), 64, ctypes.byref(seg))
    assert st != native.OK
    return st, native.last_error()


def test_segment_text():
    g = GraphBuilder()
    x = g.input("bf16", "T", 4096)
    r = g.input("bf16", "T", 4096)
    w = g.weight("f32", 4096)
    h = g.add(x, r)
    g.output(h)
    g.output(g.rms_norm(h, w, eps=1e-5))
    ir = g.to_ir()
    assert "value 0 bf16 T 4096" in ir
    assert "node Add 0,1 -> 3" in ir
    assert "node RmsNorm 3,2 -> 4 eps=1e-05" in ir
    assert "weight 2" in ir and "output 3" in ir and "output 4" in ir


def test_supports_answers():
    g = GraphBuilder()
    x = g.input("f32", "T", 4, 64)
    pos = g.input("i32", "T")
    w16 = g.weight("f16", 64)
    g.rms_norm(x, w16)                       # 0: f16 norm weight -> no (f32 weights only)
    g.rope(x, pos)                           # 1: yes
    g.emit("MatMul", [x, x], "f32", ("T", 4, 64))  # 2: not on this path
    xh = g.input("f16", "T", 64)
    g.rms_norm(xh)                           # 3: f16 rows -> no
    tbl = g.weight("q8_0", 100, 64)
    ids = g.input("i32", "T")
    g.gather(tbl, ids, out_type="bf16")      # 4: yes
    g.gather(tbl, ids, out_type="f16")       # 5: f16 output -> no
    pos2 = g.input("i32", "T", 4)
    g.rope(x, pos2)                          # 6: multi-axis positions -> no
    expect = [False, True, False, False, True, False, False]
    for k, e in enumerate(expect):
        ok, why = _supports(g, k)
        assert ok == e, (k, why)
        assert ok or why


def test_standalone_elementwise_is_rejected_at_compile():
    g = GraphBuilder()
    a = g.input("f32", "T", 64)
    b = g.input("f32", "T", 64)
    g.output(g.add(a, b))  # no norm follows: nothing to fuse it into
    st, msg = _compile_error(g)
    assert st == native.ERR_UNSUPPORTED and "standalone Add" in msg


def test_unsupported_node_is_rejected_at_compile():
    g = GraphBuilder()
    x = g.input("f32", "T", 64)
    g.output(g.emit("Softmax", [x], "f32", x.dims))
    st, msg = _compile_error(g)
    assert st == native.ERR_UNSUPPORTED and "Softmax" in msg


def test_malformed_segment_text():
    seg = ctypes.c_void_p(0)
    for bad in ["value 0 f99 4\n", "node Add 0,1 => 2\n", "output 7\n", "frobnicate\n"]:
        st = native.lib().slhip_segment_compile(bad.encode(), 8, ctypes.byref(seg))
        assert st == native.ERR_INVALID, bad
        assert "line 1" in native.last_error()


def test_availability_never_raises():
    p = HipExecutionProvider()
    a = p.check_availability()
    devs = p.get_devices()
    assert (len(devs) > 0) == a.is_available
    if not a.is_available:
        assert a.reason
        with pytest.raises(NotImplementedError):
            from sharplight_amd.provider import DeviceInfo
            p.open_device(DeviceInfo("hip", 0, "x", "DiscreteGpu", 0, "AMD", "HIP", "", (), 0))


def test_open_device_of_other_provider():
    from sharplight_amd.provider import DeviceInfo
    with pytest.raises(ValueError):
        HipExecutionProvider().open_device(DeviceInfo("vulkan", 0, "x", "DiscreteGpu", 0, "", "", "", (), 0))
