"""Provider-level host logic without a GPU: segment text, per-node support answers and compile-time
rejection of what the provider cannot run (all decided before any device memory is touched)."""
import ctypes

import pytest

from sharplight_amd import native
from sharplight_amd.provider import GraphBuilder, HipExecutionProvider, _fmt, describe, plan


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


def _canonical(g: GraphBuilder) -> str:
    """The builder's own objects written in the provider's canonical order (independent of to_ir)."""
    out = [f"value {v.id} {v.type}" + "".join(f" {d}" for d in v.dims) for v in sorted(g.values, key=lambda v: v.id)]
    for role, vals in (("input", g.inputs), ("weight", g.weights), ("output", g.outputs), ("state", g.states)):
        out += [f"{role} {i}" for i in sorted({v.id for v in vals})]
    for n in g.nodes:
        ids = lambda l: ",".join(str(v.id) for v in l) or "-"
        out.append(f"node {n.op} {ids(n.inputs)} -> {ids(n.outputs)}" +
                   "".join(f" {k}={_fmt(n.attrs[k])}" for k in sorted(n.attrs)))
    return "\n".join(out) + "\n"


def test_segment_text_round_trip():
    """to_ir() parses back (slhip_segment_describe) to the same values, roles, nodes and attributes, over
    every statement kind, the block types, the symbolic T, states, empty lists and the attribute spellings
    (floats incl. +-inf, booleans, section lists, scalar names)."""
    g = GraphBuilder()
    x = g.input("bf16", "T", 4096)
    r = g.input("f32", "T", 4096)
    pos = g.input("i32", "T", 4)
    ids = g.input("i32", "T")
    cache = g.state("f16", 32768, 8, 128)
    w = g.weight("f32", 4096)
    b = g.weight("f32", 4096)
    ff = g.weight("f32", 64)
    emb = {t: g.weight(t, 1024, 4096) for t in ("q8_0", "q4_k", "iq2_xxs", "nf4_b64", "q2_0_g128", "f8e4m3_b128")}
    h = g.add(x, r)
    y = g.rms_norm(h, w, eps=1e-6)
    g.layer_norm(y, w, b, eps=1e-5, out_type="bf16")
    q = g.value("bf16", "T", 32, 128)
    g.nodes.append(type(g.nodes[0])("Reshape", [y], [q], {}))
    k = g.rope(q, pos, ff, dims=128, base=1e6, style="normal", freq_scale=0.25, attn_factor=1.5,
               sections=[16, 24, 24, 0], interleaved=True, sections_per_element=True)
    g.cache_write(cache, k, offset="n_past", slots=2, block_size=16)
    g.output(g.clip(g.scale(y, scale=0.125, bias=-3.0), min=float("-inf"), max=6.0))
    g.output(g.binary("Mod", y, w, fmod=True))
    for t, e in emb.items():
        g.output(g.gather(e, ids, out_type="bf16"))
    g.output(g.matmul(y, emb["q4_k"], out_type="f32"))
    g.output(g.cast(y, "f16"))
    g.output(g.unary("LeakyRelu", y, alpha=0.01))
    ir = g.to_ir()
    assert describe(ir) == _canonical(g)
    # the canonical text is a fixed point
    assert describe(describe(ir)) == describe(ir)


def test_segment_text_refuses_other_symbols_and_small_buffers():
    with pytest.raises(native.SlhipArgumentError, match="neither a size nor the token count T"):
        describe("value 0 f32 N 64\n")
    with pytest.raises(native.SlhipArgumentError, match="too small"):
        buf = ctypes.create_string_buffer(8)
        native.call("slhip_segment_describe", b"value 0 f32 T 64\n", buf, len(buf))
    with pytest.raises(ValueError):
        _fmt("two words")


def test_supports_answers():
    g = GraphBuilder()
    x = g.input("f32", "T", 4, 64)
    pos = g.input("i32", "T")
    w16 = g.weight("f16", 64)
    g.rms_norm(x, w16)                       # 0: f16 norm weight -> no (f32 weights only)
    g.rope(x, pos)                           # 1: yes
    g.emit("Softmax", [x], "f32", ("T", 4, 64))  # 2: not on this path
    xh = g.input("f16", "T", 64)
    g.rms_norm(xh)                           # 3: f16 rows -> no
    tbl = g.weight("q8_0", 100, 64)
    ids = g.input("i32", "T")
    g.gather(tbl, ids, out_type="bf16")      # 4: yes
    g.gather(tbl, ids, out_type="f16")       # 5: f16 output -> no
    pos2 = g.input("i32", "T", 4)
    g.rope(x, pos2, sections=(8, 12, 12, 0))  # 6: multi-axis positions (M-RoPE) -> yes
    pos5 = g.input("i32", "T", 5)
    g.rope(x, pos5)                          # 7: five axes -> no
    g.emit("Rope", [x, pos2], "f32", x.dims, sections="1,2,3")  # 8: three sections -> no
    expect = [False, True, False, False, True, False, True, False, False]
    for k, e in enumerate(expect):
        ok, why = _supports(g, k)
        assert ok == e, (k, why)
        assert ok or why


def test_elementwise_chain_is_one_group():
    """GroupElementwiseChains (GraphLowerer.Fusion.cs:88-142): consecutive f32 elementwise nodes of one output
    shape, each reading the open group, are one generated kernel -- an Add, a bias add, a scalar Mul and a
    Silu here; a lone node is its own standalone launch; bf16 outputs are not fusable (IsFusable, :9-11)."""
    g = GraphBuilder()
    a = g.input("f32", "T", 64)
    b = g.input("f32", "T", 64)
    bias = g.weight("f32", 64)
    s = g.weight("f32", 1)
    y = g.add(g.add(a, b), bias)
    y = g.mul(y, s)
    g.output(g.silu(y))
    assert plan(g) == ["fused[Add,Add,Mul,Silu]"]
    for k in range(4):
        assert _supports(g, k)[0]
    g = GraphBuilder()
    g.output(g.add(g.input("f32", "T", 64), g.weight("f32", 64)))
    assert plan(g) == ["Add"]
    g = GraphBuilder()
    x = g.input("bf16", "T", 64)
    g.output(g.silu(g.add(x, g.input("bf16", "T", 64))))
    assert plan(g) == ["Add", "Silu"]


def test_broadcast_support_answers():
    g = GraphBuilder()
    x = g.input("bf16", "T", 8, 64)
    g.binary("Add", x, g.weight("f32", 64))             # 0: bf16 + f32 bias -> yes
    g.binary("Mul", g.weight("f32", 64), x)             # 1: f32 * bf16 commutes -> yes
    g.binary("Sub", g.weight("f32", 64), x, "bf16")      # 2: f32 - bf16 does not commute -> no
    g.emit("Add", [x, g.input("f32", "T", 7, 64)], "bf16", ("T", 8, 64))  # 3: 8 vs 7 -> no
    g.emit("Add", [x, g.input("bf16", 5, 8, 64)], "bf16", ("T", 8, 64))   # 4: T vs 5 -> no
    g.unary("Scale", x, scale=2.0, bias=1.0)            # 5: yes
    g.unary("Clip", x, min=-1.0, max=1.0)               # 6: yes
    g.emit("Relu", [x], "bf16", ("T", 64))              # 7: output shape differs -> no
    expect = [True, True, False, False, False, True, True, False]
    for k, e in enumerate(expect):
        ok, why = _supports(g, k)
        assert ok == e, (k, why)


def test_gated_unit_waits_for_up():
    """Gate MatMul (bf16 out: no dual matvec) -> Silu -> up MatMul -> Mul: the activation comes before up's
    producer, so act and Mul must not be fused at the activation (it would read up before it is written)."""
    g = GraphBuilder()
    x = g.input("bf16", "T", 256)
    wg = g.weight("bf16", 512, 256)
    wu = g.weight("bf16", 512, 256)
    gate = g.matmul(x, wg, out_type="bf16")
    act = g.silu(gate)
    up = g.matmul(x, wu, out_type="bf16")
    g.output(g.mul(act, up))
    assert plan(g) == ["matvec", "Silu", "matvec", "Mul"]
    # the usual order (both products first) still fuses
    g2 = GraphBuilder()
    x = g2.input("bf16", "T", 256)
    gate = g2.matmul(x, g2.weight("bf16", 512, 256), out_type="bf16")
    up = g2.matmul(x, g2.weight("bf16", 512, 256), out_type="bf16")
    g2.output(g2.mul(g2.silu(gate), up))
    assert plan(g2) == ["matvec", "matvec", "fused[Silu,Mul]"]


def test_dual_matvec_falls_back_when_rows_do_not_fit_lds():
    """A Q8_0 gate/up pair at K = 16384 does not fit the dual kernel's LDS staging: two matvecs plus the
    gated unit instead (a single Q8_0 matvec at that K fits)."""
    def build(K):
        g = GraphBuilder()
        x = g.input("f32", "T", K)
        gate = g.matmul(x, g.weight("q8_0", 256, K), f32_activations=True)
        up = g.matmul(x, g.weight("q8_0", 256, K), f32_activations=True)
        g.output(g.mul(g.silu(gate), up))
        return g
    assert plan(build(4096)) == ["matvec2+fused[Silu,Mul]"]
    assert plan(build(16384)) == ["matvec", "matvec", "fused[Silu,Mul]"]


def test_add_before_a_norm_folds_into_it():
    """FoldNormTails (GraphLowerer.Fusion.cs:211-238): a broadcast Add before a norm joins the norm's launch
    (the group program); two same-shape operands take the residual row-norm kernel."""
    g = GraphBuilder()
    x = g.input("f32", "T", 64)
    b = g.weight("f32", 64)
    g.output(g.rms_norm(g.add(x, b), g.weight("f32", 64)))
    assert plan(g) == ["fused[Add]+RmsNorm"]
    g = GraphBuilder()
    x = g.input("f32", "T", 64)
    g.output(g.rms_norm(g.add(x, g.input("f32", "T", 64)), g.weight("f32", 64)))
    assert plan(g) == ["fused[Add]+RmsNorm"]


def test_unsupported_node_is_rejected_at_compile():
    g = GraphBuilder()
    x = g.input("f32", "T", 64)
    g.output(g.emit("Softmax", [x], "f32", x.dims))
    st, msg = _compile_error(g)
    assert st == native.ERR_UNSUPPORTED and "Softmax" in msg


def test_malformed_segment_text():
    seg = ctypes.c_void_p(0)
    for bad in ["value 0 f99 4\n", "node Add 0,1 => 2\n", "output 7\n", "frobnicate\n",
                "value 0 f32 4\nstate 0\nnode CacheWrite 0,0 -> offset=n_past\n"]:
        st = native.lib().slhip_segment_compile(bad.encode(), 8, ctypes.byref(seg))
        assert st == native.ERR_INVALID, bad
        assert "line " in native.last_error()


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


def test_cache_write_text_and_support():
    g = GraphBuilder()
    k = g.input("bf16", "T", 2, 64)
    pos = g.input("i32", "T")
    kc = g.state("f16", 32, 2, 64)
    g.cache_write(kc, g.rope(k, pos))
    ir = g.to_ir()
    assert "state 2" in ir and "node CacheWrite 2,3 -> - offset=n_past" in ir
    assert _supports(g, 1) == (True, "")
    q8 = g.state("q8_0", 32, 128)
    x = g.input("f32", "T", 128)
    g.cache_write(q8, x)
    ok, why = _supports(g, 2)
    assert not ok and "quantized" in why
    g2 = GraphBuilder()
    notstate = g2.input("f32", 32, 64)
    g2.cache_write(notstate, g2.input("f32", "T", 64))
    ok, why = _supports(g2, 0)
    assert not ok and "state" in why


def test_state_needs_fixed_dims():
    seg = ctypes.c_void_p(0)
    st = native.lib().slhip_segment_compile(b"value 0 f32 T 4\nstate 0\n", 8, ctypes.byref(seg))
    assert st == native.ERR_INVALID and "fixed dims" in native.last_error()


def test_matmul_support_answers():
    g = GraphBuilder()
    x = g.input("f32", "T", 64)
    wq = g.weight("q8_0", 16, 64)
    wb = g.weight("bf16", 16, 64)
    w60 = g.weight("bf16", 16, 60)
    x60 = g.input("f32", "T", 60)
    g.matmul(x, wq)                          # 0: Q8_0 with K = 64 -> no (block formats need K % 256 == 0)
    g.matmul(x, wb)                          # 1: yes
    g.matmul(x60, w60)                       # 2: K not a multiple of 8 -> no
    g.emit("MatMul", [x, x60], "f32", ("T", 64))  # 3: second operand not a weight [N, K] -> no
    x256 = g.input("f32", "T", 256)
    g.matmul(x256, g.weight("q4_0", 16, 256))     # 4: yes
    g.matmul(x256, g.weight("i32", 16, 256))      # 5: integer weights -> no
    g.matmul(x256, g.weight("q4_k", 16, 256))     # 6: yes
    g.matmul(x256, g.weight("q6_k", 16, 256))     # 7: Q6_K rows of 210 bytes -> yes (2-byte staging loads)
    x2048 = g.input("f32", "T", 2048)
    g.matmul(x2048, g.weight("q6_k", 16, 2048))   # 8: yes
    g.matmul(x2048, g.weight("iq4_xs", 16, 2048))  # 9: no matvec for this format
    g.matmul(x2048, g.weight("q2_k", 16, 2048))   # 10: yes
    g.matmul(x256, g.weight("q3_k", 16, 256))     # 11: Q3_K with K = 256 -> yes (the VALU kernel at any T)
    x1024 = g.input("f32", "T", 1024)
    g.matmul(x1024, g.weight("q3_k", 16, 1024))   # 12: yes
    expect = [False, True, False, False, True, False, True, True, True, False, True, True, True]
    for k, e in enumerate(expect):
        ok, why = _supports(g, k)
        assert ok == e, (k, why)
        assert ok or why


def test_zero_and_oversized_dimensions_are_answered_not_crashed():
    """A cache write against a state or rows with a zero extent is answered (no division by the extent), and
    sizes the provider could not address are refused at parse time: a dimension above 2^40, more than 2^46
    elements without T, a token bound above 2^20. (Found by fuzzing the segment text under AddressSanitizer.)"""
    text = ("value 0 f16 0 8 128\nvalue 1 bf16 T 8 128\nvalue 2 f16 4 0 128\nstate 0\nstate 2\ninput 1\n"
            "node CacheWrite 0,1 -> -\nnode CacheWrite 2,1 -> -\n")
    answers = []
    for k in (0, 1):
        ok = ctypes.c_int(1)
        buf = ctypes.create_string_buffer(512)
        native.call("slhip_node_supports", text.encode(), k, ctypes.byref(ok), buf, len(buf))
        answers.append((ok.value, buf.value.decode()))
    assert answers[0] == (1, "")  # rows of 8 x 128 into a cache of zero slots: a shape match (the write itself
    #                                is refused at run time, every position being past the cache's end)
    assert answers[1][0] == 0 and "cache rows" in answers[1][1]
    for bad, msg in (("value 0 f32 T 1099511627777\n", "above 2"), ("value 0 f32 262144 262144 4096\n", "2\\^46"),
                     ("value 0 f32 T 99999999999999999999\n", "above 2")):
        with pytest.raises(native.SlhipArgumentError, match=msg):
            describe(bad)
    seg = ctypes.c_void_p(0)
    assert native.lib().slhip_segment_compile(b"value 0 f32 T 64\ninput 0\n", (1 << 20) + 1, ctypes.byref(seg)) != native.OK
    assert "2^20" in native.last_error()


# ---- the integer-dot matvec: which MatMuls quantize x, and the shared q8 copies ---------------------------

def _qkv(fmts, **opts):
    g = GraphBuilder()
    g.options.update(opts)
    x = g.input("f32", "T", 1024)
    for f in fmts:
        g.output(g.matmul(x, g.weight(f, 64, 1024)))
    return g


def test_int_dot_plan_shares_one_q8_copy_per_x_and_range():
    """GraphLowerer.IntDot.cs:119-220: matmuls reading the same rows share one quantized copy per row range
    (Q4_K and Q6_K: 1..8 rows; Q8_0: 2..16 rows, IntDotMinRows / IntDotMaxRows :18-19,75)."""
    assert plan(_qkv(["q4_k", "q6_k", "q4_k"])) == [
        "x->q8 rows 1..8", "matvec (int-dot rows 1..8)", "matvec (int-dot rows 1..8)", "matvec (int-dot rows 1..8)"]
    assert plan(_qkv(["q4_k", "q8_0"])) == [
        "x->q8 rows 1..8", "matvec (int-dot rows 1..8)", "x->q8 rows 2..16", "matvec (int-dot rows 2..16)"]
    # the lowerer's rule: the 32-value block formats Q4_0 / Q5_0 (SHARPLIGHT_MMVQ_BLOCK on by default), not Q4_1,
    # Q5_1 or dense weights
    assert plan(_qkv(["q4_0", "q5_0"])) == [
        "x->q8 rows 1..8", "matvec (int-dot rows 1..8)", "matvec (int-dot rows 1..8)"]
    assert plan(_qkv(["q4_1", "q5_1", "bf16", "q2_k", "q3_k"])) == ["matvec"] * 5


def test_int_dot_rules_and_f32_activations():
    # the CPU provider's rule: every IntDot.Supports format below 32 rows (MatMulOp.cs:104,138-147)
    assert plan(_qkv(["q4_1", "q8_0", "bf16", "q2_k"], int_dot="cpu")) == [
        "x->q8 rows 1..31", "matvec (int-dot rows 1..31)", "matvec (int-dot rows 1..31)", "matvec", "matvec"]
    assert plan(_qkv(["q4_k", "q8_0"], int_dot="off")) == ["matvec", "matvec"]
    # f32_activations keeps x unquantized unless the compile allows reduced precision (GraphLowerer.IntDot.cs:61-62)
    def one(**kw):
        g = GraphBuilder()
        g.options.update(kw.pop("opts", {}))
        x = g.input("f32", "T", 1024)
        g.output(g.matmul(x, g.weight("q4_k", 64, 1024), **kw))
        return g
    assert plan(one(f32_activations=True)) == ["matvec"]
    assert plan(one(f32_activations=False)) == ["x->q8 rows 1..8", "matvec (int-dot rows 1..8)"]
    assert plan(one(f32_activations=True, opts={"reduced_precision": True})) == ["x->q8 rows 1..8",
                                                                                 "matvec (int-dot rows 1..8)"]


def test_int_dot_options_are_checked_and_described():
    g = _qkv(["q4_k"], int_dot="cpu", reduced_precision=True)
    text = describe(g.to_ir())
    assert "option int_dot=cpu\n" in text and "option reduced_precision=true\n" in text
    for bad in ("option int_dot=gpu\n", "option speed=3\n", "option reduced_precision=2\n", "option x\n"):
        seg = ctypes.c_void_p(0)
        st = native.lib().slhip_segment_compile((bad + g.to_ir()).encode(), 4, ctypes.byref(seg))
        assert st == native.ERR_INVALID, bad


def test_int_dot_only_formats():
    """IQ4_NL, IQ4_XS and MXFP4 have no f32 matvec here: supported when the integer-dot path serves every row
    count from one, and compile refuses a token bound beyond the range's end."""
    def g_of(fmt, K=1024, **opts):
        g = GraphBuilder()
        g.options.update(opts)
        x = g.input("f32", "T", K)
        g.output(g.matmul(x, g.weight(fmt, 64, K)))
        return g
    for fmt in ("iq4_nl", "mxfp4"):
        assert _supports(g_of(fmt), 0)[0]
        assert plan(g_of(fmt)) == ["x->q8 rows 1..8", "matvec (int-dot rows 1..8)"]
        seg = ctypes.c_void_p(0)
        st = native.lib().slhip_segment_compile(g_of(fmt).to_ir().encode(), 9, ctypes.byref(seg))
        assert st == native.ERR_UNSUPPORTED and "up to 8 activation rows" in native.last_error()
    assert not _supports(g_of("iq4_xs"), 0)[0]           # not in the lowerer's int-dot set
    assert _supports(g_of("iq4_xs", int_dot="cpu"), 0)[0]  # the CPU provider's
    assert not _supports(g_of("mxfp4", int_dot="off"), 0)[0]
    # gpt-oss's K = 2880 (not a multiple of 256): MXFP4 yes (integer dots only), Q4_0 no (no f32 path at that K)
    assert _supports(g_of("mxfp4", K=2880), 0)[0]
    assert not _supports(g_of("q4_0", K=2880), 0)[0]


def test_matmul_bias_folds_into_the_matvec():
    """FoldMatMulBiases (GraphLowerer.Fusion.cs:355-408): an Add of a constant f32 row vector [N] that is the
    product's only reader joins the matvec launch; other Adds stay their own launch."""
    def g_of(bias_kind):
        g = GraphBuilder()
        x = g.input("f32", "T", 1024)
        p = g.matmul(x, g.weight("bf16", 64, 1024))
        b = g.input("f32", 64) if bias_kind == "input" else g.weight("f32", 64)
        g.output(g.add(b, p) if bias_kind == "swapped" else g.add(p, b))
        return g
    assert plan(g_of("weight")) == ["matvec+bias"]
    assert plan(g_of("swapped")) == ["matvec+bias"]
    assert plan(g_of("input")) == ["matvec", "Add"]
    g = GraphBuilder()
    x = g.input("f32", "T", 1024)
    p = g.output(g.matmul(x, g.weight("q4_k", 64, 1024)))  # the product is also an output: not folded
    g.output(g.add(p, g.weight("f32", 64)))
    assert plan(g) == ["x->q8 rows 1..8", "matvec (int-dot rows 1..8)", "Add"]
    g = GraphBuilder()
    x = g.input("f32", "T", 1024)
    g.output(g.add(g.matmul(x, g.weight("q4_k", 64, 1024)), g.weight("f32", 64)))
    assert plan(g) == ["x->q8 rows 1..8", "matvec+bias (int-dot rows 1..8)"]


# ---- fused elementwise groups (GraphLowerer.Fusion.cs:88-285) -----------------------------------------------

def test_bias_residual_norm_is_one_launch():
    """Add(bias) + Add(residual) + RmsNorm: one group with the norm as its tail; the sum is stored only when
    something else reads it."""
    g = GraphBuilder()
    x = g.input("f32", "T", 256)
    r = g.input("f32", "T", 256)
    h = g.add(g.add(x, g.weight("f32", 256)), r)
    g.output(g.rms_norm(h, g.weight("f32", 256), eps=1e-6))
    assert plan(g) == ["fused[Add,Add]+RmsNorm"]


def test_norm_head_and_scale():
    """FoldNormHeads (:240-284): RmsNorm -> Mul(w) -> Scale, the norm read only by the group: one launch; a norm
    that is also a segment output stays its own launch."""
    g = GraphBuilder()
    x = g.input("f32", "T", 128)
    n = g.rms_norm(x, None, eps=1e-6)
    g.output(g.scale(g.mul(n, g.weight("f32", 128)), scale=0.5, bias=0.25))
    assert plan(g) == ["RmsNorm+fused[Mul,Scale]"]
    g = GraphBuilder()
    x = g.input("f32", "T", 128)
    n = g.output(g.rms_norm(x, None, eps=1e-6))
    g.output(g.scale(g.mul(n, g.weight("f32", 128)), scale=0.5))
    assert plan(g) == ["RmsNorm", "fused[Mul,Scale]"]


def _gpt_oss_swiglu(K=256, N=512, alpha=1.702, limit=7.0):
    """gpt-oss's clamped SwiGLU with the projections' biases (the model's MLP: gate and up products, their bias
    adds, gate clamped above, up clamped both ways, gate * sigmoid(alpha gate) * (up + 1))."""
    g = GraphBuilder()
    x = g.input("f32", "T", K)
    gate = g.add(g.matmul(x, g.weight("bf16", N, K)), g.weight("f32", N))
    up = g.add(g.matmul(x, g.weight("bf16", N, K)), g.weight("f32", N))
    gc = g.clip(gate, max=limit)
    uc = g.clip(up, min=-limit, max=limit)
    glu = g.mul(gc, g.unary("Sigmoid", g.scale(gc, scale=alpha)))
    g.output(g.mul(g.scale(uc, bias=1.0), glu))
    return g


def test_gpt_oss_clamped_swiglu_merges_into_one_group():
    """MergeElementwiseGroups (:160-205): the groups split by the up projection join along data flow, so the
    bias adds, clamps and gating are one kernel after the two matvecs (the Add groups are not single-node, so
    FoldMatMulBiases leaves them in the group, as the reference does)."""
    assert plan(_gpt_oss_swiglu()) == ["matvec", "matvec",
                                       "fused[Add,Clip,Add,Clip,Scale,Sigmoid,Mul,Scale,Mul]"]


def test_group_merge_is_blocked_by_a_reader_in_between():
    g = GraphBuilder()
    x = g.input("f32", "T", 64)
    a = g.scale(x, scale=2.0)                      # group 1
    m = g.output(g.matmul(a, g.weight("bf16", 64, 64)))  # reads group 1's output: blocks the merge
    g.output(g.add(a, m))                          # group 2 reads group 1's output
    assert plan(g) == ["Scale", "matvec", "Add"]
