"""GPU parity of the fused elementwise groups (slhip_ew_program_run) and of the provider's group formation
(GraphLowerer.Fusion.cs:88-285: GroupElementwiseChains, MergeElementwiseGroups, FoldNormTails, FoldNormHeads)
against the oracle's node-by-node CPU arithmetic (BinaryOp, ScalarMath.Unary, RowOp), f32 at 1e-5 relative
(the parity rule of tests/parity.py), bf16 outputs within 2 ulp, stored intermediates included."""
import os

import numpy as np
import pytest

import oracle
from sharplight_amd import native, synth
from sharplight_amd.provider import GraphBuilder, HipExecutionProvider
from tests.devutil import Dev, log
from tests.parity import assert_bf16_close, assert_f32_close

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["generated", "interpreter"])
def path(request, device):
    """Both forms of a group's kernel: the one generated for the program (default) and the op-code interpreter
    (SLHIP_EWG_JIT=0, read at every run)."""
    old = os.environ.get("SLHIP_EWG_JIT")
    os.environ["SLHIP_EWG_JIT"] = "1" if request.param == "generated" else "0"
    yield request.param
    if old is None:
        del os.environ["SLHIP_EWG_JIT"]
    else:
        os.environ["SLHIP_EWG_JIT"] = old


def test_program_every_input_mode(path):
    rows, cols = 37, 1024
    x = synth.normal(40, 0, (rows, cols))
    b = synth.normal(40, 1, (cols,), dtype="bf16")
    s = np.array([1.75], np.float32)
    c = synth.normal(40, 2, (rows, 1))
    with Dev() as d:
        px, pb, ps, pc = d.put(x), d.put(b), d.put(s), d.put(c)
        p1 = d.empty(rows * cols * 4)
        p3 = d.empty(rows * cols * 2)
        log(f"ew_program modes {path}")
        # r4 = x + b; r5 = r4 * s; r4 = silu(r5); r6 = r4 - c  (registers reused)
        native.ew_program([(px, "f32", native.EWI_FULL), (pb, "bf16", native.EWI_ROW), (ps, "f32", native.EWI_SCALAR),
                           (pc, "f32", native.EWI_COL)],
                          [("binary", "Add", 0, 1, 4, "f32", 0, 0), ("binary", "Mul", 4, 2, 5, "f32", 0, 0),
                           ("unary", "Silu", 5, 0, 4, "f32", 0, 0), ("binary", "Sub", 4, 3, 6, "f32", 0, 0)],
                          [(p1, "f32", 5), (p3, "bf16", 6)], rows, cols)
        native.synchronize()
        y1 = d.get(p1, (rows, cols), np.float32)
        y3 = d.get(p3, (rows, cols), np.uint16)
    r1 = oracle.binary("Mul", oracle.binary("Add", x, oracle.from_bf16(b)), s.reshape(()))
    r3 = oracle.binary("Sub", oracle.unary_kind("Silu", r1), c)
    assert_f32_close(y1, r1, what="stored intermediate")
    assert_bf16_close(y3, oracle.to_bf16(r3), what="bf16 output")


def test_program_rounding_and_f16(path):
    """A node whose output type is bf16 or f16 (the value rounded where the unfused graph stores it), an f16 input
    and an f16 output."""
    rows, cols = 19, 768
    x = synth.normal(46, 0, (rows, cols))
    h = synth.normal(46, 1, (rows, cols)).astype(np.float16)
    with Dev() as d:
        px, ph = d.put(x), d.put(h)
        py = d.empty(rows * cols * 2)
        log(f"ew_program rounding f16 {path}")
        # r2 = bf16(x * 3) ; r3 = f16(r2 + h) ; r2 = tanh(r3) -> f16 output
        native.ew_program([(px, "f32", native.EWI_FULL), (ph, "f16", native.EWI_FULL)],
                          [("unary", "Scale", 0, 0, 2, "bf16", 3.0, 0.0), ("binary", "Add", 2, 1, 3, "f16", 0, 0),
                           ("unary", "Tanh", 3, 0, 2, "f32", 0, 0)],
                          [(py, "f16", 2)], rows, cols)
        native.synchronize()
        y = d.get(py, (rows, cols), np.float16)
    r2 = oracle.from_bf16(oracle.to_bf16(oracle.unary_kind("Scale", x, 3.0, 0.0)))
    r3 = oracle.binary("Add", r2, h.astype(np.float32)).astype(np.float16).astype(np.float32)
    ref = oracle.unary_kind("Tanh", r3).astype(np.float16)
    bad = np.abs(y.astype(np.float64) - ref.astype(np.float64)) > 2.0 ** -10 * np.abs(ref.astype(np.float64)) + 1e-7
    assert not bad.any(), (np.argwhere(bad)[:3], y[bad][:3], ref[bad][:3])


@pytest.mark.parametrize("dty,cols", [("f32", 4096), ("bf16", 4096), ("f32", 5000)])
def test_program_norm_tail(path, dty, cols):
    """Add(bias) + Add(residual) + RmsNorm: h stored, y = RmsNorm(h) * w (5000 columns: beyond the generated
    kernel's registers, a second pass over the row)."""
    rows = 64
    x = synth.normal(41, 0, (rows, cols))
    r = synth.normal(41, 1, (rows, cols))
    bias = synth.normal(41, 2, (cols,))
    w = synth.normal(41, 3, (cols,), mean=1.0, std=0.1)
    with Dev() as d:
        px, pr, pbias, pw = d.put(x), d.put(r), d.put(bias), d.put(w)
        ph = d.empty(rows * cols * 4)
        py = d.empty(rows * cols * (4 if dty == "f32" else 2))
        log(f"ew_program norm tail y={dty} cols={cols} {path}")
        native.ew_program([(px, "f32", native.EWI_FULL), (pbias, "f32", native.EWI_ROW), (pr, "f32", native.EWI_FULL)],
                          [("binary", "Add", 0, 1, 3, "f32", 0, 0), ("binary", "Add", 3, 2, 3, "f32", 0, 0)],
                          [(ph, "f32", 3)], rows, cols,
                          tail=dict(kind="rms", reg=3, w=pw, eps=1e-6, y=py, dtype_y=dty))
        native.synchronize()
        h = d.get(ph, (rows, cols), np.float32)
        y = d.get(py, (rows, cols), np.float32 if dty == "f32" else np.uint16)
    href = oracle.binary("Add", oracle.binary("Add", x, bias), r)
    assert np.array_equal(h.view(np.uint32), href.view(np.uint32))
    yref = oracle.rmsnorm(href, w, 1e-6)
    if dty == "f32":
        assert_f32_close(y, yref, what="y")
    else:
        assert_bf16_close(y, oracle.to_bf16(yref), what="y")


@pytest.mark.parametrize("cols", [2048, 4100])
def test_program_norm_head(path, cols):
    """RmsNorm (no weight) read only by Mul(w2) -> Scale: the norm computed in the group's launch."""
    rows = 50
    x = synth.normal(42, 0, (rows, cols), std=3.0)
    w2 = synth.normal(42, 1, (cols,))
    with Dev() as d:
        px, pw2 = d.put(x), d.put(w2)
        py = d.empty(rows * cols * 4)
        log(f"ew_program norm head cols={cols} {path}")
        native.ew_program([(px, "f32", native.EWI_FULL), (pw2, "f32", native.EWI_ROW)],
                          [("binary", "Mul", 0, 1, 2, "f32", 0, 0), ("unary", "Scale", 2, 0, 2, "f32", 0.5, 0.25)],
                          [(py, "f32", 2)], rows, cols, head=dict(kind="rms", reg=0, eps=1e-6, dtype_y="f32"))
        native.synchronize()
        y = d.get(py, (rows, cols), np.float32)
    n = oracle.rmsnorm(x, None, 1e-6)
    ref = oracle.unary_kind("Scale", oracle.binary("Mul", n, w2), 0.5, 0.25)
    assert_f32_close(y, ref, what="head")


@pytest.fixture(scope="module")
def dev(device):
    p = HipExecutionProvider()
    return p.open_device(p.get_devices()[0])


def test_provider_gpt_oss_clamped_swiglu(dev):
    """gpt-oss's clamped SwiGLU with its bias adds (from the products, given as inputs here): one launch, equal
    to the nodes run one by one on the CPU."""
    T, N, alpha, limit = 9, 2880, 1.702, 7.0
    g = GraphBuilder()
    gp, up = g.input("f32", "T", N), g.input("f32", "T", N)
    bg, bu = g.weight("f32", N), g.weight("f32", N)
    gc = g.clip(g.add(gp, bg), max=limit)
    uc = g.clip(g.add(up, bu), min=-limit, max=limit)
    glu = g.mul(gc, g.unary("Sigmoid", g.scale(gc, scale=alpha)))
    y = g.output(g.mul(g.scale(uc, bias=1.0), glu))
    G, U = synth.normal(43, 0, (T, N), std=4.0), synth.normal(43, 1, (T, N), std=4.0)
    BG, BU = synth.normal(43, 2, (N,)), synth.normal(43, 3, (N,))
    with dev.compile(g, max_tokens=16) as seg:
        assert len(seg.launches) == 1 and seg.launches[0].startswith("fused[")
        seg.set_input(gp, G)
        seg.set_input(up, U)
        seg.set_input(bg, BG)
        seg.set_input(bu, BU)
        log("provider gpt-oss swiglu group")
        seg.execute(T)
        got = seg.get_output(y)
    inf = float("inf")
    gcr = oracle.unary_kind("Clip", oracle.binary("Add", G, BG), -inf, limit)
    ucr = oracle.unary_kind("Clip", oracle.binary("Add", U, BU), -limit, limit)
    glur = oracle.binary("Mul", gcr, oracle.unary_kind("Sigmoid", oracle.unary_kind("Scale", gcr, alpha, 0.0)))
    ref = oracle.binary("Mul", oracle.unary_kind("Scale", ucr, 1.0, 1.0), glur)
    assert_f32_close(got, ref, what="gpt-oss swiglu")


@pytest.mark.parametrize("h_out", [False, True])
def test_provider_bias_residual_norm(dev, h_out):
    T, D = 17, 4096
    g = GraphBuilder()
    x, r = g.input("f32", "T", D), g.input("f32", "T", D)
    b, w = g.weight("f32", D), g.weight("f32", D)
    h = g.add(g.add(x, b), r)
    if h_out:
        g.output(h)
    y = g.output(g.rms_norm(h, w, eps=1e-5))
    xs, rs = synth.normal(44, 0, (T, D)), synth.normal(44, 1, (T, D))
    bs, ws = synth.normal(44, 2, (D,)), synth.normal(44, 3, (D,), mean=1.0, std=0.1)
    with dev.compile(g, max_tokens=32) as seg:
        assert seg.launches == ["fused[Add,Add]+RmsNorm"]
        for v, a in ((x, xs), (r, rs), (b, bs), (w, ws)):
            seg.set_input(v, a)
        log(f"provider bias+residual+norm h_out={h_out}")
        seg.execute(T)
        href = oracle.binary("Add", oracle.binary("Add", xs, bs), rs)
        assert_f32_close(seg.get_output(y), oracle.rmsnorm(href, ws, 1e-5), what="y")
        if h_out:
            assert np.array_equal(seg.get_output(h).view(np.uint32), href.view(np.uint32))


def test_provider_norm_head_and_long_chain(dev):
    """RmsNorm -> a 12-node chain over 6 inputs (register reuse) in one launch."""
    T, D = 5, 768
    g = GraphBuilder()
    x = g.input("f32", "T", D)
    ins = [g.input("f32", "T", D) for _ in range(3)] + [g.weight("f32", D) for _ in range(2)]
    v = g.rms_norm(x, None, eps=1e-6)
    for i in range(12):
        v = g.add(v, ins[i % 5]) if i % 3 == 0 else g.mul(v, ins[i % 5]) if i % 3 == 1 else g.unary("Tanh", v)
    y = g.output(v)
    vals = [synth.normal(45, i, (T, D)) for i in range(3)] + [synth.normal(45, 10 + i, (D,)) for i in range(2)]
    xs = synth.normal(45, 20, (T, D))
    with dev.compile(g, max_tokens=8) as seg:
        assert len(seg.launches) == 1 and seg.launches[0].startswith("RmsNorm+fused[")
        seg.set_input(x, xs)
        for vv, a in zip(ins, vals):
            seg.set_input(vv, a)
        log("provider norm head + long chain")
        seg.execute(T)
        got = seg.get_output(y)
    r = oracle.rmsnorm(xs, None, 1e-6)
    for i in range(12):
        a = vals[i % 5]
        r = oracle.binary("Add", r, a) if i % 3 == 0 else oracle.binary("Mul", r, a) if i % 3 == 1 else \
            oracle.unary_kind("Tanh", r)
    assert_f32_close(got, r, what="chain")
