"""Graph segments through the HIP provider (discover -> open -> compile -> set inputs -> execute -> outputs),
compared with the CPU oracle, in the manner of the reference's GPU-vs-CPU tests (tests/Sharplight.Vulkan.Tests:
NormTests.cs, RowOpTests.cs, RopeTests.cs, GatherTests.cs, FusionTests.cs:18-26,59-67,142-157). The launch
lists check that the fusions of the reference's lowerer happen."""
import numpy as np
import pytest

import oracle
from sharplight_amd import native, synth
from sharplight_amd.provider import GraphBuilder, HipExecutionProvider
from tests.devutil import log
from tests.parity import assert_bf16_close, assert_bits_equal, assert_f16_close, assert_f32_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(device):
    p = HipExecutionProvider()
    assert p.check_availability().is_available
    devices = p.get_devices()
    assert devices and devices[0].provider == "hip"
    return p.open_device(devices[0])


def test_norms_graph(dev):
    """ViewAndNormTests.Norms / NormTests: RmsNorm with and without weight, L2Norm, LayerNorm (T=5, n=70)."""
    T, n = 5, 70
    g = GraphBuilder()
    x = g.input("f32", "T", n)
    w = g.weight("f32", n)
    b = g.weight("f32", n)
    rms = g.output(g.rms_norm(x, w, eps=1e-5))
    rms0 = g.output(g.rms_norm(x, None, eps=1e-5))
    l2 = g.output(g.l2_norm(x, eps=1e-6))
    ln = g.output(g.layer_norm(x, w, b, eps=1e-5))
    xs = synth.normal(1, 0, (T, n), std=3.0)
    ws, bs = synth.normal(1, 1, (n,)), synth.normal(1, 2, (n,))
    with dev.compile(g, max_tokens=16) as seg:
        assert seg.launches == ["RmsNorm", "RmsNorm", "L2Norm", "LayerNorm"]
        seg.set_input(x, xs)
        seg.set_input(w, ws)
        seg.set_input(b, bs)
        log("provider norms")
        seg.execute(T)
        assert_f32_close(seg.get_output(rms), oracle.rmsnorm(xs, ws, 1e-5), what="rms")
        assert_f32_close(seg.get_output(rms0), oracle.rmsnorm(xs, None, 1e-5), what="rms0")
        assert_f32_close(seg.get_output(l2), oracle.rmsnorm(xs, None, 1e-6, mode=1), what="l2")
        assert_f32_close(seg.get_output(ln), oracle.layernorm(xs, ws, bs, 1e-5), what="ln")


@pytest.mark.parametrize("h_is_output", [True, False])
def test_residual_add_rmsnorm_fuses(dev, h_is_output):
    """FusionTests.cs:18-26: Add followed by RmsNorm is one launch; the sum is written only if read."""
    T, D = 33, 4096
    g = GraphBuilder()
    x = g.input("bf16", "T", D)
    r = g.input("bf16", "T", D)
    w = g.weight("f32", D)
    h = g.add(x, r)
    if h_is_output:
        g.output(h)
    y = g.output(g.rms_norm(h, w, eps=1e-5))
    c = synth.c2(rows=T, D=D)
    with dev.compile(g, max_tokens=64) as seg:
        assert seg.launches == ["fused[Add]+RmsNorm"]
        seg.set_input(x, c["x"])
        seg.set_input(r, c["res"])
        seg.set_input(w, c["w"])
        log(f"provider add+rmsnorm h_out={h_is_output}")
        seg.execute(T)
        yref, href = oracle.add_rmsnorm(c["x"], c["res"], c["w"], 1e-5, dtype="bf16")
        assert_bf16_close(seg.get_output(y), yref, what="y")
        if h_is_output:
            assert_bf16_close(seg.get_output(h), href, ulp=0, what="h")


@pytest.mark.parametrize("fmt,T,swap", [("bf16", 1, False), ("f16", 3, True), ("f32", 9, False), ("q8_0", 1, False),
                                        ("q4_0", 3, True), ("q4_k", 1, False), ("q5_k", 3, True),
                                        ("q4_k", 8, False), ("q6_k", 16, True),   # several-token matrix cores
                                        ("q3_k", 2, False)])                      # Q3_K: matrix cores always
def test_swiglu_dual_matvec_fuses(dev, fmt, T, swap):
    """FusionTests.SwiGluDualMatvec (FusionTests.cs:59-80): Mul(Silu(x Wg^T), x Wu^T) is one dual matvec launch
    (in either operand order), within the f32 dot-product bound of the unfused CPU computation. The matmuls
    carry f32_activations, so x stays f32 (the float-row path); the integer-dot form is tested below."""
    K, N = 1024, 96
    g = GraphBuilder()
    x = g.input("f32", "T", K)
    wg = g.weight(fmt, N, K)
    wu = g.weight(fmt, N, K)
    gate, up = g.matmul(x, wg, f32_activations=True), g.matmul(x, wu, f32_activations=True)
    y = g.output(g.mul(up, g.silu(gate)) if swap else g.mul(g.silu(gate), up))
    rg = synth.quant_table(fmt, N, K, seed=8, tid=1)
    ru = synth.quant_table(fmt, N, K, seed=8, tid=2)
    xs = synth.normal(8, 3, (T, K))
    with dev.compile(g, max_tokens=16) as seg:
        assert seg.launches == ["matvec2+fused[Silu,Mul]"]
        seg.set_input(x, xs)
        seg.set_input(wg, rg)
        seg.set_input(wu, ru)
        log(f"provider dual matvec {fmt} T={T}")
        seg.execute(T)
        got = seg.get_output(y).astype(np.float64)
    gr, ur = oracle.matvec(fmt, rg, N, K, xs), oracle.matvec(fmt, ru, N, K, xs)
    ref = oracle.mul(oracle.unary("silu", gr), ur).astype(np.float64)
    ax = np.abs(xs).astype(np.float64)
    # |d(silu)/dg| <= 1.1 everywhere: a first-order bound of the two products' rounding, plus the epilogue's;
    # block formats with an additive term add |a| per weight to the magnitudes summed (Q4_0: 8 |d|)
    def mags(raw):
        W = oracle.dequant(fmt, raw.reshape(-1), N * K).reshape(N, K).astype(np.float64)
        if fmt in ("q4_k", "q5_k"):  # |q * scale| + |min| per value
            from tests.test_oracle import _k_terms
            return _k_terms(fmt, raw.reshape(-1), N, K).reshape(N, K)
        if fmt != "q4_0":
            return np.abs(W)
        d = raw.reshape(N, K // 32, 18)[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
        A = np.repeat(-8.0 * d, 32, axis=1)
        return np.abs(W - A) + np.abs(A)
    tol = 2.0 ** -16 * (1.1 * np.abs(ur) * (ax @ mags(rg).T) + np.abs(gr) * (ax @ mags(ru).T)) + 1e-5 * np.abs(ref)
    assert (np.abs(got - ref) <= tol + 1e-30).all()


def test_matmul_alone_is_a_matvec(dev):
    K, N, T = 512, 40, 2
    g = GraphBuilder()
    x = g.input("f32", "T", K)
    w = g.weight("bf16", N, K)
    y = g.output(g.matmul(x, w))
    raw = synth.quant_table("bf16", N, K, seed=9, tid=1)
    xs = synth.normal(9, 2, (T, K))
    with dev.compile(g, max_tokens=4) as seg:
        assert seg.launches == ["matvec"]
        seg.set_input(x, xs)
        seg.set_input(w, raw)
        seg.execute(T)
        got = seg.get_output(y).astype(np.float64)
    W = oracle.dequant("bf16", raw.reshape(-1), N * K).reshape(N, K).astype(np.float64)
    S = np.abs(xs).astype(np.float64) @ np.abs(W).T
    assert (np.abs(got - oracle.matvec("bf16", raw, N, K, xs)) <= 2.0 ** -16 * S).all()


@pytest.mark.parametrize("y_is_output", [True, False])
def test_norm_writes_the_f16_copy(dev, y_is_output):
    """NormHalfCopyTests (tests/Sharplight.Vulkan.Tests/NormHalfCopyTests.cs): a Cast to f16 of an f32 norm
    output is the norm's own f16 copy -- one launch, the f32 values rounded once -- and the f32 rows are
    written only when read."""
    T, D = 40, 1024
    g = GraphBuilder()
    x = g.input("f32", "T", D)
    r = g.input("f32", "T", D)
    w = g.weight("f32", D)
    y = g.rms_norm(g.add(x, r), w, eps=1e-6)
    if y_is_output:
        g.output(y)
    y16 = g.output(g.cast(y, "f16"))
    xs, rs = synth.normal(4, 0, (T, D)), synth.normal(4, 1, (T, D))
    ws = synth.normal(4, 2, (D,), 1.0, 0.1)
    with dev.compile(g, max_tokens=64) as seg:
        assert seg.launches == ["fused[Add]+RmsNorm+f16copy" + ("" if y_is_output else "(no f32 rows)")]
        seg.set_input(x, xs)
        seg.set_input(r, rs)
        seg.set_input(w, ws)
        log(f"provider norm f16 copy y_out={y_is_output}")
        seg.execute(T)
        yref = oracle.rmsnorm(oracle.add(xs, rs), ws, 1e-6)
        got16 = seg.get_output(y16)
        assert_f16_close(got16.view(np.uint16), oracle.to_f16(yref), what="f16 copy")
        if y_is_output:
            y32 = seg.get_output(y)
            assert_f32_close(y32, yref, what="y")
            assert_bits_equal(got16.view(np.uint16), oracle.to_f16(y32), what="copy of y")


def test_cast_of_a_bf16_norm_stays_separate(dev):
    """The copy is the f32 value rounded once; a bf16 norm output cast to f16 is rounded twice, so it is not
    absorbed."""
    g = GraphBuilder()
    x = g.input("bf16", "T", 256)
    g.output(g.cast(g.rms_norm(x, None, out_type="bf16"), "f16"))
    with dev.compile(g, max_tokens=8) as seg:
        assert seg.launches == ["RmsNorm", "Cast"]


@pytest.mark.parametrize("act,op", [("silu", "Silu"), ("gelu_tanh", "GeluTanh"), ("gelu_erf", "Gelu")])
def test_gated_mlp_fuses(dev, act, op):
    """IMlpActivation.ActivateGated: Mul(act(gate), up) is one launch (FusionTests.cs:59-67's epilogue)."""
    T, F = 17, 14336
    g = GraphBuilder()
    gate = g.input("bf16", "T", F)
    up = g.input("bf16", "T", F)
    a = {"silu": g.silu, "gelu_tanh": g.gelu_tanh, "gelu_erf": g.gelu}[act](gate)
    y = g.output(g.mul(up, a))  # operand order must not matter
    c = synth.c3(rows=T, cols=F)
    with dev.compile(g, max_tokens=32) as seg:
        assert seg.launches == [f"fused[{op},Mul]"]
        seg.set_input(gate, c["gate"])
        seg.set_input(up, c["up"])
        log(f"provider gated {act}")
        seg.execute(T)
        assert_bf16_close(seg.get_output(y), oracle.gated(act, c["gate"], c["up"], dtype="bf16"), what=act)


def test_qwen3_qk_norm_rope_one_launch(dev):
    """The Qwen3 attention prologue (DecoderGraphBuilder.Attention.cs:146-206): RmsNorm per head then neox rope
    for q and k -- absorbed into rope (GraphLowerer.Fusion.cs:618-630) and merged into one launch."""
    T = 64
    g = GraphBuilder()
    q = g.input("bf16", "T", 32, 128)
    k = g.input("bf16", "T", 8, 128)
    pos = g.input("i32", "T")
    wq = g.weight("f32", 128)
    wk = g.weight("f32", 128)
    yq = g.output(g.rope(g.rms_norm(q, wq, eps=1e-6), pos, base=1e6, style="neox"))
    yk = g.output(g.rope(g.rms_norm(k, wk, eps=1e-6), pos, base=1e6, style="neox"))
    c = synth.c4(T=T)
    with dev.compile(g, max_tokens=T) as seg:
        assert seg.launches == ["rope+norm|rope+norm"]
        for v, a in ((q, c["q"]), (k, c["k"]), (pos, c["pos"]), (wq, c["wq"]), (wk, c["wk"])):
            seg.set_input(v, a)
        log("provider qk-norm rope")
        seg.execute(T)
        assert_bf16_close(seg.get_output(yq), oracle.qk_norm_rope(c["q"], c["pos"], c["wq"], 1e-6, dtype="bf16", base=1e6),
                          what="q")
        assert_bf16_close(seg.get_output(yk), oracle.qk_norm_rope(c["k"], c["pos"], c["wk"], 1e-6, dtype="bf16", base=1e6),
                          what="k")


def test_rope_normal_style_with_freq_factors(dev):
    """RopeTests.cs: the normal (gptj) style, frequency factors, partial dims, f32."""
    T, H, D = 9, 3, 64
    g = GraphBuilder()
    x = g.input("f32", "T", H, D)
    pos = g.input("i32", "T")
    ff = g.weight("f32", 16)
    y = g.output(g.rope(x, pos, ff, dims=32, base=1e4, style="gptj", freq_scale=0.5, attn_factor=1.25))
    xs = synth.normal(5, 0, (T, H, D))
    ps = synth.rng(5, 1).integers(0, 4000, T).astype(np.int32)
    fs = synth.rng(5, 2).uniform(1, 4, 16).astype(np.float32)
    with dev.compile(g, max_tokens=T) as seg:
        assert seg.launches == ["rope"]
        seg.set_input(x, xs)
        seg.set_input(pos, ps)
        seg.set_input(ff, fs)
        seg.execute(T)
        ref = oracle.rope(xs, ps, dims=32, neox=False, base=1e4, freq_scale=0.5, attn_factor=1.25, ff=fs)
        assert_f32_close(seg.get_output(y), ref, what="gptj rope")


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "f16", "q4_k", "q5_k", "q6_k", "iq4_xs", "tq2_0", "mxfp4", "nvfp4",
                                 "iq2_xxs", "iq3_s", "iq1_m"])
@pytest.mark.parametrize("out", ["f32", "bf16"])
def test_gather_graph(dev, fmt, out):
    """GatherTests.cs:7-25,147-163: token embedding from a quantized table (the reference's Table cases include
    q4_k, q5_k and q6_k); f32 output is the reference's default."""
    V, D, N = 300, 4096, 40
    g = GraphBuilder()
    tbl = g.weight(fmt, V, D)
    ids = g.input("i32", "T")
    y = g.output(g.gather(tbl, ids, out_type=out))
    table = synth.quant_table(fmt, V, D, seed=9)
    idv = synth.rng(9, 1).integers(0, V, N).astype(np.int32)
    with dev.compile(g, max_tokens=64) as seg:
        seg.set_input(tbl, table)
        seg.set_input(ids, idv)
        seg.execute(N)
        assert_bits_equal(seg.get_output(y), oracle.gather_as(fmt, table, V, D, idv, dtype=out), what=f"{fmt}->{out}")


def test_symbol_bound_and_index_errors(dev):
    """Execute beyond the compiled bound fails like CpuCompiledSegment.Execute; a bad id fails like GatherOp."""
    V, D = 10, 64
    g = GraphBuilder()
    tbl = g.weight("f32", V, D)
    ids = g.input("i32", "T")
    y = g.output(g.gather(tbl, ids))
    with dev.compile(g, max_tokens=4) as seg:
        seg.set_input(tbl, np.zeros((V, D), np.float32))
        with pytest.raises(ValueError, match="exceeds the compiled bound 4"):
            seg.execute(5)
        seg.set_input(ids, np.array([1, 11, 2], np.int32))
        seg.execute(3)
        with pytest.raises(IndexError, match="11"):
            seg.get_output(y)
        seg.set_input(ids, np.array([1, 2, 3], np.int32))
        seg.execute(3)
        assert seg.get_output(y).shape == (3, D)
        assert seg.device_memory_bytes >= V * D * 4


def test_symbolic_tokens_reuse_one_compilation(dev):
    """One compiled segment runs any T up to its bound (decode T=1, prefill T=bound)."""
    D = 1024
    g = GraphBuilder()
    x = g.input("f32", "T", D)
    w = g.weight("f32", D)
    y = g.output(g.rms_norm(x, w))
    ws = synth.normal(3, 1, (D,), 1.0, 0.1)
    with dev.compile(g, max_tokens=512) as seg:
        seg.set_input(w, ws)
        for T in (1, 7, 512, 3):
            xs = synth.normal(T, 0, (T, D))
            seg.set_input(x, xs)
            seg.execute(T)
            assert_f32_close(seg.get_output(y), oracle.rmsnorm(xs, ws, 1e-6), what=f"T={T}")


def _norm_rope_cache_graph(cache_type, D=128, Hq=4, Hkv=2, ctx=32, paged=False):
    """FusionTests.NormRopeIntoCache (tests/Sharplight.Vulkan.Tests/FusionTests.cs:138-175) without the
    attention read-out and with a single-axis rope: q and k RmsNorm then neox rope, k into the K cache,
    v into the V cache; the caches are states read back after the steps."""
    g = GraphBuilder()
    q = g.input("bf16", "T", Hq, D)
    k = g.input("bf16", "T", Hkv, D)
    v = g.input("bf16", "T", Hkv, D)
    pos = g.input("i32", "T")
    wq, wk = g.weight("f32", D), g.weight("f32", D)
    kc = g.state(cache_type, ctx, Hkv, D)
    vc = g.state(cache_type, ctx, Hkv, D)
    rows = pages = None
    kw = {}
    if paged:
        rows = g.input("i32", "T", 4)
        pages = g.weight("i32", 1, ctx // 8)
        kw = dict(slots=1, block_size=8)
    yq = g.output(g.rope(g.rms_norm(q, wq, eps=1e-6), pos, base=1e4, style="neox"))
    g.cache_write(kc, g.rope(g.rms_norm(k, wk, eps=1e-6), pos, base=1e4, style="neox"), rows, pages, **kw)
    g.cache_write(vc, v, rows, pages, **kw)
    return g, dict(q=q, k=k, v=v, pos=pos, wq=wq, wk=wk, kc=kc, vc=vc, yq=yq, rows=rows, pages=pages)


@pytest.mark.parametrize("cache_type,paged", [("bf16", False), ("f16", False), ("f16", True)])
def test_norm_rope_into_cache_graph(dev, cache_type, paged):
    D, Hq, Hkv, ctx = 128, 4, 2, 32
    g, h = _norm_rope_cache_graph(cache_type, D, Hq, Hkv, ctx, paged)
    wq, wk = synth.normal(7, 0, (D,), 1.0, 0.1), synth.normal(7, 1, (D,), 1.0, 0.1)
    table = np.int32([[3, 0, 2, 1]])  # paged: positions 0-7 live in block 3, 8-15 in block 0, ...
    chunks, past = [5, 1, 3, 1], 0
    ref_k = np.zeros((ctx, Hkv, D), np.float32)
    ref_v = np.zeros((ctx, Hkv, D), np.float32)
    with dev.compile(g, max_tokens=8) as seg:
        want = ["rope+norm|rope+norm+cache", "CacheWrite"] if cache_type == "bf16" else \
               ["rope+norm", "rope+norm+cache", "CacheWrite"]
        assert seg.launches == want
        seg.set_input(h["wq"], wq)
        seg.set_input(h["wk"], wk)
        if paged:
            seg.set_input(h["pages"], table)
        for i, c in enumerate(chunks):
            q = synth.normal(10 + i, 0, (c, Hq, D), dtype="bf16")
            k = synth.normal(20 + i, 0, (c, Hkv, D), dtype="bf16")
            v = synth.normal(30 + i, 0, (c, Hkv, D), dtype="bf16")
            p = np.arange(past, past + c, dtype=np.int32)
            for val, arr in ((h["q"], q), (h["k"], k), (h["v"], v), (h["pos"], p)):
                seg.set_input(val, arr)
            if paged:
                seg.set_input(h["rows"], np.stack([np.zeros(c, np.int32), p, p, p], axis=1))
            seg.set_scalar("n_past", past)
            log(f"provider cache step {i}: T={c} past={past}")
            seg.execute(c)
            assert_bf16_close(seg.get_output(h["yq"]),
                              oracle.qk_norm_rope(q, p, wq, 1e-6, dtype="bf16", base=1e4), what=f"q step {i}")
            rows = p if not paged else table[0, p // 8] * 8 + p % 8
            ref_k[rows] = oracle.rope(oracle.rmsnorm(oracle.from_bf16(k), wk, 1e-6), p, base=1e4)
            ref_v[rows] = oracle.from_bf16(v)
            past += c
        conv = oracle.to_f16 if cache_type == "f16" else oracle.to_bf16
        close = assert_f16_close if cache_type == "f16" else assert_bf16_close
        got_k = seg.get_output(h["kc"]).view(np.uint16)
        got_v = seg.get_output(h["vc"]).view(np.uint16)
        close(got_k, conv(ref_k), what="k cache")
        assert_bits_equal(got_v, conv(ref_v), what="v cache")
        seg.reset_state()
        assert not seg.get_output(h["kc"]).view(np.uint16).any()


def test_cache_write_needs_its_scalar(dev):
    g = GraphBuilder()
    x = g.input("f32", "T", 64)
    c = g.state("f32", 16, 64)
    g.cache_write(c, x)
    with dev.compile(g, max_tokens=4) as seg:
        seg.set_input(x, np.ones((2, 64), np.float32))
        with pytest.raises(ValueError, match="Runtime scalar 'n_past' was not provided"):
            seg.execute(2)
        seg.set_scalar("n_past", 15)
        with pytest.raises(native.SlhipCacheError, match=r"n_past 15 \+ T 2 > context 16"):
            seg.execute(2)


def test_standalone_elementwise_graph(dev):
    """A bias add over bf16 rows (f32 bias), a scalar Mul, a lone Silu and a Scale in one segment, each its
    own launch, against the oracle's BinaryOp/UnaryOp on the same widened values."""
    T, D = 19, 1000
    g = GraphBuilder()
    x = g.input("bf16", "T", D)
    bias = g.weight("f32", D)
    s = g.weight("f32", 1)
    h = g.add(x, bias)
    m = g.mul(h, s)
    a = g.output(g.silu(m))
    z = g.output(g.scale(a, scale=0.5, bias=-1.0))
    xs = oracle.to_bf16(synth.normal(5, 0, (T, D), std=2.0))
    bs = synth.normal(5, 1, (D,))
    ss = np.array([1.75], np.float32)
    with dev.compile(g, max_tokens=32) as seg:
        assert seg.launches == ["Add", "Mul", "Silu", "Scale"]
        seg.set_input(x, xs)
        seg.set_input(bias, bs)
        seg.set_input(s, ss)
        log("provider standalone elementwise")
        seg.execute(T)
        h32 = oracle.from_bf16(oracle.to_bf16(oracle.binary("Add", oracle.from_bf16(xs), bs)))
        m32 = oracle.from_bf16(oracle.to_bf16(oracle.binary("Mul", h32, ss)))
        a16 = oracle.to_bf16(oracle.unary_kind("Silu", m32))
        assert_bf16_close(seg.get_output(a), a16, what="silu")
        z16 = oracle.to_bf16(oracle.unary_kind("Scale", oracle.from_bf16(seg.get_output(a)).ravel(), 0.5, -1.0))
        assert_bf16_close(seg.get_output(z), z16.reshape(T, D), ulp=0, what="scale")


def test_mrope_graph_one_launch(dev):
    """A Qwen3-VL attention prologue: per-head RmsNorm then interleaved M-RoPE over [T, 3] positions for q
    and k -- absorbed and merged into one launch like the single-axis form."""
    T = 40
    g = GraphBuilder()
    q = g.input("bf16", "T", 8, 128)
    k = g.input("bf16", "T", 2, 128)
    pos = g.input("i32", "T", 3)
    wq = g.weight("f32", 128)
    wk = g.weight("f32", 128)
    kw = dict(base=5e6, style="neox", sections=(24, 20, 20, 0), interleaved=True)
    yq = g.output(g.rope(g.rms_norm(q, wq, eps=1e-6), pos, **kw))
    yk = g.output(g.rope(g.rms_norm(k, wk, eps=1e-6), pos, **kw))
    rng = np.random.default_rng(4)
    qs = oracle.to_bf16(rng.standard_normal((T, 8, 128)).astype(np.float32))
    ks = oracle.to_bf16(rng.standard_normal((T, 2, 128)).astype(np.float32))
    ps = rng.integers(0, 9000, (T, 3)).astype(np.int32)
    wqs = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    wks = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    with dev.compile(g, max_tokens=T) as seg:
        assert seg.launches == ["rope+norm|rope+norm"]
        for v, a in ((q, qs), (k, ks), (pos, ps), (wq, wqs), (wk, wks)):
            seg.set_input(v, a)
        log("provider mrope")
        seg.execute(T)
        for y, x, w in ((yq, qs, wqs), (yk, ks, wks)):
            xn = oracle.rmsnorm(oracle.from_bf16(x).reshape(-1, 128), w, 1e-6).reshape(x.shape)
            ref = oracle.to_bf16(oracle.rope_multi(xn, ps, [24, 20, 20, 0], interleaved=True, base=5e6))
            assert_bf16_close(seg.get_output(y), ref, what="mrope")


@pytest.mark.parametrize("fmt,T", [("q4_k", 1), ("q4_k", 8), ("q4_k", 9), ("q6_k", 3), ("q8_0", 1), ("q8_0", 2),
                                   ("mxfp4", 4), ("q4_0", 5)])
def test_swiglu_dual_matvec_int_dot(dev, fmt, T):
    """The decode FFN's gate/up pair by default (the lowerer's rule): x quantized once to q8, one dual int-dot
    launch for the row counts of the format's range (Q4_K/Q6_K/Q4_0/MXFP4 1..8, Q8_0 2..16), the f32 dual matvec
    outside it (GraphLowerer.MatMul.cs:150-158; GraphLowerer.IntDot.cs:18-19,52-75). Parity: against the oracle's
    integer-dot restatement inside the range, the float-row path outside."""
    K, N = 2048, 96
    g = GraphBuilder()
    x = g.input("f32", "T", K)
    wg = g.weight(fmt, N, K)
    wu = g.weight(fmt, N, K)
    y = g.output(g.mul(g.silu(g.matmul(x, wg)), g.matmul(x, wu)))
    rg = synth.quant_table(fmt, N, K, seed=12, tid=1)
    ru = synth.quant_table(fmt, N, K, seed=12, tid=2)
    xs = synth.normal(12, 3, (T, K))
    lo, hi = (2, 16) if fmt == "q8_0" else (1, 8)
    int_dot = lo <= T <= hi
    with dev.compile(g, max_tokens=8 if fmt == "mxfp4" else 16) as seg:
        assert seg.launches == [f"x->q8 rows {lo}..{hi}", f"matvec2+fused[Silu,Mul] (int-dot rows {lo}..{hi})"]
        assert seg.launches_at(T) == (["x->q8", "matvec2+fused[Silu,Mul] int-dot"] if int_dot
                                      else ["matvec2+fused[Silu,Mul] f32"])
        seg.set_input(x, xs)
        seg.set_input(wg, rg)
        seg.set_input(wu, ru)
        log(f"provider dual int-dot matvec {fmt} T={T}")
        seg.execute(T)
        got = seg.get_output(y).astype(np.float64)
    if int_dot:
        gr, Sg = oracle.matvec_q8(fmt, rg, N, K, xs, with_abs=True)
        ur, Su = oracle.matvec_q8(fmt, ru, N, K, xs, with_abs=True)
    else:
        gr, ur = oracle.matvec(fmt, rg, N, K, xs), oracle.matvec(fmt, ru, N, K, xs)
        from tests.test_gpu_matvec import _abs_terms
        ax = np.abs(xs).astype(np.float64)
        Wg = oracle.dequant(fmt, rg.reshape(-1), N * K).reshape(N, K)
        Wu = oracle.dequant(fmt, ru.reshape(-1), N * K).reshape(N, K)
        Sg, Su = ax @ _abs_terms(fmt, rg, Wg).T, ax @ _abs_terms(fmt, ru, Wu).T
    ref = oracle.mul(oracle.unary("silu", gr), ur).astype(np.float64)
    tol = 2.0 ** -16 * (1.1 * np.abs(ur) * Sg + np.abs(gr) * Su) + 1e-5 * np.abs(ref)
    assert (np.abs(got - ref) <= tol + 1e-30).all()


@pytest.mark.parametrize("fmt,T", [("q4_k", 20), ("iq4_xs", 31), ("q5_0", 6)])
def test_int_dot_cpu_rule_many_rows(dev, fmt, T):
    """The CPU provider's rule (option int_dot=cpu: every IntDot format, 1..31 rows, MatMulOp.cs:104,138-147) at
    row counts the integer matrix cores take in 16-token passes (20 = 16 + 4, 31 = 16 + 15)."""
    K, N = 1024, 80
    g = GraphBuilder()
    g.options["int_dot"] = "cpu"
    x = g.input("f32", "T", K)
    wg, wu = g.weight(fmt, N, K), g.weight(fmt, N, K)
    y = g.output(g.mul(g.silu(g.matmul(x, wg)), g.matmul(x, wu)))
    rg = synth.quant_table(fmt, N, K, seed=14, tid=1)
    ru = synth.quant_table(fmt, N, K, seed=14, tid=2)
    xs = synth.normal(14, 3, (T, K))
    with dev.compile(g, max_tokens=31) as seg:  # IQ4_XS has no f32 matvec: the bound stays in the rule's range
        assert seg.launches_at(T) == ["x->q8", "matvec2+fused[Silu,Mul] int-dot"]
        seg.set_input(x, xs)
        seg.set_input(wg, rg)
        seg.set_input(wu, ru)
        log(f"provider int-dot cpu rule {fmt} T={T}")
        seg.execute(T)
        got = seg.get_output(y).astype(np.float64)
    gr, Sg = oracle.matvec_q8(fmt, rg, N, K, xs, with_abs=True)
    ur, Su = oracle.matvec_q8(fmt, ru, N, K, xs, with_abs=True)
    ref = oracle.mul(oracle.unary("silu", gr), ur).astype(np.float64)
    tol = 2.0 ** -16 * (1.1 * np.abs(ur) * Sg + np.abs(gr) * Su) + 1e-5 * np.abs(ref)
    assert (np.abs(got - ref) <= tol + 1e-30).all()


def test_qkv_projections_share_one_q8_copy_and_fold_biases(dev):
    """Three biased projections of one x (a Qwen2-style attention input): one quantization, three int-dot
    launches with the biases folded in (FoldMatMulBiases), and a Q8_0 projection of the same x with its own
    copy for its own row range."""
    K = 1024
    Ns = [128, 64, 64]
    g = GraphBuilder()
    x = g.input("f32", "T", K)
    ws = [g.weight("q4_k", n, K) for n in Ns]
    bs = [g.weight("f32", n) for n in Ns]
    ys = [g.output(g.add(g.matmul(x, w), b)) for w, b in zip(ws, bs)]
    w8 = g.weight("q8_0", 32, K)
    y8 = g.output(g.matmul(x, w8))
    raws = [synth.quant_table("q4_k", n, K, seed=30, tid=i) for i, n in enumerate(Ns)]
    biases = [synth.normal(30, 10 + i, (n,)) for i, n in enumerate(Ns)]
    raw8 = synth.quant_table("q8_0", 32, K, seed=30, tid=9)
    T = 3
    xs = synth.normal(30, 20, (T, K))
    with dev.compile(g, max_tokens=16) as seg:
        assert seg.launches == ["x->q8 rows 1..8"] + ["matvec+bias (int-dot rows 1..8)"] * 3 + [
            "x->q8 rows 2..16", "matvec (int-dot rows 2..16)"]
        assert seg.launches_at(1) == ["x->q8"] + ["matvec+bias int-dot"] * 3 + ["matvec f32"]
        seg.set_input(x, xs)
        for w, r in zip(ws, raws):
            seg.set_input(w, r)
        for b, v in zip(bs, biases):
            seg.set_input(b, v)
        seg.set_input(w8, raw8)
        log("provider qkv int-dot + bias")
        seg.execute(T)
        for y, r, v, n in zip(ys, raws, biases, Ns):
            ref, S = oracle.matvec_q8("q4_k", r, n, K, xs, with_abs=True)
            ref = oracle.add(ref, np.broadcast_to(v, ref.shape).copy()).astype(np.float64)
            got = seg.get_output(y).astype(np.float64)
            assert (np.abs(got - ref) <= 2.0 ** -16 * S + 2.0 ** -24 * np.abs(ref) + 1e-30).all()
        ref, S = oracle.matvec_q8("q8_0", raw8, 32, K, xs, with_abs=True)
        assert (np.abs(seg.get_output(y8).astype(np.float64) - ref) <= 2.0 ** -16 * S + 1e-30).all()


def test_f32_activations_keep_x_unquantized(dev):
    K, N, T = 1024, 40, 2
    for f32_act, reduced in [(True, False), (True, True), (False, False)]:
        g = GraphBuilder()
        if reduced:
            g.options["reduced_precision"] = True
        x = g.input("f32", "T", K)
        w = g.weight("q4_k", N, K)
        y = g.output(g.matmul(x, w, f32_activations=f32_act))
        raw = synth.quant_table("q4_k", N, K, seed=31, tid=1)
        xs = synth.normal(31, 2, (T, K))
        with dev.compile(g, max_tokens=4) as seg:
            seg.set_input(x, xs)
            seg.set_input(w, raw)
            log(f"provider f32_activations={f32_act} reduced={reduced}")
            seg.execute(T)
            got = seg.get_output(y)
        q8 = not f32_act or reduced
        ref = oracle.matvec_q8("q4_k", raw, N, K, xs) if q8 else oracle.matvec("q4_k", raw, N, K, xs)
        other = oracle.matvec("q4_k", raw, N, K, xs) if q8 else oracle.matvec_q8("q4_k", raw, N, K, xs)
        # the two numerics differ visibly at this size; the result is the one the rule picks
        assert np.abs(got - ref).max() < 0.1 * np.abs(got - other).max()
