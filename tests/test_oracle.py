"""Pins the CPU oracle before it is trusted as the checker of the HIP kernels.

Each oracle function is checked against something independent of its own formula: the reference's
ggml golden vectors (tests/golden, extracted from tests/Sharplight.Cpu.Tests/Fixtures), an exhaustive
or brute-force enumeration, a closed form in f64, a library routine (numpy, torch, math.erf) or an
invariant -- chosen so that a dropped term, a wrong sign, a swapped pair index or an off-by-one in the
block layouts fails.
"""
import math
import os

import numpy as np
import pytest

import oracle
from sharplight_amd import synth

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def quant_fx():
    return np.load(os.path.join(GOLDEN, "ggml_quant.npz"))


@pytest.fixture(scope="module")
def rope_fx():
    return np.load(os.path.join(GOLDEN, "ggml_rope.npz"))


# ---- dequantization: ggml golden vectors (QuantTests.DequantizeMatchesGgml, QuantTests.cs:49-69) ----

@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q4_1", "q5_0", "q5_1"])
def test_dequant_matches_ggml(quant_fx, fmt):
    rows, cols = quant_fx[f"{fmt}_shape"]
    got = oracle.dequant(fmt, quant_fx[f"{fmt}_blocks"].reshape(-1), rows * cols).reshape(rows, cols)
    ref = quant_fx[f"{fmt}_deq"]
    # Equal as values: ggml computes (q-8)*d, which is -0 for q = 8 and d < 0; the reference (and the
    # oracle) compute fma(q, d, -8d) = +0. Every nonzero value is bit-identical.
    np.testing.assert_array_equal(got, ref)
    nz = ref != 0
    assert np.array_equal(got[nz].view(np.uint32), ref[nz].view(np.uint32))
    src = quant_fx[f"{fmt}_src"]
    assert float(np.sum((src - got) ** 2) / np.sum(src ** 2)) < 0.05  # the fixture is a real quantization


# ---- K-quants and the IQ4 codebook formats (GgmlDequantTests, tests/Sharplight.Cpu.Tests/GgmlDequantTests.cs) ----

@pytest.fixture(scope="module")
def quant_ext_fx():
    return np.load(os.path.join(GOLDEN, "ggml_quant_ext.npz"))


def _ext_records(fx, fmt):
    return sorted({k[: -len("_shape")] for k in fx.files if k.startswith(fmt + "_") and k.endswith("_shape")})


def _same_bits_or_both_nan(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return np.array_equal(a.view(np.uint32), b.view(np.uint32)) or (
        np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(a[~np.isnan(a)].view(np.uint32), b[~np.isnan(b)].view(np.uint32)))


@pytest.mark.parametrize("fmt", ["q2_k", "q3_k", "iq4_nl", "iq4_xs", "tq1_0", "tq2_0", "mxfp4", "nvfp4", "iq2_xxs",
                                 "iq2_xs", "iq2_s", "iq3_xxs", "iq3_s", "iq1_s", "iq1_m"])
def test_unfused_formats_match_ggml_bit_for_bit(quant_ext_fx, fmt):
    """The reference decodes these as ggml does (separate multiply and subtract), so ggml's own output in
    ggml_quant_ext.bin -- blocks quantized from gaussian data and random bytes -- must come out bit for bit
    (GgmlDequantTests.DequantizeMatchesGgml)."""
    recs = _ext_records(quant_ext_fx, fmt)
    assert len(recs) == 2
    for r in recs:
        rows, cols = quant_ext_fx[f"{r}_shape"]
        got = oracle.dequant(fmt, quant_ext_fx[f"{r}_blocks"].reshape(-1), rows * cols).reshape(rows, cols)
        assert _same_bits_or_both_nan(got, quant_ext_fx[f"{r}_deq"]), r


def _k_terms(fmt, blocks, rows, cols):
    """Per value the magnitudes of the decoder's two terms, |q * scale| + |offset|, recomputed in f64 from the
    block fields (an independent reading of the K-quant layouts)."""
    nb = cols // 256
    b = blocks.reshape(rows, nb, -1)
    f16 = lambda a: a.copy().view(np.float16)[..., 0].astype(np.float64)
    out = np.zeros((rows, nb, 256))
    if fmt in ("q4_k", "q5_k"):
        d, dmin, sc = f16(b[:, :, 0:2]), f16(b[:, :, 2:4]), b[:, :, 4:16].astype(np.int64)
        qs = b[:, :, 48:176] if fmt == "q5_k" else b[:, :, 16:144]
        for j in range(8):
            if j < 4:
                s_, m_ = sc[..., j] & 63, sc[..., j + 4] & 63
            else:
                s_ = (sc[..., j + 4] & 15) | ((sc[..., j - 4] >> 6) << 4)
                m_ = (sc[..., j + 4] >> 4) | ((sc[..., j] >> 6) << 4)
            g, half = j // 2, j % 2
            q = (qs[:, :, 32 * g:32 * g + 32].astype(np.int64) >> (4 * half)) & 15
            if fmt == "q5_k":
                q |= ((b[:, :, 16:48].astype(np.int64) >> j) & 1) << 4
            out[:, :, 32 * j:32 * j + 32] = np.abs(q * (d * s_)[..., None]) + np.abs((dmin * m_)[..., None])
    else:  # q6_k
        d = f16(b[:, :, 208:210])
        for n in range(2):
            for r in range(128):
                qt, i = r // 32, r % 32
                h = i // 16
                lo = b[:, :, 64 * n + (32 if qt & 1 else 0) + i].astype(np.int64)
                lo = lo >> 4 if qt >= 2 else lo & 15
                hi = (b[:, :, 128 + 32 * n + i].astype(np.int64) >> (2 * qt)) & 3
                s_ = d * b[:, :, 192 + 8 * n + h + 2 * qt].view(np.int8).astype(np.float64)
                out[:, :, 128 * n + r] = np.abs((lo | (hi << 4)) * s_) + np.abs(32 * s_)
    return out.reshape(rows, cols)


@pytest.mark.parametrize("fmt", ["q4_k", "q5_k", "q6_k"])
def test_fused_k_formats_match_ggml_within_one_rounding(quant_ext_fx, quant_fx, fmt):
    """The reference fuses q * scale + offset (one rounding) where ggml multiplies, then subtracts (two), so the
    values agree within one rounding of the larger term: |oracle - ggml| <= 2^-24 (|q scale| + |offset|) per
    value -- far tighter than QuantTests' 1e-5 (QuantTests.cs:58) -- on ggml's blocks and on random bytes."""
    cases = [(quant_ext_fx, r) for r in _ext_records(quant_ext_fx, fmt)] + [(quant_fx, fmt)]
    for fx, r in cases:
        rows, cols = fx[f"{r}_shape"]
        blocks = fx[f"{r}_blocks"]
        got = oracle.dequant(fmt, blocks.reshape(-1), rows * cols).reshape(rows, cols).astype(np.float64)
        ref = fx[f"{r}_deq"].astype(np.float64)
        fin = np.isfinite(ref)
        assert np.array_equal(np.isfinite(got), fin), r
        with np.errstate(invalid="ignore", over="ignore"):  # random-byte blocks hold inf / NaN scales
            bound = 2.0 ** -24 * _k_terms(fmt, blocks, rows, cols)
        assert (np.abs(got - ref)[fin] <= bound[fin] * (1 + 1e-12)).all(), r
        # and most values are the same bits
        assert np.mean(got[fin] == ref[fin]) > 0.5, r


def test_k_quant_fixture_is_a_real_quantization(quant_fx):
    for fmt in ("q4_k", "q5_k", "q6_k"):
        rows, cols = quant_fx[f"{fmt}_shape"]
        got = oracle.dequant(fmt, quant_fx[f"{fmt}_blocks"].reshape(-1), rows * cols).reshape(rows, cols)
        src = quant_fx[f"{fmt}_src"]
        assert float(np.sum((src - got) ** 2) / np.sum(src ** 2)) < 0.02, fmt


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q4_1", "q5_0", "q5_1", "q4_k", "q5_k", "q6_k"])
def test_gather_dequantizes_fixture_rows(quant_fx, fmt):
    """QuantTests.GatherDequantizes (QuantTests.cs:71-95): rows [3, 0, 2, 2] of the fixture table."""
    rows, cols = quant_fx[f"{fmt}_shape"]
    y = oracle.gather(fmt, quant_fx[f"{fmt}_blocks"], rows, cols, np.array([3, 0, 2, 2], np.int32))
    np.testing.assert_array_equal(y, quant_fx[f"{fmt}_deq"][[3, 0, 2, 2]])


def test_gather_out_of_range_raises():
    """QuantTests.GatherOutOfRangeThrows (QuantTests.cs:97): GatherOp checks every id."""
    t = np.zeros((4, 8), np.float32).view(np.uint8)
    for bad in (4, -1, 1 << 30):
        with pytest.raises(oracle.OutOfRange):
            oracle.gather("f32", t, 4, 8, np.array([0, bad], np.int32))


def _f16_codes():
    return np.arange(65536, dtype=np.uint32).astype(np.uint16)


def test_f16_to_f32_exhaustive():
    """All 65,536 binary16 codes against numpy's conversion (subnormals, infinities, NaN payloads)."""
    h = _f16_codes()
    got = oracle.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def _scale_codes():
    """f16 scale codes: normal, subnormal, negative, tiny and large (no inf/NaN)."""
    return np.array([0x3C00, 0x2E66, 0x1A36, 0x0001, 0x03FF, 0x0400, 0x8001, 0xBC00, 0xA0A4, 0x7BFF, 0xFBFF, 0x0000,
                     0x8000], np.uint16)


def test_q8_0_brute_force():
    """Every int8 code at every scale: q * d exactly; a zero product is +0 (fma(q, d, +0))."""
    codes = np.arange(-128, 128, dtype=np.int32)
    for s in _scale_codes():
        blocks = np.zeros((8, 34), np.uint8)
        blocks[:, 0:2] = np.frombuffer(np.uint16(s).tobytes(), np.uint8)
        blocks[:, 2:] = codes.astype(np.int8).view(np.uint8).reshape(8, 32)
        got = oracle.dequant("q8_0", blocks.reshape(-1), 256)
        d = np.float32(np.uint16(s).view(np.float16))
        ref = codes.astype(np.float32) * d
        ref[ref == 0] = 0.0
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), hex(s)


@pytest.mark.parametrize("fmt", ["q4_0", "q4_1", "q5_0", "q5_1"])
def test_nibble_formats_brute_force(fmt):
    """Every nibble (and high bit) in every position: (q - 8) d, (q - 16) d, q d + m."""
    bb = synth.BLOCK[fmt]
    qs_off = {"q4_0": 2, "q4_1": 4, "q5_0": 6, "q5_1": 8}[fmt]
    five = fmt.startswith("q5")
    rng = np.random.default_rng(7)
    for s in _scale_codes():
        m_code = np.uint16(0xB266)  # m = -0.2
        blocks = np.zeros((16, bb), np.uint8)
        blocks[:, 0:2] = np.frombuffer(np.uint16(s).tobytes(), np.uint8)
        if fmt in ("q4_1", "q5_1"):
            blocks[:, 2:4] = np.frombuffer(m_code.tobytes(), np.uint8)
        blocks[:, qs_off:] = rng.integers(0, 256, size=(16, bb - qs_off), dtype=np.uint8)
        blocks[0, qs_off:] = np.arange(16, dtype=np.uint8) * 17  # every nibble, both halves
        if five:
            blocks[:, qs_off - 4:qs_off] = rng.integers(0, 256, size=(16, 4), dtype=np.uint8)
        got = oracle.dequant(fmt, blocks.reshape(-1), 16 * 32).reshape(16, 32)
        d = np.float32(np.uint16(s).view(np.float16))
        m = np.float32(m_code.view(np.float16))
        for b in range(16):
            qs = blocks[b, qs_off:qs_off + 16].astype(np.int64)
            q = np.concatenate([qs & 15, qs >> 4])
            if five:
                qh = int(np.frombuffer(blocks[b, qs_off - 4:qs_off].tobytes(), np.uint32)[0])
                q = q | (((qh >> np.arange(32)) & 1) << 4)
            if fmt == "q4_0":
                ref = (q - 8).astype(np.float32) * d
            elif fmt == "q5_0":
                ref = (q - 16).astype(np.float32) * d
            else:
                ref = (q.astype(np.float64) * np.float64(d) + np.float64(m)).astype(np.float32)
            np.testing.assert_array_equal(got[b], ref, err_msg=f"{fmt} scale {s:#x} block {b}")


# ---- f32 -> bf16 --------------------------------------------------------------------------------------

def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * np.float32(10) ** rng.integers(-40, 38, 100000).astype(np.float32),
                        np.array([0.0, -0.0, np.inf, -np.inf, 1.0, 3.4028235e38, 1e-45, -1e-45,
                                  1.00390625, 1.01171875, 1.0039063, 1.0117188], np.float32)])
    # exact ties: mantissa ending in 0x8000 with both parities of the kept lsb
    ties = (np.arange(1000, dtype=np.uint32) << np.uint32(16) | np.uint32(0x8000)) + np.uint32(0x3F800000)
    x = np.concatenate([x, ties.view(np.float32)])
    got = oracle.to_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    assert np.array_equal(got, synth.bf16_bits(x))


def test_bf16_nan_quieting():
    """Simd.FloatToBFloat: a NaN keeps its top half with the quiet bit set."""
    nans = np.array([0x7F800001, 0x7FC00000, 0xFF800001, 0x7FBFFFFF, 0xFFFFFFFF], np.uint32).view(np.float32)
    got = oracle.to_bf16(nans)
    ref = ((nans.view(np.uint32) >> 16) | 0x40).astype(np.uint16)
    assert np.array_equal(got, ref)
    assert np.array_equal(oracle.from_bf16(got).view(np.uint32) >> 16, got.astype(np.uint32))


# ---- norms --------------------------------------------------------------------------------------------

def _rms_f64(x, w, eps, mode=0):
    x = x.astype(np.float64)
    ss = (x * x).sum(-1, keepdims=True)
    s = 1.0 / np.sqrt(ss / x.shape[-1] + eps) if mode == 0 else 1.0 / np.sqrt(ss + eps)
    y = x * s
    return y * w if w is not None else y


@pytest.mark.parametrize("n", [1, 7, 16, 70, 1024, 4099])
def test_rmsnorm_closed_form(n):
    """Ref.RmsNorm (tests/Sharplight.Cpu.Tests/Ref.cs:6-23): f64 scale; the reference tolerance is 1e-5/1e-4."""
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((5, n)) * 3).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    got = oracle.rmsnorm(x, w, 1e-5)
    np.testing.assert_allclose(got, _rms_f64(x, w, 1e-5), rtol=2e-6, atol=1e-6)
    np.testing.assert_allclose(oracle.rmsnorm(x, None, 1e-5), _rms_f64(x, None, 1e-5), rtol=2e-6, atol=1e-6)
    np.testing.assert_allclose(oracle.rmsnorm(x, None, 1e-6, mode=1), _rms_f64(x, None, 1e-6, 1), rtol=2e-6, atol=1e-7)


def test_rmsnorm_invariants():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((16, 512)).astype(np.float32)
    y = oracle.rmsnorm(x, None, 0.0)
    np.testing.assert_allclose(np.sqrt((y.astype(np.float64) ** 2).mean(-1)), 1.0, rtol=1e-6)  # unit RMS
    np.testing.assert_allclose(oracle.rmsnorm(x * np.float32(8), None, 0.0), y, rtol=1e-6, atol=1e-7)  # scale-free
    # eps is added to the mean square, not the sum: a zero row stays zero, a constant row c -> c/sqrt(c^2+eps)
    c = np.full((1, 64), 0.01, np.float32)
    np.testing.assert_allclose(oracle.rmsnorm(c, None, 1e-4), 0.01 / math.sqrt(1e-4 + 1e-4), rtol=1e-6)


def _layernorm_f64(x, w, b, eps):
    """ViewAndNormTests.Norms' LayerNorm reference (ViewAndNormTests.cs:161-182)."""
    x = x.astype(np.float64)
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    y = (x - m) / np.sqrt(v + eps)
    if w is not None:
        y = y * w
    if b is not None:
        y = y + b
    return y


@pytest.mark.parametrize("n", [1, 8, 70, 768, 5000])
def test_layernorm_closed_form(n):
    rng = np.random.default_rng(n + 1)
    x = (rng.standard_normal((5, n)) * 3 + 1).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    np.testing.assert_allclose(oracle.layernorm(x, w, b, 1e-5), _layernorm_f64(x, w, b, 1e-5), rtol=1e-5, atol=1e-5)
    y = oracle.layernorm(x, None, None, 1e-5)
    if n > 1:
        assert np.abs(y.astype(np.float64).mean(-1)).max() < 1e-5  # zero mean
        np.testing.assert_allclose((y.astype(np.float64) ** 2).mean(-1), 1.0, rtol=1e-3)


def test_row_ops_threaded_match_single_thread():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((300, 1000)).astype(np.float32)
    w = rng.standard_normal(1000).astype(np.float32)
    oracle.set_threads(4)
    try:
        assert np.array_equal(oracle.rmsnorm(x, w, 1e-6, threads=4), oracle.rmsnorm(x, w, 1e-6))
        assert np.array_equal(oracle.layernorm(x, w, w, 1e-6, threads=4), oracle.layernorm(x, w, w, 1e-6))
        g = rng.standard_normal(200000).astype(np.float32)
        assert np.array_equal(oracle.unary("silu", g, threads=4), oracle.unary("silu", g))
    finally:
        oracle.set_threads(1)


# ---- activations --------------------------------------------------------------------------------------

def _x_activations():
    rng = np.random.default_rng(11)
    return np.concatenate([rng.standard_normal(4000).astype(np.float32) * 3,
                           np.linspace(-12, 12, 4001, dtype=np.float32)[:4000]])


def test_silu_closed_form():
    x = _x_activations()
    ref = x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64)))
    np.testing.assert_allclose(oracle.unary("silu", x), ref, rtol=1e-6, atol=1e-7)  # Ref.Silu, Ref.cs:65


def test_gelu_tanh_closed_form():
    x = _x_activations()
    xd = x.astype(np.float64)
    ref = 0.5 * xd * (1 + np.tanh(0.7978845608028654 * (xd + 0.044715 * xd ** 3)))
    got = oracle.unary("gelu_tanh", x)
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-7)
    # the tail form (n % 8 elements) agrees with the vector form
    got7 = oracle.unary("gelu_tanh", x[:7])
    np.testing.assert_allclose(got7, ref[:7], rtol=2e-6, atol=1e-6)


def test_gelu_erf_closed_form():
    x = _x_activations()
    ref = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x.astype(np.float64)])
    # 1 + erf cancels for x << 0, so the f32 result carries the rational's ~1e-7 absolute error times |x|/2
    np.testing.assert_allclose(oracle.unary("gelu_erf", x), ref, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(oracle.unary("gelu_erf", x[:5]), ref[:5], rtol=1e-6, atol=2e-7)


def test_erf_implementations():
    for v in np.linspace(-7, 7, 2801):
        assert abs(oracle.lib().orc_erf(float(v)) - math.erf(v)) < 2e-15
        assert abs(oracle.lib().orc_erf_rational(float(v)) - math.erf(float(np.float32(v)))) < 4e-7


# ---- rope ---------------------------------------------------------------------------------------------

def test_rope_matches_ggml(rope_fx):
    """GgmlCrossCheckTests.RopeMatchesGgml (GgmlCrossCheckTests.cs:75-98), all seven cases: normal (mode 0),
    neox (mode 2), neox with partial dims and freq_scale 0.5, M-RoPE (mode 8, sections 2,3,3,0) and
    interleaved M-RoPE (mode 40, three section sets, one with dims 32 of D 64). Positions [T, 4] for the
    multi-axis modes, axis 0 otherwise, as the reference test passes them. Reference tolerance 2e-4."""
    for k in range(7):
        mode, dims, T, H, D = (int(v) for v in rope_fx[f"case{k}_meta"])
        fs = float(rope_fx[f"case{k}_freq_scale"][0])
        if mode >= 8:
            got = oracle.rope_multi(rope_fx[f"case{k}_x"], rope_fx[f"case{k}_pos"], rope_fx[f"case{k}_sections"],
                                    interleaved=mode == 40, dims=dims, neox=True, base=10000.0, freq_scale=fs)
        else:
            got = oracle.rope(rope_fx[f"case{k}_x"], rope_fx[f"case{k}_pos"][:, 0], dims=dims, neox=mode == 2,
                              base=10000.0, freq_scale=fs)
        ref = rope_fx[f"case{k}_y"]
        np.testing.assert_allclose(got, ref, rtol=2e-4, atol=2e-4)
        assert np.abs(got - ref).max() < 1e-5, k


def test_rope_axis_of_sector_rules():
    """RopeOp.AxisOf by hand: sectioned [2,3,3,0] and interleaved [3,2,2,1] over two periods; no sections
    -> axis 0."""
    sec = [oracle.rope_axis_of(i, [2, 3, 3, 0]) for i in range(10)]
    assert sec == [0, 0, 1, 1, 1, 2, 2, 2, 0, 0]
    il = [oracle.rope_axis_of(i, [3, 2, 2, 1], interleaved=True) for i in range(16)]
    assert il == [0, 1, 2, 0, 1, 2, 0, 3] * 2
    assert [oracle.rope_axis_of(i, [0, 0, 0, 5]) for i in range(3)] == [0, 0, 0]


def _rope_axes_f64(x, pos, ax1, ax2, dims, neox, base=10000.0):
    """f64 closed form with given axes per pair for the first and the second element."""
    T, H, D = x.shape
    half = dims // 2
    inv = base ** (-2.0 * np.arange(half) / dims)
    th1 = pos.astype(np.float64)[:, ax1] * inv[None, :]
    th2 = pos.astype(np.float64)[:, ax2] * inv[None, :]
    i0 = np.arange(half) if neox else 2 * np.arange(half)
    i1 = i0 + half if neox else i0 + 1
    y = x.astype(np.float64).copy()
    x0, x1 = x[:, :, i0].astype(np.float64), x[:, :, i1].astype(np.float64)
    y[:, :, i0] = x0 * np.cos(th1)[:, None, :] - x1 * np.sin(th1)[:, None, :]
    y[:, :, i1] = x0 * np.sin(th2)[:, None, :] + x1 * np.cos(th2)[:, None, :]
    return y


def test_rope_per_element_sections():
    """XD-RoPE: dims 8, sections [1,1,1,1], neox: pair i's first element i takes section i//2 and its second
    element i+4 section (i+4)//2, so the axes are (0,2), (0,2), (1,3), (1,3) -- worked by hand. With gptj
    pairs (2i, 2i+1) both elements take section i: per-element sections change nothing."""
    rng = np.random.default_rng(8)
    x = rng.standard_normal((5, 3, 8)).astype(np.float32)
    pos = rng.integers(0, 3000, (5, 4)).astype(np.int32)
    got = oracle.rope_multi(x, pos, [1, 1, 1, 1], per_element=True, neox=True)
    want = _rope_axes_f64(x, pos, [0, 0, 1, 1], [2, 2, 3, 3], 8, True)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
    plain = oracle.rope_multi(x, pos, [1, 1, 1, 1], neox=False)
    assert np.array_equal(oracle.rope_multi(x, pos, [1, 1, 1, 1], per_element=True, neox=False), plain)
    np.testing.assert_allclose(plain, _rope_axes_f64(x, pos, [0, 1, 2, 3], [0, 1, 2, 3], 8, False), rtol=1e-5, atol=1e-5)


def test_rope_multi_axis_with_equal_axes_is_plain_rope():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((6, 2, 16)).astype(np.float32)
    p = rng.integers(0, 30000, 6).astype(np.int32)
    pos = np.repeat(p[:, None], 4, axis=1)
    for sec, il in (([2, 3, 3, 0], False), ([3, 2, 2, 1], True)):
        assert np.array_equal(oracle.rope_multi(x, pos, sec, interleaved=il), oracle.rope(x, p))
    # one position axis broadcast to all four (RopeOp.cs:133-139)
    assert np.array_equal(oracle.rope_multi(x, p[:, None], [2, 3, 3, 0]), oracle.rope(x, p))


def _rope_f64(x, pos, dims, neox, base, fs=1.0, af=1.0, ff=None):
    T, H, D = x.shape
    half = dims // 2
    inv = base ** (-2.0 * np.arange(half) / dims) * fs
    th = pos.astype(np.float64)[:, None] * inv[None, :]
    if ff is not None:
        th = th / ff.astype(np.float64)
    c, s = np.cos(th) * af, np.sin(th) * af
    y = x.astype(np.float64).copy()
    i0 = np.arange(half) if neox else 2 * np.arange(half)
    i1 = i0 + half if neox else i0 + 1
    x0, x1 = x[:, :, i0].astype(np.float64), x[:, :, i1].astype(np.float64)
    y[:, :, i0] = x0 * c[:, None, :] - x1 * s[:, None, :]
    y[:, :, i1] = x0 * s[:, None, :] + x1 * c[:, None, :]
    return y


@pytest.mark.parametrize("neox", [True, False])
def test_rope_closed_form_large_positions(neox):
    """Qwen3 shape, theta 1e6, positions up to 32767: f64 angles keep the f32 result within 1e-5."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal((64, 4, 128)).astype(np.float32)
    pos = rng.integers(0, 32768, 64).astype(np.int32)
    pos[0] = 32767
    got = oracle.rope(x, pos, neox=neox, base=1e6)
    np.testing.assert_allclose(got, _rope_f64(x, pos, 128, neox, 1e6), rtol=1e-5, atol=1e-5)
    ff = rng.uniform(1, 8, 64).astype(np.float32)
    got = oracle.rope(x, pos, neox=neox, base=1e6, freq_scale=0.25, attn_factor=1.5, ff=ff)
    np.testing.assert_allclose(got, _rope_f64(x, pos, 128, neox, 1e6, 0.25, 1.5, ff), rtol=1e-5, atol=1e-5)


def test_rope_invariants():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((8, 3, 64)).astype(np.float32)
    assert np.array_equal(oracle.rope(x, np.zeros(8, np.int32), base=1e4), x)  # position 0: identity
    y = oracle.rope(x, rng.integers(0, 5000, 8).astype(np.int32), base=1e4)
    n0 = x[..., :32] ** 2 + x[..., 32:] ** 2
    n1 = y[..., :32] ** 2 + y[..., 32:] ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-5, atol=1e-6)  # each neox pair keeps its norm
    yp = oracle.rope(x, np.full(8, 100, np.int32), dims=16, base=1e4)
    assert np.array_equal(yp[..., 16:], x[..., 16:])  # dims past `dims` are copied


def test_qk_norm_rope_composition():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((16, 4, 128)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    pos = rng.integers(0, 32768, 16).astype(np.int32)
    got = oracle.qk_norm_rope(x, pos, w, 1e-6, base=1e6)
    ref = _rope_f64(_rms_f64(x, w, 1e-6).astype(np.float32), pos, 128, True, 1e6)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


# ---- KV cache writes (CacheWriteOp.cs, KvPages.cs) ------------------------------------------------

def test_f16_rounding_matches_numpy():
    """FloatToHalf (.NET (Half)f): IEEE round to nearest even, gradual underflow, overflow to inf --
    the same conversion numpy implements. Every finite f16 neighbourhood: the value itself, the midpoints
    to its neighbours (ties) and the f32 values one ulp either side of each midpoint; plus 2M random f32
    bit patterns over the whole exponent range."""
    h = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16)  # every finite non-negative f16
    v = h.view(np.float16).astype(np.float64)
    with np.errstate(over="ignore"):  # the largest finite f16's neighbour is inf
        nxt = np.nextafter(h.view(np.float16), np.float16(np.inf)).astype(np.float64)
    mid = ((v + nxt) / 2).astype(np.float32)  # exact in f32
    cand = np.concatenate([v.astype(np.float32), mid, np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(np.inf))])
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 1 << 32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    bits = bits[(bits & 0x7F800000) != 0x7F800000]  # finite
    cand = np.concatenate([cand, -cand, bits.view(np.float32), np.float32([0.0, -0.0, np.inf, -np.inf, 65504, 65520, -65520, 1e30])])
    with np.errstate(over="ignore"):
        ref = cand.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.to_f16(cand), ref)


def test_f16_nan_keeps_sign_and_payload_top():
    """The runtime's rule for NaN (parity unpinned: the .NET runtime is not part of the reference)."""
    nans = np.array([0x7F800001, 0x7FC00000, 0xFF800001, 0x7FBFFFFF, 0xFFFFFFFF, 0x7FA02000], np.uint32)
    got = oracle.to_f16(nans.view(np.float32))
    want = ((nans >> 16) & 0x8000) | 0x7E00 | ((nans & 0x7FFFFF) >> 13)
    assert np.array_equal(got, want.astype(np.uint16))
    assert np.isnan(got.view(np.float16)).all()


def test_cache_rows_past():
    assert list(oracle.cache_rows("past", 4, 10, n_past=6)) == [6, 7, 8, 9]
    assert list(oracle.cache_rows("past", 0, 10, n_past=10)) == []
    with pytest.raises(oracle.CacheOverflow, match=r"n_past 7 \+ T 4 > context 10"):
        oracle.cache_rows("past", 4, 10, n_past=7)


def test_cache_rows_multi_sequence():
    """Row = slot * (ctx / slots) + position (CacheWriteOp.Body, multi-sequence form)."""
    rng = np.random.default_rng(4)
    T, ctx, slots = 50, 96, 3
    seq = np.zeros((T, 4), np.int32)
    seq[:, 0] = rng.integers(0, slots, T)
    seq[:, 1] = rng.integers(0, ctx // slots, T)
    rows = oracle.cache_rows("seq", T, ctx, seq=seq, slots=slots)
    assert np.array_equal(rows, seq[:, 0] * (ctx // slots) + seq[:, 1])
    for bad in ((0, 32), (3, 0), (-1, 0), (1, -1)):
        s2 = seq.copy()
        s2[7, :2] = bad
        with pytest.raises(oracle.CacheOverflow, match="KV cache overflow: sequence row 7"):
            oracle.cache_rows("seq", T, ctx, seq=s2, slots=slots)


def test_cache_rows_paged():
    """Row = table[slot, p / bs] * bs + p % bs (KvPages.Row), brute force over every (slot, position)."""
    rng = np.random.default_rng(5)
    slots, bps, bs, ctx = 3, 4, 8, 12 * 8
    table = rng.permutation(12)[: slots * bps].reshape(slots, bps).astype(np.int32)
    seq = np.array([(s, p, 0, 0) for s in range(slots) for p in range(bps * bs)], np.int32)
    rows = oracle.cache_rows("paged", len(seq), ctx, seq=seq, pages=table, block_size=bs)
    want = [table[s, p // bs] * bs + p % bs for s, p, _, _ in seq]
    assert np.array_equal(rows, want)
    assert len(set(rows.tolist())) == len(rows)  # a permutation table maps positions to distinct rows
    with pytest.raises(oracle.CacheOverflow, match="outside the block table"):
        oracle.cache_rows("paged", 1, ctx, seq=np.int32([[0, bps * bs, 0, 0]]), pages=table, block_size=bs)
    t2 = table.copy()
    t2[1, 2] = 12  # past the cache's 12 blocks
    with pytest.raises(oracle.CacheOverflow, match="Block 12 of slot 1"):
        oracle.cache_rows("paged", 1, ctx, seq=np.int32([[1, 2 * bs + 3, 0, 0]]), pages=t2, block_size=bs)


@pytest.mark.parametrize("ct", ["f32", "f16", "bf16"])
def test_cache_write_converts_into_rows(ct):
    rng = np.random.default_rng(6)
    T, inner, ctx = 5, 24, 16
    x = rng.standard_normal((T, inner)).astype(np.float32)
    rows = np.int64([3, 9, 0, 15, 4])
    cache = np.full((ctx, inner), 7, np.float32 if ct == "f32" else np.uint16)
    oracle.cache_write(cache, x, rows, ct)
    conv = {"f32": lambda a: a, "f16": oracle.to_f16, "bf16": oracle.to_bf16}[ct]
    assert np.array_equal(cache[rows], conv(x))
    untouched = np.setdiff1d(np.arange(ctx), rows)
    assert (cache[untouched] == 7).all()


# ---- E4M3 activation rows (Kernels/e4m3.slang, Kernels/gemm_fp8.slang) ------------------------------

def _e4m3_values():
    """Every non-negative finite E4M3 code's value from the format's definition: bias 7, 3 mantissa bits,
    subnormals m * 2^-9, largest finite code 0x7E = 448 (0x7F is NaN)."""
    c = np.arange(0x7F)
    e, m = c >> 3, c & 7
    return np.where(e == 0, m * 2.0 ** -9, (1 + m / 8) * 2.0 ** (e - 7))


def _e4m3_nearest(v):
    """Brute force: the code whose value is nearest |v| (ties to the even code), saturated at 0x7E."""
    vals = _e4m3_values()
    a = np.minimum(np.abs(np.asarray(v, np.float64)), 448.0)
    d = np.abs(a[:, None] - vals[None, :])
    best = d.min(axis=1, keepdims=True)
    cand = np.where(d == best, np.arange(0x7F)[None, :], 1 << 20)
    even = np.where(cand % 2 == 0, cand, 1 << 20).min(axis=1)
    code = np.where(even < (1 << 20), even, cand.min(axis=1))
    return (code | np.where(np.asarray(v) < 0, 0x80, 0)).astype(np.uint8)


def test_e4m3_code_is_nearest_even():
    vals = _e4m3_values()
    mids = (vals[:-1] + vals[1:]) / 2
    f = np.float32
    cand = np.concatenate([vals, mids, np.nextafter(mids.astype(f), f(0)), np.nextafter(mids.astype(f), f(1e9)),
                           np.random.default_rng(8).uniform(0, 500, 20000), [448, 460, 464, 480, 1e6]]).astype(f)
    cand = np.concatenate([cand, -cand])
    got = np.array([oracle.e4m3_code(v) for v in cand], np.uint8)
    assert np.array_equal(got, _e4m3_nearest(cand))


def test_quantize_fp8_rows():
    """Per 128 values: scale amax / 448, codes nearest to v / scale (computed as v * (1/scale) in f32)."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((3, 512)).astype(np.float32) * np.float32([[1], [1e-3], [300]])
    x[1, 128:256] = 0  # an all-zero group: scale 0, codes 0
    q = oracle.quantize_fp8(x)
    assert q.shape == (3, 512 + 16)
    for r in range(3):
        d = q[r, 512:].view(np.float32)
        for g in range(4):
            v = x[r, 128 * g:128 * (g + 1)]
            assert d[g] == np.float32(np.abs(v).max()) / np.float32(448)
            inv = np.float32(1) / d[g] if d[g] > 0 else np.float32(0)
            assert np.array_equal(q[r, 128 * g:128 * (g + 1)], _e4m3_nearest(v * inv))
    assert not q[1, 128:256].any() and q[1, 512 + 4:512 + 8].view(np.float32)[0] == 0


def test_quantize_fp8_rows_threaded_matches():
    x = np.random.default_rng(10).standard_normal((300, 1024)).astype(np.float32)
    out = np.empty((300, 1024 + 32), np.uint8)
    oracle.lib().orc_quantize_fp8_rows_mt(oracle._p(x), 300, 1024, oracle._p(out))
    assert np.array_equal(out, oracle.quantize_fp8(x))


def test_f16_threaded_matches():
    x = np.random.default_rng(11).standard_normal(300_001).astype(np.float32)
    y = np.empty(x.size, np.uint16)
    oracle.lib().orc_f32_to_f16_mt(oracle._p(x), oracle._p(y), x.size)
    assert np.array_equal(y, oracle.to_f16(x))


# ---- matvec (MatMulOp's float-row path) ----------------------------------------------------------------

MV_FORMATS = ["f32", "f16", "bf16", "q8_0", "q4_0", "q4_1", "q5_0", "q5_1"]


def _deq_rows(fmt, raw, N, K):
    return oracle.dequant(fmt, raw.reshape(-1), N * K).reshape(N, K)


@pytest.mark.parametrize("fmt", MV_FORMATS)
@pytest.mark.parametrize("T", [1, 3, 6])
def test_matvec_one_hot_rows_pick_columns(fmt, T):
    """x = e_k picks column k of the dequantized W exactly, on every path (fused, chunked, paired rows):
    a transposed operand, a wrong block or chunk offset, or a dropped chunk cannot pass."""
    N, K = 13, 2080  # N not a multiple of 4; K over two 1024-value chunks and a partial third
    raw = synth.quant_table(fmt, N, K, seed=5, tid=1)
    W = _deq_rows(fmt, raw, N, K)
    ks = np.array([0, 31, 1023, 1024, 2079, 1500][:T])
    x = np.zeros((T, K), np.float32)
    x[np.arange(T), ks] = 1.0
    y = oracle.matvec(fmt, raw, N, K, x)
    assert np.array_equal(y, W[:, ks].T)


@pytest.mark.parametrize("fmt", MV_FORMATS)
@pytest.mark.parametrize("T", [1, 4, 5, 9])
def test_matvec_matches_f64_within_the_f32_bound(fmt, T):
    """Against the f64 dot of the dequantized rows: |y - y64| <= 2^-17 * sum_k |x_k w_k| (far below the
    worst-case bound of f32 summation; a dropped or doubled term shows at ~1e-3 of the sum)."""
    N, K = 37, 4096 if fmt != "f32" else 1536
    raw = synth.quant_table(fmt, N, K, seed=6, tid=2)
    W = _deq_rows(fmt, raw, N, K).astype(np.float64)
    x = synth.normal(6, 3, (T, K))
    y = oracle.matvec(fmt, raw, N, K, x)
    y64 = x.astype(np.float64) @ W.T
    bound = 2.0 ** -17 * (np.abs(x).astype(np.float64) @ np.abs(W).T)
    assert (np.abs(y - y64) <= bound).all()


def test_matvec_threaded_equals_plain():
    N, K = 301, 1024
    raw = synth.quant_table("q4_0", N, K, seed=7, tid=1)
    x = synth.normal(7, 2, (2, K))
    assert np.array_equal(oracle.matvec("q4_0", raw, N, K, x, threads=True), oracle.matvec("q4_0", raw, N, K, x))


def test_matvec_rejects_ragged_quant_rows():
    with pytest.raises(ValueError):
        oracle.matvec("q8_0", np.zeros((2, 34), np.uint8), 2, 40, np.zeros((1, 40), np.float32))


def test_fp4_scales_and_codes_closed_forms():
    """MXFP4: every E8M0 byte e gives 2^(e-128) times the doubled E2M1 value of every code; NVFP4: every
    UE4M3 byte gives (m/8 + 1) 2^(e-7) / 2 (e > 0) or m 2^-9 / 2 (e = 0), bit 7 ignored, 0x7F -> 0."""
    e2m1 = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], np.float64)
    code_vals = np.concatenate([2 * e2m1, -2 * e2m1])  # doubled, codes 8..15 negative
    # MXFP4: block = e, then 16 bytes holding codes j (low nibble) and 15 - j (high nibble)
    blocks = np.zeros((256, 17), np.uint8)
    blocks[:, 0] = np.arange(256)
    blocks[:, 1:] = (np.arange(16) | ((15 - np.arange(16)) << 4)).astype(np.uint8)
    got = oracle.dequant("mxfp4", blocks.reshape(-1), 256 * 32).reshape(256, 32).astype(np.float64)
    codes = np.concatenate([np.arange(16), 15 - np.arange(16)])
    want = np.ldexp(1.0, np.arange(256) - 128)[:, None] * code_vals[codes][None, :]
    assert np.array_equal(got, want.astype(np.float32).astype(np.float64))
    # NVFP4: four scales per block, code 2 (value 2) everywhere -> 2 * scale
    x = np.arange(256)
    e, m = (x >> 3) & 15, x & 7
    scale = np.where(e == 0, m * 2.0 ** -9, (1 + m / 8) * np.ldexp(1.0, e - 7)) / 2
    scale[(x == 0) | (x == 0x7F)] = 0
    blocks = np.zeros((64, 36), np.uint8)
    blocks[:, :4] = x.reshape(64, 4)
    blocks[:, 4:] = 0x22
    got = oracle.dequant("nvfp4", blocks.reshape(-1), 64 * 64).reshape(64, 4, 16).astype(np.float64)
    assert np.array_equal(got, np.broadcast_to(2 * scale.reshape(64, 4)[..., None], got.shape))


def test_tq1_trits_invert_the_ggml_packing():
    """Five ternary digits t0..t4 (t0 most significant) pack as q = ceil(v * 256 / 243), v = sum t_i 3^(4-i)
    (ggml's quantize_row_tq1_0); every byte of every TQ1_0 region must decode back to t_n - 1."""
    v = np.arange(243)
    q = (v * 256 + 242) // 243
    digits = np.stack([(v // 3 ** (4 - n)) % 3 for n in range(5)], 1)  # [243, 5]
    blocks = np.zeros((243, 54), np.uint8)
    blocks[:, :48] = q[:, None]
    blocks[:, 48:52] = q[:, None]
    blocks[:, 52:54] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    got = oracle.dequant("tq1_0", blocks.reshape(-1), 243 * 256).reshape(243, 256)
    want = np.empty((243, 256))
    for n in range(5):
        want[:, n * 32:(n + 1) * 32] = digits[:, n:n + 1] - 1
        want[:, 160 + n * 16:160 + (n + 1) * 16] = digits[:, n:n + 1] - 1
    for n in range(4):
        want[:, 240 + 4 * n:244 + 4 * n] = digits[:, n:n + 1] - 1
    assert np.array_equal(got, want)


def _grid(name, n, width):
    """A table of iq_grids.h as an [n, width] byte array."""
    import re
    text = open(os.path.join(os.path.dirname(__file__), "..", "sharplight_amd", "csrc", "iq_grids.h")).read()
    body = text[text.index(name + "["):]
    body = body[body.index("{") + 1:body.index("}")]
    vals = [int(v.rstrip("ul"), 16) for v in re.findall(r"0x[0-9a-f]+u?l*", body)]
    assert len(vals) == n
    dt = np.uint64 if width == 8 else np.uint32
    return np.array(vals, dt).view(np.uint8).reshape(n, width), np.array(vals, dt)


def test_iq_grid_tables_have_the_lattice_structure():
    """ggml's lattice tables: IQ2 entries take the values {8, 25, 43}, IQ3 entries {4, 12, ..., 52, 62}, IQ1
    entries {-1, 0, 1}; entries are distinct and ascending as ggml lists them (the IQ1 entries as base-3
    numbers), with the table sizes the
    index widths imply. A corrupted or shifted entry breaks one of these; the fixture records above pin the
    entries their blocks use bit for bit."""
    for name, n, w, allowed in [("kIq2xxsGrid", 256, 8, {8, 25, 43}), ("kIq2xsGrid", 512, 8, {8, 25, 43}),
                                ("kIq2sGrid", 1024, 8, {8, 25, 43}),
                                ("kIq3xxsGrid", 256, 4, {4, 12, 20, 28, 36, 44, 52, 62}),
                                ("kIq3sGrid", 512, 4, {1, 3, 5, 7, 9, 11, 13, 15}),
                                ("kIq1sGrid", 2048, 8, {0xFF, 0, 1})]:
        b, v = _grid(name, n, w)
        assert set(np.unique(b).tolist()) <= allowed, name
        if name == "kIq1sGrid":  # ascending as base-3 numbers, byte 7 the most significant digit
            key = ((b.view(np.int8)[:, ::-1].astype(np.int64) + 1) * 3 ** np.arange(7, -1, -1)).sum(1)
        else:
            key = v
        assert np.all(key[1:] > key[:-1]), name
