"""Pins of the oracle's integer-dot matvec (oracle/sl_oracle.c: orc_q8_quantize, orc_intdot_decode,
orc_intdot_dot, orc_matvec_q8): the CPU provider's few-row MatMul with q8 activations
(src/Sharplight.Cpu/MatMulOp.cs:173-213, IntDot.cs:92-126, IntDot.Decode.cs, IntDot.Kernels.cs:12-29).

No reference fixture holds int-dot outputs, so each part is pinned by what the mathematics fixes:
  * the quantizer against an independent numpy statement of the rule in f32 arithmetic, and by hand-computed
    blocks (exact ties, the f32 addition quirk of the half-away rounding, zero and subnormal blocks, NaN);
  * the decoder by a * u + b reproducing the dequantized weights (orc_dequant, itself pinned by ggml's
    fixtures) exactly or within one rounding;
  * the dot by an f64 evaluation of sum_g (a_g d s_g + b_g gs_g) with integer s_g from numpy, and, end to end,
    by the float-row matvec: the two differ by at most the quantization error sum |w| d / 2 per block;
  * x already on the int8 grid (per block d = 2^m, |q| <= 127 with 127 present) gives the float-row result
    within f32 accumulation; a one-hot x = 127 * 2^m e_k picks 127 * 2^m * (a u_k + b) of every row."""
import numpy as np
import pytest

import oracle
from sharplight_amd import synth

FORMATS = oracle.INTDOT_FORMATS


def _np_quantize(x):
    """The quantization rule of IntDot.QuantizeBlockScalar written with numpy f32 arithmetic."""
    x = np.asarray(x, np.float32).reshape(-1, 32)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        amax = np.abs(x).max(axis=1)  # numpy's max propagates NaN, as MathF.Max does
        d = (amax / np.float32(127)).astype(np.float32)
        idv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
        v = (x * idv[:, None]).astype(np.float32)
        r = (v + np.copysign(np.float32(0.5), v)).astype(np.float32)
        r = np.where(np.isnan(r), 0, np.trunc(r)).astype(np.int64)
    q = r.astype(np.int8)
    s = r.reshape(-1, 2, 16).sum(axis=2)
    gs = (d[:, None] * s.astype(np.float32)).astype(np.float32)
    return q.reshape(-1), d, gs.reshape(-1)


@pytest.mark.parametrize("seed", range(6))
def test_quantize_matches_numpy_rule(seed):
    g = np.random.default_rng(seed)
    K = 4096
    x = (g.standard_normal((3, K // 32, 32)) * np.exp2(g.integers(-30, 30, size=(3, K // 32, 1)))).reshape(3, K)
    x = x.astype(np.float32)
    q, d, gs = oracle.q8_quantize(x)
    for r in range(3):
        nq, nd, ngs = _np_quantize(x[r])
        assert np.array_equal(q[r], nq)
        assert np.array_equal(d[r].view(np.uint32), nd.view(np.uint32))
        assert np.array_equal(gs[r].view(np.uint32), ngs.view(np.uint32))


def test_quantize_hand_blocks():
    # amax 127 -> d = 1, id = 1: x = k + 0.5 rounds away from zero
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:8] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5]
    x[8] = np.float32(0.49999997)   # 0.49999997 + 0.5 rounds up to 1.0 in f32: q = 1, not 0
    x[9] = np.float32(-0.49999997)
    x[10] = 0.25
    q, d, gs = oracle.q8_quantize(x[None])
    assert d[0, 0] == 1.0
    assert list(q[0, :11]) == [127, 1, -1, 2, -2, 3, -3, 127, 1, -1, 0]
    assert gs[0, 0] == float(q[0, :16].astype(np.int64).sum())
    assert gs[0, 1] == 0.0
    # a zero block: d = 0, id = 0, every q 0
    q, d, gs = oracle.q8_quantize(np.zeros((1, 32), np.float32))
    assert not q.any() and d[0, 0] == 0.0 and not gs.any()
    # amax 2^-120: d is subnormal, 1 / d still finite, q = x / d rounded
    x = (np.arange(32, dtype=np.float32) - 16) * np.float32(2.0 ** -124)
    q, d, gs = oracle.q8_quantize(x[None])
    assert d[0, 0] == np.float32(np.float32(2.0 ** -120) / np.float32(127)) and d[0, 0] < np.finfo(np.float32).tiny
    assert q[0, 0] == -127 and q[0, 16] == 0 and q[0, 31] == round(15 * 127 / 16)
    # amax 2^-136: 1 / d overflows to inf, x * id is +-inf (0 * inf NaN), and the saturating cast gives
    # int.MaxValue (low byte 0xFF: -1) for positive values, int.MinValue (low byte 0) for negative ones and 0
    # for NaN -- what the reference's (sbyte)(int) of IntDot.QuantizeBlockScalar yields under .NET's
    # saturating conversions
    x = (np.arange(32, dtype=np.float32) - 16) * np.float32(2.0 ** -140)
    q, d, gs = oracle.q8_quantize(x[None])
    assert list(q[0]) == [0] * 17 + [-1] * 15
    # NaN in a block: amax NaN, d NaN, every code 0 (the saturating cast of NaN), the sums NaN
    x = np.ones(64, np.float32)
    x[3] = np.nan
    q, d, gs = oracle.q8_quantize(x[None])
    assert not q[0, :32].any() and np.isnan(d[0, 0]) and np.isnan(gs[0, :2]).all()
    assert (q[0, 32:] == 127).all() and d[0, 1] == np.float32(1) / np.float32(127)


@pytest.mark.parametrize("fmt", FORMATS)
def test_decode_reproduces_dequant(fmt):
    K, N = 512, 24
    raw = synth.quant_table(fmt, N, K, seed=5, tid=1)
    W = oracle.dequant(fmt, raw.reshape(-1), N * K).reshape(N, K).astype(np.float64)
    rb = raw.shape[1]
    for n in range(N):
        u, a, b = oracle.intdot_decode(fmt, raw[n], K)
        A = np.repeat(a.astype(np.float64), 16)
        B = np.repeat(b.astype(np.float64), 16)
        v = A * u + B  # exact in f64 (a 24-bit a times an 8-bit u)
        # the reference decodes K-quants with one fused rounding (Quant.cs), the others exactly
        tol = 2.0 ** -24 * (np.abs(A * u) + np.abs(B)) * 2
        assert np.all(np.abs(v - W[n]) <= tol), (fmt, n)
        assert raw[n].size == rb


def _f64_dot(fmt, raw, N, K, x):
    """sum_g a_g d s_g + b_g gs_g in f64 with exact integer s_g: the value the f32 dot approximates."""
    q, d, gs = oracle.q8_quantize(x)
    T = x.shape[0]
    y = np.zeros((T, N))
    S = np.zeros((T, N))
    for n in range(N):
        u, a, b = oracle.intdot_decode(fmt, raw[n], K)
        s = (u.astype(np.int64)[None, :] * q.astype(np.int64)).reshape(T, K // 16, 16).sum(axis=2)
        dg = np.repeat(d.astype(np.float64), 2, axis=1)
        terms = a.astype(np.float64) * dg * s
        offs = b.astype(np.float64) * gs.astype(np.float64)
        y[:, n] = (terms + offs).sum(axis=1)
        S[:, n] = (np.abs(terms) + np.abs(offs)).sum(axis=1)
    return y, S


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("T", [1, 3])
def test_dot_against_f64_and_float_rows(fmt, T):
    K, N = 1024, 20
    raw = synth.quant_table(fmt, N, K, seed=7, tid=2)
    x = synth.normal(11, 3, (T, K))
    y, yabs = oracle.matvec_q8(fmt, raw, N, K, x, with_abs=True)
    y64, S = _f64_dot(fmt, raw, N, K, x)
    assert np.allclose(yabs, S, rtol=1e-12, atol=0)
    assert np.all(np.abs(y - y64) <= 2.0 ** -17 * S + 1e-30)
    # against the float rows: |sum w (x - d q)| <= sum |w| d / 2 (each value within half a step)
    W = oracle.dequant(fmt, raw.reshape(-1), N * K).reshape(N, K).astype(np.float64)
    yf = oracle.matvec(fmt, raw, N, K, x).astype(np.float64)
    q, d, gs = oracle.q8_quantize(x)
    step = np.repeat(d.astype(np.float64), 32, axis=1) / 2  # [T, K]
    bound = step @ np.abs(W).T + 2.0 ** -16 * (np.abs(x).astype(np.float64) @ np.abs(W).T + S)
    assert np.all(np.abs(y - yf) <= bound)
    # the threaded variant equals the plain one
    assert np.array_equal(oracle.matvec_q8(fmt, raw, N, K, x, threads=True).view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("fmt", FORMATS)
def test_on_grid_x_matches_float_rows(fmt):
    K, N, T = 512, 16, 2
    g = np.random.default_rng(3)
    q = g.integers(-127, 128, size=(T, K // 32, 32))
    q[:, :, 5] = 127
    m = g.integers(-12, 6, size=(T, K // 32, 1))
    x = (q * np.exp2(m)).astype(np.float32).reshape(T, K)
    raw = synth.quant_table(fmt, N, K, seed=9, tid=1)
    qq, d, gs = oracle.q8_quantize(x)
    assert np.array_equal(qq.reshape(T, K // 32, 32), q.astype(np.int8))
    y = oracle.matvec_q8(fmt, raw, N, K, x).astype(np.float64)
    W = oracle.dequant(fmt, raw.reshape(-1), N * K).reshape(N, K).astype(np.float64)
    exact = x.astype(np.float64) @ W.T
    _, S = _f64_dot(fmt, raw, N, K, x)
    assert np.all(np.abs(y - exact) <= 2.0 ** -16 * S + 2.0 ** -22 * (np.abs(x).astype(np.float64) @ np.abs(W).T))


@pytest.mark.parametrize("fmt", FORMATS)
def test_one_hot_picks_column(fmt):
    K, N = 512, 12
    raw = synth.quant_table(fmt, N, K, seed=13, tid=1)
    for k in (0, 17, 255, 300, 511):
        c = 127.0 * 2.0 ** -3
        x = np.zeros((1, K), np.float32)
        x[0, k] = c
        y = oracle.matvec_q8(fmt, raw, N, K, x)[0].astype(np.float64)
        for n in range(N):
            u, a, b = oracle.intdot_decode(fmt, raw[n], K)
            want = c * (float(a[k // 16]) * float(u[k]) + float(b[k // 16]))
            mag = c * (abs(float(a[k // 16]) * float(u[k])) + abs(float(b[k // 16])))
            assert abs(y[n] - want) <= 2.0 ** -22 * mag, (fmt, k, n)


def test_unsupported_formats_refused():
    raw = synth.quant_table("q2_k", 4, 256, seed=1, tid=1)
    with pytest.raises(ValueError):
        oracle.matvec_q8("q2_k", raw, 4, 256, np.ones((1, 256), np.float32))
    assert [oracle.lib().orc_intdot_supported(oracle.FORMATS[f]) for f in FORMATS] == [1] * len(FORMATS)
