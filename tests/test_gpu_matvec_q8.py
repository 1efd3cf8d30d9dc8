"""GPU parity of the integer-dot matvec (slhip_quantize_q8, slhip_matvec_q8, slhip_dual_matvec_q8) against the
oracle's restatement of the CPU provider's few-row MatMul with q8 activations (src/Sharplight.Cpu/MatMulOp.cs:
173-213, IntDot.cs), followed for the dual form by the activation and Mul (the Vulkan lowerer's fused int-dot
unit, GraphLowerer.MatMul.cs:150-158).

Bars:
  * the quantized rows (codes, block scales, 16-value group sums) bit for bit;
  * y within 2^-16 * S of the oracle, S = sum over 16-value groups of |a d s| + |b gs| (the oracle's f32 sum
    is within 2^-17 * S of the exact value of those terms, tests/test_oracle_intdot.py; the kernel's integer
    sums are exact and its f32 sums run in another order); the dual form propagates that through act(g) * u to
    first order, plus 1e-5 relative for the activation; bf16 outputs 2 bf16 ulp on top."""
import math
import zlib

import numpy as np
import pytest

import oracle
from sharplight_amd import native, synth
from tests.devutil import Dev, log

pytestmark = pytest.mark.gpu

NP = {"f32": np.float32, "bf16": np.uint16}


def _seed(*parts) -> int:
    return zlib.crc32(repr(parts).encode())


def _x(dx, T, K, seed, spread=False):
    x = synth.normal(seed, 9, (T, K), dtype="f32")
    if spread:  # block magnitudes over 2^-20 .. 2^12
        g = np.random.default_rng(seed)
        x = (x.reshape(T, K // 32, 32) * np.exp2(g.integers(-20, 12, size=(T, K // 32, 1)))).reshape(T, K)
        x = x.astype(np.float32)
    if dx == "bf16":
        xb = oracle.to_bf16(x)
        return xb, oracle.from_bf16(xb)
    return x, x


def _quantize_on_gpu(d, dx, x, T, K):
    rb = native.q8_row_bytes(K)
    px = d.put(x)
    pq = d.empty(T * rb)
    native.quantize_q8(dx, px, T, K, pq)
    return pq, rb


def _unpack(buf, T, K):
    rb = K + K // 2
    b = buf.reshape(T, rb)
    q = b[:, :K].copy().view(np.int8)
    s = b[:, K:].copy().view(np.float32).reshape(T, K // 32, 4)
    return q, s


@pytest.mark.parametrize("dx", ["f32", "bf16"])
@pytest.mark.parametrize("T,K", [(1, 256), (3, 4096), (17, 1024), (5, 14336)])
def test_quantize_bits(device, dx, T, K):
    x, x32 = _x(dx, T, K, _seed("q", dx, T, K), spread=True)
    with Dev() as d:
        log(f"quantize_q8 x={dx} T={T} K={K}")
        pq, rb = _quantize_on_gpu(d, dx, x, T, K)
        native.synchronize()
        got = d.get(pq, (T * rb,), np.uint8)
    q, s = _unpack(got, T, K)
    oq, od, ogs = oracle.q8_quantize(x32)
    assert np.array_equal(q, oq)
    assert np.array_equal(s[:, :, 0].view(np.uint32), od.view(np.uint32))
    assert np.array_equal(s[:, :, 1:3].reshape(T, K // 16).view(np.uint32), ogs.view(np.uint32))
    assert not s[:, :, 3].view(np.uint32).any()


def test_quantize_edge_blocks(device):
    K = 256
    x = np.zeros((1, K), np.float32)
    x[0, 0] = 127.0  # block 0: d = 1, ties away from zero, the f32 addition quirk
    x[0, 1:11] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, np.float32(0.49999997), np.float32(-0.49999997), 0.25]
    # block 1: zeros; block 2: amax 2^-120 (subnormal d); block 3: amax 2^-136 (1/d overflows: saturating casts)
    x[0, 64:96] = (np.arange(32, dtype=np.float32) - 16) * np.float32(2.0 ** -124)
    x[0, 96:128] = (np.arange(32, dtype=np.float32) - 16) * np.float32(2.0 ** -140)
    x[0, 128:160] = 1.0
    x[0, 130] = np.nan  # block 4: NaN
    x[0, 160:192] = -3.0
    x[0, 170] = np.inf  # block 5: inf: d inf, id 0, inf * 0 NaN -> 0
    x[0, 192:224] = np.float32(3e38)  # block 6: near the f32 maximum
    x[0, 224:256] = -np.float32(3e38)
    x[0, 230] = np.float32(-3.4028235e38)
    with Dev() as d:
        log("quantize_q8 edge blocks")
        pq, rb = _quantize_on_gpu(d, "f32", x, 1, K)
        native.synchronize()
        got = d.get(pq, (rb,), np.uint8)
    q, s = _unpack(got, 1, K)
    oq, od, ogs = oracle.q8_quantize(x)
    assert np.array_equal(q, oq)
    assert np.array_equal(s[:, :, 0].view(np.uint32), od.view(np.uint32))
    g, og = s[:, :, 1:3].reshape(1, K // 16), ogs
    assert np.array_equal(np.isnan(g), np.isnan(og))
    assert np.array_equal(np.where(np.isnan(g), 0, g).view(np.uint32), np.where(np.isnan(og), 0, og).view(np.uint32))


def _run(fmt, dx, dy, x, raws, N, K, *, act=None, bias=None):
    T = x.shape[0]
    with Dev() as d:
        log(f"matvec_q8 {'dual ' + act if act else 'single'} fmt={fmt} x={dx} y={dy} T={T} K={K} N={N}"
            f"{' bias' if bias is not None else ''}")
        pq, _ = _quantize_on_gpu(d, dx, x, T, K)
        pw = [d.put(r) for r in raws]
        py = d.empty(max(T * N * np.dtype(NP[dy]).itemsize, 4))
        if act:
            native.dual_matvec_q8(act, fmt, dy, pq, T, K, pw[0], pw[1], N, py)
        else:
            native.matvec_q8(fmt, dy, pq, T, K, pw[0], N, py, bias=None if bias is None else d.put(bias))
        native.synchronize()
        return d.get(py, (T, N), NP[dy])


def _compare(got, dy, ref, tol, what):
    if dy == "bf16":
        g = oracle.from_bf16(got).astype(np.float64)
        r = oracle.from_bf16(oracle.to_bf16(ref)).astype(np.float64)
        tol = tol + 2 * 2.0 ** -8 * np.abs(r)
    else:
        g, r = got.astype(np.float64), ref.astype(np.float64)
    bad = np.abs(g - r) > tol
    if bad.any():
        i = tuple(np.argwhere(bad)[0])
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} beyond the bound; first at {i}: got {g[i]!r} "
                             f"ref {r[i]!r} tol {tol[i]!r}")


FORMATS = oracle.INTDOT_FORMATS

SINGLE_CASES = [  # (fmt, x dtype, y dtype, T, K, N)
    *[(f, "f32", "f32", 1, 4096, 96) for f in FORMATS],
    *[(f, "bf16", "bf16", 3, 1024, 37) for f in FORMATS],
    *[(f, "f32", "f32", 8, 2048, 40) for f in FORMATS],
    ("q8_0", "f32", "f32", 16, 4096, 33),    # two passes of eight tokens
    ("q4_k", "f32", "bf16", 13, 1280, 24),   # a partial second pass
    ("q6_k", "f32", "f32", 2, 3072, 40),     # rows of 2520 bytes: 4-byte staging loads
    ("q6_k", "bf16", "f32", 1, 768, 24),     # 630 bytes: 2-byte loads
    ("iq4_xs", "f32", "f32", 5, 1280, 33),   # 680 bytes: 8-byte loads
    ("mxfp4", "f32", "f32", 1, 768, 19),     # 408 bytes: 8-byte loads
    ("q4_0", "f32", "f32", 1, 14336, 20),    # a down projection's K
    ("q8_0", "bf16", "f32", 2, 14336, 17),
    ("q4_k", "f32", "f32", 1, 256, 1),       # a single row of one super-block
    ("q5_k", "f32", "f32", 31, 4096, 24),    # the CPU provider's largest int-dot row count
    ("q4_0", "f32", "f32", 2, 2880, 40),     # K a multiple of 32 only: rows of 1620 bytes, 2-byte loads
    ("q8_0", "bf16", "f32", 1, 1056, 33),    # 1122 bytes
    ("q5_1", "f32", "bf16", 3, 2080, 24),    # 1560 bytes: 8-byte loads
    ("iq4_nl", "f32", "f32", 4, 96, 17),     # three blocks
    # from 3-5 tokens (by format) with K whole stages: the integer matrix cores (16-row tiles, 512- or 1024-value stages)
    *[(f, "f32", "bf16", 9, 1024, 40) for f in FORMATS],      # one stage, a partial tile
    ("q4_k", "bf16", "f32", 16, 3072, 48),   # three stages (an odd count)
    ("q6_k", "f32", "f32", 20, 2048, 33),    # a full 16-token pass and a 4-token one
    ("q8_0", "f32", "f32", 9, 14336, 16),    # fourteen stages, one tile
    ("q4_0", "f32", "f32", 10, 1280, 24),    # K not whole stages: the VALU kernel
    # 64-value slices: Q6_K / IQ4_XS loaded straight into registers, Q4_K / Q5_K read from the row images;
    # K = 14336 is four slice groups per row (the last one half full), T = 3 pads a four-token pass
    ("q6_k", "f32", "f32", 2, 14336, 20),
    ("iq4_xs", "bf16", "f32", 3, 14336, 17),
    ("q4_k", "f32", "bf16", 3, 14336, 21),
    ("q5_k", "f32", "f32", 1, 14336, 19),
    ("q6_k", "f32", "bf16", 4, 256, 700),    # one slice group, many rows per wave
    ("q8_0", "f32", "f32", 6, 1536, 33),     # Q8_0's 512-value stages: three of them (K not a multiple of 1024)
    # three and four tokens where the matrix cores take them from 3 or 4 tokens (Q8_0, Q4_K, IQ4_NL, Q5_K, ...)
    # but K is not whole 512-value stages: the VALU kernel
    ("q8_0", "f32", "f32", 3, 1056, 33),
    ("iq4_nl", "bf16", "f32", 3, 1056, 21),
    ("q4_k", "f32", "f32", 4, 1280, 21),
    ("q5_k", "f32", "bf16", 4, 1280, 19),
    ("mxfp4", "f32", "f32", 4, 768, 18),
    ("q4_k", "f32", "bf16", 3, 14080, 21),   # 55 super-blocks: Q4_K's slices on the VALU kernel
]


@pytest.mark.parametrize("fmt,dx,dy,T,K,N", SINGLE_CASES)
def test_matvec_q8(device, fmt, dx, dy, T, K, N):
    seed = _seed(fmt, dx, dy, T, K, N)
    raw = synth.quant_table(fmt, N, K, seed=seed, tid=1)
    x, x32 = _x(dx, T, K, seed)
    y = _run(fmt, dx, dy, x, [raw], N, K)
    ref, S = oracle.matvec_q8(fmt, raw, N, K, x32, with_abs=True)
    _compare(y, dy, ref, 2.0 ** -16 * S + 1e-30, f"matvec_q8 {fmt}")


@pytest.mark.parametrize("fmt,T", [("q4_0", 3), ("q4_k", 3), ("q6_k", 3), ("iq4_nl", 3), ("q4_k", 12), ("q8_0", 7),
                                   ("q6_k", 16), ("mxfp4", 5)])
def test_matvec_q8_bias_and_spread(device, fmt, T):
    """The bias epilogue (FoldMatMulBiases: y + b in f32 after the product) and x blocks spread over 2^-20..2^12,
    on the VALU kernel (Q4_0 and Q6_K at 3 tokens) and the matrix cores (the rest: Q4_K and IQ4_NL from 3)."""
    K, N = 2048, 50
    seed = _seed("bias", fmt, T)
    raw = synth.quant_table(fmt, N, K, seed=seed, tid=1)
    x, x32 = _x("f32", T, K, seed, spread=True)
    b = synth.normal(seed, 4, (N,), dtype="f32")
    y = _run(fmt, "f32", "f32", x, [raw], N, K, bias=b)
    ref, S = oracle.matvec_q8(fmt, raw, N, K, x32, with_abs=True)
    ref = oracle.add(ref, np.broadcast_to(b, ref.shape).copy())
    _compare(y, "f32", ref, 2.0 ** -16 * S + 2.0 ** -24 * np.abs(ref) + 1e-30, f"matvec_q8 bias {fmt}")


def _act64(act, g):
    g = np.asarray(g, np.float64)
    if act == "silu":
        with np.errstate(over="ignore"):
            return g / (1.0 + np.exp(-g))
    if act == "gelu_tanh":
        return 0.5 * g * (1.0 + np.tanh(0.7978845608028654 * (g + 0.044715 * g ** 3)))
    return 0.5 * g * (1.0 + np.vectorize(math.erf)(g / math.sqrt(2.0)))


DUAL_CASES = [  # (act, fmt, x dtype, y dtype, T, K, N)
    ("silu", "q4_k", "f32", "f32", 1, 4096, 14336),   # a Q4_K_M decode FFN's gate/up at one token
    ("silu", "q4_k", "f32", "bf16", 8, 4096, 14336),  # and at eight
    ("silu", "q6_k", "f32", "f32", 1, 4096, 14336),
    ("silu", "q6_k", "bf16", "f32", 8, 4096, 14336),
    ("gelu_tanh", "q8_0", "f32", "f32", 2, 2048, 40),
    ("gelu_erf", "q4_0", "bf16", "bf16", 4, 1024, 72),
    ("silu", "q5_k", "f32", "f32", 3, 2048, 33),
    ("silu", "q4_1", "f32", "f32", 1, 4096, 40),
    ("silu", "q5_0", "bf16", "f32", 6, 1024, 24),
    ("silu", "q5_1", "f32", "bf16", 1, 1024, 24),
    ("gelu_tanh", "iq4_nl", "f32", "f32", 2, 2048, 33),
    ("silu", "iq4_xs", "f32", "f32", 1, 1280, 40),
    ("silu", "mxfp4", "f32", "f32", 5, 2880, 33),       # gpt-oss's hidden size (rows of 1530 bytes)
    ("silu", "q6_k", "f32", "f32", 16, 3072, 17),
    ("gelu_erf", "q5_k", "bf16", "bf16", 12, 4096, 100),   # matrix cores, dual
    ("silu", "iq4_xs", "f32", "f32", 11, 2048, 64),
    ("gelu_tanh", "mxfp4", "f32", "bf16", 9, 1024, 16),
    ("silu", "q8_0", "f32", "f32", 16, 4096, 14336),        # the lowerer's largest Q8_0 int-dot batch
]


@pytest.mark.parametrize("act,fmt,dx,dy,T,K,N", DUAL_CASES)
def test_dual_matvec_q8(device, act, fmt, dx, dy, T, K, N):
    seed = _seed(act, fmt, dx, dy, T, K, N)
    rg = synth.quant_table(fmt, N, K, seed=seed, tid=1)
    ru = synth.quant_table(fmt, N, K, seed=seed, tid=2)
    x, x32 = _x(dx, T, K, seed)
    y = _run(fmt, dx, dy, x, [rg, ru], N, K, act=act)
    g, Sg = oracle.matvec_q8(fmt, rg, N, K, x32, with_abs=True)
    u, Su = oracle.matvec_q8(fmt, ru, N, K, x32, with_abs=True)
    ref = oracle.mul(oracle.unary(act, g), u)
    g64 = g.astype(np.float64)
    h = 1e-4 * np.maximum(1.0, np.abs(g64))
    dact = np.abs((_act64(act, g64 + h) - _act64(act, g64 - h)) / (2 * h)) * 1.5 + 1e-3
    e = 2.0 ** -16
    tol = dact * np.abs(u) * e * Sg + np.abs(_act64(act, g64)) * e * Su + 1e-5 * np.abs(ref) + 1e-30
    if act == "gelu_erf":
        tol = tol + 0.5 * np.abs(g64 * u) * 4.2e-7
    _compare(y, dy, ref, tol, f"dual_matvec_q8 {act} {fmt}")


@pytest.mark.parametrize("fmt,dx,T,K,N", [
    ("q4_k", "f32", 3, 4096, 200), ("q8_0", "bf16", 12, 2048, 64),
    # few tokens on the VALU kernel
    ("q4_k", "f32", 1, 4096, 300), ("q6_k", "bf16", 1, 4096, 130), ("q4_0", "bf16", 2, 2048, 70),
    ("q5_1", "f32", 4, 1056, 33), ("q8_0", "f32", 2, 96, 17), ("mxfp4", "f32", 1, 768, 40),
    # the register-piece kernel (IQ4_XS) and the matrix cores
    ("iq4_xs", "f32", 1, 4096, 90), ("q5_k", "bf16", 4, 2048, 48)])
def test_dual_matvec_int8_one_call(device, fmt, dx, T, K, N):
    """slhip_dual_matvec_int8 (quantize into the caller's workspace, then the dual matvec) equals the two calls
    bit for bit; a workspace below T q8 rows is refused."""
    seed = _seed("one_call", fmt, dx, T)
    rg = synth.quant_table(fmt, N, K, seed=seed, tid=1)
    ru = synth.quant_table(fmt, N, K, seed=seed, tid=2)
    x, _ = _x(dx, T, K, seed)
    two = _run(fmt, dx, "f32", x, [rg, ru], N, K, act="silu")
    with Dev() as d:
        px, pg, pu = d.put(x), d.put(rg), d.put(ru)
        py = d.empty(T * N * 4)
        wb = T * native.q8_row_bytes(K)
        work = d.empty(wb)
        log(f"dual_matvec_int8 fmt={fmt} x={dx} T={T} K={K} N={N}")
        native.dual_matvec_int8("silu", fmt, dx, "f32", px, T, K, pg, pu, N, py, work, wb)
        native.synchronize()
        one = d.get(py, (T, N), np.float32)
        with pytest.raises(native.SlhipArgumentError, match="workspace"):
            native.dual_matvec_int8("silu", fmt, dx, "f32", px, T, K, pg, pu, N, py, work, wb - 1)
    assert np.array_equal(one.view(np.uint32), two.view(np.uint32))


def test_refusals(device):
    with Dev() as d:
        p = d.empty(4096)
        for fn, args in [
            ("slhip_matvec_q8", (native.FORMATS["q2_k"], native.DTYPES["f32"], p, 1, 256, p, 1, p, 1, None, None)),
            ("slhip_matvec_q8", (native.FORMATS["q4_0"], native.DTYPES["f32"], p, 1, 80, p, 1, p, 1, None, None)),
            ("slhip_matvec_q8", (native.FORMATS["q4_k"], native.DTYPES["f32"], p, 1, 288, p, 1, p, 1, None, None)),
            ("slhip_matvec_q8", (native.FORMATS["mxfp4"], native.DTYPES["f32"], p, 1, 96, p, 1, p, 1, None, None)),
            ("slhip_quantize_q8", (native.DTYPES["f32"], p, 100, 1, 100, p, None)),
        ]:
            st = getattr(native.lib(), fn)(*args)
            assert st == native.ERR_UNSUPPORTED, (fn, st)
        native.matvec_q8("q4_0", "f32", None, 0, 256, None, 10, None)  # T = 0: nothing to do
