"""GPU parity of the decode matvec and the dual gate/up matvec with the gating epilogue (slhip_matvec,
slhip_dual_matvec) against the oracle's restatement of the CPU provider's MatMul float-row path followed by
the activation and Mul -- the reference's FusionTests.SwiGluDualMatvec (tests/Sharplight.Vulkan.Tests/
FusionTests.cs:59-80: the fused dual matvec against the CPU provider, T in 1..140, K 1024 and 256).

Tolerance (f32 sums in a different order): for a dot product with terms x_k w_k the kernel and the oracle
each stay within 2^-17 * S of the exact value (the oracle's own pin), so they are held to 2^-16 * S of each
other, with S = sum_k |x_k w_k| for dense and Q8_0 weights and, for the formats with an additive term
(w = q d + a, summed as d * sum x q + a * sum x, the form of the reference's fused Q4_0 dot),
S = sum_k |x_k| (|q_k d| + |a|); the dual epilogue propagates that through act(g) * u (first order, with act'
evaluated in f64), plus 1e-5 relative for the activation itself. bf16 outputs: 2 bf16 ulp of the rounded
reference on top. A one-hot x picks a weight column and must come out exactly."""
import math
import zlib

import numpy as np
import pytest

import oracle
from sharplight_amd import native, synth
from tests.devutil import Dev, log
from tests.parity import assert_bits_equal

pytestmark = pytest.mark.gpu

NP = {"f32": np.float32, "bf16": np.uint16}


def _seed(*parts) -> int:
    return zlib.crc32(repr(parts).encode())


def _weights(fmt, N, K, seed, tid):
    raw = synth.quant_table(fmt, N, K, seed=seed, tid=tid)
    W = oracle.dequant(fmt, raw.reshape(-1), N * K).reshape(N, K)
    return raw, W


def _act64(act, g):
    g = np.asarray(g, np.float64)
    if act == "silu":
        with np.errstate(over="ignore"):  # exp(-g) = inf for very negative g: g / inf = -0, as wanted
            return g / (1.0 + np.exp(-g))
    if act == "gelu_tanh":
        return 0.5 * g * (1.0 + np.tanh(0.7978845608028654 * (g + 0.044715 * g ** 3)))
    return 0.5 * g * (1.0 + np.vectorize(math.erf)(g / math.sqrt(2.0)))


def _run(fmt, dx, dy, x, raws, N, K, *, act=None, x_stride=None, y_stride=None, pad=0):
    T = x.shape[0]
    xs = K if x_stride is None else x_stride
    ys = N if y_stride is None else y_stride
    xp = np.zeros((T, xs), x.dtype)
    xp[:, :K] = x
    with Dev() as d:
        px = d.put(xp, pad)
        pw = [d.put(r) for r in raws]
        py = d.empty(max(T * ys * np.dtype(NP[dy]).itemsize, 4))
        log(f"matvec {'dual ' + act if act else 'single'} fmt={fmt} x={dx} y={dy} T={T} K={K} N={N} "
            f"xs={xs} ys={ys}")
        if act:
            native.dual_matvec(act, fmt, dx, dy, px, T, K, pw[0], pw[1], N, py, x_stride=xs, y_stride=ys)
        else:
            native.matvec(fmt, dx, dy, px, T, K, pw[0], N, py, x_stride=xs, y_stride=ys)
        native.synchronize()
        y = d.get(py, (T, ys), NP[dy])
    return y[:, :N]


BLOCK_ADD = {"q4_0": -8, "q5_0": -16}  # additive term OFF * d; q4_1 / q5_1 carry m


def _abs_terms(fmt, raw, W):
    """|q d| + |a| per weight (= |w| for dense and Q8_0 weights): the magnitudes the kernel's sums add."""
    if fmt in ("f32", "f16", "bf16", "q8_0"):
        return np.abs(W).astype(np.float64)
    if fmt == "q3_k":  # d (s - 32) (q - 4): one term per value
        return np.abs(W).astype(np.float64)
    if fmt == "q2_k":  # |q d sc| + |dmin m| per value (ggml's Q2_K layout)
        N, K = W.shape
        b = raw.reshape(N, K // 256, 84)
        f16 = lambda a: a.copy().view(np.float16)[..., 0].astype(np.float64)
        d, dmin = f16(b[:, :, 80:82]), f16(b[:, :, 82:84])
        out = np.zeros((N, K // 256, 256))
        for n in range(2):
            for j in range(4):
                for h in range(2):
                    sc = b[:, :, 8 * n + 2 * j + h].astype(np.int64)
                    q = (b[:, :, 16 + 32 * n + 16 * h:16 + 32 * n + 16 * h + 16].astype(np.int64) >> (2 * j)) & 3
                    v0 = 128 * n + 32 * j + 16 * h
                    out[:, :, v0:v0 + 16] = np.abs(q * (d * (sc & 15))[..., None]) + np.abs((dmin * (sc >> 4))[..., None])
        return out.reshape(N, K)
    if fmt in ("q4_k", "q5_k", "q6_k"):  # |q * scale| + |offset| per value, from the block fields
        from tests.test_oracle import _k_terms
        N, K = W.shape
        return _k_terms(fmt, raw.reshape(-1), N, K).reshape(N, K)
    N, K = W.shape
    bb = {"q4_0": 18, "q4_1": 20, "q5_0": 22, "q5_1": 24}[fmt]
    blocks = raw.reshape(N, K // 32, bb)
    d = blocks[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    a = BLOCK_ADD[fmt] * d if fmt in BLOCK_ADD else blocks[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    A = np.repeat(a, 32, axis=1)
    return np.abs(W.astype(np.float64) - A) + np.abs(A)


def _x(dx, T, K, seed):
    x = synth.normal(seed, 9, (T, K), dtype=dx)
    return x, (oracle.from_bf16(x) if dx == "bf16" else x)


def _check_single(got, dy, ref, S, what):
    tol = 2.0 ** -16 * S + 1e-30
    if dy == "bf16":
        g = oracle.from_bf16(got).astype(np.float64)
        r = oracle.from_bf16(oracle.to_bf16(ref)).astype(np.float64)
        tol = tol + 2 * 2.0 ** -8 * np.abs(r)
    else:
        g, r = got.astype(np.float64), ref.astype(np.float64)
    bad = np.abs(g - r) > tol
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} beyond the bound; first at {np.argwhere(bad)[0]}"


SINGLE_CASES = [  # (fmt, x dtype, y dtype, T, K, N)
    ("bf16", "f32", "f32", 1, 4096, 96),
    ("bf16", "f32", "f32", 3, 1024, 96),
    ("f16", "f32", "f32", 8, 1024, 37),
    ("f32", "f32", "f32", 9, 256, 40),
    ("bf16", "bf16", "bf16", 16, 4096, 70),
    ("f16", "bf16", "f32", 20, 512, 33),
    ("f32", "f32", "bf16", 2, 8, 5),        # one vector per row: most lanes clamp
    ("bf16", "f32", "f32", 1, 14336, 24),   # K split over waves
    ("f32", "f32", "f32", 1, 16384, 8),     # the largest staged K
    ("q8_0", "f32", "f32", 1, 4096, 96),
    ("q4_0", "f32", "f32", 3, 1024, 96),
    ("q4_1", "bf16", "f32", 8, 1024, 37),
    ("q5_0", "f32", "bf16", 9, 256, 40),
    ("q5_1", "f32", "f32", 16, 4096, 33),
    ("q8_0", "f32", "f32", 2, 14336, 20),   # a down projection's K: LDS beyond 64 KiB
    ("q4_k", "f32", "f32", 1, 4096, 96),
    ("q4_0", "f32", "f32", 1, 4096, 90),    # one token
    ("q4_0", "bf16", "bf16", 1, 14336, 33),
    ("q5_k", "bf16", "f32", 3, 2048, 37),
    ("q6_k", "f32", "bf16", 9, 4096, 40),
    ("q4_k", "f32", "f32", 2, 14336, 20),
    ("q6_k", "f32", "f32", 1, 14336, 24),
    ("q4_k", "bf16", "f32", 1, 256, 33),    # one token on the matrix cores: one super-block, a partial tile
    ("q4_k", "f32", "bf16", 1, 2048, 17),
    ("q4_k", "bf16", "bf16", 1, 14336, 40),
    ("q6_k", "bf16", "f32", 1, 2048, 33),    # one token on the matrix cores: one segment, a partial tile
    ("q6_k", "f32", "bf16", 1, 4096, 17),
    ("q6_k", "f32", "f32", 1, 3072, 40),     # rows of 2520 bytes: 8-byte staging loads
    ("q6_k", "f32", "f32", 2, 2560, 33),     # 2100 bytes: 4-byte loads
    ("q6_k", "bf16", "f32", 1, 768, 24),     # 630 bytes: 2-byte loads
    ("q6_k", "f32", "bf16", 5, 5120, 19),    # 4200 bytes
    ("bf16", "bf16", "f32", 2, 2048, 40),    # bf16 x at two tokens: the matrix cores
    ("q4_0", "bf16", "bf16", 16, 4096, 50),  # block formats from three tokens on the matrix cores
    ("q8_0", "bf16", "f32", 3, 1024, 33),
    ("q4_0", "f32", "f32", 2, 2048, 33),     # two tokens: the VALU kernel
    ("q8_0", "f32", "bf16", 17, 2048, 40),   # two token groups, the second of one token
    ("q4_0", "f32", "f32", 5, 1536, 24),     # K not a whole number of 1024-value stages: the VALU kernel
    ("q4_0", "bf16", "f32", 1, 8192, 17),    # one token, a partial block of rows
    ("q4_0", "f32", "bf16", 1, 4096, 1),     # a single row
    ("q4_k", "f32", "f32", 5, 1024, 33),     # Q4_K from five tokens on the matrix cores: one stage
    ("q4_k", "bf16", "bf16", 16, 4096, 50),
    ("q4_k", "f32", "bf16", 17, 2048, 40),   # two token groups, the second of one token
    ("q4_k", "f32", "f32", 4, 1280, 24),     # K not a whole number of 1024-value stages: the VALU kernel
    ("q6_k", "f32", "f32", 5, 1024, 33),     # Q6_K from five tokens on the matrix cores: one 840-byte stage
    ("q6_k", "bf16", "bf16", 16, 4096, 50),
    ("q6_k", "f32", "bf16", 17, 3072, 40),   # two token groups, the second of one token; three stages
    ("q5_0", "f32", "f32", 6, 2048, 33),     # the other block formats on the matrix cores (Q5: qh bits)
    ("q4_1", "bf16", "f32", 16, 1024, 40),
    ("q5_1", "f32", "bf16", 3, 3072, 24),
    ("q5_k", "f32", "f32", 16, 4096, 40),
    ("q5_k", "bf16", "bf16", 7, 1024, 17),
    ("q2_k", "f32", "f32", 1, 4096, 40),     # Q2_K and Q3_K: the VALU kernel below five tokens
    ("q2_k", "bf16", "f32", 4, 2048, 24),
    ("q3_k", "f32", "bf16", 2, 3072, 33),    # rows of 1320 bytes: 8-byte staging loads
    ("q3_k", "bf16", "bf16", 3, 2048, 33),
    ("q2_k", "f32", "bf16", 16, 1024, 17),
    ("q3_k", "f32", "f32", 17, 1024, 24),
    ("q2_k", "f32", "f32", 1, 1280, 33),     # rows of 420 bytes (not 16-byte multiples): 4-byte staging loads
    ("q2_k", "bf16", "bf16", 3, 512, 17),    # 168 bytes
    ("q2_k", "f32", "f32", 6, 1280, 19),     # five tokens or more, K not a multiple of 1024: the VALU kernel
]


@pytest.mark.parametrize("fmt,dx,dy,T,K,N", SINGLE_CASES)
def test_matvec(device, fmt, dx, dy, T, K, N):
    seed = _seed(fmt, dx, dy, T, K, N)
    raw, W = _weights(fmt, N, K, seed, 1)
    x, x32 = _x(dx, T, K, seed)
    y = _run(fmt, dx, dy, x, [raw], N, K)
    ref = oracle.matvec(fmt, raw, N, K, x32)
    S = np.abs(x32).astype(np.float64) @ _abs_terms(fmt, raw, W).T
    _check_single(y, dy, ref, S, f"matvec {fmt}")


@pytest.mark.parametrize("fmt,dx,T", [("bf16", "f32", 1), ("bf16", "f32", 5), ("q4_k", "f32", 1), ("q4_k", "f32", 4),
                                    ("q4_k", "bf16", 16), ("q6_k", "f32", 7), ("q4_0", "f32", 3), ("q8_0", "bf16", 12),
                                    ("q3_k", "f32", 9), ("q5_1", "f32", 2)])
def test_matvec_bias(device, fmt, dx, T):
    """slhip_matvec_bias: y = x . W^T + bias in the matvec's launch (FoldMatMulBiases: the f32 sum, then the Add
    of the f32 row vector), on every path (one token, the VALU kernels, the matrix cores)."""
    K, N = 2048, 56
    seed = _seed("bias", fmt, dx, T)
    raw, W = _weights(fmt, N, K, seed, 1)
    x, x32 = _x(dx, T, K, seed)
    b = synth.normal(seed, 5, (N,))
    with Dev() as d:
        px, pw, pb = d.put(x), d.put(raw), d.put(b)
        py = d.empty(T * N * 4)
        log(f"matvec_bias fmt={fmt} x={dx} T={T}")
        native.matvec_bias(fmt, dx, "f32", px, T, K, pw, N, pb, py)
        native.synchronize()
        y = d.get(py, (T, N), np.float32)
    ref = oracle.add(oracle.matvec(fmt, raw, N, K, x32), np.broadcast_to(b, (T, N)).copy())
    S = np.abs(x32).astype(np.float64) @ _abs_terms(fmt, raw, W).T
    _check_single(y, "f32", ref, S + 2.0 ** -8 * np.abs(ref.astype(np.float64)), f"matvec_bias {fmt}")


@pytest.mark.parametrize("fmt", ["f32", "f16", "bf16", "q8_0", "q4_0", "q4_1", "q5_0", "q5_1", "q6_k", "q2_k", "q3_k"])
def test_one_hot_rows_pick_columns_exactly(device, fmt):
    """x = e_k: every 8-value group but one sums to zero and the one holds q_k * 1 exactly, so y = d q_k + a
    exactly -- the dequantized weight -- whatever the summation order."""
    N, K = 29, 2048
    raw, W = _weights(fmt, N, K, 3, 1)
    ks = [0, 7, 511, 512, 2047]
    x = np.zeros((len(ks), K), np.float32)
    x[np.arange(len(ks)), ks] = 1.0
    y = _run(fmt, "f32", "f32", x, [raw], N, K)
    # + 0.0 makes -0 +0: a dot product that starts from +0 (the CPU MatMul's) turns a -0 weight (Q3_K's
    # (q - 4) d s with q = 4 and a negative scale) into +0
    assert_bits_equal(y + np.float32(0.0), np.ascontiguousarray(W[:, ks].T) + np.float32(0.0), what="one-hot columns")


@pytest.mark.parametrize("fmt", ["q2_k", "q3_k"])
def test_one_hot_columns_below_five_tokens(device, fmt):
    """The same exactness on the VALU kernel (two tokens): each half's terms d0 sum(x q) - m sum(x) (Q2_K) or
    d0 (sum(x q) - 4 sum(x)) (Q3_K) give the dequantized weight with one rounding."""
    N, K = 21, 2048
    raw, W = _weights(fmt, N, K, 4, 1)
    ks = [3, 1553]
    x = np.zeros((len(ks), K), np.float32)
    x[np.arange(len(ks)), ks] = 1.0
    y = _run(fmt, "f32", "f32", x, [raw], N, K)
    assert_bits_equal(y + np.float32(0.0), np.ascontiguousarray(W[:, ks].T) + np.float32(0.0), what="one-hot columns")


DUAL_CASES = [  # (act, fmt, x dtype, y dtype, T, K, N): FusionTests.SwiGluDualMatvec's K/N plus decode shapes
    ("silu", "bf16", "f32", "f32", 1, 1024, 96),
    ("silu", "f16", "f32", "f32", 3, 1024, 96),
    ("silu", "f32", "f32", "f32", 8, 1024, 96),
    ("silu", "bf16", "f32", "f32", 9, 256, 40),
    ("silu", "bf16", "f32", "bf16", 16, 1024, 96),
    ("silu", "f16", "bf16", "bf16", 20, 256, 40),
    ("silu", "bf16", "f32", "f32", 70, 1024, 96),
    ("gelu_tanh", "bf16", "f32", "f32", 1, 4096, 64),
    ("gelu_erf", "f16", "f32", "f32", 4, 4096, 64),
    ("silu", "bf16", "bf16", "bf16", 1, 4096, 14336),  # the Llama-3-8B decode FFN (C3's model)
    ("silu", "bf16", "bf16", "f32", 2, 4096, 72),      # bf16 x at two tokens: the matrix cores
    ("gelu_tanh", "bf16", "bf16", "bf16", 16, 1024, 40),  # bf16 x at 16 tokens: one tile per block
    ("silu", "bf16", "f32", "f32", 13, 1024, 72),      # f32 x above 12 tokens: two tiles per block
    ("silu", "q8_0", "f32", "f32", 1, 1024, 96),
    ("silu", "q8_0", "f32", "f32", 9, 1024, 96),
    ("silu", "q4_0", "f32", "f32", 1, 4096, 14336),
    ("silu", "q4_0", "f32", "f32", 16, 4096, 14336),  # batched decode on the matrix cores
    ("gelu_erf", "q8_0", "bf16", "bf16", 4, 2048, 72),
    ("gelu_tanh", "q4_1", "f32", "bf16", 3, 1024, 96),
    ("silu", "q5_0", "bf16", "f32", 20, 256, 40),
    ("gelu_erf", "q5_1", "f32", "f32", 4, 2048, 64),
    ("silu", "q4_k", "f32", "f32", 1, 4096, 14336),   # a Q4_K_M decode FFN (Mistral-7B / Llama-3-8B shapes)
    ("silu", "q6_k", "f32", "f32", 1, 4096, 14336),
    ("silu", "q5_k", "f32", "bf16", 5, 4096, 96),
    ("gelu_tanh", "q4_k", "bf16", "f32", 9, 2048, 40),
    ("silu", "q6_k", "f32", "f32", 12, 2048, 33),
    # one token, a gate/up pair per x read, each block format
    ("silu", "q4_1", "f32", "f32", 1, 2048, 64),
    ("gelu_erf", "q5_0", "bf16", "f32", 1, 1024, 96),
    ("silu", "q5_1", "f32", "bf16", 1, 4096, 40),
    ("silu", "q5_k", "f32", "f32", 1, 2048, 33),
    ("gelu_tanh", "q4_k", "bf16", "bf16", 1, 14336, 24),
    ("silu", "q6_k", "f32", "f32", 1, 3072, 40),          # Q6_K rows not 16-byte multiples
    ("gelu_erf", "q6_k", "bf16", "f32", 3, 768, 33),
    ("silu", "q4_k", "f32", "f32", 16, 4096, 14336),  # batched Q4_K_M decode FFN on the matrix cores
    ("gelu_erf", "q4_k", "bf16", "bf16", 6, 1024, 72),
    ("silu", "q4_k", "f32", "f32", 4, 1024, 40),       # four tokens: still the VALU kernel
    ("silu", "q6_k", "f32", "f32", 16, 4096, 14336),  # batched decode with Q6_K weights on the matrix cores
    ("gelu_tanh", "q6_k", "bf16", "f32", 8, 2048, 40),
    ("silu", "q5_k", "f32", "f32", 16, 4096, 14336),  # a Q5_K_M decode FFN at 16 tokens
    ("silu", "q5_0", "f32", "f32", 16, 1024, 64),
    ("gelu_erf", "q4_1", "bf16", "bf16", 5, 2048, 33),
    ("silu", "q3_k", "f32", "f32", 1, 4096, 1024),    # a Q3_K_M decode FFN's gate/up
    ("gelu_tanh", "q2_k", "bf16", "f32", 8, 2048, 40),
    ("silu", "q2_k", "f32", "f32", 1, 1280, 40),          # Q2_K rows of 420 bytes: 4-byte staging loads
    ("silu", "q2_k", "bf16", "bf16", 2, 768, 24),         # 252 bytes
]


@pytest.mark.parametrize("act,fmt,dx,dy,T,K,N", DUAL_CASES)
def test_dual_matvec(device, act, fmt, dx, dy, T, K, N):
    seed = _seed(act, fmt, dx, dy, T, K, N)
    rg, Wg = _weights(fmt, N, K, seed, 1)
    ru, Wu = _weights(fmt, N, K, seed, 2)
    x, x32 = _x(dx, T, K, seed)
    y = _run(fmt, dx, dy, x, [rg, ru], N, K, act=act)
    g = oracle.matvec(fmt, rg, N, K, x32)
    u = oracle.matvec(fmt, ru, N, K, x32)
    ref = oracle.mul(oracle.unary(act, g), u)
    ax = np.abs(x32).astype(np.float64)
    Sg = ax @ _abs_terms(fmt, rg, Wg).T
    Su = ax @ _abs_terms(fmt, ru, Wu).T
    g64 = g.astype(np.float64)
    h = 1e-4 * np.maximum(1.0, np.abs(g64))
    dact = (_act64(act, g64 + h) - _act64(act, g64 - h)) / (2 * h)
    # the slope of the implemented activation too: where the reference's erf rational is clamped (|g| > 5.4)
    # 1 + erf(g) is a constant, so GELU-erf is linear in g there, unlike the exact function
    h2 = 1e-3 * np.maximum(1.0, np.abs(g64))
    gp, gm = (g64 + h2).astype(np.float32), (g64 - h2).astype(np.float32)
    dimpl = (oracle.unary(act, gp).astype(np.float64) - oracle.unary(act, gm).astype(np.float64)) / (
        gp.astype(np.float64) - gm.astype(np.float64))
    dact = np.maximum(np.abs(dact), 1.5 * np.abs(dimpl))
    e = 2.0 ** -16
    tol = np.abs(dact * u) * e * Sg + np.abs(_act64(act, g64)) * e * Su + 1e-5 * np.abs(ref) + 1e-30
    if act == "gelu_erf":  # the erf rational evaluated in f32: within 4e-7 of the f64 evaluation
        tol = tol + 0.5 * np.abs(g64 * u) * 4.2e-7
    if dy == "bf16":
        got = oracle.from_bf16(y).astype(np.float64)
        r = oracle.from_bf16(oracle.to_bf16(ref)).astype(np.float64)
        tol = tol + 2 * 2.0 ** -8 * np.abs(r)
    else:
        got, r = y.astype(np.float64), ref.astype(np.float64)
    bad = np.abs(got - r) > tol
    if bad.any():
        i = tuple(np.argwhere(bad)[0])
        raise AssertionError(f"{bad.sum()} of {bad.size} beyond the bound; first at {i}: got {got[i]!r} ref {r[i]!r} "
                             f"tol {tol[i]!r} g {g[i]!r} u {u[i]!r} Sg {Sg[i]!r} Su {Su[i]!r}")


def test_strided_rows(device):
    """x and y with row strides beyond the row (views of wider buffers): only the row's own values count
    and only [T, N] of y is written."""
    fmt, T, K, N = "bf16", 5, 1024, 50
    raw, W = _weights(fmt, N, K, 4, 1)
    x, x32 = _x("f32", T, K, 4)
    y = _run(fmt, "f32", "f32", x, [raw], N, K, x_stride=K + 16, y_stride=N + 7)
    S = np.abs(x32).astype(np.float64) @ np.abs(W).astype(np.float64).T
    _check_single(y, "f32", oracle.matvec(fmt, raw, N, K, x32), S, "strided")


def test_empty_shapes_are_noops(device):
    native.matvec("bf16", "f32", "f32", None, 0, 64, None, 10, None)
    native.dual_matvec("silu", "bf16", "f32", "f32", None, 3, 64, None, None, 0, None)


@pytest.mark.parametrize("min_t", ["0", "1"])  # 0: the VALU kernel for every T; 1: the matrix cores for every T
@pytest.mark.parametrize("dual,dx,T,K,N", [
    (False, "f32", 1, 1024, 48), (False, "f32", 4, 2048, 40), (True, "f32", 5, 4096, 64),
    (True, "bf16", 17, 1024, 33), (False, "bf16", 33, 256, 17),
    (True, "f32", 9, 320, 40),  # K not a multiple of the 256-value stage: operands loaded directly
])
def test_bf16_paths_agree_with_oracle(device, monkeypatch, min_t, dual, dx, T, K, N):
    """bf16 weights take the MFMA kernels from SLHIP_MATVEC_MFMA_MIN_T tokens on; every kernel meets the same
    bound whichever T it is forced onto (ragged token and row tiles, one and two 16-row tiles per block, the
    LDS-staged kernel and, for K off its stage size, the directly loaded one)."""
    monkeypatch.setenv("SLHIP_MATVEC_MFMA_MIN_T", min_t)
    seed = _seed("paths", min_t, dual, dx, T, K, N)
    rg, Wg = _weights("bf16", N, K, seed, 1)
    x, x32 = _x(dx, T, K, seed)
    if not dual:
        y = _run("bf16", dx, "f32", x, [rg], N, K)
        S = np.abs(x32).astype(np.float64) @ _abs_terms("bf16", rg, Wg).T
        _check_single(y, "f32", oracle.matvec("bf16", rg, N, K, x32), S, f"bf16 min_t={min_t}")
        return
    ru, Wu = _weights("bf16", N, K, seed, 2)
    y = _run("bf16", dx, "f32", x, [rg, ru], N, K, act="silu")
    g = oracle.matvec("bf16", rg, N, K, x32)
    u = oracle.matvec("bf16", ru, N, K, x32)
    ref = oracle.mul(oracle.unary("silu", g), u).astype(np.float64)
    ax = np.abs(x32).astype(np.float64)
    Sg, Su = ax @ _abs_terms("bf16", rg, Wg).T, ax @ _abs_terms("bf16", ru, Wu).T
    g64 = g.astype(np.float64)
    s = 1 / (1 + np.exp(-g64))
    dsilu = np.abs(s * (1 + g64 * (1 - s))) * 1.5 + 1e-3
    e = 2.0 ** -16
    tol = dsilu * np.abs(u) * e * Sg + np.abs(g64 * s) * e * Su + 1e-5 * np.abs(ref) + 1e-30
    bad = np.abs(y.astype(np.float64) - ref) > tol
    assert not bad.any(), f"dual min_t={min_t}: {bad.sum()} beyond the bound; first at {np.argwhere(bad)[0]}"


def test_q6k_one_token_rows_of_code_32_give_exactly_zero(device):
    """At one token (the integer matrix-core kernel) a Q6_K row whose codes are all 32 -- zero weights, as in
    padded or pruned rows -- gives exactly 0: its sum is formed as sum q d - 32 sum d in integers. Other rows
    of the same tile stay within the f32 bound."""
    N, K = 40, 4096
    raw, _ = _weights("q6_k", N, K, 23, 1)
    b = raw.reshape(N, K // 256, 210)
    b[0:5, :, 0:128] = 0x00          # low nibbles 0
    b[0:5, :, 128:192] = 0xAA        # high 2-bit fields 2: every code 32
    W = oracle.dequant("q6_k", raw.reshape(-1), N * K).reshape(N, K)
    assert not np.any(W[0:5])
    x = synth.normal(3, 9, (1, K)) * 5 + 2
    y = _run("q6_k", "f32", "f32", x, [raw], N, K)
    assert np.all(y[0, 0:5] == 0.0), y[0, 0:5]
    S = np.abs(x).astype(np.float64) @ _abs_terms("q6_k", raw, W).T
    _check_single(y, "f32", oracle.matvec("q6_k", raw, N, K, x), S, "q6_k one token")


def test_q40_one_token_rows_of_code_8_and_wide_range(device):
    """Q4_0 at one token: rows whose codes are all 8 (zero weights), blocks with d = 0 or a large d among
    ordinary ones, and x spanning 2^-20 .. 2^12 with zeros and an outlier stay within the f32 bound, single and
    dual. (The kernel folds the offset as d (sum q x - 8 sum x) per block, so a zero row gives a residual of
    f32 rounding size, ~2^-24 8 d sum |x| per block, not an exact 0; the bound's |a| term covers it.)"""
    N, K = 40, 4096
    raw, _ = _weights("q4_0", N, K, 29, 1)
    b = raw.reshape(N, K // 32, 18)
    b[0:5, :, 2:] = 0x88             # every code 8
    b[6, ::3, 0:2] = 0               # d = +0 on every third block of row 6
    b[7, 5, 0:2] = np.frombuffer(np.float16(6.0e4).tobytes(), np.uint8)
    W = oracle.dequant("q4_0", raw.reshape(-1), N * K).reshape(N, K)
    assert not np.any(W[0:5])
    r = synth.rng(7, 7)
    x = (r.standard_normal((1, K)) * 2.0 ** r.integers(-20, 13, (1, K))).astype(np.float32)
    x[0, ::41] = 0.0
    x[0, 300] = -2.5e4
    y = _run("q4_0", "f32", "f32", x, [raw], N, K)
    S = np.abs(x).astype(np.float64) @ _abs_terms("q4_0", raw, W).T
    _check_single(y, "f32", oracle.matvec("q4_0", raw, N, K, x), S, "q4_0 one token")
    assert np.all(np.abs(y[0, 0:5]) <= 2.0 ** -16 * S[0, 0:5])
    g = oracle.matvec("q4_0", raw, N, K, x)
    y2 = _run("q4_0", "f32", "f32", x, [raw, raw], N, K, act="silu")
    sig = 0.5 * (1.0 + np.tanh(0.5 * g.astype(np.float64)))  # the logistic function, without overflow
    ref = g * sig * g
    assert np.all(np.abs(y2 - ref) <= 2.0 ** -14 * (S * (np.abs(g) + S) + 1e-30)), "dual q4_0 one token"


def test_q4k_one_token_wide_range_and_zero_rows(device):
    """The one-token Q4_K kernel (integer matrix cores, x as four 7-bit digits per value against its 32-value
    block's exponent): x spanning 2^-20 .. 2^12 inside each block, exact zeros and a huge outlier stay within
    the f32 bound; rows whose codes and minima are all zero give exactly 0, and so do rows whose codes are
    zero with a minimum, exactly -m * sum(x) per sub-block (checked against the oracle's value)."""
    N, K = 48, 2048
    raw, W = _weights("q4_k", N, K, 17, 1)
    blocks = raw.reshape(N, K // 256, 144)
    blocks[0:8, :, 16:] = 0          # codes 0
    blocks[0:4, :, 2:4] = 0          # and dmin 0: the row's weights are exactly 0
    W = oracle.dequant("q4_k", raw.reshape(-1), N * K).reshape(N, K)
    r = synth.rng(5, 5)
    x = (r.standard_normal((1, K)) * 2.0 ** r.integers(-20, 13, (1, K))).astype(np.float32)
    x[0, ::37] = 0.0
    x[0, 100] = 3.0e4
    for dual in (False, True):
        y = _run("q4_k", "f32", "f32", x, [raw, raw] if dual else [raw], N, K, act="silu" if dual else None)
        g = oracle.matvec("q4_k", raw, N, K, x)
        if dual:
            assert np.all(y[0, 0:4] == 0.0)  # silu(0) * 0
            continue
        assert np.all(y[0, 0:4] == 0.0), y[0, 0:4]
        S = np.abs(x).astype(np.float64) @ _abs_terms("q4_k", raw, W).T
        _check_single(y, "f32", g, S, "q4_k one token, wide x")


def test_q4k_several_tokens_wide_range_and_zero_rows(device):
    """The several-token Q4_K kernel (bf16 codes on the matrix cores, f32 x as two bf16 parts, the minimum
    applied as -m * sum(x) per sub-block on the VALU): x spanning 2^-20 .. 2^12 within a block, exact zeros and
    an outlier stay within the f32 bound per token; rows whose codes and minima are all zero give exactly 0."""
    N, K, T = 40, 2048, 5
    raw, W = _weights("q4_k", N, K, 23, 1)
    blocks = raw.reshape(N, K // 256, 144)
    blocks[0:8, :, 16:] = 0          # codes 0
    blocks[0:4, :, 2:4] = 0          # and dmin 0: the row's weights are exactly 0
    W = oracle.dequant("q4_k", raw.reshape(-1), N * K).reshape(N, K)
    r = synth.rng(6, 6)
    x = (r.standard_normal((T, K)) * 2.0 ** r.integers(-20, 13, (T, K))).astype(np.float32)
    x[:, ::37] = 0.0
    x[1, 100] = 3.0e4
    y = _run("q4_k", "f32", "f32", x, [raw], N, K)
    assert np.all(y[:, 0:4] == 0.0), y[:, 0:4]
    S = np.abs(x).astype(np.float64) @ _abs_terms("q4_k", raw, W).T
    _check_single(y, "f32", oracle.matvec("q4_k", raw, N, K, x), S, "q4_k several tokens, wide x")


@pytest.mark.parametrize("T", [1, 3, 6])
@pytest.mark.parametrize("dual", [False, True])
def test_q6k_codes_near_32_with_offset_x(device, dual, T):
    """Q6_K's -32 is applied to the sums of x over each 16-value half (sum x q - 32 sum x, the decomposition of
    the reference's integer dot, IntDot.Decode.cs:216-221): codes 32..34 and x of mean 4 make sum x q about 33
    times the result. Checked against the strict bound 2^-16 * sum |x| |w| (|w| itself, not the code and
    offset terms): an f32 emulation of the kernel's order stays below 2^-21 of it."""
    N, K = 48, 4096
    rng = np.random.default_rng(17)
    raws = []
    for tid in (1, 2):
        raw, _ = _weights("q6_k", N, K, 5, tid)
        b = raw.reshape(-1, 210).copy()
        nib = rng.integers(0, 3, (b.shape[0], 128, 2))
        b[:, 0:128] = (nib[..., 0] | (nib[..., 1] << 4)).astype(np.uint8)  # low nibbles 0..2
        b[:, 128:192] = 0xAA                                               # every 2-bit high field 2
        b[:, 208:210] = np.frombuffer(np.float16(0.0123).tobytes(), np.uint8)
        raws.append(b.reshape(raw.shape))
    x = (4.0 + 0.25 * rng.standard_normal((T, K))).astype(np.float32)
    W = [oracle.dequant("q6_k", r.reshape(-1), N * K).reshape(N, K).astype(np.float64) for r in raws]
    if not dual:
        y = _run("q6_k", "f32", "f32", x, raws[:1], N, K)
        ref = oracle.matvec("q6_k", raws[0], N, K, x)
        _check_single(y, "f32", ref, np.abs(x).astype(np.float64) @ np.abs(W[0]).T, "q6_k near 32")
        return
    y = _run("q6_k", "f32", "f32", x, raws, N, K, act="silu").astype(np.float64)
    g = x.astype(np.float64) @ W[0].T
    u = x.astype(np.float64) @ W[1].T
    Sg = np.abs(x).astype(np.float64) @ np.abs(W[0]).T
    Su = np.abs(x).astype(np.float64) @ np.abs(W[1]).T
    # |d(silu(g) u)| <= |silu'(g)| |dg| |u| + |silu(g)| |du| with |silu'| <= 1.1; plus one f32 rounding
    ref = _act64("silu", g) * u
    tol = 1.1 * 2.0 ** -16 * Sg * np.abs(u) + 2.0 ** -16 * Su * np.abs(_act64("silu", g)) + 2.0 ** -23 * np.abs(ref)
    assert (np.abs(y - ref) <= tol).all()


@pytest.mark.parametrize("dual", [False, True])
def test_q8_0_codes_near_0_with_offset_x(device, dual):
    """Codes -2..2 and x of mean 4, against the strict bound 2^-16 * sum |x| |w|: a guard for any rewrite that
    sums offset codes q + 128 and applies -128 d to the sum of x (the reference's integer-dot form,
    IntDot.Decode.cs:75-81), which would cancel about 128-fold here (f32 emulation: 2^-20 of the bound)."""
    N, K, T = 40, 4096, 3
    rng = np.random.default_rng(23)
    raws = []
    for tid in (1, 2):
        raw, _ = _weights("q8_0", N, K, 5, tid)
        b = raw.reshape(-1, 34).copy()
        b[:, 2:34] = rng.integers(-2, 3, (b.shape[0], 32)).astype(np.int8).view(np.uint8)
        b[:, 0:2] = np.frombuffer(np.float16(0.0123).tobytes(), np.uint8)
        raws.append(b.reshape(raw.shape))
    x = (4.0 + 0.25 * rng.standard_normal((T, K))).astype(np.float32)
    W = [oracle.dequant("q8_0", r.reshape(-1), N * K).reshape(N, K).astype(np.float64) for r in raws]
    if not dual:
        y = _run("q8_0", "f32", "f32", x, raws[:1], N, K)
        ref = oracle.matvec("q8_0", raws[0], N, K, x)
        _check_single(y, "f32", ref, np.abs(x).astype(np.float64) @ np.abs(W[0]).T, "q8_0 near 0")
        return
    y = _run("q8_0", "f32", "f32", x, raws, N, K, act="silu").astype(np.float64)
    g = x.astype(np.float64) @ W[0].T
    u = x.astype(np.float64) @ W[1].T
    Sg = np.abs(x).astype(np.float64) @ np.abs(W[0]).T
    Su = np.abs(x).astype(np.float64) @ np.abs(W[1]).T
    ref = _act64("silu", g) * u
    tol = 1.1 * 2.0 ** -16 * Sg * np.abs(u) + 2.0 ** -16 * Su * np.abs(_act64("silu", g)) + 2.0 ** -23 * np.abs(ref)
    assert (np.abs(y - ref) <= tol).all()
