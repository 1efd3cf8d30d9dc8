"""Pins of the oracle's standalone elementwise ops (BinaryOp with broadcasting, every UnaryKind) against
mathematics that does not go through the oracle: numpy's own broadcasting and IEEE f32 arithmetic for the
exact ops, f64 closed forms (math / numpy) for the transcendental ones, and the reference's rules that
differ from numpy (MathF.Max/Min on -0 and NaN, Python-style Mod, Pow's row-constant exponent forms,
vector-vs-tail forms of Scale/HardSwish/HardSigmoid)."""
import math

import numpy as np
import pytest

import oracle

RNG = np.random.default_rng(1234)

SHAPES = [  # a, b: every broadcast pattern of BinaryOp.Align
    ((6, 16), (6, 16)),
    ((6, 16), (16,)),          # bias over rows
    ((6, 16), (6, 1)),         # one value per row
    ((6, 16), ()),             # scalar
    ((1, 16), (6, 1)),         # both broadcast: outer product shape
    ((2, 3, 16), (3, 1)),      # middle dim
    ((2, 1, 5), (1, 4, 1)),
    ((7,), (2, 3, 7)),         # a broadcast over leading dims
    ((), ()),                  # rank 0
]


def _rand(shape, lo=-4, hi=4):
    return RNG.uniform(lo, hi, size=shape).astype(np.float32)


@pytest.mark.parametrize("sa,sb", SHAPES)
@pytest.mark.parametrize("kind,ref", [
    ("Add", np.add), ("Sub", np.subtract), ("Mul", np.multiply), ("Div", np.divide),
    ("Max", np.maximum), ("Min", np.minimum), ("Equal", np.equal), ("Less", np.less),
    ("GreaterEqual", np.greater_equal), ("PRelu", lambda a, b: np.where(a < 0, a * b, a)),
    ("FMod", np.fmod), ("Mod", np.mod),
])
def test_binary_broadcast_matches_numpy(sa, sb, kind, ref):
    a, b = _rand(sa), _rand(sb)
    if kind in ("Mod", "FMod", "Div"):
        b = np.where(np.abs(b) < 0.5, np.float32(1.5), b).astype(np.float32)
    with np.errstate(all="ignore"):
        want = np.asarray(ref(a, b)).astype(np.float32)
    got = oracle.binary(kind, a, b)
    assert got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), kind


def test_align_gives_zero_strides_to_broadcast_dims():
    assert list(oracle.align((4, 1), 3)) == [0, 1, 0]
    assert list(oracle.align((2, 3, 4), 3)) == [12, 4, 1]
    assert list(oracle.align((1, 4), 2)) == [0, 1]


def test_max_min_follow_ieee_2019():
    """MathF.Max/Min: NaN wins, +0 is above -0 (numpy's maximum keeps the first of equal operands)."""
    a = np.array([-0.0, 0.0, np.nan, 1.0, -np.inf], np.float32)
    b = np.array([0.0, -0.0, 1.0, np.nan, np.inf], np.float32)
    mx, mn = oracle.binary("Max", a, b), oracle.binary("Min", a, b)
    assert [math.copysign(1, v) for v in mx[:2]] == [1, 1]
    assert [math.copysign(1, v) for v in mn[:2]] == [-1, -1]
    assert np.isnan(mx[2]) and np.isnan(mx[3]) and np.isnan(mn[2]) and np.isnan(mn[3])
    assert mx[4] == np.inf and mn[4] == -np.inf


def test_mod_sign_of_divisor_and_fmod_sign_of_dividend():
    a = np.array([7, -7, 7, -7, 6], np.float32)
    b = np.array([3, 3, -3, -3, 3], np.float32)
    assert list(oracle.binary("Mod", a, b)) == [1, 2, -2, -1, 0]
    assert list(oracle.binary("FMod", a, b)) == [1, -1, 1, -1, 0]


def test_pow_row_constant_exponent_forms():
    """Apply's special exponents (BinaryOp.cs:153-196): -0 ** 0.5 is sqrt(-0) = -0 (powf gives +0), and a
    per-element exponent goes through powf."""
    a = np.array([[-0.0, 4.0, 2.0, -8.0]], np.float32)
    y = oracle.binary("Pow", a, np.float32(0.5))
    assert math.copysign(1, y[0, 0]) == -1 and y[0, 1] == 2.0
    y2 = oracle.binary("Pow", a, np.full((1, 4), 0.5, np.float32))
    assert math.copysign(1, y2[0, 0]) == 1
    x = _rand((3, 9), 0.1, 3)
    assert np.array_equal(oracle.binary("Pow", x, np.float32(2)), x * x)
    assert np.array_equal(oracle.binary("Pow", x, np.float32(3)), x * x * x)
    e = np.float32(1.7)
    np.testing.assert_allclose(oracle.binary("Pow", x, e), np.power(x.astype(np.float64), 1.7), rtol=2e-7)


EXACT = {  # kinds whose result is one correctly rounded f32 operation (or none) of x
    "Neg": lambda x: -x, "Sqrt": np.sqrt, "Abs": np.abs, "Square": lambda x: x * x, "Recip": lambda x: 1 / x,
    "Relu": lambda x: np.where(x > 0, x, np.float32(0)), "Floor": np.floor, "Ceil": np.ceil, "Round": np.rint,
    "Sign": np.sign, "Not": lambda x: (x == 0).astype(np.float32), "IsNaN": lambda x: np.isnan(x).astype(np.float32),
    "IsInf": lambda x: np.isinf(x).astype(np.float32),
}


@pytest.mark.parametrize("kind", sorted(EXACT))
def test_unary_exact_kinds(kind):
    x = np.concatenate([_rand(997, -6, 6), np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 2.5, -2.5, 0.5], np.float32)])
    with np.errstate(all="ignore"):
        want = EXACT[kind](x).astype(np.float32)
    got = oracle.unary_kind(kind, x)
    assert np.array_equal(got, want, equal_nan=True), kind


F64 = {
    "Exp": np.exp, "Log": np.log, "Rsqrt": lambda x: 1 / np.sqrt(x), "Sigmoid": lambda x: 1 / (1 + np.exp(-x)),
    "Silu": lambda x: x / (1 + np.exp(-x)), "Tanh": np.tanh, "Softplus": lambda x: np.log1p(np.exp(x)),
    "Gelu": lambda x: 0.5 * x * (1 + np.vectorize(math.erf)(x / math.sqrt(2))),
    "GeluTanh": lambda x: 0.5 * x * (1 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3))),
    "Erf": np.vectorize(math.erf), "Sin": np.sin, "Cos": np.cos, "Atan": np.arctan, "Sinh": np.sinh,
    "Asinh": np.arcsinh, "Softsign": lambda x: x / (1 + np.abs(x)),
    "Mish": lambda x: x * np.tanh(np.log1p(np.exp(x))), "Elu": lambda x: np.where(x >= 0, x, np.expm1(x)),
    "HardSwish": lambda x: x * np.clip(x / 6 + 0.5, 0, 1), "HardSigmoid": lambda x: np.clip(0.2 * x + 0.5, 0, 1),
}


@pytest.mark.parametrize("kind", sorted(F64))
def test_unary_closed_forms(kind):
    lo = 0.05 if kind in ("Log", "Rsqrt") else -6
    x = _rand(1003, lo, 6)  # 1003: vector groups and a tail
    p0, p1 = (0.2, 0.5) if kind == "HardSigmoid" else (1.0, 0.0)
    want = F64[kind](x.astype(np.float64))
    got = oracle.unary_kind(kind, x, p0, p1).astype(np.float64)
    err = np.abs(got - want)
    tol = 4e-7 * np.abs(want) + 1e-30
    if kind in ("Gelu", "Erf", "Mish", "GeluTanh", "Softplus", "Elu", "HardSwish", "HardSigmoid"):
        # absolute terms: the rational erf's ~1e-7 approximation error (times x/2 in Gelu), and the
        # cancellation in 1 + erf, 1 + tanh, x/6 + 0.5 near the zeros of these forms
        tol = tol + 1.5e-7 * np.maximum(np.abs(x), 1)
    assert (err <= tol).all(), (kind, float(err.max()))


def test_scale_vector_and_tail_forms():
    """Scale (ScalarMath.cs:460-484): fma on whole groups of 8, v*s + b on the tail."""
    x = _rand(11)
    s, b = np.float32(1.1), np.float32(0.3)
    y = oracle.unary_kind("Scale", x, float(s), float(b))
    fused = (x.astype(np.float64) * float(s) + float(b)).astype(np.float32)
    split = (x * s + b).astype(np.float32)
    assert np.array_equal(y[:8], fused[:8]) and np.array_equal(y[8:], split[8:])


def test_clip_and_leaky_relu_parameters():
    x = np.array([-3, -1, 0, 1, 3, np.nan], np.float32)
    assert np.array_equal(oracle.unary_kind("Clip", x, -1.5, 2.0), np.array([-1.5, -1, 0, 1, 2, np.nan], np.float32),
                          equal_nan=True)
    assert np.array_equal(oracle.unary_kind("LeakyRelu", x[:5], 0.1), np.where(x[:5] >= 0, x[:5], np.float32(0.1) * x[:5]))
    assert np.array_equal(oracle.unary_kind("ThresholdedRelu", x[:5], 1.0), np.array([0, 0, 0, 0, 3], np.float32))
