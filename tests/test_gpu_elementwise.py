"""GPU parity of the standalone elementwise ops (slhip_binary with broadcasting, slhip_unary over every
UnaryKind) against the oracle's BinaryOp / ScalarMath.Unary restatement -- the reference's ElementwiseTests
pattern (GPU vs CPU provider), with the reference's broadcast shapes (a bias over rows, one value per row,
a scalar, outer-product shapes)."""
import os

import numpy as np
import pytest

import oracle
from sharplight_amd import native
from tests.devutil import Dev, log
from tests.parity import assert_bf16_close, assert_f32_close

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

NP = {"f32": np.float32, "bf16": np.uint16, "f16": np.float16}
RNG = np.random.default_rng(77)

EXACT_BIN = ["Add", "Sub", "Mul", "Div", "Max", "Min", "Mod", "FMod", "PRelu", "Equal", "NotEqual", "Less",
             "LessEqual", "Greater", "GreaterEqual", "And", "Or", "Xor"]
ALL_BIN = EXACT_BIN + ["Pow", "Atan2"]


def _to(x32, dt):
    if dt == "f32":
        return x32.astype(np.float32)
    if dt == "bf16":
        return oracle.to_bf16(x32)
    return x32.astype(np.float16)


def _f32(x, dt):
    if dt == "f32":
        return np.asarray(x, np.float32)
    if dt == "bf16":
        return oracle.from_bf16(x)
    return np.asarray(x, np.float16).astype(np.float32)


def _check(got, ref32, dt, exact, what):
    if dt == "f32":
        nan = np.isnan(ref32)
        assert np.array_equal(np.isnan(got), nan), f"{what}: NaN positions"
        if exact:
            assert np.array_equal(got[~nan].view(np.uint32), ref32[~nan].view(np.uint32)), what
        else:
            assert_f32_close(np.where(nan, 0, got), np.where(nan, 0, ref32), what=what)
    elif dt == "bf16":
        assert_bf16_close(got, oracle.to_bf16(ref32), ulp=0 if exact else 2, what=what)
    else:
        ref16 = ref32.astype(np.float16)
        if exact:
            assert np.array_equal(got.view(np.uint16), ref16.view(np.uint16)), what
        else:
            np.testing.assert_allclose(got.astype(np.float32), ref16.astype(np.float32), rtol=2e-3, atol=1e-6)


def _binary(op, da, db, do, a, b, *, a_strides=None, b_strides=None, pad=0, in_place=False):
    """a, b: arrays in their storage dtype (broadcastable); returns y [broadcast shape] from the GPU."""
    shape = np.broadcast_shapes(np.shape(a), np.shape(b)) if a_strides is None else a.shape
    r = len(shape)
    sa = list(oracle.align(np.shape(a), r)) if a_strides is None else a_strides
    sb = list(oracle.align(np.shape(b), r)) if b_strides is None else b_strides
    with Dev() as d:
        pa = d.put(np.asarray(a), pad)
        pb = d.put(np.asarray(b), pad)
        n = int(np.prod(shape)) if r else 1
        py = pa if in_place else d.empty(n * np.dtype(NP[do]).itemsize, pad)
        log(f"binary {op} {da},{db}->{do} a{np.shape(a)} b{np.shape(b)} y{shape} pad={pad} in_place={in_place}")
        native.binary(op, da, db, do, pa, pb, py, list(shape), a_strides=sa, b_strides=sb)
        native.synchronize()
        return d.get(py, shape, NP[do])


SHAPES = [((6, 64), (6, 64)), ((6, 64), (64,)), ((6, 64), (6, 1)), ((6, 64), ()), ((1, 64), (6, 1)),
          ((2, 3, 64), (3, 1)), ((2, 1, 40), (1, 4, 1)), ((24,), (2, 3, 24)), ((), ()), ((5, 13), (13,)),
          ((3, 7, 5), (7, 1))]


@pytest.mark.parametrize("sa,sb", SHAPES)
@pytest.mark.parametrize("op", ALL_BIN)
def test_binary_broadcast_f32(device, sa, sb, op):
    a = RNG.uniform(-4, 4, sa).astype(np.float32)
    b = RNG.uniform(-4, 4, sb).astype(np.float32)
    if op in ("Mod", "FMod", "Div"):
        b = np.where(np.abs(b) < 0.5, np.float32(1.5), b).astype(np.float32)
    if op == "Pow":
        a = np.abs(a) + np.float32(0.1)
    y = _binary(op, "f32", "f32", "f32", a, b)
    _check(y, oracle.binary(op, a, b), "f32", op in EXACT_BIN, f"{op} {sa} {sb}")


@pytest.mark.parametrize("da,db,do", [("bf16", "bf16", "bf16"), ("bf16", "f32", "bf16"), ("bf16", "bf16", "f32"),
                                      ("f16", "f16", "f16"), ("f16", "f32", "f32"), ("f32", "f32", "bf16")])
@pytest.mark.parametrize("op", ["Add", "Mul", "Sub", "Div", "Max", "Pow"])
def test_binary_dtypes(device, da, db, do, op):
    """A bf16 residual stream plus an f32 bias, a bf16 scalar Mul, f16 tensors: f32 arithmetic on the
    widened values, rounded once."""
    a32 = RNG.normal(size=(9, 512)).astype(np.float32)
    b32 = RNG.normal(size=(512,)).astype(np.float32) + np.float32(2.5)
    if op == "Pow":
        a32 = np.abs(a32) + np.float32(0.1)
        b32 = np.float32(0.5) * np.ones(1, np.float32)
    a, b = _to(a32, da), _to(b32, db)
    y = _binary(op, da, db, do, a, b)
    ref = oracle.binary(op, _f32(a, da), _f32(b, db))
    _check(y, ref, do, op != "Pow", f"{op} {da},{db}->{do}")


def test_bias_add_at_prefill_size(device):
    """A bias add over a [4096, 4096] bf16 activation with an f32 [4096] bias: every element bit-exact."""
    a32 = RNG.normal(size=(4096, 4096)).astype(np.float32)
    b = RNG.normal(size=(4096,)).astype(np.float32)
    a = oracle.to_bf16(a32)
    y = _binary("Add", "bf16", "f32", "bf16", a, b)
    assert_bf16_close(y, oracle.to_bf16(oracle.binary("Add", oracle.from_bf16(a), b)), ulp=0, what="bias add")


def test_binary_index_forms_agree(device):
    """The row index of a wave divided out in 32 bits (every size a launch can take today) and in 64 bits
    (the form for more than 2^32 waves, forced at start-up by SLHIP_EW_INDEX64 in a child process) give the
    same outputs over the broadcast shapes."""
    import json
    import subprocess
    import sys
    cases = [(sa, sb) for sa, sb in SHAPES if np.prod(sa, dtype=int) >= 8]
    script = (
        "import json, sys, numpy as np\n"
        "sys.path.insert(0, %r)\n"
        "from tests.test_gpu_elementwise import _binary, SHAPES\n"
        "from sharplight_amd import native\n"
        "native.set_device(0)\n"
        "rng = np.random.default_rng(5)\n"
        "out = []\n"
        "for sa, sb in %r:\n"
        "    a = rng.uniform(-4, 4, sa).astype(np.float32); b = rng.uniform(-4, 4, sb).astype(np.float32)\n"
        "    out.append(_binary('Add', 'f32', 'f32', 'f32', a, b).tobytes().hex())\n"
        "print(json.dumps(out))\n") % (ROOT, [(list(a), list(b)) for a, b in cases])
    res = []
    for force in ("0", "1"):
        env = dict(os.environ, SLHIP_EW_INDEX64=force)
        log(f"elementwise index form, SLHIP_EW_INDEX64={force} (child process)")
        r = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=100, env=env)
        assert r.returncode == 0, r.stderr[-2000:]
        res.append(json.loads(r.stdout.strip().splitlines()[-1]))
    assert res[0] == res[1]


def test_binary_strided_and_unaligned(device):
    """b a transposed view (explicit strides), then both operands 4 bytes off 16-byte alignment."""
    a = RNG.normal(size=(16, 24)).astype(np.float32)
    bt = RNG.normal(size=(24, 16)).astype(np.float32)  # b = bt.T as a [16, 24] view: strides (1, 16)
    y = _binary("Mul", "f32", "f32", "f32", a, bt, a_strides=[24, 1], b_strides=[1, 16])
    assert np.array_equal(y, a * bt.T)
    b = RNG.normal(size=(16, 24)).astype(np.float32)
    y = _binary("Sub", "f32", "f32", "f32", a, b, pad=4)
    assert np.array_equal(y, a - b)


def test_binary_in_place(device):
    a = RNG.normal(size=(33, 136)).astype(np.float32)
    b = RNG.normal(size=(136,)).astype(np.float32)
    y = _binary("Add", "f32", "f32", "f32", a, b, in_place=True)
    assert np.array_equal(y, a + b)


def test_binary_rejects_mixed_input_types(device):
    with pytest.raises(NotImplementedError):
        native.binary("Add", "bf16", "f16", "bf16", 16, 16, 16, [8])
    native.binary("Add", "f32", "f32", "f32", None, None, None, [0, 8])  # empty: nothing to do


UNARY_EXACT = {"Neg", "Sqrt", "Rsqrt", "Relu", "Abs", "Square", "Recip", "Scale", "HardSwish", "HardSigmoid", "Clip",
               "Floor", "Ceil", "Round", "Sign", "Softsign", "LeakyRelu", "ThresholdedRelu", "Not", "IsNaN", "IsInf",
               "Softplus"}
PARAMS = {"Scale": (1.25, -0.5), "HardSigmoid": (0.2, 0.5), "Clip": (-1.5, 2.0), "Elu": (1.0, 0.0),
          "Celu": (1.3, 0.0), "Selu": (1.6732632, 1.050701), "LeakyRelu": (0.01, 0.0), "ThresholdedRelu": (1.0, 0.0)}
DOMAIN = {"Log": (0.01, 8), "Sqrt": (0, 8), "Rsqrt": (0.01, 8), "Asin": (-0.99, 0.99), "Acos": (-0.99, 0.99),
          "Atanh": (-0.99, 0.99), "Acosh": (1.01, 8), "Exp": (-20, 20), "Sinh": (-10, 10), "Cosh": (-10, 10),
          "Tan": (-1.4, 1.4)}


@pytest.mark.parametrize("op", list(native.UNARY_OPS))
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_unary_kinds(device, op, dt):
    """Every UnaryKind at [37, 1000] (whole vector groups: the oracle takes the vector forms throughout)."""
    lo, hi = DOMAIN.get(op, (-6, 6))
    x32 = RNG.uniform(lo, hi, (37, 1000)).astype(np.float32)
    if op in ("Round", "Floor", "Ceil", "Sign", "Not"):
        x32[:, :64] = np.round(x32[:, :64] * 2) / 2  # halves and integers
    x = _to(x32, dt)
    p0, p1 = PARAMS.get(op, (1.0, 0.0))
    with Dev() as d:
        px, py = d.put(x), d.empty(x32.size * np.dtype(NP[dt]).itemsize)
        log(f"unary {op} {dt}")
        native.unary(op, dt, dt, px, py, 37, 1000, p0=p0, p1=p1)
        native.synchronize()
        y = d.get(py, (37, 1000), NP[dt])
    ref = oracle.unary_kind(op, _f32(x, dt), p0, p1)
    _check(y, ref, dt, op in UNARY_EXACT, f"{op} {dt}")


def test_erf_dense_grid_error_bound(device):
    """Erf and Gelu evaluate the reference's f64 rational (ScalarMath.cs:51-98) in f32: over 2^24 points of
    [-6, 6] (beyond the clamp at 3.8325 on both sides) erf stays within 4e-7 absolute and 8 ulp of the f64
    evaluation narrowed to f32, and Gelu within 0.5|x| times that; erf(NaN) is NaN."""
    n = 1 << 24
    x = np.linspace(-6, 6, n, dtype=np.float32).reshape(1024, n // 1024)
    x[0, :3] = [np.nan, np.inf, -np.inf]
    out = {}
    with Dev() as d:
        px, py = d.put(x), d.empty(x.nbytes)
        for op in ("Erf", "Gelu"):
            log(f"unary {op} dense grid")
            native.unary(op, "f32", "f32", px, py, x.shape[0], x.shape[1])
            native.synchronize()
            out[op] = d.get(py, x.shape, np.float32)
    ref = oracle.unary_kind("Erf", x)
    got = out["Erf"]
    assert np.isnan(got[0, 0])
    f = ~np.isnan(x)  # +-inf clamp like any |x| > 3.8325
    err = np.abs(got[f].astype(np.float64) - ref[f])
    ulp = np.abs(got[f].view(np.int32).astype(np.int64) - ref[f].view(np.int32))
    assert err.max() <= 4e-7 and ulp.max() <= 8, (err.max(), ulp.max())
    gref = oracle.unary_kind("Gelu", x)
    f = np.isfinite(x)
    gerr = np.abs(out["Gelu"][f].astype(np.float64) - gref[f])
    assert np.all(gerr <= 0.5 * np.abs(x[f]) * 4.2e-7 + 1e-7 * np.abs(gref[f])), gerr.max()


def test_unary_ragged_strided_and_special_values(device):
    """cols = 13 (the element kernel), padded row strides, and inf/NaN/-0 through Relu, Silu and Clip."""
    x = RNG.normal(size=(5, 16)).astype(np.float32) * 4
    x[0, :6] = [np.inf, -np.inf, np.nan, -0.0, 0.0, 88.0]
    for op in ("Relu", "Silu", "Clip", "Sigmoid"):
        p0, p1 = PARAMS.get(op, (1.0, 0.0))
        with Dev() as d:
            px, py = d.put(x), d.empty(5 * 20 * 4)
            log(f"unary ragged {op}")
            native.unary(op, "f32", "f32", px, py, 5, 13, x_stride=16, y_stride=20, p0=p0, p1=p1)
            native.synchronize()
            y = d.get(py, (5, 20), np.float32)[:, :13]
        ref = np.stack([oracle.unary_kind(op, x[r, :13], p0, p1) for r in range(5)])
        _check(y, ref, "f32", op in UNARY_EXACT, f"ragged {op}")
