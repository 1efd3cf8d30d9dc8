"""GPU parity of the GEMM activation copies a row norm writes (slhip_rownorm_copies): the f16 rows and the
E4M3 rows of the fp8 GEMM (D codes, then one f32 scale per 128 values), from the same f32 values as y
(RowNormKernelSource.cs:45-57,108-124; quantize_fp8, Kernels/gemm_fp8.slang:36-55), after the reference's
NormHalfCopyTests (tests/Sharplight.Vulkan.Tests/NormHalfCopyTests.cs: the norm's copies against the
values the unfused graph computes).

The copies are a function of the kernel's f32 norm values, which are only close to the oracle's. So each
case also runs with f32 y: the oracle's f16 conversion and quantize_fp8 applied to that y must give the
copies bit for bit, and the copies must not depend on y's dtype or on whether y is written at all. The
norm values themselves are held to the f32 tolerance against the oracle, and the E4M3 rows decode to
within E4M3's half step of them."""
import os
import subprocess
import zlib

import numpy as np
import pytest

import oracle
from sharplight_amd import native, synth
from tests.devutil import Dev, log
from tests.parity import assert_bits_equal, assert_f32_close

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

NP = {"f32": np.float32, "bf16": np.uint16}


def _seed(*parts) -> int:
    return zlib.crc32(repr(parts).encode())


def _e4m3_value(codes):
    """The value of E4M3 codes (OCP E4M3FN: bias 7, no infinities, 0x7F/0xFF NaN)."""
    c = codes.astype(np.int32)
    e, m = (c >> 3) & 0xF, c & 7
    v = np.where(e == 0, m * 2.0 ** -9, (8 + m) * 2.0 ** (e - 10))
    return np.where(c & 0x80, -v, v)


def _run(kind, din, dout, x, r, w, eps, *, y, y16, yq, x_pad=0, y16_stride=None, yq_stride=None):
    """One launch; returns (y, y16 rows, yq rows) with the padding of strided copies included."""
    rows, D = x.shape
    s16 = D if y16_stride is None else y16_stride
    sq = D + D // 32 if yq_stride is None else yq_stride
    with Dev() as d:
        px = d.put(x, x_pad)
        pr = d.put(r) if r is not None else None
        pw = d.put(w) if w is not None else None
        py = d.empty(rows * D * np.dtype(NP[dout]).itemsize) if y else None
        p16 = d.empty(rows * s16 * 2) if y16 else None
        pq = d.empty(rows * sq) if yq else None
        log(f"rownorm copies kind={kind} {din}->{dout} rows={rows} D={D} res={r is not None} y={y} y16={y16} "
            f"yq={yq} x_pad={x_pad} strides={s16},{sq}")
        native.rownorm(kind, din, dout, px, py, rows, D, res=pr, w=pw, eps=eps, y16=p16, y16_stride=s16, yq=pq,
                       yq_stride=sq)
        native.synchronize()
        out_y = d.get(py, (rows, D), NP[dout]) if y else None
        out_16 = d.get(p16, (rows, s16), np.uint16) if y16 else None
        out_q = d.get(pq, (rows, sq), np.uint8) if yq else None
    return out_y, out_16, out_q


def _oracle_norm(kind, din, x, r, w, eps):
    xf = oracle.from_bf16(x) if din == "bf16" else x
    if r is not None:
        xf = oracle.add(xf, oracle.from_bf16(r) if din == "bf16" else r)
    return oracle.rmsnorm(xf, w if kind == "rms" else None, eps, mode=0 if kind == "rms" else 1)


CASES = [  # (kind, din, D, rows, residual)
    ("rms", "bf16", 4096, 37, True),
    ("rms", "bf16", 128, 5, False),    # one group per row: most lanes of the wave repeat the last group
    ("rms", "f32", 128, 9, True),
    ("rms", "f32", 1024, 33, False),
    ("l2", "bf16", 640, 17, False),    # 5 groups: a partly filled wave
    ("rms", "bf16", 14336, 6, True),   # several vectors per lane
    ("rms", "f32", 6144, 4, True),
]


@pytest.mark.parametrize("kind,din,D,rows,res", CASES)
def test_copies_follow_the_f32_norm(device, kind, din, D, rows, res):
    seed = _seed(kind, din, D, rows, res)
    x = synth.normal(seed, 0, (rows, D), dtype=din)
    r = synth.normal(seed, 1, (rows, D), dtype=din) if res else None
    w = synth.normal(seed, 2, (D,), 1.0, 0.1) if kind == "rms" else None
    y32, y16, yq = _run(kind, din, "f32", x, r, w, 1e-6, y=True, y16=True, yq=True)
    # the f32 values against the oracle, then the copies against the oracle's conversions of those values
    yref = _oracle_norm(kind, din, x, r, w, 1e-6)
    assert_f32_close(y32, yref, what="norm values")
    assert_bits_equal(y16, oracle.to_f16(y32), what="f16 copy")
    assert_bits_equal(yq, oracle.quantize_fp8(y32), what="E4M3 rows")
    # the E4M3 rows decode to the norm values within half a step of the format (2^-4 relative; 2^-10 of the
    # scale below E4M3's smallest normal)
    codes, scales = yq[:, :D], yq[:, D:].copy().view(np.float32)
    dec = _e4m3_value(codes).reshape(rows, D // 128, 128) * scales.reshape(rows, D // 128, 1)
    g = yref.reshape(rows, D // 128, 128).astype(np.float64)
    tol = np.maximum(np.abs(g) * 2.0 ** -4, scales.reshape(rows, -1, 1) * 2.0 ** -10) * (1 + 1e-4)
    assert (np.abs(dec - g) <= tol).all()
    # the copies do not depend on y's dtype or on whether y is written
    y_bf, y16b, yqb = _run(kind, din, "bf16", x, r, w, 1e-6, y=True, y16=True, yq=True)
    assert_bits_equal(y_bf, oracle.to_bf16(y32), what="bf16 y of the same values")
    assert_bits_equal(y16b, y16, what="f16 copy beside bf16 y")
    assert_bits_equal(yqb, yq, what="E4M3 rows beside bf16 y")
    _, y16n, yqn = _run(kind, din, "bf16", x, r, w, 1e-6, y=False, y16=True, yq=True)
    assert_bits_equal(y16n, y16, what="f16 copy without y")
    assert_bits_equal(yqn, yq, what="E4M3 rows without y")


@pytest.mark.parametrize("din", ["bf16", "f32"])
def test_scalar_path_copies(device, din):
    """A misaligned x takes the block-per-row kernel; its copies obey the same rule."""
    rows, D = 7, 384
    seed = _seed("scalar", din)
    x = synth.normal(seed, 0, (rows, D), dtype=din)
    w = synth.normal(seed, 2, (D,), 1.0, 0.1)
    y32, y16, yq = _run("rms", din, "f32", x, None, w, 1e-6, y=True, y16=True, yq=True, x_pad=4)
    assert_f32_close(y32, _oracle_norm("rms", din, x, None, w, 1e-6), what="norm values")
    assert_bits_equal(y16, oracle.to_f16(y32), what="f16 copy")
    assert_bits_equal(yq, oracle.quantize_fp8(y32), what="E4M3 rows")


@pytest.mark.parametrize("din,D,res", [("bf16", 1004, True), ("bf16", 4100, False)])
def test_f16_copy_of_rows_with_8_byte_vectors(device, din, D, res):
    """2-byte rows of a length that is a multiple of 4 but not of 8 (8-byte vectors): the f16 copy follows
    the kernel's f32 values as on the 16-byte path (no E4M3 rows: they need D % 128 == 0)."""
    rows = 13
    seed = _seed("vec8", din, D, res)
    x = synth.normal(seed, 0, (rows, D), dtype=din)
    r = synth.normal(seed, 1, (rows, D), dtype=din) if res else None
    w = synth.normal(seed, 2, (D,), 1.0, 0.1)
    y32, y16, _ = _run("rms", din, "f32", x, r, w, 1e-6, y=True, y16=True, yq=False)
    assert_f32_close(y32, _oracle_norm("rms", din, x, r, w, 1e-6), what="norm values")
    assert_bits_equal(y16, oracle.to_f16(y32), what="f16 copy")
    y_bf, y16b, _ = _run("rms", din, "bf16", x, r, w, 1e-6, y=True, y16=True, yq=False)
    assert_bits_equal(y_bf, oracle.to_bf16(y32), what="bf16 y of the same values")
    assert_bits_equal(y16b, y16, what="f16 copy beside bf16 y")


def test_strided_copies_leave_the_padding(device):
    """Row strides beyond the row: the copies land at their rows and the bytes between stay untouched."""
    rows, D = 11, 512
    x = synth.normal(7, 0, (rows, D), dtype="bf16")
    w = synth.normal(7, 2, (D,), 1.0, 0.1)
    s16, sq = D + 64, D + D // 32 + 48
    y32, y16, yq = _run("rms", "bf16", "f32", x, None, w, 1e-6, y=True, y16=True, yq=True, y16_stride=s16,
                        yq_stride=sq)
    assert_bits_equal(y16[:, :D], oracle.to_f16(y32), what="f16 copy")
    assert_bits_equal(yq[:, :D + D // 32], oracle.quantize_fp8(y32), what="E4M3 rows")
    assert (y16[:, D:] == 0xABAB).all() and (yq[:, D + D // 32:] == 0xAB).all()


def test_zero_group_has_zero_scale_and_codes(device):
    """A 128-value group of zeros: d = 0, so 1/d is taken as 0 and every code is 0 (e4m3_pack4)."""
    rows, D = 3, 256
    x = synth.normal(3, 0, (rows, D), dtype="f32")
    w = np.ones(D, np.float32)
    w[:128] = 0.0  # the first group of every row is all zeros after the weight
    y32, _, yq = _run("rms", "f32", "f32", x, None, w, 1e-6, y=True, y16=False, yq=True)
    assert (yq[:, :128] == 0).all()
    assert (yq[:, D:D + 4].copy().view(np.float32) == 0).all()
    assert_bits_equal(yq, oracle.quantize_fp8(y32), what="E4M3 rows")


def _code_grid():
    """Every positive E4M3 value, every midpoint between neighbours (the ties), each midpoint one f32 ulp
    either side, and the edges of the subnormal range: all within [0, 448], so that 448 stays each group's
    amax."""
    vals = _e4m3_value(np.arange(0x7F)).astype(np.float32)  # codes 0..0x7E
    mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2).astype(np.float32)
    grid = np.concatenate([vals, mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1000)),
                           np.float32([2.0 ** -10, 2.0 ** -11, 2.0 ** -20, 1e-30, 0.015625 * (1 - 2 ** -24),
                                       0.015625, 447.99997, 440.0, 447.0])])
    return grid[(grid >= 0) & (grid <= 448)]


@pytest.mark.parametrize("din", ["f32", "bf16"])
def test_e4m3_code_grid_through_the_norm(device, din):
    """RmsNorm with eps 0 of rows of +-1 has scale exactly 1, so y = +-w exactly; with 448 in every group
    the E4M3 scale is 1 and the codes are e4m3_code(+-w) themselves: each code value, each tie (to even),
    each tie +-1 ulp, on both signs, and -0 (code 0x00, v < 0 being false)."""
    grid = _code_grid()
    per = 127
    n_groups = -(-grid.size // per)
    w = np.zeros((n_groups, 128), np.float32)
    w[:, 0] = 448.0
    w.reshape(-1)[np.arange(grid.size) // per * 128 + 1 + np.arange(grid.size) % per] = grid
    w = w.reshape(-1)
    D = w.size
    rows = np.ones((2, D), np.float32)
    rows[1] = -1.0
    wz = w.copy()
    wz[2] = -0.0  # row 0: +1 * -0 = -0
    x = oracle.to_bf16(rows) if din == "bf16" else rows
    y32, _, yq = _run("rms", din, "f32", x, None, wz, 0.0, y=True, y16=False, yq=True)
    assert np.array_equal(y32, rows * wz)
    assert (yq[:, D:].copy().view(np.float32) == 1.0).all()
    want = np.array([[oracle.e4m3_code(float(v)) for v in r] for r in (rows * wz)], np.uint8)
    assert_bits_equal(yq[:, :D], want, what="E4M3 codes of the grid")
    assert yq[0, 2] == 0x00 and yq[1, 2] == 0x00  # -0 (row 0) and +0 (row 1: -1 * -0)
    assert_bits_equal(yq, oracle.quantize_fp8(y32), what="E4M3 rows")


def test_e4m3_conversion_exhaustive(device):
    """The kernels' E4M3 conversion against the reference's integer rule on all 2^32 f32 inputs, and their
    group scale (d = amax/448, 1/d) against IEEE division for every non-negative amax (a check program
    built beside the library: tests/e4m3_exhaustive.hip)."""
    exe = os.path.join(ROOT, "tests", "_bin", "e4m3_exhaustive")
    assert os.path.exists(exe), "tests/_bin/e4m3_exhaustive is not built: run the package build"
    log("e4m3 exhaustive check program")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=100)
    out = r.stdout.split()
    assert r.returncode == 0, r.stdout + r.stderr
    assert out[0] == "checked" and int(out[1]) == 1 << 32 and int(out[3]) == 0, r.stdout
    assert int(out[7]) > 0, "the bare conversion must differ somewhere (-0, NaN, inf): the checker compared nothing"
    assert out[8] == "scale_checked" and int(out[9]) == 0x7F800001 and int(out[11]) == 0, r.stdout
