"""GPU parity of slhip_rownorm (RMSNorm / L2Norm / LayerNorm, optional fused residual add) against the CPU
oracle's unfused decomposition (Add, then RowOp), mirroring the reference's NormTests.cs, RowOpTests.cs
and FusionTests.cs:18-26 (GPU vs CPU provider)."""
import numpy as np
import pytest

import oracle
from sharplight_amd import native, synth
from tests.devutil import Dev, log
from tests.parity import FLOOR_ONLY, assert_bf16_close, assert_f32_close

pytestmark = pytest.mark.gpu

NP = {"f32": np.float32, "bf16": np.uint16}


def _inputs(rows, D, din, seed, scale=1.0):
    x = synth.normal(seed, 0, (rows, D), std=scale, dtype=din)
    r = synth.normal(seed, 1, (rows, D), std=scale, dtype=din)
    w = synth.normal(seed, 2, (D,), 1.0, 0.1)
    b = synth.normal(seed, 3, (D,), 0.0, 0.5)
    return x, r, w, b


def _run(kind, din, dout, x, r, w, b, eps, *, with_res, with_h, pad=0, x_stride=None):
    rows, D = x.shape
    with Dev() as d:
        xs = D if x_stride is None else x_stride
        if xs != D:
            xp = np.zeros((rows, xs), x.dtype)
            xp[:, :D] = x
        else:
            xp = x
        px = d.put(xp, pad)
        pr = d.put(r, pad) if with_res else None
        pw = d.put(w) if w is not None else None
        pb = d.put(b) if b is not None else None
        osz = np.dtype(NP[dout]).itemsize
        py = d.empty(rows * D * osz, pad)
        ph = d.empty(rows * D * np.dtype(NP[din]).itemsize, pad) if with_h else None
        log(f"rownorm kind={kind} {din}->{dout} rows={rows} D={D} res={with_res} h={with_h} pad={pad} xs={xs}")
        native.rownorm(kind, din, dout, px, py, rows, D, res=pr, w=pw, b=pb, h_out=ph, eps=eps, x_stride=xs)
        native.synchronize()
        y = d.get(py, (rows, D), NP[dout])
        h = d.get(ph, (rows, D), NP[din]) if with_h else None
    return y, h


def _reference(kind, din, dout, x, r, w, b, eps, with_res):
    xf = oracle.from_bf16(x) if din == "bf16" else x
    if with_res:
        rf = oracle.from_bf16(r) if din == "bf16" else r
        hf = oracle.add(xf, rf)
    else:
        hf = xf
    if kind == "layer":
        yf = oracle.layernorm(hf, w, b, eps)
    else:
        yf = oracle.rmsnorm(hf, w if kind == "rms" else None, eps, mode=0 if kind == "rms" else 1)
    y = oracle.to_bf16(yf) if dout == "bf16" else yf
    h = oracle.to_bf16(hf) if din == "bf16" else hf
    return y, h, yf


def _check(dout, y, yref, what):
    if dout == "bf16":
        assert_bf16_close(y, yref, what=what)
    else:
        assert_f32_close(y, yref, what=what)


def test_c1_rmsnorm_f32(device):
    """RMSNorm f32 [512, 1024], gamma ~ N(1, 0.1), eps 1e-6, seed 0."""
    c = synth.c1()
    y, _ = _run("rms", "f32", "f32", c["x"], None, c["w"], None, c["eps"], with_res=False, with_h=False)
    yref, _, _ = _reference("rms", "f32", "f32", c["x"], None, c["w"], None, c["eps"], False)
    rel = assert_f32_close(y, yref, what="C1")
    assert rel < 1e-5


# elements of the full-shape configs that may pass only through the bf16 rule's absolute floor (measured on
# MI355X; the norm's outputs are products, nothing cancels)
C2_FLOOR_ONLY = 0


def test_c2_add_rmsnorm_bf16(device):
    """residual add + RMSNorm bf16 [8192, 4096], gamma f32, eps 1e-5; y and h both bf16."""
    c = synth.c2()
    y, h = _run("rms", "bf16", "bf16", c["x"], c["res"], c["w"], None, c["eps"], with_res=True, with_h=True)
    yref, href, _ = _reference("rms", "bf16", "bf16", c["x"], c["res"], c["w"], None, c["eps"], True)
    assert_bf16_close(h, href, ulp=0, what="C2 h (x+res rounded once: exact)")
    assert_bf16_close(y, yref, what="C2 y", max_floor_only=C2_FLOOR_ONLY)
    log(f"C2 y: {FLOOR_ONLY['C2 y'][0]} of {FLOOR_ONLY['C2 y'][1]} pass only through the absolute floor")


CASES = [
    # kind, din, dout, rows, D
    ("rms", "f32", "f32", 3, 1),
    ("rms", "f32", "f32", 5, 70),
    ("rms", "f32", "f32", 33, 1024),
    ("rms", "f32", "f32", 2, 2048),
    ("rms", "bf16", "bf16", 7, 4096),
    ("rms", "bf16", "f32", 9, 896),
    ("rms", "f32", "bf16", 9, 5120),
    ("rms", "bf16", "bf16", 1, 40960),
    ("rms", "f32", "f32", 2, 70000),   # beyond the vector path: scalar kernel
    ("l2", "f32", "f32", 6, 256),
    ("l2", "bf16", "bf16", 6, 4100),   # D % 8 == 4: 8-byte vectors
    ("rms", "bf16", "bf16", 5, 4100),
    ("rms", "bf16", "f32", 9, 1004),
    ("layer", "bf16", "bf16", 3, 1004),
    ("layer", "bf16", "f32", 2, 12),
    ("rms", "bf16", "bf16", 2, 32764),  # 8191 vectors of 8 bytes: one 16-wave group, 8 vectors per lane
    ("rms", "bf16", "bf16", 4, 4102),   # D % 4 == 2: scalar kernel
    ("layer", "bf16", "bf16", 3, 1001),
    ("layer", "f32", "f32", 5, 70),
    ("layer", "f32", "f32", 197, 768),
    ("layer", "f32", "f32", 4, 5000),
    ("layer", "bf16", "bf16", 16, 4096),
]


@pytest.mark.parametrize("kind,din,dout,rows,D", CASES)
@pytest.mark.parametrize("with_res", [False, True])
def test_rownorm_matrix(device, kind, din, dout, rows, D, with_res):
    x, r, w, b = _inputs(rows, D, din, seed=rows * 1000 + D, scale=3.0)
    w = None if kind == "l2" else w
    b = b if kind == "layer" else None
    eps = 1e-5
    y, h = _run(kind, din, dout, x, r, w, b, eps, with_res=with_res, with_h=with_res)
    yref, href, _ = _reference(kind, din, dout, x, r, w, b, eps, with_res)
    _check(dout, y, yref, f"{kind} {din}->{dout} [{rows},{D}] res={with_res}")
    if with_res:
        if din == "bf16":
            assert_bf16_close(h, href, ulp=0, what="h")
        else:
            assert np.array_equal(h.view(np.uint32), href.view(np.uint32))


def test_rownorm_without_weight_and_unaligned(device):
    """RmsNorm without weight (RowOp's Simd.Scale branch) on tensors misaligned by 4 bytes (scalar path),
    and with a padded x row stride (strided view of a wider tensor)."""
    x, r, w, _ = _inputs(11, 512, "f32", seed=5)
    y, _ = _run("rms", "f32", "f32", x, r, None, None, 1e-6, with_res=False, with_h=False, pad=4)
    yref, _, _ = _reference("rms", "f32", "f32", x, r, None, None, 1e-6, False)
    assert_f32_close(y, yref, what="unaligned")
    y, _ = _run("rms", "f32", "f32", x, r, w, None, 1e-6, with_res=False, with_h=False, x_stride=520)
    yref, _, _ = _reference("rms", "f32", "f32", x, r, w, None, 1e-6, False)
    assert_f32_close(y, yref, what="strided")


def test_rownorm_in_place_residual(device):
    """y written over x and h over res (the residual stream updated in place), bf16."""
    rows, D = 64, 4096
    x, r, w, _ = _inputs(rows, D, "bf16", seed=9)
    with Dev() as d:
        px = d.put(x)
        pr = d.put(r)
        pw = d.put(w)
        log("rownorm in-place residual")
        native.rownorm("rms", "bf16", "bf16", px, px, rows, D, res=pr, w=pw, h_out=pr, eps=1e-6)
        native.synchronize()
        y = d.get(px, (rows, D), np.uint16)
        h = d.get(pr, (rows, D), np.uint16)
    yref, href, _ = _reference("rms", "bf16", "bf16", x, r, w, None, 1e-6, True)
    assert_bf16_close(y, yref, what="in-place y")
    assert_bf16_close(h, href, ulp=0, what="in-place h")


IN_PLACE = [
    # kind, dtype, rows, D, residual, forced row-group width (0: the dispatcher's choice)
    ("rms", "f32", 4097, 1024, False, 0),   # one wave per row, 4 rows per block: 3 surplus groups
    ("rms", "bf16", 4099, 512, True, 0),    # one wave per row with a residual; 3 surplus groups
    ("rms", "bf16", 37, 896, True, 0),      # 112 vectors: surplus lanes of the same wave
    ("rms", "bf16", 37, 896, True, 2),      # surplus lanes in the second wave of a two-wave group
    ("rms", "bf16", 4099, 896, True, 2),    # two-wave groups, two groups per block, one surplus group
    ("rms", "f32", 5, 1000, True, 4),       # 250 vectors over 256 lanes: surplus lanes in the fourth wave
    ("layer", "bf16", 4099, 512, True, 0),  # LayerNorm's two reductions with one wave per row
    ("layer", "f32", 37, 1000, True, 2),
    ("rms", "bf16", 9, 4100, True, 0),      # D % 8 == 4: 8-byte vectors, surplus lanes
    ("layer", "bf16", 4099, 1004, True, 0),  # 8-byte vectors, one wave per row, surplus groups
    ("rms", "bf16", 4099, 1004, False, 1),
    ("rms", "bf16", 37, 1004, True, 4),
    ("rms", "bf16", 9, 4102, True, 0),      # D % 4 == 2: the scalar kernel
]


@pytest.mark.parametrize("kind,din,rows,D,with_res,wpr", IN_PLACE)
def test_rownorm_in_place_shapes(device, monkeypatch, kind, din, rows, D, with_res, wpr):
    """y written over x and h over res at shapes whose launch has lanes past the row's end or row groups past
    the last row, which re-read the row's last vector or last row: those must not observe the owner's
    stores (every value compared with the oracle on the unmodified inputs)."""
    if wpr:
        monkeypatch.setenv("SLHIP_ROWNORM_WPR", str(wpr))
    x, r, w, b = _inputs(rows, D, din, seed=rows + D, scale=2.0)
    b = b if kind == "layer" else None
    with Dev() as d:
        px = d.put(x)
        pr = d.put(r) if with_res else None
        log(f"rownorm in-place kind={kind} {din} [{rows},{D}] res={with_res} wpr={wpr}")
        native.rownorm(kind, din, din, px, px, rows, D, res=pr, w=d.put(w), b=d.put(b) if b is not None else None,
                       h_out=pr, eps=1e-5)
        native.synchronize()
        y = d.get(px, (rows, D), NP[din])
        h = d.get(pr, (rows, D), NP[din]) if with_res else None
    yref, href, _ = _reference(kind, din, din, x, r, w, b, 1e-5, with_res)
    _check(din, y, yref, f"in-place y {kind} [{rows},{D}]")
    if with_res:
        assert np.array_equal(h.view(np.uint16 if din == "bf16" else np.uint32),
                              href.view(np.uint16 if din == "bf16" else np.uint32)), "in-place h"


def test_rownorm_zero_rows_is_noop(device):
    native.rownorm("rms", "f32", "f32", None, None, 0, 1024)
    native.synchronize()


def test_rownorm_forced_row_groups(device, monkeypatch):
    """Every row-group width of the vector kernel gives the same result (tuning override)."""
    x, r, w, _ = _inputs(37, 4096, "bf16", seed=3)
    yref, href, _ = _reference("rms", "bf16", "bf16", x, r, w, None, 1e-5, True)
    for wpr in (1, 2, 4, 8, 16):
        monkeypatch.setenv("SLHIP_ROWNORM_WPR", str(wpr))
        y, h = _run("rms", "bf16", "bf16", x, r, w, None, 1e-5, with_res=True, with_h=True)
        assert_bf16_close(y, yref, what=f"wpr={wpr}")
        assert_bf16_close(h, href, ulp=0, what=f"h wpr={wpr}")


@pytest.mark.parametrize("kind,rows,D,with_w", [
    ("rms", 1, 4096, True),        # one row pair, half empty
    ("rms", 1001, 4096, True),     # many pairs per persistent group, an odd last row
    ("rms", 3000, 64, True),       # one-wave groups, one vector per lane
    ("rms", 37, 16384, True),      # 16-wave groups, two vectors per lane
    ("rms", 9, 8200, False),       # 1025 vectors: the last lane of the group holds a second, partial vector set
    ("l2", 515, 2048, False),
])
def test_rownorm_persistent_rows(device, kind, rows, D, with_w):
    """bf16 RMS / L2 rows without a residual on the persistent row groups (weights held for the launch,
    row pairs walked with the next pair in flight)."""
    x, r, w, _ = _inputs(rows, D, "bf16", seed=rows * 7 + D, scale=2.0)
    w = w if with_w else None
    y, _ = _run(kind, "bf16", "bf16", x, r, w, None, 1e-6, with_res=False, with_h=False)
    yref, _, _ = _reference(kind, "bf16", "bf16", x, r, w, None, 1e-6, False)
    assert_bf16_close(y, yref, what=f"persistent {kind} [{rows},{D}] w={with_w}")


@pytest.mark.parametrize("rows,D,offset", [
    (33, 3000, 0.0),    # 375 vectors over two waves: lanes own 2 or 3 of them
    (17, 520, 0.0),     # 65 vectors on one wave: lane 0 owns two, the rest one
    (64, 4096, 300.0),  # rows whose mean (300) dwarfs their spread (~1): the variance must not cancel
    (9, 4096, -2000.0),
])
def test_layernorm_rows_one_exchange(device, rows, D, offset):
    """bf16 LayerNorm rows without a residual (two rows per row group, mean and variance combined across the
    group's waves in one exchange), against the oracle's two-pass LayerNorm."""
    x, r, w, b = _inputs(rows, D, "f32", seed=rows * 13 + D)
    xb = oracle.to_bf16((x + np.float32(offset)).astype(np.float32))
    y, _ = _run("layer", "bf16", "bf16", xb, r, w, b, 1e-5, with_res=False, with_h=False)
    yref, _, _ = _reference("layer", "bf16", "bf16", xb, r, w, b, 1e-5, False)
    assert_bf16_close(y, yref, what=f"layernorm rows [{rows},{D}] offset={offset}")
