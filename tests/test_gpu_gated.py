"""GPU parity of slhip_gated_act (SwiGLU, GeGLU with tanh-GELU, GELU-erf gating) against the oracle's
unfused Unary-then-Mul (the reference's FusionTests.cs:59-67 / ElementwiseTests.cs pattern: GPU vs CPU)."""
import numpy as np
import pytest

import oracle
from sharplight_amd import native, synth
from tests.devutil import Dev, log
from tests.parity import FLOOR_ONLY, assert_bf16_close, assert_f32_close

pytestmark = pytest.mark.gpu

NP = {"f32": np.float32, "bf16": np.uint16}


def _run(act, din, dout, g, u, *, gs=None, us=None, os_=None, pad=0):
    rows, cols = g.shape
    with Dev() as d:
        pg = d.put(g, pad)
        pu = d.put(u, pad)
        ocols = os_ or cols
        po = d.empty(rows * ocols * np.dtype(NP[dout]).itemsize, pad)
        log(f"gated {act} {din}->{dout} rows={rows} cols={cols} pad={pad}")
        native.gated_act(act, din, dout, pg, pu, po, rows, cols, gate_stride=gs, up_stride=us, out_stride=os_)
        native.synchronize()
        return d.get(po, (rows, ocols), NP[dout])


# elements of C3 that may pass only through the bf16 rule's absolute floor, about twice the MI355X count:
# SiLU and GELU-tanh none; GELU-erf 204 of 117M (0.5 g (1 + erf(g / sqrt 2)) cancels for very negative g)
C3_FLOOR_ONLY = {"silu": 0, "gelu_tanh": 0, "gelu_erf": 400}


@pytest.mark.parametrize("act", ["silu", "gelu_tanh", "gelu_erf"])
def test_c3_full_shape(device, act):
    """BASELINE config 3 at [8192, 14336] bf16 (SwiGLU, GeGLU, and the GELU-erf gate at the same shape): every
    element against the oracle's threaded Unary-then-Mul, within 2 bf16 ulp."""
    c = synth.c3()
    y = _run(act, "bf16", "bf16", c["gate"], c["up"])
    yref = oracle.gated(act, c["gate"], c["up"], dtype="bf16", threads=16)
    assert_bf16_close(y, yref, what=f"C3 {act}", max_floor_only=C3_FLOOR_ONLY[act])
    log(f"C3 {act}: {FLOOR_ONLY[f'C3 {act}'][0]} of {FLOOR_ONLY[f'C3 {act}'][1]} pass only through the absolute floor")


@pytest.mark.parametrize("act", ["silu", "gelu_tanh", "gelu_erf"])
@pytest.mark.parametrize("din,dout", [("bf16", "bf16"), ("f32", "f32"), ("bf16", "f32"), ("f32", "bf16")])
def test_gated_dtypes(device, act, din, dout):
    rows, cols = 37, 1000
    g = synth.normal(11, 0, (rows, cols), std=3.0, dtype=din)
    u = synth.normal(11, 1, (rows, cols), dtype=din)
    y = _run(act, din, dout, g, u)
    gf = oracle.from_bf16(g) if din == "bf16" else g
    uf = oracle.from_bf16(u) if din == "bf16" else u
    yf = oracle.mul(oracle.unary(act, gf), uf)
    if dout == "bf16":
        assert_bf16_close(y, oracle.to_bf16(yf), what=f"{act} {din}->{dout}")
    else:
        assert_f32_close(y, yf, what=f"{act} {din}->{dout}")
    if act == "gelu_erf" and dout == "f32":
        # the reference's rational evaluated in f32 rather than f64: erf within 4e-7 absolute, so the
        # result within 0.5 |g| |u| 4e-7 (+ the f32 roundings of the product)
        bound = 0.5 * np.abs(gf) * np.abs(uf) * 4.2e-7 + 2e-7 * np.abs(yf)
        assert np.all(np.abs(y.astype(np.float64) - yf) <= bound), "gelu_erf beyond the erf error bound"


def test_gated_extreme_inputs(device):
    """Saturation and special values: large |g|, zeros, infinities and NaN propagate like the reference."""
    g = np.array([0.0, -0.0, 1e-30, -1e-30, 20, -20, 88, -88, 100, -100, 1e4, -1e4, np.inf, -np.inf, np.nan, 3],
                 np.float32)
    g = np.tile(g, 4).reshape(4, 16)
    u = np.ones_like(g)
    for act in ("silu", "gelu_tanh", "gelu_erf"):
        y = _run(act, "f32", "f32", g, u)
        ref = oracle.mul(oracle.unary(act, g), u)
        fin = np.isfinite(ref)
        assert_f32_close(np.where(fin, y, 0), np.where(fin, ref, 0), what=act)
        assert np.array_equal(np.isnan(y), np.isnan(ref)), act
        inf = np.isinf(ref)
        assert np.array_equal(y[inf], ref[inf]), act


def test_gated_merged_projection_strides(device):
    """gate and up as the two halves of one [rows, 2*cols] tensor (row stride 2*cols), output padded."""
    rows, cols = 64, 1024
    gu = synth.normal(4, 0, (rows, 2 * cols), dtype="bf16")
    with Dev() as d:
        p = d.put(gu)
        po = d.empty(rows * (cols + 64) * 2)
        log("gated merged projection")
        native.gated_act("silu", "bf16", "bf16", p, p + cols * 2, po, rows, cols, gate_stride=2 * cols,
                         up_stride=2 * cols, out_stride=cols + 64)
        native.synchronize()
        y = d.get(po, (rows, cols + 64), np.uint16)[:, :cols]
    assert_bf16_close(y, oracle.gated("silu", gu[:, :cols], gu[:, cols:], dtype="bf16"), what="merged")


def test_gated_unaligned_and_ragged(device):
    """Odd column counts and 2-byte misalignment take the scalar kernel."""
    for rows, cols, pad in [(3, 7, 0), (5, 1001, 2), (1, 1, 0), (2, 64, 2)]:
        g = synth.normal(cols, 0, (rows, cols), std=2.0, dtype="bf16")
        u = synth.normal(cols, 1, (rows, cols), dtype="bf16")
        y = _run("silu", "bf16", "bf16", g, u, pad=pad)
        assert_bf16_close(y, oracle.gated("silu", g, u, dtype="bf16"), what=f"[{rows},{cols}] pad {pad}")


def test_gated_empty(device):
    native.gated_act("silu", "bf16", "bf16", None, None, None, 0, 14336)
    native.synchronize()
