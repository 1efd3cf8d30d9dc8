"""GPU parity of slhip_rope (neox / normal RoPE, fused per-head q/k RMSNorm, q and k in one launch) against
the oracle's RmsNorm-then-Rope (the reference's RopeTests.cs, GgmlCrossCheckTests.RopeMatchesGgml and
FusionTests.cs:142-157 pattern: GPU vs CPU)."""
import os

import numpy as np
import pytest

import oracle
from sharplight_amd import native, synth
from tests.devutil import Dev, log
from tests.parity import FLOOR_ONLY, assert_bf16_close, assert_f32_close

pytestmark = pytest.mark.gpu

NP = {"f32": np.float32, "bf16": np.uint16}
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _run(din, dout, tensors, pos, D, *, pads=None, ff=None, **cfg):
    """tensors: list of (x [T,H,D], w or None); returns list of outputs."""
    T = len(pos)
    with Dev() as d:
        specs, outs = [], []
        for i, (x, w) in enumerate(tensors):
            pad = pads[i] if pads else 0
            H = x.shape[1]
            px = d.put(x, pad)
            py = d.empty(x.size * np.dtype(NP[dout]).itemsize, pad)
            specs.append(dict(x=px, y=py, heads=H, norm_w=d.put(w) if w is not None else None))
            outs.append((py, x.shape))
        pp = d.put(np.asarray(pos, np.int32))
        pf = d.put(ff) if ff is not None else None
        log(f"rope {din}->{dout} T={T} D={D} heads={[t[0].shape[1] for t in tensors]} cfg={cfg}")
        native.rope(din, dout, specs, pp, T, D, ff=pf, **cfg)
        native.synchronize()
        return [d.get(py, shp, NP[dout]) for py, shp in outs]


def _ref(din, dout, x, pos, w, eps, **kw):
    y = oracle.qk_norm_rope(x, pos, w, eps, dtype="bf16" if din == "bf16" else "f32", **kw)
    if din == "bf16" and dout == "f32":
        return oracle.qk_norm_rope(oracle.from_bf16(x), pos, w, eps, **kw)
    if din == "f32" and dout == "bf16":
        return oracle.to_bf16(y)
    return y


def _check(dout, y, ref, what):
    if dout == "bf16":
        assert_bf16_close(y, ref, what=what)
    else:
        assert_f32_close(y, ref, what=what)


# elements of C4 (q, k) that may pass only through the bf16 rule's absolute floor, about twice the MI355X
# count (13 of 16.8M for q, 6 of 4.2M for k): the rotation's x0 c - x1 s cancels for a few pairs, whose
# result then sits far below its row's scale
C4_FLOOR_ONLY = (26, 12)


def test_c4_qk_norm_rope(device):
    """Qwen3-8B attention prologue, q [4096,32,128] and k [4096,8,128] bf16 in one launch:
    per-head RMSNorm (eps 1e-6) then neox RoPE, theta 1e6, positions ~ U{0..32767}."""
    c = synth.c4()
    yq, yk = _run("bf16", "bf16", [(c["q"], c["wq"]), (c["k"], c["wk"])], c["pos"], 128, neox=True, base=c["base"],
                  norm=True, eps=c["eps"])
    assert_bf16_close(yq, oracle.qk_norm_rope(c["q"], c["pos"], c["wq"], c["eps"], dtype="bf16", base=c["base"]),
                      what="C4 q", max_floor_only=C4_FLOOR_ONLY[0])
    assert_bf16_close(yk, oracle.qk_norm_rope(c["k"], c["pos"], c["wk"], c["eps"], dtype="bf16", base=c["base"]),
                      what="C4 k", max_floor_only=C4_FLOOR_ONLY[1])
    for w in ("C4 q", "C4 k"):
        log(f"{w}: {FLOOR_ONLY[w][0]} of {FLOOR_ONLY[w][1]} pass only through the absolute floor")


def test_rope_matches_ggml_fixture(device):
    """The reference's ggml rope cases (normal, neox, neox with dims 8 of 16 and freq_scale 0.5), f32."""
    fx = np.load(os.path.join(GOLDEN, "ggml_rope.npz"))
    for k in range(3):
        mode, dims, T, H, D = (int(v) for v in fx[f"case{k}_meta"])
        fs = float(fx[f"case{k}_freq_scale"][0])
        (y,) = _run("f32", "f32", [(fx[f"case{k}_x"], None)], fx[f"case{k}_pos"][:, 0], D, dims=dims,
                    neox=mode == 2, base=10000.0, freq_scale=fs)
        np.testing.assert_allclose(y, fx[f"case{k}_y"], rtol=2e-4, atol=2e-4)  # GgmlCrossCheckTests.cs:96
        ref = oracle.rope(fx[f"case{k}_x"], fx[f"case{k}_pos"][:, 0], dims=dims, neox=mode == 2, base=10000.0,
                          freq_scale=fs)
        assert_f32_close(y, ref, what=f"ggml case {k}")


@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("din,dout", [("f32", "f32"), ("bf16", "bf16"), ("bf16", "f32"), ("f32", "bf16")])
@pytest.mark.parametrize("norm", [False, True])
def test_rope_variants(device, neox, din, dout, norm):
    T, D = 29, 128
    x = synth.normal(3, 0, (T, 4, D), std=2.0, dtype=din)
    k = synth.normal(3, 1, (T, 2, D), dtype=din)
    wq = synth.normal(3, 2, (D,), 1.0, 0.1) if norm else None
    wk = synth.normal(3, 3, (D,), 1.0, 0.1) if norm else None
    pos = synth.rng(3, 4).integers(0, 40000, T).astype(np.int32)
    yq, yk = _run(din, dout, [(x, wq), (k, wk)], pos, D, neox=neox, base=1e6, norm=norm, eps=1e-6)
    kw = dict(neox=neox, base=1e6)
    eps = 1e-6
    if norm:
        _check(dout, yq, _ref(din, dout, x, pos, wq, eps, **kw), "q")
        _check(dout, yk, _ref(din, dout, k, pos, wk, eps, **kw), "k")
    else:
        _check(dout, yq, _ref(din, dout, x, pos, None, eps, **kw), "q")
        _check(dout, yk, _ref(din, dout, k, pos, None, eps, **kw), "k")


@pytest.mark.parametrize("D,dims", [(64, 64), (256, 256), (16, 8), (96, 64), (80, 80), (128, 32)])
def test_rope_head_sizes_and_partial_dims(device, D, dims):
    """Other head sizes (vector path for dims == D with D/2 a multiple of the vector width, general path
    otherwise) and partial rotation (dims < D: the tail is copied, normed when the norm is fused)."""
    T = 13
    x = synth.normal(D, 0, (T, 3, D), dtype="bf16")
    w = synth.normal(D, 1, (D,), 1.0, 0.1)
    pos = synth.rng(D, 2).integers(0, 32768, T).astype(np.int32)
    for neox in (True, False):
        for norm in (False, True):
            (y,) = _run("bf16", "bf16", [(x, w if norm else None)], pos, D, dims=dims, neox=neox, base=1e4,
                        norm=norm, eps=1e-6)
            ref = oracle.qk_norm_rope(x, pos, w if norm else None, 1e-6, dtype="bf16", dims=dims, neox=neox,
                                      base=1e4)
            assert_bf16_close(y, ref, what=f"D={D} dims={dims} neox={neox} norm={norm}")


def test_rope_freq_factors_and_scaling(device):
    T, D = 17, 128
    x = synth.normal(8, 0, (T, 2, D))
    ff = synth.rng(8, 1).uniform(1, 8, D // 2).astype(np.float32)
    pos = synth.rng(8, 2).integers(0, 100000, T).astype(np.int32)
    (y,) = _run("f32", "f32", [(x, None)], pos, D, ff=ff, base=5e5, freq_scale=0.25, attn_factor=1.3)
    ref = oracle.rope(x, pos, base=5e5, freq_scale=0.25, attn_factor=1.3, ff=ff)
    assert_f32_close(y, ref, what="ff")


def test_rope_unaligned_and_single_token(device):
    x = synth.normal(1, 0, (1, 8, 128), dtype="bf16")
    (y,) = _run("bf16", "bf16", [(x, None)], np.array([32767], np.int32), 128, pads=[2], base=1e6)
    assert_bf16_close(y, oracle.qk_norm_rope(x, np.array([32767]), None, dtype="bf16", base=1e6), what="pad")


def test_rope_position_zero_is_identity(device):
    x = synth.normal(2, 0, (5, 4, 128))
    (y,) = _run("f32", "f32", [(x, None)], np.zeros(5, np.int32), 128, base=1e6)
    assert np.array_equal(y, x)


def test_rope_empty(device):
    native.rope("bf16", "bf16", [dict(x=16, y=16, heads=4)], 16, 0, 128)
    native.synchronize()


# ---- multi-axis rope (M-RoPE, interleaved, per-element sections) ----------------------------------------

def test_rope_multi_axis_matches_ggml(device):
    """GgmlCrossCheckTests.RopeMatchesGgml's seven cases through slhip_rope (f32): the four-axis positions
    with sections for modes 8 (M-RoPE) and 40 (interleaved), against ggml's output at the reference's 2e-4
    and against the oracle within the f32 tolerance."""
    fx = np.load(os.path.join(GOLDEN, "ggml_rope.npz"))
    for k in range(7):
        mode, dims, T, H, D = (int(v) for v in fx[f"case{k}_meta"])
        multi = mode >= 8
        x = fx[f"case{k}_x"]
        pos = fx[f"case{k}_pos"] if multi else np.ascontiguousarray(fx[f"case{k}_pos"][:, 0])
        sec = [int(v) for v in fx[f"case{k}_sections"]] if multi else None
        fs = float(fx[f"case{k}_freq_scale"][0])
        (y,) = _run("f32", "f32", [(x, None)], pos, D, dims=dims, neox=mode != 0, base=10000.0, freq_scale=fs,
                    pos_axes=4 if multi else 1, sections=sec, interleaved=mode == 40)
        np.testing.assert_allclose(y, fx[f"case{k}_y"], rtol=2e-4, atol=2e-4)
        ref = oracle.rope_multi(x, pos, sec, interleaved=mode == 40, dims=dims, neox=mode != 0, freq_scale=fs)
        assert_f32_close(y, ref, what=f"ggml case {k}")


@pytest.mark.parametrize("interleaved,per_element,neox", [(False, False, True), (True, False, True),
                                                          (False, True, True), (True, True, False)])
def test_rope_multi_axis_qk_norm_bf16(device, interleaved, per_element, neox):
    """A Qwen3-VL-style prologue: q [256, 16, 128] and k [256, 4, 128] bf16 with the per-head RMSNorm fused,
    three position axes (t, h, w) with sections [24, 20, 20, 0], theta 5e6 -- the vector kernel's
    multi-axis variant, against the oracle's RmsNorm then multi-axis RopeOp."""
    rng = np.random.default_rng(31)
    T = 256
    q = oracle.to_bf16(rng.standard_normal((T, 16, 128)).astype(np.float32))
    k = oracle.to_bf16(rng.standard_normal((T, 4, 128)).astype(np.float32))
    wq = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    wk = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    pos = rng.integers(0, 32768, (T, 3)).astype(np.int32)
    sec = [24, 20, 20, 0]
    yq, yk = _run("bf16", "bf16", [(q, wq), (k, wk)], pos, 128, neox=neox, base=5e6, norm=True, eps=1e-6,
                  pos_axes=3, sections=sec, interleaved=interleaved, per_element=per_element)
    for y, x, w, name in ((yq, q, wq, "q"), (yk, k, wk, "k")):
        xn = oracle.rmsnorm(oracle.from_bf16(x).reshape(-1, 128), w, 1e-6).reshape(x.shape)
        ref = oracle.to_bf16(oracle.rope_multi(xn, pos, sec, interleaved=interleaved, per_element=per_element,
                                               neox=neox, base=5e6))
        assert_bf16_close(y, ref, what=f"{name} il={interleaved} pe={per_element}")


def test_rope_multi_axis_general_path(device):
    """Partial dims (48 of D 72) and a single position axis broadcast to the sections: the general kernel."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((9, 3, 72)).astype(np.float32)
    p = rng.integers(0, 20000, 9).astype(np.int32)
    pos4 = rng.integers(0, 20000, (9, 4)).astype(np.int32)
    (y1,) = _run("f32", "f32", [(x, None)], p, 72, dims=48, neox=True, base=1e4, sections=[4, 8, 8, 4])
    assert_f32_close(y1, oracle.rope_multi(x, p[:, None], [4, 8, 8, 4], dims=48, base=1e4), what="one axis")
    (y4,) = _run("f32", "f32", [(x, None)], pos4, 72, dims=48, neox=True, base=1e4, pos_axes=4,
                 sections=[4, 8, 8, 4], per_element=True)
    assert_f32_close(y4, oracle.rope_multi(x, pos4, [4, 8, 8, 4], per_element=True, dims=48, base=1e4),
                     what="four axes, per element")


def test_recip_exhaustive(device):
    """The reciprocal behind the fused q/k-norm scale (hardware reciprocal + one Newton step, division outside
    [2^-125, 2^125]) equals IEEE 1.0f / s on all 2^32 f32 inputs, and the bare hardware reciprocal does not
    (a check program built beside the library: tests/recip_exhaustive.hip)."""
    import subprocess
    exe = os.path.join(os.path.dirname(GOLDEN), "_bin", "recip_exhaustive")
    assert os.path.exists(exe), "tests/_bin/recip_exhaustive is not built: run the package build"
    log("recip exhaustive check program")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=100)
    out = r.stdout.split()
    assert out[0] == "checked" and int(out[1]) == 1 << 32, r.stdout + r.stderr
    assert int(out[3]) == 0 and int(out[5]) == 0, r.stdout
    assert int(out[7]) > 0, "the bare reciprocal must differ somewhere: the checker compared nothing"
    assert r.returncode == 0, r.stdout + r.stderr
