"""GPU parity of slhip_gather (embedding rows with on-the-fly Q8_0 / Q4_0 / Q4_1 / Q5_0 / Q5_1, K-quant
Q2_K..Q6_K, IQ4_NL / IQ4_XS and F16 / BF16 / F32 dequantization): bit-exact against the oracle's GatherOp,
mirroring the reference's GatherTests.cs:7-25,147-163, QuantTests.cs:49-97 and GgmlDequantTests."""
import os

import numpy as np
import pytest

import oracle
from sharplight_amd import native, synth
from tests.devutil import Dev, log
from tests.parity import assert_bits_equal

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
NP = {"f32": np.float32, "bf16": np.uint16}


def _run(fmt, table, V, D, ids, dout, *, table_pad=0, y_stride=None):
    N = len(ids)
    ys = D if y_stride is None else y_stride
    with Dev() as d:
        pt = d.put(table, table_pad)
        pi = d.put(np.asarray(ids, np.int32))
        py = d.empty(max(N, 1) * ys * np.dtype(NP[dout]).itemsize)
        log(f"gather {fmt}->{dout} V={V} D={D} N={N} pad={table_pad} ys={ys}")
        native.gather(fmt, pt, V, D, pi, N, dout, py, y_stride=ys)
        native.synchronize()
        return d.get(py, (N, ys), NP[dout])[:, :D]


def _ref(fmt, table, V, D, ids, dout):
    return oracle.gather_as(fmt, table, V, D, np.asarray(ids, np.int32), dtype=dout)


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "f16"])
def test_c5_full_shape(device, fmt):
    """16384 ids uniform over a [151936, 4096] table -> bf16, bit-exact on every row."""
    c = synth.c5(fmt)
    y = _run(fmt, c["table"], c["V"], c["D"], c["ids"], "bf16")
    assert_bits_equal(y, _ref(fmt, c["table"], c["V"], c["D"], c["ids"], "bf16"), what=f"C5 {fmt}")


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q4_1", "q5_0", "q5_1"])
@pytest.mark.parametrize("dout", ["f32", "bf16"])
def test_ggml_fixture_rows(device, fmt, dout):
    """The reference's ggml fixture table, rows [3, 0, 2, 2] (QuantTests.GatherDequantizes)."""
    fx = np.load(os.path.join(GOLDEN, "ggml_quant.npz"))
    rows, cols = (int(v) for v in fx[f"{fmt}_shape"])
    ids = [3, 0, 2, 2]
    y = _run(fmt, fx[f"{fmt}_blocks"], rows, cols, ids, dout)
    assert_bits_equal(y, _ref(fmt, fx[f"{fmt}_blocks"], rows, cols, ids, dout), what=fmt)
    if dout == "f32":
        np.testing.assert_array_equal(y, fx[f"{fmt}_deq"][ids])  # ggml's own values (+0 vs -0 aside)


KFMTS = ["q2_k", "q3_k", "q4_k", "q5_k", "q6_k", "iq4_nl", "iq4_xs", "tq1_0", "tq2_0", "mxfp4", "nvfp4", "iq2_xxs",
         "iq2_xs", "iq2_s", "iq3_xxs", "iq3_s", "iq1_s", "iq1_m"]


@pytest.mark.parametrize("fmt", ["f32", "f16", "bf16", "q8_0", "q4_0", "q4_1", "q5_0", "q5_1"] + KFMTS)
@pytest.mark.parametrize("dout", ["f32", "bf16"])
@pytest.mark.parametrize("D", [32, 256, 4096, 5120, 8192 + 32])
def test_gather_formats(device, fmt, dout, D):
    """Every format, both outputs: a single block, whole and partial 4096-value chunks, rows that are not
    a whole number of 16-byte vectors (the general kernel). Formats with larger blocks take D rounded to
    their block size."""
    bs = synth.block_values(fmt)
    if bs > 32:  # D rounded to the block size; the ragged case keeps one extra block past 8192
        D = max(bs, D // bs * bs) + (bs if D == 8192 + 32 else 0)
    V, N = 300, 97
    t = synth.quant_table(fmt, V, D, seed=D, tid=0)
    ids = synth.rng(D, 1).integers(0, V, N).astype(np.int32)
    ids[:3] = [0, V - 1, 0]  # first, last, duplicate
    y = _run(fmt, t, V, D, ids, dout)
    assert_bits_equal(y, _ref(fmt, t, V, D, ids, dout), what=f"{fmt}->{dout} D={D}")


@pytest.mark.parametrize("fmt", KFMTS)
@pytest.mark.parametrize("dout", ["f32", "bf16"])
def test_ggml_ext_fixture_rows(device, fmt, dout):
    """ggml's own blocks and random bytes (ggml_quant_ext.bin, GgmlDequantTests): every row, bit-exact against
    the oracle -- whose values are ggml's bit for bit (Q2_K, Q3_K, IQ4_*) or within one rounding (Q4_K..Q6_K)
    -- including the NaN and infinite scales random bytes produce."""
    fx = np.load(os.path.join(GOLDEN, "ggml_quant_ext.npz"))
    for r in sorted({k[:-6] for k in fx.files if k.startswith(fmt + "_") and k.endswith("_shape")}):
        rows, cols = (int(v) for v in fx[f"{r}_shape"])
        ids = np.arange(rows, dtype=np.int32)[::-1].copy()
        y = _run(fmt, fx[f"{r}_blocks"], rows, cols, ids, dout)
        ref = _ref(fmt, fx[f"{r}_blocks"], rows, cols, ids, dout)
        # NaNs compare as NaNs: a random-byte block with an infinite scale makes inf * 0 = NaN, whose sign is
        # the platform's default NaN (negative on x86, where the reference runs; positive on the GPU)
        yf = y if dout == "f32" else oracle.from_bf16(y)
        rf = ref if dout == "f32" else oracle.from_bf16(ref)
        nan = np.isnan(rf)
        assert np.array_equal(np.isnan(yf), nan), r
        assert np.array_equal(yf[~nan].view(np.uint32), rf[~nan].view(np.uint32)), r


def test_gather_every_f16_code(device):
    """All 65,536 binary16 codes through the f16 table path to f32 (exact, NaNs as NaN) and to bf16 (bit-exact)."""
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(16, 4096)
    t = codes.view(np.uint8)
    ids = np.arange(16, dtype=np.int32)
    y32 = _run("f16", t, 16, 4096, ids, "f32")
    ref32 = _ref("f16", t, 16, 4096, ids, "f32")
    nan = np.isnan(ref32)
    assert np.array_equal(np.isnan(y32), nan)
    assert np.array_equal(y32[~nan].view(np.uint32), ref32[~nan].view(np.uint32))
    assert_bits_equal(_run("f16", t, 16, 4096, ids, "bf16"), _ref("f16", t, 16, 4096, ids, "bf16"), what="f16 codes")


def test_gather_every_q8_code_and_scale(device):
    """Every int8 code under normal, subnormal, negative and zero f16 scales, to f32 and bf16."""
    scales = np.array([0x3C00, 0x2E66, 0x0001, 0x03FF, 0x8001, 0xBC00, 0x7BFF, 0x0000, 0x8000], np.uint16)
    blocks = np.zeros((len(scales), 128, 34), np.uint8)
    for i, s in enumerate(scales):
        blocks[i, :, 0:2] = np.frombuffer(s.tobytes(), np.uint8)
        blocks[i, :, 2:] = np.tile(np.arange(-128, 128, dtype=np.int32).astype(np.int8).view(np.uint8), 16).reshape(128, 32)
    t = blocks.reshape(len(scales), -1)
    ids = np.arange(len(scales), dtype=np.int32)
    for dout in ("f32", "bf16"):
        assert_bits_equal(_run("q8_0", t, len(scales), 4096, ids, dout), _ref("q8_0", t, len(scales), 4096, ids, dout),
                          what=dout)


def test_gather_unaligned_table_and_strided_output(device):
    """A table misaligned by 2 bytes and an odd row length take the general kernel; a padded output row
    stride keeps the vector kernel."""
    V, D = 50, 4096
    t = synth.quant_table("q4_0", V, D, seed=1)
    ids = synth.rng(1, 1).integers(0, V, 33).astype(np.int32)
    ref = _ref("q4_0", t, V, D, ids, "bf16")
    assert_bits_equal(_run("q4_0", t, V, D, ids, "bf16", table_pad=2), ref, what="pad")
    assert_bits_equal(_run("q4_0", t, V, D, ids, "bf16", y_stride=D + 64), ref, what="stride")
    t2 = synth.quant_table("q8_0", V, 96, seed=2)  # 3 blocks = 102 bytes per row: not 16-byte rows
    assert_bits_equal(_run("q8_0", t2, V, 96, ids, "bf16"), _ref("q8_0", t2, V, 96, ids, "bf16"), what="ragged")


def test_gather_out_of_range_raises_on_sync(device):
    """GatherOp throws ArgumentOutOfRangeException (GatherOp.cs:60-63): the kernel zeroes the row, the next
    slhip_stream_sync raises, and the error is cleared afterwards."""
    V, D = 20, 256
    t = synth.quant_table("q8_0", V, D, seed=3)
    for bad in (V, -1, 1 << 30):
        ids = np.array([1, bad, 2], np.int32)
        with Dev() as d:
            pt, pi = d.put(t), d.put(ids)
            py = d.empty(3 * D * 2)
            log(f"gather out-of-range id={bad}")
            native.gather("q8_0", pt, V, D, pi, 3, "bf16", py)
            with pytest.raises(native.SlhipIndexError, match=str(bad)):
                native.synchronize()
            native.synchronize()  # cleared
            y = d.get(py, (3, D), np.uint16)
        assert np.all(y[1] == 0)
        ref = _ref("q8_0", t, V, D, [1, 2], "bf16")
        assert_bits_equal(y[[0, 2]], ref, what="good rows")


def test_gather_empty(device):
    native.gather("q8_0", None, 10, 4096, None, 0, "bf16", None)
    native.synchronize()


def _nan_aware_equal(y, ref, dout, what):
    yf = y if dout == "f32" else oracle.from_bf16(y)
    rf = ref if dout == "f32" else oracle.from_bf16(ref)
    nan = np.isnan(rf)
    assert np.array_equal(np.isnan(yf), nan), what
    assert np.array_equal(yf[~nan].view(np.uint32), rf[~nan].view(np.uint32)), what


@pytest.mark.parametrize("fmt", oracle.REF_FORMATS)
@pytest.mark.parametrize("dout", ["f32", "bf16"])
@pytest.mark.parametrize("D", [128, 4096, 5120 + 128])
def test_gather_reference_formats(device, fmt, dout, D):
    """The reference's own formats (Q1_0 .. F8E4M3_B128, src/Sharplight.Cpu/Quant.cs:287-362): random code
    bytes with sane scales, bit-exact against the oracle's restatement of each decoder (NaNs -- from E5M2's
    NaN codes -- compared as NaNs), on a single block, whole work items and a partial last item."""
    bs = synth.block_values(fmt)
    D = max(bs, D // bs * bs)
    V, N = 257, 61
    t = synth.quant_table(fmt, V, D, seed=D + 7, tid=len(fmt))
    ids = synth.rng(D, 3).integers(0, V, N).astype(np.int32)
    ids[:3] = [0, V - 1, 0]
    y = _run(fmt, t, V, D, ids, dout)
    _nan_aware_equal(y, _ref(fmt, t, V, D, ids, dout), dout, f"{fmt}->{dout} D={D}")


def test_gather_trellis_reference_fixture(device):
    """The reference's trellis fixture (tests/golden/trellis_ref.bin: the fork's decoders' values) gathered on
    the GPU, every row of every record, bit for bit against the fixture itself."""
    from tests.test_oracle_formats import trellis_fixture
    for fmt, rows, cols, blocks, expected in trellis_fixture():
        ids = np.arange(rows, dtype=np.int32)[::-1].copy()
        y = _run(fmt, np.ascontiguousarray(blocks), rows, cols, ids, "f32")
        assert np.array_equal(y.view(np.uint32), expected[ids].view(np.uint32)), fmt


@pytest.mark.parametrize("fmt", ["f8e4m3", "f8e5m2"])
def test_gather_every_fp8_code(device, fmt):
    """All 256 codes of the plain FP8 tables to f32, exact (NaN codes as NaN)."""
    t = np.tile(np.arange(256, dtype=np.uint8), 16).reshape(1, 4096)
    y = _run(fmt, t, 1, 4096, np.zeros(1, np.int32), "f32")
    _nan_aware_equal(y, _ref(fmt, t, 1, 4096, np.zeros(1, np.int32), "f32"), "f32", fmt)


@pytest.mark.parametrize("fmt", ["nvfp4_gs", "q4z_g32", "q8z_g128", "nf4_b64", "q8a_g32", "f8e4m3_b32",
                                 "trellis_v4k6_g128", "trellis_v2k5_g128"])
def test_gather_reference_formats_unaligned(device, fmt):
    """A table 2 bytes off 16-byte alignment: the general kernel, same bits."""
    bs = synth.block_values(fmt)
    V, D = 9, 2 * max(bs, 64)
    t = synth.quant_table(fmt, V, D, seed=3, tid=1)
    ids = np.array([3, 0, 8, 3], np.int32)
    with Dev() as d:
        pt = d.put(t, 2)
        py = d.empty(4 * D * 4)
        log(f"gather unaligned {fmt}")
        native.gather(fmt, pt, V, D, d.put(ids), 4, "f32", py)
        native.synchronize()
        y = d.get(py, (4, D), np.float32)
    _nan_aware_equal(y, _ref(fmt, t, V, D, ids, "f32"), "f32", fmt)
