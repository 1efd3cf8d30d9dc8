"""GPU parity of slhip_convert: f32 -> bf16 rounding (ties, NaN payloads, infinities, subnormals) bit-exact
against the reference's Simd.FloatToBFloat as restated by the oracle; the widening directions exact."""
import numpy as np
import pytest

import oracle
from tests.devutil import Dev, log
from tests.parity import assert_bits_equal
from sharplight_amd import native

pytestmark = pytest.mark.gpu


def _convert(din, dout, x, pad=0):
    sizes = {"f32": 4, "f16": 2, "bf16": 2}
    np_out = {"f32": np.float32, "f16": np.float16, "bf16": np.uint16}[dout]
    with Dev() as d:
        px = d.put(x, pad)
        py = d.empty(x.size * sizes[dout], pad)
        log(f"convert {din}->{dout} n={x.size} pad={pad}")
        native.convert(din, dout, px, py, x.size)
        native.synchronize()
        return d.get(py, x.shape, np_out)


def _special_f32():
    rng = np.random.default_rng(0)
    bits = np.concatenate([
        rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32),           # every class, NaN payloads
        (np.arange(4096, dtype=np.uint32) << np.uint32(16)) | np.uint32(0x8000),       # exact ties
        (np.arange(4096, dtype=np.uint32) << np.uint32(16)) | np.uint32(0x7FFF),
        np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7F800001, 0x7FC00000, 0xFFFFFFFF, 0x00000001,
                  0x007FFFFF, 0x7F7FFFFF, 0x7F7F8000, 0x3F808000], np.uint32),
    ])
    return bits[: bits.size - bits.size % 8].view(np.float32)


@pytest.mark.parametrize("pad", [0, 4])
def test_f32_to_bf16_bits(device, pad):
    x = _special_f32()
    assert_bits_equal(_convert("f32", "bf16", x, pad), oracle.to_bf16(x), what=f"f32->bf16 pad {pad}")


def test_bf16_to_f32_exact(device):
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    assert_bits_equal(_convert("bf16", "f32", codes), oracle.from_bf16(codes), what="bf16->f32")


def test_f16_to_f32_exact(device):
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    y = _convert("f16", "f32", codes.view(np.float16))
    ref = oracle.f16_bits_to_f32(codes)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(y), nan)
    assert np.array_equal(y[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy(device):
    x = _special_f32()
    x = x[np.isfinite(x)]
    x = x[: x.size - x.size % 8]
    y = _convert("f32", "f16", x)
    with np.errstate(over="ignore"):  # values beyond f16's range round to infinity
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(y.view(np.uint16), ref)


def test_f32_to_f16_nans(device):
    """NaN payloads through f32 -> f16 against the oracle's rule (the .NET runtime's (Half) conversion:
    sign | 0x7E00 | mantissa >> 13)."""
    nans = np.array([0x7F800001, 0x7FC00000, 0xFF800001, 0x7FBFFFFF, 0xFFFFFFFF, 0x7FA02000, 0xFFC12345,
                     0x7F812000], np.uint32).view(np.float32)
    y = _convert("f32", "f16", nans)
    assert_bits_equal(y.view(np.uint16), oracle.to_f16(nans), what="f32->f16 NaN")
