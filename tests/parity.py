"""Comparison rules of the parity tests.

* f32 outputs: the reference's own rule ``|d| <= atol + rtol*|ref|`` (tests/Sharplight.Vulkan.Tests/Diff.cs:206)
  with rtol = 1e-5 and atol = 1e-5 * RMS of the reference row, so near-zero outputs are not over-weighted.
* bf16 outputs: at most ``ulp`` (default 2) units in the last place from bf16_RNE(oracle f32 result),
  counted on the ordered integer line of bf16 codes (so -0 and +0 are 0 apart), with the f32 rule's
  absolute floor for results far below their row's scale (see assert_bf16_close).
* f16 outputs (KV caches): the same rule on the f16 code line (assert_f16_close).
* integer / byte / dequantized outputs: bit-exact.
"""
from __future__ import annotations

import numpy as np

F32_RTOL = 1e-5
F32_ATOL_ROW = 1e-5
BF16_ULP = 2


def bf16_ordered(bits: np.ndarray) -> np.ndarray:
    b = np.asarray(bits, dtype=np.uint16).astype(np.int64)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


def bf16_ulp_diff(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    return np.abs(bf16_ordered(a) - bf16_ordered(b))


def _bf16_f32(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def _f16_f32(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def assert_f16_close(got, ref, ulp: int = BF16_ULP, what: str = "", atol_row: float | None = None,
                     max_floor_only: int | None = None):
    """The bf16 rule (assert_bf16_close) on f16 codes: at most ``ulp`` f16 ulp from f16_RNE(oracle f32
    result), with the same absolute floor."""
    return _assert_half_close(got, ref, ulp, what, atol_row, _f16_f32, "f16", max_floor_only)


def assert_bf16_close(got, ref, ulp: int = BF16_ULP, what: str = "", atol_row: float | None = None,
                      max_floor_only: int | None = None):
    """At most ``ulp`` bf16 ulp from ``ref``. An element further away still passes when it is within the f32
    rule's absolute floor, ``atol_row`` (default 1e-5) x the RMS of its reference row: for results far below
    the row's scale -- the cancellation in a rotated pair, exp() underflowing into subnormals -- the ulp of
    the result is finer than the f32 rounding of the terms that produced it, and the reference's own
    comparison (Diff.cs:206, ``atol + rtol*|ref|``) is absolute there too. ``ulp=0`` disables the floor
    (bit-exact comparison). The elements that pass only through the floor are counted (FLOOR_ONLY[what]);
    ``max_floor_only`` bounds that count, so a regression that moves many elements there fails."""
    return _assert_half_close(got, ref, ulp, what, atol_row, _bf16_f32, "bf16", max_floor_only)


FLOOR_ONLY: dict = {}  # what -> (elements beyond ulp that passed through the absolute floor, elements compared)


def _assert_half_close(got, ref, ulp, what, atol_row, to_f32, name, max_floor_only=None):
    got = np.asarray(got, np.uint16)
    ref = np.asarray(ref, np.uint16)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    if atol_row is None:
        atol_row = 0.0 if ulp == 0 else F32_ATOL_ROW
    d = bf16_ulp_diff(got, ref)
    over = d > ulp
    beyond = int(over.sum())
    if over.any() and atol_row > 0:
        rf = to_f32(ref).astype(np.float64)
        gf = to_f32(got).astype(np.float64)
        r2 = rf.reshape(-1, ref.shape[-1]) if ref.ndim else rf.reshape(1, 1)
        rms = np.sqrt(np.mean(r2 * r2, axis=1, keepdims=True))
        floor = np.broadcast_to(atol_row * rms, r2.shape).reshape(ref.shape)
        over &= ~(np.abs(gf - rf) <= floor)
    floor_only = beyond - int(over.sum())
    FLOOR_ONLY[what] = (floor_only, int(d.size))
    if max_floor_only is not None and floor_only > max_floor_only:
        raise AssertionError(f"{what}: {floor_only} of {d.size} {name} values pass only through the absolute floor "
                             f"(at most {max_floor_only} allowed)")
    if over.any():
        i = np.unravel_index(np.argmax(np.where(over, d, -1)), d.shape)
        raise AssertionError(f"{what}: {int(over.sum())} of {d.size} {name} values beyond {ulp} ulp (and beyond the "
                             f"absolute floor); worst at {i}: got {got[i]:#06x} ref {ref[i]:#06x} ({int(d[i])} ulp)")
    return int(d.max()) if d.size else 0


def assert_f32_close(got, ref, rtol=F32_RTOL, atol_row=F32_ATOL_ROW, what: str = ""):
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    if ref.size == 0:
        return 0.0
    r2 = (ref.reshape(-1, ref.shape[-1]) if ref.ndim else ref.reshape(1, 1)).astype(np.float64)
    rms = np.sqrt(np.mean(r2 * r2, axis=1, keepdims=True))
    atol = atol_row * np.broadcast_to(rms, r2.shape).reshape(ref.shape)
    d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    bad = ~(d <= atol + rtol * np.abs(ref.astype(np.float64))) & ~(got == ref)  # equal infinities match
    if bad.any():
        i = np.unravel_index(np.argmax(bad), bad.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} f32 values out of tolerance; first at {i}: "
                             f"got {got[i]!r} ref {ref[i]!r}")
    big = np.abs(ref) > 1e-3
    return float((d[big] / np.abs(ref[big])).max()) if big.any() else 0.0


def assert_bits_equal(got, ref, what: str = ""):
    got = np.ascontiguousarray(got)
    ref = np.ascontiguousarray(ref)
    assert got.shape == ref.shape and got.dtype == ref.dtype, (got.shape, got.dtype, ref.shape, ref.dtype)
    gv = got.view(np.uint8).reshape(-1, got.dtype.itemsize)
    rv = ref.view(np.uint8).reshape(-1, ref.dtype.itemsize)
    neq = np.any(gv != rv, axis=1)
    if neq.any():
        i = int(np.argmax(neq))
        raise AssertionError(f"{what}: {int(neq.sum())} of {neq.size} values differ bitwise; first flat index {i}: "
                             f"got {got.reshape(-1)[i]!r} ref {ref.reshape(-1)[i]!r}")
