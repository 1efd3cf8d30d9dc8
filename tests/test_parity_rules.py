"""The comparison rules themselves (tests/parity.py): ulp distance, the absolute floor, exactness."""
import numpy as np
import pytest

from tests.parity import assert_bf16_close, assert_f32_close, bf16_ulp_diff


def test_ulp_distance_is_ordered_across_zero():
    a = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x3F80, 0x3F81], np.uint16)
    b = np.array([0x8000, 0x0000, 0x8001, 0x0001, 0x3F82, 0x3F80], np.uint16)
    assert bf16_ulp_diff(a, b).tolist() == [0, 0, 2, 2, 2, 1]


def test_bf16_rule_floor_and_exact_mode():
    ref = np.full((2, 64), 0x3F80, np.uint16)  # rows of 1.0
    got = ref.copy()
    got[0, 0] = 0x3F83  # 3 ulp at 1.0: fails
    with pytest.raises(AssertionError):
        assert_bf16_close(got, ref)
    ref[1, 5], got[1, 5] = 0x3400, 0x3410  # 1.19e-7 vs 1.34e-7: 16 ulp but 1.5e-8 << 1e-5 * RMS(1)
    got[0, 0] = 0x3F82
    assert_bf16_close(got, ref)
    with pytest.raises(AssertionError):
        assert_bf16_close(got, ref, ulp=0)


def test_f32_rule():
    ref = np.ones((3, 10), np.float32)
    assert_f32_close(ref * np.float32(1 + 9e-6), ref)
    with pytest.raises(AssertionError):
        assert_f32_close(ref * np.float32(1 + 3e-5), ref)
