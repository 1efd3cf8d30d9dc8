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


def test_floor_only_elements_are_counted_and_bounded():
    """assert_bf16_close counts the elements that pass only through the absolute floor, and max_floor_only
    bounds them: a regression moving many elements there fails even though each passes the floor."""
    import numpy as np
    import pytest

    from tests import parity
    ref = np.full((2, 256), 0x3F80, np.uint16)  # 1.0
    ref[0, :4] = 0x0001                         # four results far below the row's scale (1e-5 x RMS = 1e-5)
    got = ref.copy()
    got[0, :4] = 0x0003                          # 2 codes away, but |d| is ~1e-45: within the floor
    got[1, 7] = 0x3F81                           # 1 ulp: within the ulp rule
    parity.assert_bf16_close(got, ref, what="t")
    assert parity.FLOOR_ONLY["t"] == (0, 512)    # 2 ulp is within ulp=2: nothing needed the floor
    got[0, :4] = 0x0007                          # 6 codes away: the floor alone passes them
    parity.assert_bf16_close(got, ref, what="t")
    assert parity.FLOOR_ONLY["t"] == (4, 512)
    parity.assert_bf16_close(got, ref, what="t", max_floor_only=4)
    with pytest.raises(AssertionError, match="only through the absolute floor"):
        parity.assert_bf16_close(got, ref, what="t", max_floor_only=3)
