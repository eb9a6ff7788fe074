"""The fp16 ulp metric of the nbit parity check (tests/nbit_helpers.py) on
values whose distance is known: neighbours are 1 apart, +0 and -0 are 0
apart, the two smallest subnormals of opposite sign are 2 apart, and a
2-ulp difference fails the check while a 1-ulp one passes."""

import numpy as np
import pytest

from nbit_helpers import assert_nbit_close, fp16_ulp_distance


def test_ulp_distance_known_values():
    x = np.array([1.0, 0.5, 65504.0, 6e-8, 0.0], np.float16)
    up = np.nextafter(x, np.float16(np.inf))
    assert fp16_ulp_distance(x, up).tolist() == [1, 1, 1, 1, 1]
    assert fp16_ulp_distance(np.float16(0.0), np.float16(-0.0)) == 0
    tiny = np.float16(2.0 ** -24)
    assert fp16_ulp_distance(tiny, -tiny) == 2
    assert fp16_ulp_distance(np.float16(1.0), np.float16(2.0)) == 1024


def test_check_accepts_one_ulp_and_rejects_two():
    exp = np.linspace(-3, 3, 1001).astype(np.float16)
    one = np.nextafter(exp, np.float16(np.inf))
    assert_nbit_close(one, exp)
    two = np.nextafter(one, np.float16(np.inf))
    with pytest.raises(AssertionError):
        assert_nbit_close(two, exp)
