"""The nbit parity check (tests/nbit_helpers.py) itself.  Its fp16 ulp metric
on values whose distance is known: neighbours are 1 apart, +0 and -0 are 0
apart, the two smallest subnormals of opposite sign are 2 apart, and a
2-ulp difference fails the check while a 1-ulp one passes.  Then mistakes
planted in the oracle's own output (CPU only) that the check must reject: a
truncating fp16 conversion instead of round-to-nearest-even, a dropped bias
term, and SUM where MEAN was asked for."""

import numpy as np
import pytest

import oracle as orc
from nbit_helpers import assert_nbit_close, build_weights, fp16_ulp_distance
from tbe_helpers import random_tbe


def test_ulp_distance_known_values():
    x = np.array([1.0, 0.5, 65504.0, 6e-8, 0.0], np.float16)
    with np.errstate(over="ignore"):  # 65504's neighbour is +inf
        up = np.nextafter(x, np.float16(np.inf))
    assert fp16_ulp_distance(x, up).tolist() == [1, 1, 1, 1, 1]
    assert fp16_ulp_distance(np.float16(0.0), np.float16(-0.0)) == 0
    tiny = np.float16(2.0 ** -24)
    assert fp16_ulp_distance(tiny, -tiny) == 2
    assert fp16_ulp_distance(np.float16(1.0), np.float16(2.0)) == 1024


def test_check_accepts_one_ulp_and_rejects_two():
    exp = np.linspace(-3, 3, 1001).astype(np.float16)
    one = np.nextafter(exp, np.float16(np.inf))
    assert_nbit_close(one, exp, min_exact=0.0)
    two = np.nextafter(one, np.float16(np.inf))
    with pytest.raises(AssertionError, match="more than 1 fp16 ulp"):
        assert_nbit_close(two, exp, min_exact=0.0)


def _f16_toward_zero(x32: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 rounding toward zero (a plausible wrong output rounding)."""
    h = x32.astype(np.float16)
    over = np.abs(h.astype(np.float32)) > np.abs(x32)
    h[over] = np.nextafter(h[over], np.float16(0))
    return h


@pytest.fixture(scope="module")
def nbit_case():
    rng = np.random.default_rng(77)
    tys = [orc.INT8, orc.INT4, orc.INT2, orc.FP16]
    dims = [64, 128, 32, 96]
    rows = [300, 500, 200, 100]
    inp = random_tbe(rng, len(tys), 64, dims, rows, 25)
    buf, w_off = build_weights(rng, tys, dims, rows)
    return tys, dims, rows, inp, buf, w_off


@pytest.mark.parametrize("pooling", [0, 1])
def test_planted_mistakes_are_rejected(nbit_case, pooling):
    tys, dims, rows, inp, buf, w_off = nbit_case
    exp = orc.nbit_forward(buf, w_off, tys, inp.D_offsets, inp.B, inp.indices, inp.offsets,
                           pooling)
    f32 = orc.nbit_forward(buf, w_off, tys, inp.D_offsets, inp.B, inp.indices, inp.offsets,
                           pooling, out_f16=False)
    # The oracle's fp16 output is its fp32 sum rounded to nearest even.
    assert np.array_equal(f32.astype(np.float16).view(np.uint16), exp.view(np.uint16))
    assert_nbit_close(exp.copy(), exp)

    trunc = _f16_toward_zero(f32)
    assert fp16_ulp_distance(trunc, exp).max() <= 1  # within one ulp: only the share catches it
    with pytest.raises(AssertionError, match="equal the oracle"):
        assert_nbit_close(trunc, exp)

    no_bias = buf.copy()
    for t, (ty, D, E) in enumerate(zip(tys, dims, rows)):
        if ty in (orc.INT8, orc.INT4, orc.INT2):
            s = orc.nbit_row_bytes(ty, D, 16)
            tab = no_bias[w_off[t]: w_off[t] + E * s].reshape(E, s)
            tab[:, 2:4] = 0
    dropped = orc.nbit_forward(no_bias, w_off, tys, inp.D_offsets, inp.B, inp.indices,
                               inp.offsets, pooling)
    with pytest.raises(AssertionError):
        assert_nbit_close(dropped, exp)

    other = orc.nbit_forward(buf, w_off, tys, inp.D_offsets, inp.B, inp.indices, inp.offsets,
                             1 - pooling)
    with pytest.raises(AssertionError):
        assert_nbit_close(other, exp)
