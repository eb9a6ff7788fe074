"""The backward's parity checks (tests/adagrad_bounds.py) themselves, on the
CPU.  A numpy copy of the rowwise-Adagrad rule, in fp32, that adds each run's
gradient terms in the kernels' documented order (sequential up to 24 terms;
32-term chunks, strided groups, then the groups in order above) must pass the
reordering bound against the C oracle; the same copy with a mistake planted
in it must fail it:

* one term of the longest run dropped;
* one occurrence's term scaled by 1/2 (a wrong bag-length scale);
* the momentum increment not divided by D.

And the eps pin: on the eps-pin case (sqrt(h) about eps), the copy with eps
outside the root passes the pin's rtol 1e-5 comparison against the oracle,
while eps inside the root, or no eps at all, fails it."""

import numpy as np
import pytest

import oracle as orc
from adagrad_bounds import (KCHUNK, KLONG, assert_eps_pin_close, assert_reordered_adagrad_close,
                            eps_pin_case, long_run_groups, run_terms)
from tbe_helpers import random_tbe, weight_offsets


def _seq32(x: np.ndarray) -> np.ndarray:
    acc = np.zeros(x.shape[1], np.float32)
    for row in x:
        acc = acc + row
    return acc


def _kernel_sum32(x: np.ndarray, ng: int) -> np.ndarray:
    if x.shape[0] <= KLONG:
        return _seq32(x)
    chunks = [_seq32(x[i:i + KCHUNK]) for i in range(0, x.shape[0], KCHUNK)]
    groups = [_seq32(np.array(chunks[j::ng])) if chunks[j::ng] else np.zeros(x.shape[1], np.float32)
              for j in range(ng)]
    return _seq32(np.array(groups))


def adagrad_copy(inp, W0, m0, m1_off, grad, pooling, lr, eps, *, eps_mode="outside",
                 drop_term=False, half_term=False, h_not_mean=False):
    """fp32 rowwise Adagrad with the kernels' summation order; the keyword
    switches plant one mistake each."""
    W, m = W0.astype(np.float32).copy(), m0.astype(np.float32).copy()
    w_off = weight_offsets(inp)
    ng = long_run_groups(max(inp.D))
    runs = list(run_terms(inp, grad, pooling))
    longest = max(range(len(runs)), key=lambda i: runs[i][2].shape[0])
    lr32, eps32 = np.float32(lr), np.float32(eps)
    for i, (t, row, x) in enumerate(runs):
        x = x.astype(np.float32)
        if drop_term and i == longest:
            x = x[:-1]
        if half_term and i == longest:
            x = x.copy()
            x[0] = x[0] * np.float32(0.5)
        D = x.shape[1]
        g = _kernel_sum32(x, ng)
        ss = np.float32(0.0)
        for v in g * g:
            ss = np.float32(ss + v)
        mi = int(m1_off[t]) + row
        inc = ss if h_not_mean else np.float32(ss / np.float32(D))
        h = np.float32(m[mi] + inc)
        if eps_mode == "outside":
            mult = lr32 / np.float32(np.sqrt(h) + eps32)
        elif eps_mode == "inside":
            mult = lr32 / np.float32(np.sqrt(np.float32(h + eps32)))
        else:
            mult = lr32 / np.float32(np.sqrt(h))
        w0 = int(w_off[t]) + row * D
        # fma(-m, g, w): the product is exact in float64, then one rounding.
        W[w0:w0 + D] = (-np.float64(mult) * g.astype(np.float64)
                        + W[w0:w0 + D].astype(np.float64)).astype(np.float32)
        m[mi] = h
    return W, m


CASES = [  # T, B, dims, rows, max_L, pooling, dup (runs of hundreds to thousands)
    (2, 120, [208, 132], [1, 300], 40, 1, False),
    (3, 80, [56, 104, 104], [50, 1, 1], 42, 0, False),
    (2, 90, [64, 48], [3, 2000], 30, 0, True),
]


@pytest.fixture(scope="module", params=range(len(CASES)))
def extreme(request):
    T, B, dims, rows, max_L, pooling, dup = CASES[request.param]
    rng = np.random.default_rng(B + T)
    inp = random_tbe(rng, T, B, dims, rows, max_L, dup_heavy=dup)
    rng = np.random.default_rng(B)
    W = rng.uniform(-0.01, 0.01, size=sum(E * D for E, D in zip(inp.E, inp.D))).astype(np.float32)
    m1 = rng.uniform(0, 1e-4, size=sum(inp.E)).astype(np.float32)
    m1_off = np.concatenate([[0], np.cumsum(inp.E)[:-1]]).astype(np.int64)
    grad = rng.normal(0, 1e-2, size=(inp.B, inp.total_D)).astype(np.float32)
    lr, eps = 0.01, 1e-8
    W_exp, m_exp = orc.backward_rowwise_adagrad(
        W, weight_offsets(inp), inp.D_offsets, inp.B, inp.hash_size_cumsum,
        inp.total_hash_size_bits, inp.indices, inp.offsets, pooling, grad, m1, m1_off, lr, eps,
        0.0, 0, orc.info_B_num_bits(inp.T, inp.B))
    return inp, W, m1, m1_off, grad, pooling, lr, eps, W_exp, m_exp


def _check(extreme, got):
    inp, W, m1, m1_off, grad, pooling, lr, eps, W_exp, m_exp = extreme
    return assert_reordered_adagrad_close(got[0], got[1], W_exp, m_exp, W, m1, weight_offsets(inp),
                                          m1_off, inp, grad, pooling, lr, eps)


def test_kernel_order_copy_passes(extreme):
    inp, W, m1, m1_off, grad, pooling, lr, eps, W_exp, m_exp = extreme
    longest = max(x.shape[0] for _, _, x in run_terms(inp, grad, pooling))
    assert longest > 200  # the case has long runs: chunked sums in a different order
    got = adagrad_copy(inp, W, m1, m1_off, grad, pooling, lr, eps)
    # The orders differ for real: the copy is not bit-identical to the oracle.
    assert not np.array_equal(got[0], W_exp)
    _check(extreme, got)
    # The oracle against itself: difference 0, within any bound.
    _check(extreme, (W_exp, m_exp))


@pytest.mark.parametrize("mistake", ["drop_term", "half_term", "h_not_mean"])
def test_planted_mistakes_fail_the_bound(extreme, mistake):
    inp, W, m1, m1_off, grad, pooling, lr, eps, W_exp, m_exp = extreme
    got = adagrad_copy(inp, W, m1, m1_off, grad, pooling, lr, eps, **{mistake: True})
    with pytest.raises(AssertionError):
        _check(extreme, got)


@pytest.fixture(scope="module")
def eps_case():
    rng = np.random.default_rng(71)
    inp = random_tbe(rng, 3, 64, [64, 64, 64], [400, 900, 50], 12)
    W, m1, grad = eps_pin_case(np.random.default_rng(72), inp)
    m1_off = np.concatenate([[0], np.cumsum(inp.E)[:-1]]).astype(np.int64)
    lr, eps = 0.01, 1e-8
    W_exp, m_exp = orc.backward_rowwise_adagrad(
        W, weight_offsets(inp), inp.D_offsets, inp.B, inp.hash_size_cumsum,
        inp.total_hash_size_bits, inp.indices, inp.offsets, 0, grad, m1, m1_off, lr, eps,
        0.0, 0, orc.info_B_num_bits(inp.T, inp.B))
    return inp, W, m1, m1_off, grad, lr, eps, W_exp, m_exp


def test_eps_pin_case_puts_sqrt_h_at_eps(eps_case):
    inp, W, m1, m1_off, grad, lr, eps, W_exp, m_exp = eps_case
    r = np.sqrt(m_exp[m_exp > 0]) / eps
    assert 0.25 < np.median(r) < 4


def test_eps_pin_accepts_eps_outside_the_root(eps_case):
    inp, W, m1, m1_off, grad, lr, eps, W_exp, m_exp = eps_case
    got = adagrad_copy(inp, W, m1, m1_off, grad, 0, lr, eps, eps_mode="outside")
    assert_eps_pin_close(*got, W_exp, m_exp)


@pytest.mark.parametrize("eps_mode", ["inside", "none"])
def test_eps_pin_rejects_other_placements(eps_case, eps_mode):
    inp, W, m1, m1_off, grad, lr, eps, W_exp, m_exp = eps_case
    got = adagrad_copy(inp, W, m1, m1_off, grad, 0, lr, eps, eps_mode=eps_mode)
    with pytest.raises(AssertionError):
        assert_eps_pin_close(*got, W_exp, m_exp)
