"""Comparison of two fp32 evaluations of the exact rowwise-Adagrad update whose
per-row gradient sums add the same fp32 terms in different orders.

Both the oracle (orc_backward_rowwise_adagrad) and the kernels compute, per
run r = (table t, row i): the terms x_j = grad[b_j, D_off[t]:D_off[t+1]]
(times fp32 1/L_j under MEAN), the sum g = sum_j x_j in fp32,
h' = h + sum_d g_d^2 / D, m = lr / (sqrt(h') + eps) and w' = fma(-m, g, w).
They differ only in the order of the additions of g and of sum_d g_d^2:

* the oracle adds a run's terms one after another in sorted order (occurrence
  order) and the squares in column order;
* the kernels add runs of at most KLONG occurrences in that same order (equal
  results), and longer runs in KCHUNK-occurrence chunks (each summed in
  order), the chunk sums in NG strided groups (group j: chunks j, j+NG, ...,
  in order), then the NG group sums in group order; NG follows the launch
  width (`long_run_groups`); the squares by per-lane sums and a lane tree.

A pure relative tolerance on w' fails wherever g has cancelled to near zero,
however correct both sides are.  The check here uses the first-order
rounding-error bound of recursive summation (Higham, Accuracy and Stability
of Numerical Algorithms, 2nd ed., 2002, section 4.2, eq. (4.3)): an fp32 sum
computed along a tree of additions is within u * sum over the additions of
|partial result| of the exact sum, u = 2^-24.  That bound is evaluated from
the float64 partial sums of each side's own order (e_d per column), and it
is carried through the update:

* |g_A - g_B| <= e_d = u (P_oracle_d + P_kernel_d);
* |h_A - h_B| <= (sum_d 2 |g|_d e_d + 2 D u ss) / D + 4 u h', where ss is
  sum_d |g|_d^2 (each side's sum of D positive squares in any order: at most
  D - 1 additions of partial sums <= ss, plus one rounding per square) and
  4 u h' the two roundings per side of ss / D and h + ss / D;
* |m_A - m_B| <= m |h_A - h_B| / (2 sqrt(h') (sqrt(h') + eps)) + 6 u m
  (the measured h difference moved through d m / d h; sqrt, add and divide
  each round once per side);
* |w_A - w_B| <= m e_d + |g|_d |m_A - m_B| + u (|w_A| + |w_B|) (the fused
  multiply-add rounds once per side);

each with a factor 1.01 for the second-order terms the first-order bound
drops.  So the comparison is against the oracle itself, element by element,
with no float64 referee: it fails when the two sides disagree by more than
the rounding of two correct evaluations can explain.  In the form
|w_A - w_B| <= k u (sum_j |x_j|) m, the effective k is
(P_oracle + P_kernel) / sum_j |x_j|, printed by the tests (typically a few
to a few tens for runs of thousands of terms)."""

from __future__ import annotations

import numpy as np

U = 2.0 ** -24
KLONG, KCHUNK = 24, 32  # the kernels' long-run threshold and chunk length
SLACK = 1.01


def long_run_groups(max_D: int) -> int:
    """Groups that sum a long run's chunk partials: 256 threads / lanes per
    group, the lanes per group following the call's widest table (16 lanes up
    to D = 64, 32 up to 128, 64 above)."""
    if max_D <= 64:
        return 16
    if max_D <= 128:
        return 8
    return 4


def _seq_bound(terms: np.ndarray) -> np.ndarray:
    """sum over the additions (the second term on) of |partial sum|, for terms
    [n, D] (float64) added one after another from zero."""
    if terms.shape[0] <= 1:
        return np.zeros(terms.shape[1])
    return np.abs(np.cumsum(terms, axis=0)[1:]).sum(axis=0)


def kernel_order_bound(terms: np.ndarray, ng: int) -> np.ndarray:
    n, D = terms.shape
    if n <= KLONG:
        return _seq_bound(terms)
    chunks = [terms[i:i + KCHUNK] for i in range(0, n, KCHUNK)]
    P = sum(_seq_bound(c) for c in chunks)
    csum = np.array([c.sum(axis=0) for c in chunks])
    groups = [csum[j::ng] for j in range(ng)]
    P = P + sum(_seq_bound(gq) for gq in groups if len(gq))
    gsum = np.array([gq.sum(axis=0) if len(gq) else np.zeros(D) for gq in groups])
    return P + _seq_bound(gsum)


def run_terms(inp, grad: np.ndarray, pooling: int):
    """Yields (t, row, terms [n, D] float64 in occurrence order) for every
    row the batch touches (features do not share tables here)."""
    B, Doff = inp.B, inp.D_offsets
    L = np.diff(inp.offsets)
    for t in range(inp.T):
        s, e = int(inp.offsets[t * B]), int(inp.offsets[(t + 1) * B])
        if e == s:
            continue
        Lt = L[t * B:(t + 1) * B]
        bags = np.repeat(np.arange(B), Lt)
        x = grad[bags, Doff[t]:Doff[t + 1]].astype(np.float32)
        if pooling == 1:  # the fp32 scale both sides use: x * fp32(1/L)
            x = x * (np.float32(1.0) / Lt[bags].astype(np.float32))[:, None]
        idx = inp.indices[s:e]
        order = np.argsort(idx, kind="stable")
        rows, starts = np.unique(idx[order], return_index=True)
        ends = np.append(starts[1:], len(order))
        for row, a, b in zip(rows, starts, ends):
            yield t, int(row), x[order[a:b]].astype(np.float64)


def assert_reordered_adagrad_close(got_W, got_m, exp_W, exp_m, W0, m0, w_off, m1_off, inp,
                                   grad, pooling: int, lr: float, eps: float) -> float:
    """Asserts the GPU update (got) against the oracle's (exp) under the
    bound above; rows the batch does not touch must be bit-identical to the
    start values on both sides.  Returns the largest |w_A - w_B| / bound and
    prints the largest effective k."""
    got_W, got_m = np.asarray(got_W, np.float32), np.asarray(got_m, np.float32)
    exp_W, exp_m = np.asarray(exp_W, np.float32), np.asarray(exp_m, np.float32)
    ng = long_run_groups(max(inp.D))
    touched_w = np.zeros(got_W.size, bool)
    touched_m = np.zeros(got_m.size, bool)
    worst, worst_k = 0.0, 0.0
    for t, row, x in run_terms(inp, grad, pooling):
        D = x.shape[1]
        g = x.sum(axis=0)
        e = SLACK * U * (_seq_bound(x) + kernel_order_bound(x, ng))
        gabs = np.abs(g) + e
        ss = float((gabs * gabs).sum())
        mi = int(m1_off[t]) + row
        h0 = float(m0[mi])
        h = h0 + float((g * g).sum()) / D
        hb = h0 + ss / D
        dh_bound = SLACK * ((2.0 * gabs * e).sum() / D + 2.0 * U * ss + 4.0 * U * hb)
        dh = abs(float(got_m[mi]) - float(exp_m[mi]))
        assert dh <= dh_bound, (
            f"table {t} row {row}: momentum differs by {dh:.3e}, bound {dh_bound:.3e}")
        sq = np.sqrt(h)
        m = lr / (sq + eps)
        dm = SLACK * (m * dh / (2.0 * sq * (sq + eps)) if h > 0 else 0.0) + SLACK * 6.0 * U * m
        w0 = int(w_off[t]) + row * D
        wa = got_W[w0:w0 + D].astype(np.float64)
        wb = exp_W[w0:w0 + D].astype(np.float64)
        bound = SLACK * (m * e + gabs * dm + U * (np.abs(wa) + np.abs(wb)))
        diff = np.abs(wa - wb)
        bad = diff > bound
        assert not bad.any(), (
            f"table {t} row {row} ({x.shape[0]} terms): {int(bad.sum())} of {D} weights past the "
            f"reordering bound (worst diff {diff[bad].max():.3e}, bound there "
            f"{bound[bad][np.argmax(diff[bad])]:.3e})")
        worst = max(worst, float((diff / np.maximum(bound, 1e-300)).max()))
        sabs = np.abs(x).sum(axis=0)
        k = (e / SLACK / U) / np.maximum(sabs, 1e-300)
        worst_k = max(worst_k, float(k.max()))
        touched_w[w0:w0 + D] = True
        touched_m[mi] = True
    W0 = np.asarray(W0, np.float32)
    m0 = np.asarray(m0, np.float32)
    assert np.array_equal(got_W[~touched_w].view(np.uint32), W0[~touched_w].view(np.uint32))
    assert np.array_equal(exp_W[~touched_w].view(np.uint32), W0[~touched_w].view(np.uint32))
    assert np.array_equal(got_m[~touched_m].view(np.uint32), m0[~touched_m].view(np.uint32))
    print(f"  reordering bound: worst |dw| / bound {worst:.3f}, largest effective k {worst_k:.1f}",
          flush=True)
    return worst


def eps_pin_case(rng: np.random.Generator, inp, sigma: float = 1e-8):
    """Start values where Adagrad's eps is of the size of sqrt(h): zero
    momentum and upstream gradients N(0, sigma) with sigma = eps = 1e-8 (SUM;
    under MEAN the caller multiplies sigma by the mean bag length), so a row
    touched once has sqrt(h') = |g| ~ eps.  Then sqrt(h') + eps and
    sqrt(h' + eps) (~1e-4) differ by four orders of magnitude, and dropping
    eps halves the denominator."""
    W = rng.uniform(-0.01, 0.01, size=sum(E * D for E, D in zip(inp.E, inp.D))).astype(np.float32)
    m1 = np.zeros(sum(inp.E), np.float32)
    grad = rng.normal(0, sigma, size=(inp.B, inp.total_D)).astype(np.float32)
    return W, m1, grad


def assert_eps_pin_close(got_W, got_m, exp_W, exp_m):
    """The eps-pin comparison: weights rtol 1e-5 (atol 1e-7), momentum rtol
    1e-5."""
    np.testing.assert_allclose(np.asarray(got_W, np.float32), exp_W, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(np.asarray(got_m, np.float32), exp_m, rtol=1e-5, atol=0)
