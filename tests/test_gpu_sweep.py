"""Seeded random sweep over the TBE ops' argument space, against the oracle.

Each round draws one forward case (1-6 tables of widths 4..1024, 1-300 bags,
0-80 indices per bag, SUM/MEAN, per-sample weights or not, fp32 or fp16
weight rows, int32 or int64 indices; bit-exact), one transpose case (1-8
features of up to 200,000 rows; bit-exact over the whole run layout) and one
backward case (unweighted with any run lengths, under the reordering bound of
adagrad_bounds.py; or weighted, L2 or decoupled weight decay on rows of at
least 200, at rtol 1e-5).  A quarter of the cases draw their indices from
three rows per table, so long runs and repeated rows are common.  A second
sweep draws sequence lookups (PoolingMode NONE: forward, nbit, backward),
cumsums and feature permutes."""

import numpy as np
import pytest
import torch

import oracle as orc
from adagrad_bounds import assert_reordered_adagrad_close
from tbe_helpers import random_tbe, tbe_forward_gpu, weight_offsets
from test_gpu_backward import _backward_case, _backward_gpu, _check_transpose
from test_gpu_tbe_forward import _exact

pytestmark = pytest.mark.gpu

DIMS = [4, 8, 12, 36, 64, 100, 128, 132, 256, 260, 512, 1000, 1024]
ROUNDS = 15


def _shape(rng, max_T, max_B, max_L, rows_lo, rows_hi):
    T = int(rng.integers(1, max_T + 1))
    B = int(rng.integers(1, max_B + 1))
    dims = [int(rng.choice(DIMS)) for _ in range(T)]
    rows = [int(rng.integers(rows_lo, rows_hi + 1)) for _ in range(T)]
    return T, B, dims, rows, int(rng.integers(0, max_L + 1))


def _forward(dev, rng, i):
    T, B, dims, rows, L = _shape(rng, 6, 300, 80, 1, 5000)
    pooling, weighted = int(rng.integers(0, 2)), bool(rng.integers(0, 2))
    f16 = bool(rng.integers(0, 2))
    itype = torch.int32 if rng.integers(0, 2) else torch.int64
    print(f"[case] sweep fwd {i}: T={T} B={B} dims={dims} rows={rows} L={L} pool={pooling} "
          f"weighted={weighted} fp16={f16} {itype}", flush=True)
    inp = random_tbe(rng, T, B, dims, rows, L, dup_heavy=bool(rng.integers(0, 4) == 0))
    W = rng.uniform(-1, 1, size=sum(E * D for E, D in zip(rows, dims)))
    W = W.astype(np.float16 if f16 else np.float32)
    iw = rng.uniform(-2, 2, size=inp.N).astype(np.float32) if weighted else None
    exp = orc.tbe_forward_f32(W, weight_offsets(inp), inp.D_offsets, B, inp.indices, inp.offsets,
                              pooling, iw)
    got = tbe_forward_gpu(dev, torch.from_numpy(W).to(dev), inp, pooling, itype,
                          indice_weights=None if iw is None else torch.from_numpy(iw))
    _exact(got, exp)


def _transpose(dev, rng, i):
    T, B, _, rows, L = _shape(rng, 8, 400, 60, 1, 200000)
    itype = torch.int32 if rng.integers(0, 2) else torch.int64
    print(f"[case] sweep transpose {i}: T={T} B={B} rows={rows} L={L} {itype}", flush=True)
    inp = random_tbe(rng, T, B, [4] * T, rows, L, dup_heavy=bool(rng.integers(0, 4) == 0))
    _check_transpose(dev, inp, itype)


def _backward(dev, rng, i, seed):
    T, B, dims, rows, L = _shape(rng, 5, 300, 50, 1, 3000)
    pooling, mode = int(rng.integers(0, 2)), int(rng.integers(0, 4))
    print(f"[case] sweep bwd {i}: T={T} B={B} dims={dims} rows={rows} L={L} pool={pooling} "
          f"mode={mode}", flush=True)
    if mode == 0:  # unweighted, any run lengths
        inp = random_tbe(rng, T, B, dims, rows, L, dup_heavy=bool(rng.integers(0, 3) == 0))
        W = rng.uniform(-0.01, 0.01, size=sum(E * D for E, D in zip(rows, dims)))
        W = W.astype(np.float32)
        m1 = rng.uniform(0, 1e-4, size=sum(rows)).astype(np.float32)
        m1_off = np.concatenate([[0], np.cumsum(rows)[:-1]]).astype(np.int64)
        grad = rng.normal(0, 1e-2, size=(B, inp.total_D)).astype(np.float32)
        Wg, mg = _backward_gpu(dev, inp, W, m1, m1_off, grad, pooling, 0.01, 1e-8)
        W_exp, m_exp = orc.backward_rowwise_adagrad(
            W, weight_offsets(inp), inp.D_offsets, B, inp.hash_size_cumsum,
            inp.total_hash_size_bits, inp.indices, inp.offsets, pooling, grad, m1, m1_off, 0.01,
            1e-8, 0.0, 0, orc.info_B_num_bits(T, B))
        assert_reordered_adagrad_close(Wg, mg, W_exp, m_exp, W, m1, weight_offsets(inp), m1_off,
                                       inp, grad, pooling, 0.01, 1e-8)
        return
    # Runs stay short (at least 200 rows per table), where rtol 1e-5 holds.
    inp = random_tbe(rng, T, B, dims, [max(r, 200) for r in rows], min(L, 20))
    if mode == 1:
        _backward_case(dev, inp, pooling, weighted=True, seed=seed + i)
    elif mode == 2:
        _backward_case(dev, inp, pooling, wd=0.1, wd_mode=1, seed=seed + i)
    else:
        _backward_case(dev, inp, pooling, wd=0.05, wd_mode=2, seed=seed + i,
                       index_dtype=torch.int32)


@pytest.mark.parametrize("seed", [101, 202, 303, 404])
def test_random_sweep(dev, seed):
    rng = np.random.default_rng(seed)
    for i in range(ROUNDS):
        _forward(dev, rng, i)
        _transpose(dev, rng, i)
        _backward(dev, rng, i, seed)


SEQ_ROUNDS = 10


def _sequence_and_sparse(dev, rng, i):
    """One round: a sequence-lookup forward, an nbit sequence lookup, a
    sequence-lookup backward, a cumsum and a feature permute, each against the
    oracle (bit-exact; the backward at rtol 1e-5, 1e-4 on momentum when long
    runs reorder the sums)."""
    from nbit_helpers import build_weights
    from test_gpu_nobag import _backward_nobag, _forward_nobag, _nbit_nobag

    T = int(rng.integers(1, 6))
    B = int(rng.integers(1, 200))
    D = int(rng.choice([4, 8, 16, 36, 64, 128, 256, 512]))
    rows = [int(rng.integers(1, 3000)) for _ in range(T)]
    dup = bool(rng.integers(0, 3) == 0)
    itype = torch.int32 if rng.integers(0, 2) else torch.int64
    f16 = bool(rng.integers(0, 2))
    print(f"[case] sweep seq {i}: T={T} B={B} D={D} rows={rows} dup={dup} {itype} f16={f16}",
          flush=True)
    inp = random_tbe(rng, T, B, [D] * T, rows, int(rng.integers(0, 40)), dup_heavy=dup)
    W = rng.uniform(-0.5, 0.5, size=sum(E * D for E in rows)).astype(np.float32)
    Wd = torch.from_numpy(W).to(dev).to(torch.float16 if f16 else torch.float32)
    got = _forward_nobag(dev, Wd, inp, D, 0, itype)
    exp = orc.tbe_forward_nobag(Wd.cpu().numpy(), weight_offsets(inp), D, B, inp.indices,
                                inp.offsets)
    np.testing.assert_array_equal(got.cpu().numpy(), exp)

    Dq = int(rng.choice([8, 16, 32, 64, 128, 256]))
    tys = [int(rng.choice([orc.INT8, orc.INT4, orc.INT2, orc.FP16, orc.FP32, orc.FP8]))
           for _ in range(T)]
    inq = random_tbe(rng, T, B, [Dq] * T, rows, int(rng.integers(0, 30)))
    buf, w_off = build_weights(rng, tys, [Dq] * T, rows)
    out_dtype = int(rng.choice([0, 1, 5]))
    kind = {0: 0, 1: 1, 5: 2}[out_dtype]
    g = _nbit_nobag(dev, buf, w_off, tys, Dq, inq, out_dtype, itype).cpu()
    e = orc.nbit_forward_nobag(buf, w_off, tys, Dq, B, inq.indices, inq.offsets, out_kind=kind)
    g = g.view(torch.int16).numpy().view(np.uint16) if kind else g.numpy().view(np.uint32)
    np.testing.assert_array_equal(g, e.view(np.uint32) if kind == 0 else e.view(np.uint16))

    m1 = rng.uniform(0, 0.01, size=sum(rows)).astype(np.float32)
    m1_off = np.concatenate([[0], np.cumsum(rows)[:-1]]).astype(np.int64)
    grad = rng.normal(0, 0.01, size=(inp.N, D)).astype(np.float32)
    Wb, mb = torch.from_numpy(W).to(dev), torch.from_numpy(m1).to(dev)
    _backward_nobag(dev, Wb, mb, m1_off, inp, D, grad, 0.05, 1e-8, 0.0, 0, itype)
    W_exp, m_exp = orc.backward_rowwise_adagrad_nobag(
        W, weight_offsets(inp), D, B, inp.hash_size_cumsum, inp.total_hash_size_bits,
        inp.indices, inp.offsets, grad, m1, m1_off, 0.05, 1e-8)
    np.testing.assert_allclose(mb.cpu().numpy(), m_exp, rtol=1e-4 if dup else 1e-5, atol=0)
    np.testing.assert_allclose(Wb.cpu().numpy(), W_exp, rtol=1e-5, atol=1e-6 if dup else 1e-7)

    n = int(rng.choice([0, 1, 100, 8191, 8193, 50_000, 400_000]))
    ck = int(rng.integers(0, 3))
    cdt = np.int32 if rng.integers(0, 2) else np.int64
    x = rng.integers(-5, 60, n).astype(cdt)
    op = ("asynchronous_exclusive_cumsum", "asynchronous_inclusive_cumsum",
          "asynchronous_complete_cumsum")[ck]
    np.testing.assert_array_equal(getattr(torch.ops.fbgemm, op)(torch.from_numpy(x).to(dev)).cpu().numpy(),
                                  orc.cumsum(x, ck))

    Tp = int(rng.integers(1, 10))
    lengths = rng.integers(0, 20, (T, B))
    idx = rng.integers(0, 10**6, int(lengths.sum()))
    permute = rng.integers(0, T, Tp).astype(np.int32)
    el, ei, _ = orc.permute_2d_sparse_data(permute, lengths, idx)
    pl, pi, _ = torch.ops.fbgemm.permute_2D_sparse_data(
        torch.from_numpy(permute).to(dev), torch.from_numpy(lengths).to(dev),
        torch.from_numpy(idx).to(dev, itype))
    np.testing.assert_array_equal(pl.cpu().numpy(), el)
    np.testing.assert_array_equal(pi.cpu().numpy(), ei)


@pytest.mark.parametrize("seed", [11, 22])
def test_random_sweep_sequence_and_sparse(dev, seed):
    rng = np.random.default_rng(seed)
    for i in range(SEQ_ROUNDS):
        _sequence_and_sparse(dev, rng, i)
