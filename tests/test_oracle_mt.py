"""The multithreaded C++ restatement of the backward (oracle/backward_mt.cpp,
the backward's CPU baseline) is bit-identical to the single-threaded C
restatement it follows, for any thread count: unweighted and weighted, SUM
and MEAN, the three weight-decay modes, features sharing a table, long runs
and empty bags; at config-3 shapes too (reduced batch)."""

import numpy as np
import pytest

import oracle as orc
from mx_fbgemm import bench_inputs
from tbe_helpers import random_tbe, weight_offsets


def _both(inp, W, m1, m1_off, grad, pooling, lr, eps, wd=0.0, wd_mode=0, iw=None, w_off=None,
          hsc=None, bits=None, nthreads=(1, 3, 8)):
    w_off = weight_offsets(inp) if w_off is None else w_off
    hsc = inp.hash_size_cumsum if hsc is None else hsc
    bits = inp.total_hash_size_bits if bits is None else bits
    exp = orc.backward_rowwise_adagrad(W, w_off, inp.D_offsets, inp.B, hsc, bits, inp.indices,
                                       inp.offsets, pooling, grad, m1, m1_off, lr, eps, wd,
                                       wd_mode, orc.info_B_num_bits(inp.T, inp.B),
                                       indice_weights=iw)
    for n in nthreads:
        got = orc.backward_rowwise_adagrad_mt(W, w_off, inp.D_offsets, inp.B, hsc, bits,
                                              inp.indices, inp.offsets, pooling, grad, m1, m1_off,
                                              lr, eps, wd, wd_mode, indice_weights=iw, nthreads=n)
        assert np.array_equal(got[0].view(np.uint32), exp[0].view(np.uint32)), f"{n} threads: W"
        assert np.array_equal(got[1].view(np.uint32), exp[1].view(np.uint32)), f"{n} threads: h"


@pytest.mark.parametrize("pooling", [0, 1])
@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("wd_mode,wd", [(0, 0.0), (1, 0.01), (2, 0.02)])
def test_mt_equals_single_thread(pooling, weighted, wd_mode, wd):
    rng = np.random.default_rng(10 * pooling + 3 * weighted + wd_mode)
    inp = random_tbe(rng, 4, 97, [8, 64, 132, 4], [50, 3, 7000, 1], 30, empty_frac=0.15)
    W = rng.uniform(-0.05, 0.05, size=sum(E * D for E, D in zip(inp.E, inp.D))).astype(np.float32)
    m1 = rng.uniform(0, 1e-3, size=sum(inp.E)).astype(np.float32)
    m1_off = np.concatenate([[0], np.cumsum(inp.E)[:-1]]).astype(np.int64)
    grad = rng.normal(0, 1e-2, size=(inp.B, inp.total_D)).astype(np.float32)
    iw = rng.uniform(-2, 2, inp.N).astype(np.float32) if weighted else None
    _both(inp, W, m1, m1_off, grad, pooling, 0.05, 1e-8, wd, wd_mode, iw)


def test_mt_shared_tables():
    rng = np.random.default_rng(5)
    ftm, rows, dims = [0, 1, 0], [30, 20], [16, 8]
    inp = random_tbe(rng, 3, 40, [dims[t] for t in ftm], [rows[t] for t in ftm], 9)
    t_off = np.array([0, rows[0] * dims[0]], np.int64)
    t_hsc = np.array([0, rows[0]], np.int64)
    hsc = np.concatenate([t_hsc[ftm], [sum(rows)]]).astype(np.int64)
    W = rng.uniform(-0.5, 0.5, size=sum(E * D for E, D in zip(rows, dims))).astype(np.float32)
    m1 = rng.uniform(0, 0.01, size=sum(rows)).astype(np.float32)
    grad = rng.normal(0, 1, size=(inp.B, inp.total_D)).astype(np.float32)
    _both(inp, W, m1, t_hsc[ftm], grad, 1, 0.1, 1e-6, w_off=t_off[ftm], hsc=hsc, bits=6)


def test_mt_config3_shapes():
    """Config-3 batch (8 features, B = 4096, Zipf(1.05) runs of up to
    thousands) with each table cut to the rows the batch touches, renumbered
    in order (the same runs in the same order, without 4 GB of weights)."""
    full = bench_inputs.config2()
    B = full.B
    idx = np.empty_like(full.indices)
    rows = []
    for t in range(full.T):
        s, e = int(full.offsets[t * B]), int(full.offsets[(t + 1) * B])
        u, inv = np.unique(full.indices[s:e], return_inverse=True)
        idx[s:e] = inv
        rows.append(int(u.size))
    inp = bench_inputs.TbeInput(T=full.T, E=rows, D=full.D, B=B, indices=idx,
                                offsets=full.offsets)
    rng = np.random.default_rng(3)
    W = rng.uniform(-0.01, 0.01, size=sum(E * D for E, D in zip(inp.E, inp.D))).astype(np.float32)
    m1 = np.zeros(sum(inp.E), np.float32)
    m1_off = np.concatenate([[0], np.cumsum(inp.E)[:-1]]).astype(np.int64)
    grad = rng.normal(0, 1e-2, size=(inp.B, inp.total_D)).astype(np.float32)
    _both(inp, W, m1, m1_off, grad, 0, 0.01, 1e-8, nthreads=(8,))


def test_mt_empty_batch():
    inp = bench_inputs.TbeInput(T=2, E=[5, 6], D=[4, 4], B=3, indices=np.zeros(0, np.int64),
                                offsets=np.zeros(7, np.int64))
    W = np.ones(44, np.float32)
    m1 = np.zeros(11, np.float32)
    grad = np.ones((3, 8), np.float32)
    _both(inp, W, m1, np.array([0, 5], np.int64), grad, 0, 0.1, 1e-8)
