"""Seeded random sweep over the TBE ops' argument space, against the oracle.

Each round draws one forward case (1-6 tables of widths 4..1024, 1-300 bags,
0-80 indices per bag, SUM/MEAN, per-sample weights or not, fp32 or fp16
weight rows, int32 or int64 indices; bit-exact), one transpose case (1-8
features of up to 200,000 rows; bit-exact over the whole run layout) and one
backward case (unweighted with any run lengths, under the reordering bound of
adagrad_bounds.py; or weighted, L2 or decoupled weight decay on rows of at
least 200, at rtol 1e-5).  A quarter of the cases draw their indices from
three rows per table, so long runs and repeated rows are common."""

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
