"""Zero-size batches through every op: no indices (all bags empty) and no
bags at all.  Outputs have the documented shapes and values (pooled zeros,
untouched weights and momentum, zero runs, nothing repaired)."""

import numpy as np
import pytest
import torch

import oracle as orc
from nbit_helpers import build_weights, nbit_forward_gpu
from tbe_helpers import tbe_forward_gpu, weight_offsets

from mx_fbgemm import bench_inputs

pytestmark = pytest.mark.gpu


def _batch(T, B, dims, rows):
    off = np.zeros(T * B + 1, dtype=np.int64)
    return bench_inputs.TbeInput(T=T, E=list(rows), D=list(dims), B=B,
                                 indices=np.zeros(0, dtype=np.int64), offsets=off)


@pytest.mark.parametrize("B", [0, 5])
@pytest.mark.parametrize("pooling", [0, 1])
def test_forward_no_indices(dev, B, pooling):
    print(f"[case] empty forward B={B} pool={pooling}", flush=True)
    inp = _batch(2, B, [8, 16], [4, 4])
    W = torch.ones(sum(E * D for E, D in zip(inp.E, inp.D)), device=dev)
    out = tbe_forward_gpu(dev, W, inp, pooling)
    assert tuple(out.shape) == (B, 24)
    assert not out.any()


@pytest.mark.parametrize("B", [0, 5])
def test_backward_no_indices(dev, B):
    """No indices: weights and momentum untouched; transpose gives no runs."""
    print(f"[case] empty backward B={B}", flush=True)
    inp = _batch(2, B, [8, 16], [4, 4])
    nb = orc.info_B_num_bits(inp.T, max(B, 1))
    lin, srt, infos, run, lengths, num_runs, cum = torch.ops.fbgemm.transpose_embedding_input(
        torch.from_numpy(inp.hash_size_cumsum).to(dev), inp.total_hash_size_bits,
        torch.zeros(0, dtype=torch.int64, device=dev), torch.from_numpy(inp.offsets).to(dev),
        False, None, nb)
    assert int(num_runs.item()) == 0 and srt.numel() == 0
    W = torch.full((sum(E * D for E, D in zip(inp.E, inp.D)),), 0.5, device=dev)
    m1 = torch.full((sum(inp.E),), 0.25, device=dev)
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(inp.T, dtype=torch.int32, device=dev)
    torch.ops.fbgemm.split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_cuda(
        torch.zeros((B, inp.total_D), device=dev), W, empty, empty, pl,
        torch.from_numpy(weight_offsets(inp)).to(dev), torch.from_numpy(inp.D_offsets).to(dev),
        max(inp.D), torch.from_numpy(inp.hash_size_cumsum).to(dev), inp.total_hash_size_bits,
        torch.zeros(0, dtype=torch.int64, device=dev), torch.from_numpy(inp.offsets).to(dev), 0,
        torch.zeros(0, dtype=torch.int32, device=dev), 0, 0, False, m1, empty, pl,
        torch.tensor([0, 4], dtype=torch.int64, device=dev), 1e-8, 0.01, 0.0, 0, 0.0)
    assert bool((W == 0.5).all()) and bool((m1 == 0.25).all())


def test_grad_indice_weights_no_indices(dev):
    print("[case] empty grad_indice_weights", flush=True)
    inp = _batch(2, 3, [8, 16], [4, 4])
    empty = torch.zeros(0, device=dev)
    got = torch.ops.fbgemm.split_embedding_codegen_grad_indice_weights_cuda(
        torch.ones((3, inp.total_D), device=dev),
        torch.ones(sum(E * D for E, D in zip(inp.E, inp.D)), device=dev), empty, empty,
        torch.zeros(2, dtype=torch.int32, device=dev),
        torch.from_numpy(weight_offsets(inp)).to(dev), torch.from_numpy(inp.D_offsets).to(dev), 16,
        torch.zeros(0, dtype=torch.int64, device=dev), torch.from_numpy(inp.offsets).to(dev),
        torch.zeros(0, dtype=torch.int32, device=dev), None, 0)
    assert got.numel() == 0


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_bounds_check_no_indices(dev, mode):
    """N = 0: every offset must repair to 0 (counted, except under FATAL,
    which raises on any); a clean empty batch passes every mode."""
    print(f"[case] empty bounds check mode={mode}", flush=True)
    rows = torch.tensor([4, 4], dtype=torch.int64, device=dev)
    idx = torch.zeros(0, dtype=torch.int64, device=dev)
    clean = torch.zeros(7, dtype=torch.int64, device=dev)
    warn = torch.zeros(1, dtype=torch.int64, device=dev)
    torch.ops.fbgemm.bounds_check_indices(rows, idx, clean, mode, warn)
    assert int(warn.item()) == 0 and not clean.any()
    bad = torch.tensor([0, 3, -1, 2, 0, 5, 9], dtype=torch.int64, device=dev)
    exp_idx, exp_off, exp_n = orc.bounds_check_indices(np.array([4, 4]), np.zeros(0, np.int64),
                                                       bad.cpu().numpy(), mode)
    if mode == 0:
        with pytest.raises(RuntimeError, match="out-of-range"):
            torch.ops.fbgemm.bounds_check_indices(rows, idx, bad, mode, warn)
        return
    torch.ops.fbgemm.bounds_check_indices(rows, idx, bad, mode, warn)
    np.testing.assert_array_equal(bad.cpu().numpy(), exp_off)
    assert not bad.any() and int(warn.item()) == exp_n == 5


@pytest.mark.parametrize("B", [0, 3])
def test_nbit_no_indices(dev, B):
    print(f"[case] empty nbit B={B}", flush=True)
    rng = np.random.default_rng(1)
    tys, dims, rows = [orc.INT8, orc.INT4, orc.FP16], [16, 32, 8], [5, 5, 5]
    buf, w_off = build_weights(rng, tys, dims, rows)
    for pooling in (0, 1):
        got = nbit_forward_gpu(dev, torch.from_numpy(buf).to(dev), w_off, tys, dims,
                               np.zeros(0, np.int64), np.zeros(3 * B + 1, np.int64), pooling)
        assert tuple(got.shape) == (B, sum(dims)) and not got.any()


def test_jagged_no_rows_and_no_values(dev):
    """B = 0 rows, and rows that are all empty (total_L = 0)."""
    print("[case] empty jagged", flush=True)
    for off in ([0], [0, 0, 0]):
        o = torch.tensor(off, dtype=torch.int64, device=dev)
        v = torch.zeros((0, 8), device=dev)
        dense = torch.ops.fbgemm.jagged_to_padded_dense(v, [o], [4], 1.5)
        assert tuple(dense.shape) == (len(off) - 1, 4, 8) and bool((dense == 1.5).all())
        back, _ = torch.ops.fbgemm.dense_to_jagged(dense, [o], 0)
        assert tuple(back.shape) == (0, 8)
        s, _ = torch.ops.fbgemm.jagged_dense_elementwise_add_jagged_output(v, [o], dense)
        assert tuple(s.shape) == (0, 8)


@pytest.mark.parametrize("weighted", [False, True])
def test_module_step_no_indices(dev, weighted):
    """A training step of the TBE module over a batch with no indices: the
    pooled output is zero, loss.backward() leaves weights and momentum as
    they were, and the per-sample-weight gradient is empty."""
    print(f"[case] empty module step weighted={weighted}", flush=True)
    from mx_fbgemm import ComputeDevice, EmbeddingLocation, PoolingMode
    from mx_fbgemm.split_table_batched_embeddings_ops_training import (
        SplitTableBatchedEmbeddingBagsCodegen,
    )

    specs = [(50, 32, EmbeddingLocation.DEVICE, ComputeDevice.CUDA),
             (20, 64, EmbeddingLocation.DEVICE, ComputeDevice.CUDA)]
    tbe = SplitTableBatchedEmbeddingBagsCodegen(specs, pooling_mode=PoolingMode.SUM,
                                                learning_rate=0.05, eps=1e-6, device=dev)
    W0 = tbe.weights_dev.detach().clone()
    idx = torch.zeros(0, dtype=torch.int64, device=dev)
    off = torch.zeros(2 * 4 + 1, dtype=torch.int64, device=dev)
    psw = torch.zeros(0, device=dev, requires_grad=True) if weighted else None
    out = tbe(idx, off, per_sample_weights=psw)
    assert tuple(out.shape) == (4, 96) and not out.detach().any()
    out.backward(torch.ones_like(out))
    assert torch.equal(tbe.weights_dev.detach(), W0)
    assert not tbe.momentum1_dev.any()
    if weighted:
        assert psw.grad is not None and psw.grad.numel() == 0
