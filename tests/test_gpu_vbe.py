"""GPU parity of variable batch size per feature (VBE).

Expected values come from the dense oracle on the padded equivalent of each
case (every table padded to max_B bags with empty bags: same index order,
same per-row sums) mapped through an independent numpy construction of the
VBE layout (tests/tbe_helpers.VbeCase): metadata and forward bit-exact,
backward and per-sample-weight gradients at the dense path's tolerances."""

import numpy as np
import pytest
import torch

import oracle as orc
from tbe_helpers import VbeCase, weight_offsets

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-7

CASES = [
    # bs[t][r], dims, rows, max_L
    ([[3, 0, 2], [1, 4, 1]], [8, 4], [10, 20], 5),
    ([[40], [7], [0], [129]], [128, 64, 32, 256], [500, 70, 9, 3000], 12),   # one rank, an empty table
    ([[5, 9, 1, 30], [0, 0, 2, 2], [17, 3, 3, 3]], [36, 128, 4], [60, 2000, 11], 30),
    # several 3072-key sort tiles per feature segment, an empty feature between
    ([[900, 300], [0, 0], [1200, 40]], [64, 32, 128], [5000, 40, 300], 12),
]


def _meta_gpu(dev, c: VbeCase, nb: int):
    return torch.ops.fbgemm.generate_vbe_metadata(
        torch.from_numpy(c.B_offsets).to(dev), torch.from_numpy(c.rpf).to(dev),
        torch.from_numpy(c.out_ofr).to(dev), torch.from_numpy(c.dense.D_offsets).to(dev), -1,
        False, max(max(r) for r in c.bs), nb, c.total_B)


@pytest.mark.parametrize("bs,dims,rows,max_L", CASES)
def test_generate_vbe_metadata(dev, bs, dims, rows, max_L):
    print(f"[case] vbe metadata bs={bs}", flush=True)
    c = VbeCase(np.random.default_rng(1), bs, dims, rows, max_L)
    nb = orc.info_B_num_bits(c.T, c.max_B)
    row_out, btm = _meta_gpu(dev, c, nb)
    assert np.array_equal(row_out.cpu().numpy(), c.row_out)
    assert np.array_equal(btm.cpu().numpy(), c.b_t_map(nb))


def _forward(dev, c, W, pooling, iw, nb, idt=torch.int64, out_dtype=0):
    row_out, btm = _meta_gpu(dev, c, nb)
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(c.T, dtype=torch.int32, device=dev)
    common = (W, empty, empty, pl, torch.from_numpy(weight_offsets(c.dense)).to(dev),
              torch.from_numpy(c.dense.D_offsets).to(dev), c.dense.total_D, max(c.dims),
              torch.from_numpy(c.indices).to(dev, idt), torch.from_numpy(c.offsets).to(dev, idt),
              pooling)
    tail = (torch.zeros(0, dtype=torch.int32, device=dev), empty, out_dtype, row_out, btm,
            c.output_size, nb, (1 << nb) - 1, False)
    if iw is None:
        return torch.ops.fbgemm.split_embedding_codegen_forward_unweighted_vbe_cuda(*common, *tail)
    return torch.ops.fbgemm.split_embedding_codegen_forward_weighted_vbe_cuda(
        *common, torch.from_numpy(iw).to(dev), *tail)


@pytest.mark.parametrize("bs,dims,rows,max_L", CASES)
@pytest.mark.parametrize("pooling", [0, 1])
@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("w16", [False, True])
def test_vbe_forward(dev, bs, dims, rows, max_L, pooling, weighted, w16):
    print(f"[case] vbe fwd bs={bs} pool={pooling} w={weighted} fp16w={w16}", flush=True)
    rng = np.random.default_rng(2)
    c = VbeCase(rng, bs, dims, rows, max_L)
    W = rng.uniform(-1, 1, size=sum(E * D for E, D in zip(rows, dims))).astype(
        np.float16 if w16 else np.float32)
    iw = rng.uniform(0, 2, c.N).astype(np.float32) if weighted else None
    exp = c.dense_to_flat(orc.tbe_forward_f32(W, weight_offsets(c.dense), c.dense.D_offsets,
                                              c.max_B, c.indices, c.dense.offsets, pooling, iw))
    nb = orc.info_B_num_bits(c.T, c.max_B)
    for idt in (torch.int64, torch.int32):
        got = _forward(dev, c, torch.from_numpy(W).to(dev), pooling, iw, nb, idt).cpu().numpy()
        assert got.shape == (c.output_size,)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_vbe_forward_uniform_batch_equals_dense(dev):
    """One rank, the same batch for every feature: the flat VBE output is the
    dense [B, total_D] output taken feature block by feature block."""
    print("[case] vbe uniform batch == dense", flush=True)
    rng = np.random.default_rng(3)
    c = VbeCase(rng, [[16], [16], [16]], [8, 64, 128], [100, 50, 80], 9)
    W = rng.uniform(-1, 1, size=sum(E * D for E, D in zip(c.rows, c.dims))).astype(np.float32)
    nb = orc.info_B_num_bits(c.T, c.max_B)
    got = _forward(dev, c, torch.from_numpy(W).to(dev), 0, None, nb).cpu().numpy()
    dense = torch.ops.fbgemm.split_embedding_codegen_forward_unweighted_cuda(
        torch.from_numpy(W).to(dev), torch.zeros(0, device=dev), torch.zeros(0, device=dev),
        torch.zeros(3, dtype=torch.int32, device=dev),
        torch.from_numpy(weight_offsets(c.dense)).to(dev),
        torch.from_numpy(c.dense.D_offsets).to(dev), c.dense.total_D, 128,
        torch.from_numpy(c.indices).to(dev), torch.from_numpy(c.offsets).to(dev), 0,
        torch.zeros(0, dtype=torch.int32, device=dev), torch.zeros(0, device=dev), 0,
        False).cpu().numpy()
    blocks = [dense[:, c.dense.D_offsets[t]: c.dense.D_offsets[t + 1]].reshape(-1)
              for t in range(3)]
    assert np.array_equal(got, np.concatenate(blocks))


@pytest.mark.parametrize("bs,dims,rows,max_L", CASES[1:])
def test_vbe_transpose(dev, bs, dims, rows, max_L):
    """Sorted layout with the b_t map equals the dense-padded one (same info
    words: b is the feature-global sample index in both)."""
    print(f"[case] vbe transpose bs={bs}", flush=True)
    c = VbeCase(np.random.default_rng(4), bs, dims, rows, max_L)
    nb = orc.info_B_num_bits(c.T, c.max_B)
    exp = orc.transpose_embedding_input(c.dense.hash_size_cumsum, c.max_B, nb,
                                        c.dense.total_hash_size_bits, c.indices,
                                        c.dense.offsets)
    _, btm = _meta_gpu(dev, c, nb)
    lin, srt, infos, run, lengths, num_runs, cum = torch.ops.fbgemm.transpose_embedding_input(
        torch.from_numpy(c.dense.hash_size_cumsum).to(dev), c.dense.total_hash_size_bits,
        torch.from_numpy(c.indices).to(dev), torch.from_numpy(c.offsets).to(dev), False, btm, nb)
    r = int(num_runs.item())
    assert r == exp["num_runs"]
    np.testing.assert_array_equal(lin.cpu().numpy(), exp["linear_indices"])
    np.testing.assert_array_equal(srt.cpu().numpy(), exp["sorted_linear_indices"])
    np.testing.assert_array_equal(infos.cpu().numpy(), exp["infos_sorted"])
    np.testing.assert_array_equal(run.cpu().numpy()[:r], exp["run"])
    np.testing.assert_array_equal(cum.cpu().numpy()[: r + 1], exp["cumulative_run_lengths"])


@pytest.mark.parametrize("bs,dims,rows,max_L", CASES)
@pytest.mark.parametrize("pooling", [0, 1])
@pytest.mark.parametrize("weighted", [False, True])
def test_vbe_backward(dev, bs, dims, rows, max_L, pooling, weighted):
    print(f"[case] vbe backward bs={bs} pool={pooling} w={weighted}", flush=True)
    rng = np.random.default_rng(5)
    c = VbeCase(rng, bs, dims, rows, max_L)
    W = rng.uniform(-0.5, 0.5, size=sum(E * D for E, D in zip(rows, dims))).astype(np.float32)
    m1 = rng.uniform(0, 1e-3, size=sum(rows)).astype(np.float32)
    m1_off = np.concatenate([[0], np.cumsum(rows)[:-1]]).astype(np.int64)
    gflat = rng.normal(0, 0.1, size=c.output_size).astype(np.float32)
    iw = rng.uniform(-1.5, 1.5, c.N).astype(np.float32) if weighted else None
    nb = orc.info_B_num_bits(c.T, c.max_B)
    W_exp, m_exp = orc.backward_rowwise_adagrad(
        W, weight_offsets(c.dense), c.dense.D_offsets, c.max_B, c.dense.hash_size_cumsum,
        c.dense.total_hash_size_bits, c.indices, c.dense.offsets, pooling,
        c.flat_to_dense(gflat), m1, m1_off, 0.05, 1e-6, 0.0, 0, nb, indice_weights=iw)
    row_out, btm = _meta_gpu(dev, c, nb)
    Wd, m1d = torch.from_numpy(W).to(dev), torch.from_numpy(m1).to(dev)
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(c.T, dtype=torch.int32, device=dev)
    head = (torch.from_numpy(gflat).to(dev), Wd, empty, empty, pl,
            torch.from_numpy(weight_offsets(c.dense)).to(dev),
            torch.from_numpy(c.dense.D_offsets).to(dev), max(dims),
            torch.from_numpy(c.dense.hash_size_cumsum).to(dev), c.dense.total_hash_size_bits,
            torch.from_numpy(c.indices).to(dev), torch.from_numpy(c.offsets).to(dev), pooling)
    mid = (torch.zeros(0, dtype=torch.int32, device=dev), 0, 0, False, nb, (1 << nb) - 1,
           torch.from_numpy(c.B_offsets).to(dev), row_out, btm)
    tail = (m1d, empty, pl, torch.from_numpy(m1_off).to(dev), 1e-6, 0.05, 0.0, 0, 0.0)
    if weighted:
        torch.ops.fbgemm.split_embedding_backward_codegen_rowwise_adagrad_weighted_exact_vbe_cuda(
            *head, torch.from_numpy(iw).to(dev), *mid, *tail)
    else:
        torch.ops.fbgemm.split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_vbe_cuda(
            *head, *mid, *tail)
    np.testing.assert_allclose(m1d.cpu().numpy(), m_exp, rtol=RTOL, atol=0)
    Wg = Wd.cpu().numpy()
    np.testing.assert_allclose(Wg, W_exp, rtol=RTOL, atol=ATOL)
    untouched = W_exp == W
    assert np.array_equal(Wg[untouched], W[untouched])


@pytest.mark.parametrize("pooling", [0, 1])
def test_vbe_grad_indice_weights(dev, pooling):
    print(f"[case] vbe grad_indice_weights pool={pooling}", flush=True)
    rng = np.random.default_rng(6)
    c = VbeCase(rng, CASES[2][0], CASES[2][1], CASES[2][2], CASES[2][3])
    W = rng.uniform(-1, 1, size=sum(E * D for E, D in zip(c.rows, c.dims))).astype(np.float32)
    gflat = rng.normal(0, 1, size=c.output_size).astype(np.float32)
    frg = np.array([1, 0, 1], np.int32)
    gd = c.flat_to_dense(gflat)
    exp = orc.grad_indice_weights(gd, W, weight_offsets(c.dense), c.dense.D_offsets, c.max_B,
                                  c.indices, c.dense.offsets, pooling, frg)
    mag = orc.grad_indice_weights(np.abs(gd), np.abs(W), weight_offsets(c.dense),
                                  c.dense.D_offsets, c.max_B, c.indices, c.dense.offsets, pooling)
    nb = orc.info_B_num_bits(c.T, c.max_B)
    row_out, btm = _meta_gpu(dev, c, nb)
    empty = torch.zeros(0, device=dev)
    got = torch.ops.fbgemm.split_embedding_codegen_grad_indice_weights_vbe_cuda(
        torch.from_numpy(gflat).to(dev), torch.from_numpy(W).to(dev), empty, empty,
        torch.zeros(c.T, dtype=torch.int32, device=dev),
        torch.from_numpy(weight_offsets(c.dense)).to(dev),
        torch.from_numpy(c.dense.D_offsets).to(dev), max(c.dims),
        torch.from_numpy(c.indices).to(dev), torch.from_numpy(c.offsets).to(dev),
        torch.zeros(0, dtype=torch.int32, device=dev), torch.from_numpy(frg).to(dev), row_out,
        btm, nb, (1 << nb) - 1, pooling).cpu().numpy()
    assert np.all(np.abs(got - exp) <= 1e-5 * mag + 1e-30)


def _bounds_brute_vbe(rows, B_offsets, idx, off, mode):
    """The bounds-check contract with the table of bag i given by B_offsets."""
    idx, off = [int(x) for x in idx], [int(x) for x in off]
    N = len(idx)
    rep, run = [], 0
    for o in off:
        run = max(run, min(max(o, 0), N))
        rep.append(run)
    bad, out_idx = 0, list(idx)
    for bag in range(len(off) - 1):
        t = int(np.searchsorted(B_offsets, bag, side="right")) - 1
        for l in range(rep[bag], rep[bag + 1]):
            if not (0 <= idx[l] < rows[t]):
                bad += 1
                if mode != 0:
                    out_idx[l] = 0
    bad += sum(1 for a, b in zip(rep, off) if a != b)
    return (out_idx if mode != 0 else idx), (rep if mode != 0 else off), bad


@pytest.mark.parametrize("mode", [1, 2])
def test_vbe_bounds_check(dev, mode):
    print(f"[case] vbe bounds check mode={mode}", flush=True)
    rng = np.random.default_rng(7)
    c = VbeCase(rng, CASES[2][0], CASES[2][1], CASES[2][2], CASES[2][3])
    idx = c.indices.copy()
    bad_pos = rng.choice(c.N, 25, replace=False)
    idx[bad_pos] = rng.choice([-3, 10_000, 2**40], 25)
    off = c.offsets.copy()
    off[5] = off[4] - 2  # overlapping bag
    off[-3] = c.N + 7    # past the end
    ei, eo, ebad = _bounds_brute_vbe(c.rows, c.B_offsets, idx, off, mode)
    it, ot = torch.from_numpy(idx).to(dev), torch.from_numpy(off).to(dev)
    warning = torch.zeros(1, dtype=torch.int64, device=dev)
    torch.ops.fbgemm.bounds_check_indices(
        torch.tensor(c.rows, dtype=torch.int64, device=dev), it, ot, mode, warning, None,
        torch.from_numpy(c.B_offsets).to(dev), c.max_B)
    assert it.cpu().tolist() == ei and ot.cpu().tolist() == eo
    assert int(warning.item()) == ebad


@pytest.mark.parametrize("weighted", [False, True])
def test_module_vbe_training_step(dev, weighted):
    """batch_size_per_feature_per_rank through the training module: flat
    forward output, fused update and per-sample-weight gradient vs the dense
    oracle on the padded equivalent."""
    print(f"[case] module vbe training step weighted={weighted}", flush=True)
    from mx_fbgemm import ComputeDevice, EmbeddingLocation, PoolingMode
    from mx_fbgemm.split_table_batched_embeddings_ops_training import (
        SplitTableBatchedEmbeddingBagsCodegen,
    )

    bs, dims, rows = [[4, 7], [0, 3], [12, 1]], [64, 128, 32], [300, 200, 90]
    tbe = SplitTableBatchedEmbeddingBagsCodegen(
        [(E, D, EmbeddingLocation.DEVICE, ComputeDevice.CUDA) for E, D in zip(rows, dims)],
        pooling_mode=PoolingMode.MEAN, learning_rate=0.05, eps=1e-6, device=dev)
    rng = np.random.default_rng(8)
    c = VbeCase(rng, bs, dims, rows, 10)
    iw = rng.uniform(0.5, 1.5, c.N).astype(np.float32) if weighted else None
    psw = torch.from_numpy(iw).to(dev).requires_grad_() if weighted else None
    W0 = tbe.weights_dev.detach().cpu().numpy().copy()
    out = tbe(torch.from_numpy(c.indices).to(dev), torch.from_numpy(c.offsets).to(dev), psw,
              batch_size_per_feature_per_rank=bs)
    exp = c.dense_to_flat(orc.tbe_forward_f32(W0, weight_offsets(c.dense), c.dense.D_offsets,
                                              c.max_B, c.indices, c.dense.offsets, 1, iw))
    assert out.shape == (c.output_size,)
    assert np.array_equal(out.detach().cpu().numpy(), exp)
    gflat = rng.normal(0, 1, size=c.output_size).astype(np.float32)
    out.backward(torch.from_numpy(gflat).to(dev))
    nb = orc.info_B_num_bits(c.T, c.max_B)
    gd = c.flat_to_dense(gflat)
    W_exp, m_exp = orc.backward_rowwise_adagrad(
        W0, weight_offsets(c.dense), c.dense.D_offsets, c.max_B, c.dense.hash_size_cumsum,
        c.dense.total_hash_size_bits, c.indices, c.dense.offsets, 1, gd,
        np.zeros(sum(rows), np.float32), np.concatenate([[0], np.cumsum(rows)[:-1]]), 0.05,
        1e-6, 0.0, 0, nb, indice_weights=iw)
    np.testing.assert_allclose(tbe.weights_dev.detach().cpu().numpy(), W_exp, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(tbe.momentum1_dev.cpu().numpy(), m_exp, rtol=RTOL, atol=0)
    if weighted:
        giw = orc.grad_indice_weights(gd, W0, weight_offsets(c.dense), c.dense.D_offsets,
                                      c.max_B, c.indices, c.dense.offsets, 1)
        mag = orc.grad_indice_weights(np.abs(gd), np.abs(W0), weight_offsets(c.dense),
                                      c.dense.D_offsets, c.max_B, c.indices, c.dense.offsets, 1)
        assert np.all(np.abs(psw.grad.cpu().numpy() - giw) <= 1e-5 * mag + 1e-30)
