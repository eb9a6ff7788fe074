"""GPU parity of the sequence lookups (PoolingMode NONE) against the oracle:
the training forward and the nbit lookup bit-exact, the nobag transpose
bit-exact, the nobag rowwise-Adagrad backward at rtol 1e-5 with untouched
rows bit-identical, and the module / autograd paths that call them."""

import numpy as np
import pytest
import torch

import oracle as orc
from mx_fbgemm import ComputeDevice, EmbeddingLocation, PoolingMode, SparseType, bench_inputs
from mx_fbgemm.split_table_batched_embeddings_ops_inference import (
    IntNBitTableBatchedEmbeddingBagsCodegen,
)
from mx_fbgemm.split_table_batched_embeddings_ops_training import (
    SplitTableBatchedEmbeddingBagsCodegen,
)
from nbit_helpers import build_weights
from tbe_helpers import random_tbe, weight_offsets

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-7


def _forward_nobag(dev, W, inp, D, out_dtype, index_dtype):
    empty = torch.zeros(0, device=dev)
    return torch.ops.fbgemm.split_embedding_nobag_codegen_forward_unweighted_cuda(
        W, empty, empty, torch.zeros(inp.T, dtype=torch.int32, device=dev),
        torch.from_numpy(weight_offsets(inp)).to(dev), D,
        torch.from_numpy(inp.indices).to(dev, index_dtype),
        torch.from_numpy(inp.offsets).to(dev, index_dtype),
        torch.zeros(0, dtype=torch.int32, device=dev), empty, out_dtype, False)


@pytest.mark.parametrize("D", [4, 16, 64, 128, 200, 512, 1024])
@pytest.mark.parametrize("wdtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("out_f16", [False, True])
@pytest.mark.parametrize("index_dtype", [torch.int64, torch.int32])
def test_forward_nobag(dev, D, wdtype, out_f16, index_dtype):
    print(f"[case] nobag forward D={D} w={wdtype} f16out={out_f16} idx={index_dtype}", flush=True)
    rng = np.random.default_rng(D + 3 * out_f16)
    rows = [37, 5, 60]
    inp = random_tbe(rng, 3, 21, [D] * 3, rows, 30, empty_frac=0.2)
    W = rng.uniform(-1, 1, size=sum(E * D for E in rows)).astype(np.float32)
    Wd = torch.from_numpy(W).to(dev).to(wdtype)
    got = _forward_nobag(dev, Wd, inp, D, 1 if out_f16 else 0, index_dtype)
    assert got.shape == (inp.N, D)
    exp = orc.tbe_forward_nobag(Wd.cpu().numpy(), weight_offsets(inp), D, inp.B, inp.indices,
                                inp.offsets)
    if out_f16:
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint16),
                                      exp.astype(np.float16).view(np.uint16))
    else:
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), exp.view(np.uint32))


def test_forward_nobag_many_tables(dev):
    """More tables than the kernel stages in LDS (positions searched in memory)."""
    print("[case] nobag forward T=1100", flush=True)
    rng = np.random.default_rng(8)
    T, D = 1100, 8
    rows = [int(x) for x in rng.integers(1, 6, T)]
    inp = random_tbe(rng, T, 2, [D] * T, rows, 4, empty_frac=0.3)
    W = rng.uniform(-1, 1, size=sum(E * D for E in rows)).astype(np.float32)
    got = _forward_nobag(dev, torch.from_numpy(W).to(dev), inp, D, 0, torch.int64)
    exp = orc.tbe_forward_nobag(W, weight_offsets(inp), D, inp.B, inp.indices, inp.offsets)
    np.testing.assert_array_equal(got.cpu().numpy(), exp)


def _nbit_nobag(dev, buf, w_off, tys, D, inp, out_dtype, index_dtype=torch.int64, maxima=None,
                dims=None):
    T = len(tys)
    dims = [D] * T if dims is None else dims
    if maxima is None:
        def m(ty):
            return D if ty in tys else 0
        maxima = [m(orc.INT2), m(orc.INT4), m(orc.INT8), m(orc.FP16), m(orc.FP32), m(orc.FP8)]
    D_off = np.concatenate([[0], np.cumsum(dims)]).astype(np.int32)
    empty = torch.zeros(0, dtype=torch.uint8, device=dev)
    return torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function(
        torch.from_numpy(buf).to(dev), empty, torch.zeros(T, dtype=torch.int32, device=dev),
        torch.as_tensor(w_off, device=dev), torch.as_tensor(np.asarray(tys, np.uint8), device=dev),
        torch.as_tensor(D_off, device=dev), int(D_off[-1]), *maxima[:5],
        torch.from_numpy(inp.indices).to(dev, index_dtype),
        torch.from_numpy(inp.offsets).to(dev, index_dtype), int(PoolingMode.NONE), None,
        out_dtype, None, None, 16, maxima[5], 4, 7)


ALL_TYPES = [orc.INT8, orc.INT4, orc.INT2, orc.FP16, orc.FP32, orc.FP8]


@pytest.mark.parametrize("ty", ALL_TYPES)
@pytest.mark.parametrize("out_dtype", [0, 1, 5])
@pytest.mark.parametrize("D", [8, 32, 128, 136, 1024])
def test_nbit_nobag(dev, ty, out_dtype, D):
    print(f"[case] nbit nobag ty={ty} out={out_dtype} D={D}", flush=True)
    rng = np.random.default_rng(ty * 31 + D + out_dtype)
    rows = [33, 7, 50]
    inp = random_tbe(rng, 3, 19, [D] * 3, rows, 25, empty_frac=0.2)
    tys = [ty] * 3
    buf, w_off = build_weights(rng, tys, [D] * 3, rows)
    kind = {0: 0, 1: 1, 5: 2}[out_dtype]
    got = _nbit_nobag(dev, buf, w_off, tys, D, inp, out_dtype, torch.int32 if D == 32 else
                      torch.int64)
    exp = orc.nbit_forward_nobag(buf, w_off, tys, D, inp.B, inp.indices, inp.offsets,
                                 out_kind=kind)
    assert got.shape == (inp.N, D)
    g = got.cpu()
    g = g.view(torch.int16).numpy().view(np.uint16) if kind else g.numpy().view(np.uint32)
    np.testing.assert_array_equal(g, exp.view(np.uint32) if kind == 0 else exp.view(np.uint16))


def test_nbit_nobag_mixed_types(dev):
    """Tables of all six types in one call (one launch per type)."""
    print("[case] nbit nobag mixed types", flush=True)
    rng = np.random.default_rng(91)
    D = 64
    tys = ALL_TYPES + [orc.INT4, orc.FP16]
    rows = [int(x) for x in rng.integers(5, 60, len(tys))]
    inp = random_tbe(rng, len(tys), 23, [D] * len(tys), rows, 20)
    buf, w_off = build_weights(rng, tys, [D] * len(tys), rows)
    got = _nbit_nobag(dev, buf, w_off, tys, D, inp, 1)
    exp = orc.nbit_forward_nobag(buf, w_off, tys, D, inp.B, inp.indices, inp.offsets, out_kind=1)
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint16), exp.view(np.uint16))


def test_nbit_nobag_table_of_other_width_is_zeroed_and_reported(dev):
    """A table narrower than the call's D has its positions written as zeros
    (not left as allocated), the others match the oracle, and the next nbit
    call on the device raises, once."""
    print("[case] nbit nobag table of another width", flush=True)
    rng = np.random.default_rng(5)
    D = 32
    dims = [D, 16, D]
    tys = [orc.INT8, orc.INT8, orc.FP16]
    rows = [40, 30, 20]
    inp = random_tbe(rng, 3, 17, dims, rows, 9)
    buf, w_off = build_weights(rng, tys, dims, rows)
    maxima = [0, 0, D, D, 0, 0]
    junk = torch.full((inp.N, D), float("nan"), dtype=torch.float16, device=dev)
    del junk
    got = _nbit_nobag(dev, buf, w_off, tys, D, inp, 1, maxima=maxima, dims=dims)
    torch.cuda.synchronize()
    g = got.cpu().numpy().view(np.uint16)
    o1, o2 = int(inp.offsets[inp.B]), int(inp.offsets[2 * inp.B])
    assert np.all(g[o1:o2] == 0), "positions of the narrow table not zeroed"
    exp = orc.nbit_forward_nobag(buf, w_off, tys, D, inp.B, inp.indices, inp.offsets, out_kind=1)
    keep = np.r_[0:o1, o2:inp.N]
    np.testing.assert_array_equal(g[keep], exp.view(np.uint16)[keep])
    with pytest.raises(RuntimeError, match="cannot serve"):
        _nbit_nobag(dev, buf, w_off, tys, D, inp, 1, maxima=maxima, dims=dims)
    # Reported once: a valid call (the two D-wide tables alone) then runs normally.
    lens = np.diff(inp.offsets).reshape(3, inp.B)
    sub = bench_inputs.TbeInput(
        T=2, indices=np.concatenate([inp.indices[:o1], inp.indices[o2:]]),
        offsets=bench_inputs.offsets_from_lengths(lens[[0, 2]].reshape(-1)), B=inp.B,
        E=[rows[0], rows[2]], D=[D, D])
    ok = _nbit_nobag(dev, buf, w_off[[0, 2]], [tys[0], tys[2]], D, sub, 1, maxima=maxima)
    np.testing.assert_array_equal(ok.cpu().numpy().view(np.uint16), exp.view(np.uint16)[keep])


def _backward_nobag(dev, Wd, m1d, m1_off, inp, D, grad, lr, eps, wd, wd_mode, index_dtype):
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(inp.T, dtype=torch.int32, device=dev)
    torch.ops.fbgemm.split_embedding_nobag_backward_codegen_rowwise_adagrad_unweighted_exact_cuda(
        torch.from_numpy(grad).to(dev), Wd, empty, empty, pl,
        torch.from_numpy(weight_offsets(inp)).to(dev), D,
        torch.from_numpy(inp.hash_size_cumsum).to(dev), inp.total_hash_size_bits,
        torch.from_numpy(inp.indices).to(dev, index_dtype),
        torch.from_numpy(inp.offsets).to(dev, index_dtype),
        torch.zeros(0, dtype=torch.int32, device=dev), 0, 0, False, m1d, empty, pl,
        torch.from_numpy(m1_off).to(dev), eps, lr, wd, wd_mode, 0.0)


@pytest.mark.parametrize("D", [8, 64, 128, 256, 1024])
@pytest.mark.parametrize("wd_mode,wd", [(0, 0.0), (1, 0.05), (2, 0.02)])
@pytest.mark.parametrize("dup", [False, True])
def test_backward_nobag(dev, D, wd_mode, wd, dup):
    print(f"[case] nobag backward D={D} wd_mode={wd_mode} dup={dup}", flush=True)
    rng = np.random.default_rng(D * 7 + wd_mode + 50 * dup)
    rows = [3, 400, 60] if dup else [300, 400, 60]  # dup: a 3-row table makes long runs
    inp = random_tbe(rng, 3, 40, [D] * 3, rows, 30, empty_frac=0.2)
    W = rng.uniform(-0.5, 0.5, size=sum(E * D for E in rows)).astype(np.float32)
    m1 = rng.uniform(0, 0.01, size=sum(rows)).astype(np.float32)
    m1_off = np.concatenate([[0], np.cumsum(rows)[:-1]]).astype(np.int64)
    grad = rng.normal(0, 0.01, size=(inp.N, D)).astype(np.float32)
    lr, eps = 0.05, 1e-8
    Wd, m1d = torch.from_numpy(W).to(dev), torch.from_numpy(m1).to(dev)
    _backward_nobag(dev, Wd, m1d, m1_off, inp, D, grad, lr, eps, wd, wd_mode,
                    torch.int32 if D == 64 else torch.int64)
    W_exp, m_exp = orc.backward_rowwise_adagrad_nobag(
        W, weight_offsets(inp), D, inp.B, inp.hash_size_cumsum, inp.total_hash_size_bits,
        inp.indices, inp.offsets, grad, m1, m1_off, lr, eps, wd, wd_mode)
    Wg, mg = Wd.cpu().numpy(), m1d.cpu().numpy()
    # Long runs (dup) sum their rows in 32-row chunks, then the chunks in order:
    # another association of the same terms than the oracle's sequential sum.
    np.testing.assert_allclose(mg, m_exp, rtol=1e-4 if dup else RTOL, atol=0)
    np.testing.assert_allclose(Wg, W_exp, rtol=RTOL, atol=1e-6 if dup else ATOL)
    untouched = W_exp == W
    assert np.array_equal(Wg[untouched], W[untouched])


@pytest.mark.parametrize("index_dtype", [torch.int64, torch.int32])
def test_transpose_nobag(dev, index_dtype):
    print(f"[case] nobag transpose idx={index_dtype}", flush=True)
    rng = np.random.default_rng(17)
    inp = random_tbe(rng, 4, 50, [8] * 4, [500, 30, 2000, 7], 25)
    out = torch.ops.fbgemm.transpose_embedding_input(
        torch.from_numpy(inp.hash_size_cumsum).to(dev), inp.total_hash_size_bits,
        torch.from_numpy(inp.indices).to(dev, index_dtype),
        torch.from_numpy(inp.offsets).to(dev, index_dtype), True)
    linear, srt, infos, run, lengths, num_runs, cum = [o.cpu().numpy() for o in out]
    exp = orc.transpose_embedding_input_nobag(inp.hash_size_cumsum, inp.B,
                                              inp.total_hash_size_bits, inp.indices, inp.offsets)
    r = int(num_runs[0])
    assert infos.dtype == np.int64 and r == exp["num_runs"]
    np.testing.assert_array_equal(linear, exp["linear_indices"])
    np.testing.assert_array_equal(srt, exp["sorted_linear_indices"])
    np.testing.assert_array_equal(infos, exp["infos_sorted"])
    np.testing.assert_array_equal(run[:r], exp["run"])
    np.testing.assert_array_equal(lengths[:r], exp["run_lengths"])
    np.testing.assert_array_equal(cum[:r + 1], exp["cumulative_run_lengths"])
    assert np.all(lengths[r:] == 0) and np.all(cum[r + 1:] == inp.N)


def test_training_module_nobag_step(dev):
    """SplitTableBatchedEmbeddingBagsCodegen(pooling_mode=NONE): the forward
    is the gather, loss.backward() the nobag update, both against the oracle;
    features 0 and 2 share a table."""
    print("[case] nobag training module step", flush=True)
    rng = np.random.default_rng(44)
    D = 32
    specs = [(500, D, EmbeddingLocation.DEVICE, ComputeDevice.CUDA),
             (60, D, EmbeddingLocation.DEVICE, ComputeDevice.CUDA)]
    m = SplitTableBatchedEmbeddingBagsCodegen(specs, feature_table_map=[0, 1, 0],
                                              pooling_mode=PoolingMode.NONE, device=dev,
                                              learning_rate=0.05, eps=1e-8,
                                              weights_init=(-0.5, 0.5))
    inp = random_tbe(rng, 3, 30, [D] * 3, [500, 60, 500], 12)
    W0 = m.weights_dev.detach().cpu().numpy().copy()
    idx = torch.from_numpy(inp.indices).to(dev)
    off = torch.from_numpy(inp.offsets).to(dev)
    out = m(idx, off)
    w_off = m.weights_offsets.cpu().numpy()
    exp = orc.tbe_forward_nobag(W0, w_off, D, inp.B, inp.indices, inp.offsets)
    np.testing.assert_array_equal(out.detach().cpu().numpy(), exp)
    grad = rng.normal(0, 0.01, size=(inp.N, D)).astype(np.float32)
    (out * torch.from_numpy(grad).to(dev)).sum().backward()
    torch.cuda.synchronize()
    m1_off = m.momentum1_offsets.cpu().numpy()
    W_exp, m_exp = orc.backward_rowwise_adagrad_nobag(
        W0, w_off, D, inp.B, m.hash_size_cumsum.cpu().numpy(), m.total_hash_size_bits,
        inp.indices, inp.offsets, grad, np.zeros(560, np.float32), m1_off, 0.05, 1e-8)
    np.testing.assert_allclose(m.momentum1_dev.cpu().numpy(), m_exp, rtol=RTOL, atol=0)
    np.testing.assert_allclose(m.weights_dev.detach().cpu().numpy(), W_exp, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("out", [SparseType.FP16, SparseType.FP32, SparseType.BF16])
def test_inference_module_nobag(dev, out):
    print(f"[case] nobag inference module out={out}", flush=True)
    rng = np.random.default_rng(12)
    D = 64
    specs = [("a", 100, D, SparseType.INT8, EmbeddingLocation.DEVICE),
             ("b", 50, D, SparseType.INT4, EmbeddingLocation.DEVICE),
             ("c", 30, D, SparseType.FP16, EmbeddingLocation.DEVICE)]
    m = IntNBitTableBatchedEmbeddingBagsCodegen(specs, pooling_mode=PoolingMode.NONE,
                                                output_dtype=out, device=dev)
    tys = [orc.INT8, orc.INT4, orc.FP16]
    buf, w_off = build_weights(rng, tys, [D] * 3, [100, 50, 30])
    m.weights_dev.copy_(torch.from_numpy(buf))
    inp = random_tbe(rng, 3, 25, [D] * 3, [100, 50, 30], 10)
    got = m(torch.from_numpy(inp.indices).to(dev), torch.from_numpy(inp.offsets).to(dev))
    kind = {SparseType.FP32: 0, SparseType.FP16: 1, SparseType.BF16: 2}[out]
    exp = orc.nbit_forward_nobag(buf, w_off, tys, D, inp.B, inp.indices, inp.offsets,
                                 out_kind=kind)
    g = got.cpu()
    g = g.view(torch.int16).numpy().view(np.uint16) if kind else g.numpy().view(np.uint32)
    np.testing.assert_array_equal(g, exp.view(np.uint32) if kind == 0 else exp.view(np.uint16))


@pytest.mark.parametrize("layout", ["empty_first", "empty_middle", "empty_last", "shared_table"])
def test_nobag_sort_segments(dev, layout):
    """The recast batch sorts in per-feature segments: whole features without
    positions (first, middle, last) and two features sharing one table (equal
    hash_size_cumsum entries: one segment), each feature over several
    3072-key sort tiles; backward and transpose against the oracle."""
    print(f"[case] nobag sort segments {layout}", flush=True)
    seed = {"empty_first": 1, "empty_middle": 2, "empty_last": 3, "shared_table": 4}[layout]
    rng = np.random.default_rng(700 + seed)
    T, B, D = 4, 1500, 64
    rows = [300, 400, 400, 60]
    lengths = rng.integers(0, 11, size=(T, B))
    lengths[rng.random((T, B)) < 0.2] = 0
    if layout != "shared_table":
        lengths[{"empty_first": 0, "empty_middle": 2, "empty_last": 3}[layout]] = 0
    offsets = bench_inputs.offsets_from_lengths(lengths.reshape(-1))
    indices = np.concatenate([rng.integers(0, rows[t], int(lengths[t].sum())) for t in range(T)])
    if layout == "shared_table":  # features 1 and 2 look up the same 400-row table
        hsc = np.array([0, 300, 300, 700, 760], np.int64)
        w_off = np.array([0, 300 * D, 300 * D, 700 * D], np.int64)
        m1_off = np.array([0, 300, 300, 700], np.int64)
        n_rows = 760
    else:
        hsc = bench_inputs.offsets_from_lengths(np.asarray(rows, np.int64))
        w_off = hsc[:-1] * D
        m1_off = hsc[:-1].copy()
        n_rows = int(hsc[-1])
    bits = max(1, int(hsc[-1] - 1).bit_length())
    N = indices.size
    W = rng.uniform(-0.5, 0.5, size=n_rows * D).astype(np.float32)
    m1 = rng.uniform(0, 0.01, size=n_rows).astype(np.float32)
    grad = rng.normal(0, 0.01, size=(N, D)).astype(np.float32)
    lr, eps = 0.05, 1e-8
    Wd, m1d = torch.from_numpy(W).to(dev), torch.from_numpy(m1).to(dev)
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(T, dtype=torch.int32, device=dev)
    hsc_d = torch.from_numpy(hsc).to(dev)
    idx_d, off_d = torch.from_numpy(indices).to(dev), torch.from_numpy(offsets).to(dev)
    torch.ops.fbgemm.split_embedding_nobag_backward_codegen_rowwise_adagrad_unweighted_exact_cuda(
        torch.from_numpy(grad).to(dev), Wd, empty, empty, pl, torch.from_numpy(w_off).to(dev),
        D, hsc_d, bits, idx_d, off_d, torch.zeros(0, dtype=torch.int32, device=dev), 0, 0,
        False, m1d, empty, pl, torch.from_numpy(m1_off).to(dev), eps, lr, 0.0, 0, 0.0)
    W_exp, m_exp = orc.backward_rowwise_adagrad_nobag(
        W, w_off, D, B, hsc, bits, indices, offsets, grad, m1, m1_off, lr, eps)
    Wg, mg = Wd.cpu().numpy(), m1d.cpu().numpy()
    # Runs past 24 occurrences sum in 32-row chunks: another association of the terms.
    np.testing.assert_allclose(mg, m_exp, rtol=1e-4, atol=0)
    np.testing.assert_allclose(Wg, W_exp, rtol=RTOL, atol=1e-6)
    untouched = W_exp == W
    assert np.array_equal(Wg[untouched], W[untouched])
    out = torch.ops.fbgemm.transpose_embedding_input(hsc_d, bits, idx_d, off_d, True)
    linear, srt, infos, run, lens, num_runs, cum = [o.cpu().numpy() for o in out]
    exp = orc.transpose_embedding_input_nobag(hsc, B, bits, indices, offsets)
    r = int(num_runs[0])
    assert r == exp["num_runs"]
    np.testing.assert_array_equal(linear, exp["linear_indices"])
    np.testing.assert_array_equal(srt, exp["sorted_linear_indices"])
    np.testing.assert_array_equal(infos, exp["infos_sorted"])
    np.testing.assert_array_equal(run[:r], exp["run"])
    np.testing.assert_array_equal(lens[:r], exp["run_lengths"])
    np.testing.assert_array_equal(cum[:r + 1], exp["cumulative_run_lengths"])
