"""GPU parity of the TBE backward: transpose_embedding_input (sorted keys,
infos and run layout: bit-exact) and the fused exact rowwise-Adagrad update
(weights and momentum within rtol 1e-5 of the oracle; rows the batch does
not touch bit-identical)."""

import numpy as np
import pytest
import torch

import oracle as orc
from mx_fbgemm import bench_inputs
from adagrad_bounds import assert_eps_pin_close, assert_reordered_adagrad_close, eps_pin_case
from tbe_helpers import random_tbe, weight_offsets

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-7


def _transpose_gpu(dev, inp, info_bits, index_dtype=torch.int64):
    return torch.ops.fbgemm.transpose_embedding_input(
        torch.from_numpy(inp.hash_size_cumsum).to(dev), inp.total_hash_size_bits,
        torch.from_numpy(inp.indices).to(dev, index_dtype),
        torch.from_numpy(inp.offsets).to(dev, index_dtype), False, None, info_bits)


def _check_transpose(dev, inp, index_dtype=torch.int64):
    nb = orc.info_B_num_bits(inp.T, inp.B)
    exp = orc.transpose_embedding_input(inp.hash_size_cumsum, inp.B, nb, inp.total_hash_size_bits,
                                        inp.indices, inp.offsets)
    lin, srt, infos, run, lengths, num_runs, cum = _transpose_gpu(dev, inp, nb, index_dtype)
    r = int(num_runs.item())
    assert r == exp["num_runs"]
    np.testing.assert_array_equal(lin.cpu().numpy(), exp["linear_indices"])
    np.testing.assert_array_equal(srt.cpu().numpy(), exp["sorted_linear_indices"])
    np.testing.assert_array_equal(infos.cpu().numpy(), exp["infos_sorted"])
    np.testing.assert_array_equal(run.cpu().numpy()[:r], exp["run"])
    np.testing.assert_array_equal(lengths.cpu().numpy()[:r], exp["run_lengths"])
    np.testing.assert_array_equal(cum.cpu().numpy()[: r + 1], exp["cumulative_run_lengths"])
    # Whole arrays: past num_runs, run lengths 0 and the cumsum N.
    np.testing.assert_array_equal(lengths.cpu().numpy(), exp["run_lengths_full"])
    np.testing.assert_array_equal(cum.cpu().numpy(), exp["cumulative_run_lengths_full"])


@pytest.mark.parametrize("T,B,rows,max_L,dup", [
    (1, 1, [1], 1, False),
    (3, 50, [10, 1000, 70000], 20, False),
    (2, 300, [5000, 5000], 40, True),      # runs far longer than 64 occurrences
    (5, 700, [2 ** 20, 3, 100, 9, 2 ** 21], 10, False),  # 22+ key bits: 3 radix passes
])
def test_transpose_bit_exact(dev, T, B, rows, max_L, dup):
    print(f"[case] transpose T={T} B={B} rows={rows}", flush=True)
    rng = np.random.default_rng(T * 7 + B)
    inp = random_tbe(rng, T, B, [4] * T, rows, max_L, dup_heavy=dup)
    _check_transpose(dev, inp)
    _check_transpose(dev, inp, torch.int32)


def test_transpose_keys_outside_their_table_sort_globally(dev):
    """The sort handles each table's positions on its own only when every key
    lies in its table's range; indices past a table's rows (keys in the next
    table's range) make it sort all keys together, so the layout stays the
    global stable order, bit-exact against the oracle."""
    print("[case] transpose, keys outside their table's range", flush=True)
    rng = np.random.default_rng(31)
    inp = random_tbe(rng, 3, 400, [4] * 3, [1000, 1000, 1000], 30)
    s0, e0 = int(inp.offsets[0]), int(inp.offsets[400])
    inp.indices[s0:e0] = rng.integers(0, 1100, size=e0 - s0)  # up to 100 rows past table 0
    _check_transpose(dev, inp)
    _check_transpose(dev, inp, torch.int32)


def test_transpose_too_few_key_bits(dev):
    """With total_hash_size_bits below the keys' width the sort orders keys by
    their low bits (as a radix sort over those bits does, across features):
    per-feature segments would not, so the sort runs over the whole batch and
    matches the oracle's masked stable sort."""
    print("[case] transpose, 11 key bits for 3,000 rows", flush=True)
    rng = np.random.default_rng(11)
    inp = random_tbe(rng, 3, 300, [4] * 3, [1000, 1000, 1000], 20)
    bits = 11  # 2^11 = 2048 < 3000 rows
    nb = orc.info_B_num_bits(inp.T, inp.B)
    exp = orc.transpose_embedding_input(inp.hash_size_cumsum, inp.B, nb, bits, inp.indices,
                                        inp.offsets)
    for idt in (torch.int64, torch.int32):
        got = torch.ops.fbgemm.transpose_embedding_input(
            torch.from_numpy(inp.hash_size_cumsum).to(dev), bits,
            torch.from_numpy(inp.indices).to(dev, idt), torch.from_numpy(inp.offsets).to(dev, idt),
            False, None, nb)
        r = int(got[5].item())
        assert r == exp["num_runs"]
        np.testing.assert_array_equal(got[1].cpu().numpy(), exp["sorted_linear_indices"])
        np.testing.assert_array_equal(got[2].cpu().numpy(), exp["infos_sorted"])
        np.testing.assert_array_equal(got[6].cpu().numpy()[: r + 1], exp["cumulative_run_lengths"])


@pytest.mark.parametrize("T", [63, 64])
def test_transpose_feature_segments(dev, T):
    """Up to 63 features sort as per-feature segments, 64 as one batch.  The
    batch mixes empty features (first, middle, last), a feature of exactly
    one 3072-key sort tile, one of two tiles plus one key, and many short
    ones: the layout is the global stable order either way."""
    print(f"[case] transpose feature segments T={T}", flush=True)
    rng = np.random.default_rng(6300 + T)
    B = 64
    lengths = rng.integers(0, 9, size=(T, B))
    lengths[[0, 7, T - 1]] = 0
    lengths[1] = 48                      # 3072 positions
    lengths[2] = 96
    lengths[2, 5] += 1                   # 6145 positions
    rows = [int(r) for r in rng.integers(1, 5000, T)]
    rows[1], rows[2] = 3, 70000          # long runs; a wide table
    off = bench_inputs.offsets_from_lengths(lengths.reshape(-1))
    idx = np.empty(int(off[-1]), dtype=np.int64)
    for t in range(T):
        s, e = int(off[t * B]), int(off[(t + 1) * B])
        idx[s:e] = rng.integers(0, rows[t], size=e - s)
    inp = bench_inputs.TbeInput(T=T, E=rows, D=[4] * T, B=B, indices=idx, offsets=off)
    _check_transpose(dev, inp)
    _check_transpose(dev, inp, torch.int32)


def _bag_input(rng, E, idx, B):
    """One table of E rows whose B bags hold the indices idx in a random order."""
    idx = rng.permutation(np.asarray(idx, dtype=np.int64))
    cuts = np.sort(rng.integers(0, idx.size + 1, size=B - 1))
    off = np.concatenate([[0], cuts, [idx.size]]).astype(np.int64)
    return bench_inputs.TbeInput(T=1, E=[E], D=[4], B=B, indices=idx, offsets=off)


def test_transpose_concentrated_keys(dev):
    """16-bit keys, two thirds of them within one 256-key range (one value of
    the second radix digit): the passes' digit counts are far from uniform,
    the layout stays bit-exact."""
    print("[case] transpose, 16384 of 25384 keys in [0, 256)", flush=True)
    rng = np.random.default_rng(16384)
    E = 1 << 16
    idx = np.concatenate([rng.integers(0, 256, size=16384), rng.integers(256, E, size=9000)])
    inp = _bag_input(rng, E, idx, 1500)
    _check_transpose(dev, inp)
    _check_transpose(dev, inp, torch.int32)


@pytest.mark.parametrize("E", [1 << 24, (1 << 24) + 1])
def test_transpose_key_bits_24_and_25(dev, E):
    """24 key bits sort in three 8-bit passes, 25 in four (the widest
    histogram slot)."""
    print(f"[case] transpose, E={E}", flush=True)
    rng = np.random.default_rng(E % 1000)
    inp = _bag_input(rng, E, rng.integers(0, E, size=60000), 3000)
    assert inp.total_hash_size_bits == (24 if E == 1 << 24 else 25)
    _check_transpose(dev, inp)


def _zipf_batch(rng, T, B, E, D, max_L, permute):
    """Zipf(1.05) indices; without the per-table row permutation each table's
    first rows are its hot ones (frequency-ordered ids)."""
    lengths = rng.integers(1, max_L + 1, size=T * B)
    off = bench_inputs.offsets_from_lengths(lengths)
    parts = []
    for t in range(T):
        z = bench_inputs.bounded_zipf(rng, E, 1.05, int(off[(t + 1) * B] - off[t * B]))
        parts.append(rng.permutation(E)[z] if permute else z)
    return bench_inputs.TbeInput(T=T, E=[E] * T, D=[D] * T, B=B, indices=np.concatenate(parts),
                                 offsets=off)


@pytest.mark.parametrize("pooling", [0, 1])
def test_unpermuted_zipf_batch(dev, pooling):
    """Frequency-ordered ids: every table's hot rows are its first ones, so
    most keys share their high digits.  Transpose bit-exact, backward against
    the oracle."""
    print(f"[case] unpermuted Zipf batch pooling={pooling}", flush=True)
    rng = np.random.default_rng(105 + pooling)
    inp = _zipf_batch(rng, 2, 2048, 200_000, 64, 40, permute=False)
    _check_transpose(dev, inp)
    _backward_case(dev, inp, pooling, seed=7)


@pytest.mark.parametrize("weighted", [False, True])
def test_permuted_zipf_backward(dev, weighted):
    """A permuted Zipf batch of three tables: transpose bit-exact and the
    backward, weighted or not, against the oracle."""
    print(f"[case] permuted Zipf batch weighted={weighted}", flush=True)
    rng = np.random.default_rng(41 + weighted)
    inp = _zipf_batch(rng, 3, 2048, 200_000, 64, 40, permute=True)
    _check_transpose(dev, inp)
    _backward_case(dev, inp, 0, seed=9, weighted=weighted)


@pytest.mark.parametrize("T,B,rows,max_L,dup", [
    (3, 50, [10, 1000, 70000], 20, False),
    (2, 300, [5000, 5000], 40, True),
    (5, 700, [2 ** 20, 3, 100, 9, 2 ** 21], 10, False),
])
def test_transpose_wide_sort_words(dev, T, B, rows, max_L, dup):
    """The sort keeps its look-back counts in 32-bit words below 2^30 keys and
    in 64-bit words from there on; a test hook selects the 64-bit form here,
    at sizes the oracle checks bit for bit, and the backward is checked in
    the same form."""
    print(f"[case] transpose, 64-bit sort words T={T} B={B} rows={rows}", flush=True)
    rng = np.random.default_rng(T * 11 + B)
    inp = random_tbe(rng, T, B, [64] * T, rows, max_L, dup_heavy=dup)
    torch.ops.mx_fbgemm.test_force_wide_sort_words(True)
    try:
        _check_transpose(dev, inp)
        _check_transpose(dev, inp, torch.int32)
        _backward_case(dev, inp, 0, seed=T + B)
    finally:
        torch.ops.mx_fbgemm.test_force_wide_sort_words(False)


def _backward_case(dev, inp, pooling, wd=0.0, wd_mode=0, lr=0.01, eps=1e-8, seed=0,
                   weighted=False, index_dtype=torch.int64):
    rng = np.random.default_rng(seed)
    W = rng.uniform(-0.01, 0.01, size=sum(E * D for E, D in zip(inp.E, inp.D))).astype(np.float32)
    m1 = rng.uniform(0, 1e-4, size=sum(inp.E)).astype(np.float32)
    m1_off = np.concatenate([[0], np.cumsum(inp.E)[:-1]]).astype(np.int64)
    grad = rng.normal(0, 1e-2, size=(inp.B, inp.total_D)).astype(np.float32)
    iw = rng.uniform(-2.0, 2.0, inp.N).astype(np.float32) if weighted else None
    nb = orc.info_B_num_bits(inp.T, inp.B)
    W_exp, m1_exp = orc.backward_rowwise_adagrad(
        W, weight_offsets(inp), inp.D_offsets, inp.B, inp.hash_size_cumsum,
        inp.total_hash_size_bits, inp.indices, inp.offsets, pooling, grad, m1, m1_off, lr, eps,
        wd, wd_mode, nb, indice_weights=iw)
    Wd = torch.from_numpy(W).to(dev)
    m1d = torch.from_numpy(m1).to(dev)
    empty = torch.zeros(0, device=dev)
    head = (torch.from_numpy(grad).to(dev), Wd, empty, empty,
            torch.zeros(inp.T, dtype=torch.int32, device=dev),
            torch.from_numpy(weight_offsets(inp)).to(dev), torch.from_numpy(inp.D_offsets).to(dev),
            max(inp.D), torch.from_numpy(inp.hash_size_cumsum).to(dev), inp.total_hash_size_bits,
            torch.from_numpy(inp.indices).to(dev, index_dtype),
            torch.from_numpy(inp.offsets).to(dev, index_dtype), pooling)
    tail = (torch.zeros(0, dtype=torch.int32, device=dev), 0, 0, False, m1d, empty,
            torch.zeros(inp.T, dtype=torch.int32, device=dev), torch.from_numpy(m1_off).to(dev),
            eps, lr, wd, wd_mode, 0.0)
    if weighted:
        torch.ops.fbgemm.split_embedding_backward_codegen_rowwise_adagrad_weighted_exact_cuda(
            *head, torch.from_numpy(iw).to(dev), *tail)
    else:
        torch.ops.fbgemm.split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_cuda(
            *head, *tail)
    Wg, mg = Wd.cpu().numpy(), m1d.cpu().numpy()
    np.testing.assert_allclose(mg, m1_exp, rtol=RTOL, atol=0)
    np.testing.assert_allclose(Wg, W_exp, rtol=RTOL, atol=ATOL)
    untouched = W_exp == W  # rows the batch never touched must stay bit-identical
    assert np.array_equal(Wg[untouched], W[untouched])
    return Wg, W_exp


@pytest.mark.parametrize("pooling", [0, 1])
@pytest.mark.parametrize("T,B,dims,rows,max_L,dup", [
    (2, 40, [128, 128], [300, 300], 20, False),
    (3, 64, [4, 64, 256], [50, 2000, 40], 30, False),
    (2, 200, [128, 1024], [4, 4], 40, True),       # long runs -> chunked path
    (1, 3, [128], [1], 2, False),                  # single row, single table
])
def test_backward_rowwise_adagrad(dev, pooling, T, B, dims, rows, max_L, dup):
    print(f"[case] backward T={T} B={B} dims={dims} pool={pooling} dup={dup}", flush=True)
    rng = np.random.default_rng(B + T)
    inp = random_tbe(rng, T, B, dims, rows, max_L, dup_heavy=dup)
    _backward_case(dev, inp, pooling, seed=B)


@pytest.mark.parametrize("D", [64, 256, 512, 1024])
@pytest.mark.parametrize("pooling,weighted", [(0, False), (1, False), (0, True)])
def test_backward_full_width(dev, D, pooling, weighted):
    """Every table of width D (the kernels' full-width instances, whose rows
    have no partial column chunks), with runs long enough for the chunked
    path: against the oracle."""
    print(f"[case] full-width backward D={D} pool={pooling} weighted={weighted}", flush=True)
    rng = np.random.default_rng(D + pooling + 2 * weighted)
    inp = random_tbe(rng, 3, 96, [D] * 3, [40, 3, 900], 40, dup_heavy=False)
    _backward_case(dev, inp, pooling, seed=D, weighted=weighted)


@pytest.mark.parametrize("pooling", [0, 1])
@pytest.mark.parametrize("T,B,dims,rows,max_L,dup", [
    (3, 64, [4, 64, 256], [50, 2000, 40], 30, False),
    (2, 200, [128, 1024], [4, 4], 40, True),       # long runs -> chunked path
    (2, 500, [128, 32], [3, 20000], 25, True),     # one row per >1000 occurrences
])
def test_backward_weighted(dev, pooling, T, B, dims, rows, max_L, dup):
    """Weighted backward: every occurrence's gradient slice is scaled by its
    per-sample weight (after the MEAN 1/L); weights of both signs."""
    print(f"[case] weighted backward T={T} B={B} dims={dims} pool={pooling}", flush=True)
    rng = np.random.default_rng(B * 3 + T)
    inp = random_tbe(rng, T, B, dims, rows, max_L, dup_heavy=dup)
    _backward_case(dev, inp, pooling, seed=B + 1, weighted=True)
    _backward_case(dev, inp, pooling, seed=B + 2, weighted=True, index_dtype=torch.int32)


@pytest.mark.parametrize("pooling", [0, 1])
@pytest.mark.parametrize("dims", [[8, 36, 64], [128, 4], [256, 512, 1024]])
def test_grad_indice_weights(dev, pooling, dims):
    """split_embedding_codegen_grad_indice_weights_cuda vs the oracle (fp64
    dot product): rtol 1e-5 of sum_d |g_d * w_d|; masked tables exactly 0."""
    print(f"[case] grad_indice_weights dims={dims} pool={pooling}", flush=True)
    T = len(dims)
    rng = np.random.default_rng(sum(dims) + pooling)
    inp = random_tbe(rng, T, 70, dims, [300] * T, 25, empty_frac=0.1)
    W = rng.uniform(-1, 1, size=sum(E * D for E, D in zip(inp.E, inp.D))).astype(np.float32)
    grad = rng.normal(0, 1, size=(inp.B, inp.total_D)).astype(np.float32)
    frg = (np.arange(T) % 2 == 0).astype(np.int32)
    w_off = weight_offsets(inp)
    exp = orc.grad_indice_weights(grad, W, w_off, inp.D_offsets, inp.B, inp.indices, inp.offsets,
                                  pooling, frg)
    mag = orc.grad_indice_weights(np.abs(grad), np.abs(W), w_off, inp.D_offsets, inp.B,
                                  inp.indices, inp.offsets, pooling)
    empty = torch.zeros(0, device=dev)
    for idt, f in ((torch.int64, frg), (torch.int32, frg), (torch.int64, None)):
        got = torch.ops.fbgemm.split_embedding_codegen_grad_indice_weights_cuda(
            torch.from_numpy(grad).to(dev), torch.from_numpy(W).to(dev), empty, empty,
            torch.zeros(T, dtype=torch.int32, device=dev), torch.from_numpy(w_off).to(dev),
            torch.from_numpy(inp.D_offsets).to(dev), max(dims),
            torch.from_numpy(inp.indices).to(dev, idt), torch.from_numpy(inp.offsets).to(dev, idt),
            torch.zeros(0, dtype=torch.int32, device=dev),
            None if f is None else torch.from_numpy(f).to(dev), pooling).cpu().numpy()
        ref = exp if f is not None else orc.grad_indice_weights(
            grad, W, w_off, inp.D_offsets, inp.B, inp.indices, inp.offsets, pooling)
        assert np.all(np.abs(got - ref) <= 1e-5 * mag + 1e-30), np.max(np.abs(got - ref) / mag)
        if f is not None:
            for t in np.flatnonzero(f == 0):
                o = inp.offsets[t * inp.B], inp.offsets[(t + 1) * inp.B]
                assert not got[o[0]:o[1]].any()


@pytest.mark.parametrize("pooling", [0, 1])
def test_backward_many_tables(dev, pooling):
    """700 tables (past the 512 whose metadata the kernels stage in LDS; the
    info word then needs 10 table bits), mixed D, some rows hit by long runs:
    transpose bit-exact, update within rtol 1e-5."""
    print(f"[case] backward 700 tables pool={pooling}", flush=True)
    rng = np.random.default_rng(7000 + pooling)
    T, B = 700, 40
    dims = [int(d) for d in rng.choice([4, 32, 64, 128], T)]
    rows = [int(r) for r in rng.integers(1, 40, T)]
    inp = random_tbe(rng, T, B, dims, rows, 6)
    _check_transpose(dev, inp)
    _backward_case(dev, inp, pooling, seed=pooling)


def _shared_tables(rng, ftm, rows, dims, B, max_L, dup=False):
    """A batch whose features share tables (fbgemm's feature_table_map): per
    feature weight offsets, hash offsets and momentum offsets point at its
    table; D_offsets lay the features' columns side by side."""
    fr, fd = [rows[t] for t in ftm], [dims[t] for t in ftm]
    inp = random_tbe(rng, len(ftm), B, fd, fr, max_L, dup_heavy=dup)
    t_off = np.concatenate([[0], np.cumsum([E * D for E, D in zip(rows, dims)])[:-1]])
    t_hsc = np.concatenate([[0], np.cumsum(rows)[:-1]])
    w_off = t_off[ftm].astype(np.int64)
    hsc = np.concatenate([t_hsc[ftm], [sum(rows)]]).astype(np.int64)
    m1_off = t_hsc[ftm].astype(np.int64)
    bits = int(np.ceil(np.log2(max(sum(rows), 2))))
    return inp, w_off, hsc, m1_off, bits


@pytest.mark.parametrize("pooling", [0, 1])
@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("dup", [False, True])
@pytest.mark.parametrize("ftm", [[0, 1, 0, 2, 1], [0, 0, 1, 1, 2]])
def test_backward_shared_tables(dev, pooling, weighted, dup, ftm):
    """Features sharing tables (fbgemm's feature_table_map; hash_size_cumsum
    then decreases, and the sort runs over the whole batch, or repeats, and
    each table's features sort as one segment): one run per row of a shared
    table, each occurrence summing its own feature's
    gradient columns (MEAN: its own bag length); duplicate-heavy batches reach
    the chunked long-run path.  Transpose bit-exact, update within rtol 1e-5."""
    print(f"[case] shared tables ftm={ftm} pool={pooling} weighted={weighted} dup={dup}",
          flush=True)
    rng = np.random.default_rng(50 + pooling + 2 * weighted + 4 * dup + 8 * ftm[1])
    rows, dims = [300, 200, 50], [64, 32, 128]
    inp, w_off, hsc, m1_off, bits = _shared_tables(rng, ftm, rows, dims, 120, 30, dup)
    nb = orc.info_B_num_bits(inp.T, inp.B)
    exp = orc.transpose_embedding_input(hsc, inp.B, nb, bits, inp.indices, inp.offsets)
    got = torch.ops.fbgemm.transpose_embedding_input(
        torch.from_numpy(hsc).to(dev), bits, torch.from_numpy(inp.indices).to(dev),
        torch.from_numpy(inp.offsets).to(dev), False, None, nb)
    r = int(got[5].item())
    assert r == exp["num_runs"]
    np.testing.assert_array_equal(got[1].cpu().numpy(), exp["sorted_linear_indices"])
    np.testing.assert_array_equal(got[2].cpu().numpy(), exp["infos_sorted"])
    W = rng.uniform(-0.5, 0.5, size=sum(E * D for E, D in zip(rows, dims))).astype(np.float32)
    m1 = rng.uniform(0, 0.01, size=sum(rows)).astype(np.float32)
    grad = rng.normal(0, 1e-1, size=(inp.B, inp.total_D)).astype(np.float32)
    iw = rng.uniform(-1.5, 1.5, inp.N).astype(np.float32) if weighted else None
    W_exp, m1_exp = orc.backward_rowwise_adagrad(
        W, w_off, inp.D_offsets, inp.B, hsc, bits, inp.indices, inp.offsets, pooling, grad, m1,
        m1_off, 0.05, 1e-6, 0.0, 0, nb, indice_weights=iw)
    Wd, m1d = torch.from_numpy(W).to(dev), torch.from_numpy(m1).to(dev)
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(inp.T, dtype=torch.int32, device=dev)
    head = (torch.from_numpy(grad).to(dev), Wd, empty, empty, pl, torch.from_numpy(w_off).to(dev),
            torch.from_numpy(inp.D_offsets).to(dev), max(dims), torch.from_numpy(hsc).to(dev),
            bits, torch.from_numpy(inp.indices).to(dev), torch.from_numpy(inp.offsets).to(dev),
            pooling)
    tail = (torch.zeros(0, dtype=torch.int32, device=dev), 0, 0, False, m1d, empty, pl,
            torch.from_numpy(m1_off).to(dev), 1e-6, 0.05, 0.0, 0, 0.0)
    if weighted:
        torch.ops.fbgemm.split_embedding_backward_codegen_rowwise_adagrad_weighted_exact_cuda(
            *head, torch.from_numpy(iw).to(dev), *tail)
    else:
        torch.ops.fbgemm.split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_cuda(
            *head, *tail)
    np.testing.assert_allclose(m1d.cpu().numpy(), m1_exp, rtol=RTOL, atol=0)
    # Rows here are O(0.5) (a wrong gradient column would show at once), so
    # the absolute floor is scaled from the 1e-7 used for O(0.01) rows: an
    # update that nearly cancels the row keeps only the absolute accuracy of
    # its operands, and the chunked long runs sum in another order.
    np.testing.assert_allclose(Wd.cpu().numpy(), W_exp, rtol=RTOL, atol=1e-6)


@pytest.mark.parametrize("weighted", [False, True])
def test_module_training_step_shared_tables(dev, weighted):
    """SplitTableBatchedEmbeddingBagsCodegen(specs, feature_table_map=[0, 1, 0]):
    forward bit-exact against the oracle on the per-feature arrays, and one
    fused update per row of the shared table (vs the oracle pinned to torch
    autograd on shared tables)."""
    print(f"[case] module shared tables weighted={weighted}", flush=True)
    from mx_fbgemm import ComputeDevice, EmbeddingLocation, PoolingMode
    from mx_fbgemm.split_table_batched_embeddings_ops_training import (
        SplitTableBatchedEmbeddingBagsCodegen,
    )

    ftm, rows, dims = [0, 1, 0], [200, 80], [64, 32]
    specs = [(E, D, EmbeddingLocation.DEVICE, ComputeDevice.CUDA) for E, D in zip(rows, dims)]
    tbe = SplitTableBatchedEmbeddingBagsCodegen(specs, ftm, pooling_mode=PoolingMode.SUM,
                                                learning_rate=0.05, eps=1e-6, device=dev,
                                                weights_init=(-0.5, 0.5))
    rng = np.random.default_rng(61 + weighted)
    inp, w_off, hsc, m1_off, bits = _shared_tables(rng, ftm, rows, dims, 24, 12, dup=True)
    assert tbe.weights_offsets.tolist() == w_off.tolist()
    assert tbe.hash_size_cumsum.tolist() == hsc.tolist()
    W0 = tbe.weights_dev.detach().cpu().numpy().copy()
    iw = rng.uniform(0.5, 1.5, inp.N).astype(np.float32) if weighted else None
    out = tbe(torch.from_numpy(inp.indices).to(dev), torch.from_numpy(inp.offsets).to(dev),
              per_sample_weights=None if iw is None else torch.from_numpy(iw).to(dev))
    exp = orc.tbe_forward_f32(W0, w_off, inp.D_offsets, inp.B, inp.indices, inp.offsets, 0,
                              indice_weights=iw)
    assert np.array_equal(out.detach().cpu().numpy(), exp)
    gout = rng.normal(0, 1e-1, size=out.shape).astype(np.float32)
    out.backward(torch.from_numpy(gout).to(dev))
    W_exp, m_exp = orc.backward_rowwise_adagrad(
        W0, w_off, inp.D_offsets, inp.B, hsc, bits, inp.indices, inp.offsets, 0, gout,
        np.zeros(sum(rows), np.float32), m1_off, 0.05, 1e-6, 0.0, 0,
        orc.info_B_num_bits(inp.T, inp.B), indice_weights=iw)
    np.testing.assert_allclose(tbe.weights_dev.detach().cpu().numpy(), W_exp, rtol=RTOL, atol=1e-6)
    np.testing.assert_allclose(tbe.momentum1_dev.cpu().numpy(), m_exp, rtol=RTOL, atol=0)


@pytest.mark.parametrize("wd_mode,wd", [(1, 0.1), (2, 0.05)])
def test_backward_weight_decay(dev, wd_mode, wd):
    print(f"[case] backward weight decay mode {wd_mode}", flush=True)
    rng = np.random.default_rng(3)
    inp = random_tbe(rng, 2, 50, [64, 128], [100, 100], 15)
    _backward_case(dev, inp, 0, wd=wd, wd_mode=wd_mode)


def _update_fp64(inp, pooling, W, m1, m1_off, grad, lr, eps):
    """Rowwise Adagrad (no weight decay) evaluated in float64: exact sums of
    the (MEAN-scaled) gradient slices per row, then h += mean(g^2) and
    w -= lr * g / (sqrt(h) + eps)."""
    W64, m64 = W.astype(np.float64), m1.astype(np.float64)
    w_off, Doff, B = weight_offsets(inp), inp.D_offsets, inp.B
    L = np.diff(inp.offsets)
    for t in range(inp.T):
        D, E = int(Doff[t + 1] - Doff[t]), inp.E[t]
        s, e = int(inp.offsets[t * B]), int(inp.offsets[(t + 1) * B])
        bags = np.repeat(np.arange(B), L[t * B:(t + 1) * B])
        g = grad[bags, Doff[t]:Doff[t + 1]].astype(np.float64)
        if pooling == 1:  # the scale the kernels use: fp32 1/L
            g *= (np.float32(1.0) / L[t * B:(t + 1) * B][bags].astype(np.float32))[:, None]
        acc = np.zeros((E, D))
        np.add.at(acc, inp.indices[s:e], g)
        hit = np.zeros(E, bool)
        hit[inp.indices[s:e]] = True
        h = m64[m1_off[t]:m1_off[t] + E] + np.mean(acc * acc, axis=1)
        rows = W64[w_off[t]:w_off[t] + E * D].reshape(E, D)
        upd = rows - (lr / (np.sqrt(h) + eps))[:, None] * acc
        rows[hit] = upd[hit]
        m64[m1_off[t]:m1_off[t] + E][hit] = h[hit]
    return W64, m64


@pytest.mark.parametrize("T,B,dims,rows,max_L,pooling,dup", [
    (3, 259, [20, 216, 232], [2000, 300, 1], 43, 1, True),
    (2, 298, [208, 132], [1, 300], 40, 1, False),
    (3, 156, [516, 760, 536], [4, 1, 50], 37, 1, True),
    (4, 252, [648, 772, 248, 556], [4, 300, 1, 1], 42, 1, False),
    (3, 291, [56, 104, 104], [50, 1, 1], 42, 0, False),
    (4, 195, [156, 56, 144, 12], [300, 1, 50, 70000], 44, 0, False),
    (1, 174, [564], [1], 44, 1, False),  # one row: every occurrence in one run
])
def test_extreme_runs_against_oracle_and_fp64(dev, T, B, dims, rows, max_L, pooling, dup):
    """Tables of 1-4 rows: runs of thousands of occurrences, where the kernels
    (chunked sums) and the oracle (one sequential sum per run) add each
    row's gradient terms in very different orders.  Checked against the
    oracle element by element under the first-order reordering bound of the
    two summation orders carried through the update (tests/adagrad_bounds.py;
    a pure rtol fails near cancelled sums by construction), and against a
    float64 evaluation of the same update: the kernels' fp32 error stays
    within 3e-8 there, while the oracle's sequential sum drifts up to ~3e-7."""
    print(f"[case] extreme runs T={T} B={B} dims={dims} rows={rows} pool={pooling}", flush=True)
    rng = np.random.default_rng(B + T)
    inp = random_tbe(rng, T, B, dims, rows, max_L, dup_heavy=dup)
    rng = np.random.default_rng(B)
    lr, eps = 0.01, 1e-8
    W = rng.uniform(-0.01, 0.01, size=sum(E * D for E, D in zip(inp.E, inp.D))).astype(np.float32)
    m1 = rng.uniform(0, 1e-4, size=sum(inp.E)).astype(np.float32)
    m1_off = np.concatenate([[0], np.cumsum(inp.E)[:-1]]).astype(np.int64)
    grad = rng.normal(0, 1e-2, size=(inp.B, inp.total_D)).astype(np.float32)
    W64, m64 = _update_fp64(inp, pooling, W, m1, m1_off, grad, lr, eps)
    Wd, m1d = torch.from_numpy(W).to(dev), torch.from_numpy(m1).to(dev)
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(T, dtype=torch.int32, device=dev)
    torch.ops.fbgemm.split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_cuda(
        torch.from_numpy(grad).to(dev), Wd, empty, empty, pl,
        torch.from_numpy(weight_offsets(inp)).to(dev), torch.from_numpy(inp.D_offsets).to(dev),
        max(dims), torch.from_numpy(inp.hash_size_cumsum).to(dev), inp.total_hash_size_bits,
        torch.from_numpy(inp.indices).to(dev), torch.from_numpy(inp.offsets).to(dev), pooling,
        torch.zeros(0, dtype=torch.int32, device=dev), 0, 0, False, m1d, empty, pl,
        torch.from_numpy(m1_off).to(dev), eps, lr, 0.0, 0, 0.0)
    W_exp, m_exp = orc.backward_rowwise_adagrad(
        W, weight_offsets(inp), inp.D_offsets, inp.B, inp.hash_size_cumsum,
        inp.total_hash_size_bits, inp.indices, inp.offsets, pooling, grad, m1, m1_off, lr, eps,
        0.0, 0, orc.info_B_num_bits(T, inp.B))
    Wg, mg = Wd.cpu().numpy(), m1d.cpu().numpy()
    assert_reordered_adagrad_close(Wg, mg, W_exp, m_exp, W, m1, weight_offsets(inp), m1_off, inp,
                                   grad, pooling, lr, eps)
    assert np.abs(Wg.astype(np.float64) - W64).max() <= 3e-8
    np.testing.assert_allclose(mg, m64, rtol=1e-5, atol=0)


def _backward_gpu(dev, inp, W, m1, m1_off, grad, pooling, lr, eps):
    Wd, m1d = torch.from_numpy(W).to(dev), torch.from_numpy(m1).to(dev)
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(inp.T, dtype=torch.int32, device=dev)
    torch.ops.fbgemm.split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_cuda(
        torch.from_numpy(grad).to(dev), Wd, empty, empty, pl,
        torch.from_numpy(weight_offsets(inp)).to(dev), torch.from_numpy(inp.D_offsets).to(dev),
        max(inp.D), torch.from_numpy(inp.hash_size_cumsum).to(dev), inp.total_hash_size_bits,
        torch.from_numpy(inp.indices).to(dev), torch.from_numpy(inp.offsets).to(dev), pooling,
        torch.zeros(0, dtype=torch.int32, device=dev), 0, 0, False, m1d, empty, pl,
        torch.from_numpy(m1_off).to(dev), eps, lr, 0.0, 0, 0.0)
    return Wd.cpu().numpy(), m1d.cpu().numpy()


def _eps_pin(dev, inp, seed, pooling=0):
    rng = np.random.default_rng(seed)
    # MEAN scales each slice by 1/L: a gradient L times larger keeps sqrt(h') at eps.
    L = np.diff(inp.offsets)
    sigma = 1e-8 * (float(L[L > 0].mean()) if pooling == 1 else 1.0)
    W, m1, grad = eps_pin_case(rng, inp, sigma)
    m1_off = np.concatenate([[0], np.cumsum(inp.E)[:-1]]).astype(np.int64)
    lr, eps = 0.01, 1e-8
    W_exp, m_exp = orc.backward_rowwise_adagrad(
        W, weight_offsets(inp), inp.D_offsets, inp.B, inp.hash_size_cumsum,
        inp.total_hash_size_bits, inp.indices, inp.offsets, pooling, grad, m1, m1_off, lr, eps,
        0.0, 0, orc.info_B_num_bits(inp.T, inp.B))
    touched = m_exp > 0
    ratio = np.sqrt(m_exp[touched]) / eps
    # The case is one where eps matters: sqrt(h') within a factor 4 of eps
    # for most touched rows.
    assert np.median(ratio) > 0.25 and np.median(ratio) < 4, np.median(ratio)
    Wg, mg = _backward_gpu(dev, inp, W, m1, m1_off, grad, pooling, lr, eps)
    assert_eps_pin_close(Wg, mg, W_exp, m_exp)
    # Rows the batch does not touch: bit-identical.
    keep = np.concatenate([np.repeat(~touched[m1_off[t]:m1_off[t] + E], D)
                           for t, (E, D) in enumerate(zip(inp.E, inp.D))])
    assert np.array_equal(Wg[keep], W[keep])


@pytest.mark.parametrize("pooling", [0, 1])
def test_eps_pin_small(dev, pooling):
    """Adagrad's eps where it matters: zero momentum, gradients N(0, 1e-8),
    so sqrt(h') is about eps and the update's denominator sqrt(h') + eps is
    about 2 eps.  A kernel with eps inside the root, or without it, is off by
    orders of magnitude or by 2x; the same check rejects those placements in
    a CPU copy of the rule (tests/test_adagrad_bounds.py)."""
    print(f"[case] eps pin small pooling={pooling}", flush=True)
    rng = np.random.default_rng(71 + pooling)
    inp = random_tbe(rng, 3, 64, [64, 64, 64], [400, 900, 50], 12)
    _eps_pin(dev, inp, 72 + pooling, pooling)


def test_eps_pin_config3_table(dev):
    """The eps pin on one full-size config-3 table: table 0 of config 2
    (E = 1M, D = 128, B = 4096, Zipf(1.05) indices with runs of thousands),
    gradients N(0, 1e-8), zero momentum, SUM; weights and momentum vs the
    oracle at rtol 1e-5."""
    print("[case] eps pin config3 table 0", flush=True)
    full = bench_inputs.config2()
    B = full.B
    inp = bench_inputs.TbeInput(T=1, E=[full.E[0]], D=[full.D[0]], B=B,
                                indices=full.indices[: int(full.offsets[B])].copy(),
                                offsets=full.offsets[: B + 1].copy())
    _eps_pin(dev, inp, 73)


@pytest.mark.parametrize("pooling", [0, 1])
def test_config3_full(dev, pooling):
    """Config 3: config-2 indices (Zipf 1.05, up to ~8k duplicates of one row),
    8 x 1M x 128 fp32 tables, grad N(0, 1e-2), lr 0.01, eps 1e-8, zero momentum
    (SUM, the config, and MEAN).  Transpose bit-exact; updated weights/momentum
    vs oracle at rtol 1e-5."""
    print(f"[case] config3 full size pooling={pooling}", flush=True)
    inp = bench_inputs.config2()
    _check_transpose(dev, inp)
    rng = np.random.default_rng(33)
    E, D, T = 1_000_000, 128, 8
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    Wd = torch.empty(T * E * D, device=dev).uniform_(-0.01, 0.01, generator=g)
    W = Wd.cpu().numpy()
    m1 = np.zeros(T * E, np.float32)
    m1d = torch.zeros(T * E, device=dev)
    grad = rng.normal(0, 1e-2, size=(inp.B, inp.total_D)).astype(np.float32)
    m1_off = (np.arange(T) * E).astype(np.int64)
    W_exp, m1_exp = orc.backward_rowwise_adagrad(
        W, weight_offsets(inp), inp.D_offsets, inp.B, inp.hash_size_cumsum,
        inp.total_hash_size_bits, inp.indices, inp.offsets, pooling, grad, m1, m1_off, 0.01, 1e-8,
        0.0, 0, orc.info_B_num_bits(T, inp.B))
    empty = torch.zeros(0, device=dev)
    torch.ops.fbgemm.split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_cuda(
        torch.from_numpy(grad).to(dev), Wd, empty, empty, torch.zeros(T, dtype=torch.int32, device=dev),
        torch.from_numpy(weight_offsets(inp)).to(dev), torch.from_numpy(inp.D_offsets).to(dev), D,
        torch.from_numpy(inp.hash_size_cumsum).to(dev), inp.total_hash_size_bits,
        torch.from_numpy(inp.indices).to(dev), torch.from_numpy(inp.offsets).to(dev), pooling,
        torch.zeros(0, dtype=torch.int32, device=dev), 0, 0, False, m1d, empty,
        torch.zeros(T, dtype=torch.int32, device=dev), torch.from_numpy(m1_off).to(dev),
        1e-8, 0.01, 0.0, 0, 0.0)
    mg = m1d.cpu().numpy()
    np.testing.assert_allclose(mg, m1_exp, rtol=RTOL, atol=0)
    touched = np.flatnonzero(m1_exp)
    Wg = Wd.cpu().numpy().reshape(T * E, D)
    np.testing.assert_allclose(Wg[touched], W_exp.reshape(T * E, D)[touched], rtol=RTOL, atol=ATOL)
    untouched = np.ones(T * E, bool)
    untouched[touched] = False
    assert np.array_equal(Wg[untouched], W.reshape(T * E, D)[untouched])


def test_module_training_step(dev):
    """SplitTableBatchedEmbeddingBagsCodegen: forward, loss.backward() applies
    the fused update; equals forward + oracle update."""
    print("[case] module training step", flush=True)
    from mx_fbgemm import ComputeDevice, EmbeddingLocation, PoolingMode
    from mx_fbgemm.split_table_batched_embeddings_ops_training import (
        SplitTableBatchedEmbeddingBagsCodegen,
    )

    specs = [(500, 64, EmbeddingLocation.DEVICE, ComputeDevice.CUDA),
             (300, 128, EmbeddingLocation.DEVICE, ComputeDevice.CUDA)]
    tbe = SplitTableBatchedEmbeddingBagsCodegen(specs, pooling_mode=PoolingMode.MEAN,
                                                learning_rate=0.05, eps=1e-6, device=dev)
    rng = np.random.default_rng(9)
    inp = random_tbe(rng, 2, 32, [64, 128], [500, 300], 10)
    W0 = tbe.weights_dev.detach().cpu().numpy().copy()
    out = tbe(torch.from_numpy(inp.indices).to(dev), torch.from_numpy(inp.offsets).to(dev))
    exp = orc.tbe_forward_f32(W0, weight_offsets(inp), inp.D_offsets, inp.B, inp.indices,
                              inp.offsets, 1)
    assert np.array_equal(out.detach().cpu().numpy(), exp)
    gout = torch.from_numpy(rng.normal(0, 1, size=out.shape).astype(np.float32)).to(dev)
    out.backward(gout)
    W_exp, m_exp = orc.backward_rowwise_adagrad(
        W0, weight_offsets(inp), inp.D_offsets, inp.B, inp.hash_size_cumsum,
        inp.total_hash_size_bits, inp.indices, inp.offsets, 1, gout.cpu().numpy(),
        np.zeros(800, np.float32), np.array([0, 500], np.int64), 0.05, 1e-6, 0.0, 0,
        orc.info_B_num_bits(2, 32))
    np.testing.assert_allclose(tbe.weights_dev.detach().cpu().numpy(), W_exp, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(tbe.momentum1_dev.cpu().numpy(), m_exp, rtol=RTOL, atol=0)


@pytest.mark.parametrize("pooling", [0, 1])
def test_module_training_step_weighted(dev, pooling):
    """Weighted training lookup through the module: forward bit-exact vs the
    oracle, per-sample weight gradient (table 1 masked by
    feature_requires_grad) and the fused weighted update vs the oracle."""
    print(f"[case] module weighted training step pool={pooling}", flush=True)
    from mx_fbgemm import ComputeDevice, EmbeddingLocation, PoolingMode
    from mx_fbgemm.split_table_batched_embeddings_ops_training import (
        SplitTableBatchedEmbeddingBagsCodegen,
    )

    specs = [(400, 32, EmbeddingLocation.DEVICE, ComputeDevice.CUDA),
             (200, 128, EmbeddingLocation.DEVICE, ComputeDevice.CUDA),
             (90, 256, EmbeddingLocation.DEVICE, ComputeDevice.CUDA)]
    tbe = SplitTableBatchedEmbeddingBagsCodegen(specs, pooling_mode=PoolingMode(pooling),
                                                learning_rate=0.05, eps=1e-6, device=dev)
    rng = np.random.default_rng(19)
    inp = random_tbe(rng, 3, 24, [32, 128, 256], [400, 200, 90], 12, empty_frac=0.1)
    iw = rng.uniform(0.1, 2.0, inp.N).astype(np.float32)
    psw = torch.from_numpy(iw).to(dev).requires_grad_()
    frg = torch.tensor([1, 0, 1], dtype=torch.int32, device=dev)
    W0 = tbe.weights_dev.detach().cpu().numpy().copy()
    out = tbe(torch.from_numpy(inp.indices).to(dev), torch.from_numpy(inp.offsets).to(dev), psw,
              frg)
    exp = orc.tbe_forward_f32(W0, weight_offsets(inp), inp.D_offsets, inp.B, inp.indices,
                              inp.offsets, pooling, iw)
    assert np.array_equal(out.detach().cpu().numpy(), exp)
    gout_np = rng.normal(0, 1, size=out.shape).astype(np.float32)
    out.backward(torch.from_numpy(gout_np).to(dev))
    giw = orc.grad_indice_weights(gout_np, W0, weight_offsets(inp), inp.D_offsets, inp.B,
                                  inp.indices, inp.offsets, pooling, frg.cpu().numpy())
    mag = orc.grad_indice_weights(np.abs(gout_np), np.abs(W0), weight_offsets(inp),
                                  inp.D_offsets, inp.B, inp.indices, inp.offsets, pooling)
    got = psw.grad.cpu().numpy()
    assert np.all(np.abs(got - giw) <= 1e-5 * mag + 1e-30)
    W_exp, m_exp = orc.backward_rowwise_adagrad(
        W0, weight_offsets(inp), inp.D_offsets, inp.B, inp.hash_size_cumsum,
        inp.total_hash_size_bits, inp.indices, inp.offsets, pooling, gout_np,
        np.zeros(690, np.float32), np.array([0, 400, 600], np.int64), 0.05, 1e-6, 0.0, 0,
        orc.info_B_num_bits(3, 24), indice_weights=iw)
    np.testing.assert_allclose(tbe.weights_dev.detach().cpu().numpy(), W_exp, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(tbe.momentum1_dev.cpu().numpy(), m_exp, rtol=RTOL, atol=0)


# ---- fp16 weights: round-to-nearest-even or stochastic rounding -------------

def _f16_bracket(u: np.ndarray, w_old: np.ndarray, rel: float = 2e-6):
    """fp16 values bracketing fp32 ``u`` = w_old - m*g, widened by ``rel``
    times the operands' magnitude |w_old| + |u| (the GPU's fp32 update may
    differ from the oracle's in the last bits of m*g -- its sum of squares is
    reduced in another order -- which matters most when u nearly cancels):
    (lower, upper)."""
    widen = (np.abs(u) + np.abs(w_old.astype(np.float32))) * rel
    a = u - widen
    b = u + widen
    la = a.astype(np.float16)
    la = np.where(la.astype(np.float32) > a, np.nextafter(la, np.float16(-np.inf)), la)
    hb = b.astype(np.float16)
    hb = np.where(hb.astype(np.float32) < b, np.nextafter(hb, np.float16(np.inf)), hb)
    return la, hb


def _fp16_update(dev, inp, sr, seed=0, lr=0.05, eps=1e-6, pooling=0, weighted=False):
    rng = np.random.default_rng(seed)
    W16 = rng.uniform(-1, 1, size=sum(E * D for E, D in zip(inp.E, inp.D))).astype(np.float16)
    m1 = rng.uniform(0, 1e-3, size=sum(inp.E)).astype(np.float32)
    m1_off = np.concatenate([[0], np.cumsum(inp.E)[:-1]]).astype(np.int64)
    grad = rng.normal(0, 1e-1, size=(inp.B, inp.total_D)).astype(np.float32)
    iw = rng.uniform(0.5, 1.5, inp.N).astype(np.float32) if weighted else None
    u, m1_exp = orc.backward_rowwise_adagrad(
        W16.astype(np.float32), weight_offsets(inp), inp.D_offsets, inp.B, inp.hash_size_cumsum,
        inp.total_hash_size_bits, inp.indices, inp.offsets, pooling, grad, m1, m1_off, lr, eps,
        0.0, 0, orc.info_B_num_bits(inp.T, inp.B), indice_weights=iw)
    Wd = torch.from_numpy(W16).to(dev)
    m1d = torch.from_numpy(m1).to(dev)
    empty = torch.zeros(0, device=dev)
    head = (torch.from_numpy(grad).to(dev), Wd, empty, empty,
            torch.zeros(inp.T, dtype=torch.int32, device=dev),
            torch.from_numpy(weight_offsets(inp)).to(dev), torch.from_numpy(inp.D_offsets).to(dev),
            max(inp.D), torch.from_numpy(inp.hash_size_cumsum).to(dev), inp.total_hash_size_bits,
            torch.from_numpy(inp.indices).to(dev), torch.from_numpy(inp.offsets).to(dev), pooling)
    tail = (torch.zeros(0, dtype=torch.int32, device=dev), 0, 0, sr, m1d, empty,
            torch.zeros(inp.T, dtype=torch.int32, device=dev), torch.from_numpy(m1_off).to(dev),
            eps, lr, 0.0, 0, 0.0)
    if weighted:
        torch.ops.fbgemm.split_embedding_backward_codegen_rowwise_adagrad_weighted_exact_cuda(
            *head, torch.from_numpy(iw).to(dev), *tail)
    else:
        torch.ops.fbgemm.split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_cuda(
            *head, *tail)
    np.testing.assert_allclose(m1d.cpu().numpy(), m1_exp, rtol=RTOL, atol=0)
    got = Wd.cpu().numpy()
    untouched = u == W16.astype(np.float32)
    assert np.array_equal(got[untouched].view(np.uint16), W16[untouched].view(np.uint16))
    lo, hi = _f16_bracket(u, W16)
    gf = got.astype(np.float32)
    out = (gf < lo.astype(np.float32)) | (gf > hi.astype(np.float32))
    assert not out.any(), f"{out.sum()} fp16 results outside the bracket of the fp32 update"
    return got, u, ~untouched


@pytest.mark.parametrize("pooling", [0, 1])
@pytest.mark.parametrize("weighted", [False, True])
def test_fp16_weights_round_to_nearest(dev, pooling, weighted):
    """stochastic_rounding=False: the fp16 result is the fp32 update rounded
    to nearest even (equal to numpy's rounding of the oracle's fp32 update
    except within a few fp32 ulps of a tie)."""
    print(f"[case] fp16 weights RNE pool={pooling} weighted={weighted}", flush=True)
    rng = np.random.default_rng(41)
    inp = random_tbe(rng, 2, 300, [128, 64], [2000, 500], 20)
    got, u, touched = _fp16_update(dev, inp, False, seed=3, pooling=pooling, weighted=weighted)
    rn = u.astype(np.float16)
    same = got[touched].view(np.uint16) == rn[touched].view(np.uint16)
    assert same.mean() > 0.995, same.mean()


def _sr_statistics(got, u, touched):
    """Fraction of elements rounded away from zero, per decile of their
    distance from the toward-zero neighbour (in fp16 places)."""
    uz = u[touched]
    g = got[touched].astype(np.float32)
    rz = uz.astype(np.float16)  # RNE first, then step toward zero where it overshot
    rz = np.where(np.abs(rz.astype(np.float32)) > np.abs(uz),
                  np.nextafter(rz, np.float16(0)), rz)
    ulp = np.abs(np.nextafter(rz, np.sign(uz).astype(np.float16) * np.float16(np.inf))
                 .astype(np.float32) - rz.astype(np.float32))
    f = (np.abs(uz) - np.abs(rz.astype(np.float32))) / ulp
    away = g != rz.astype(np.float32)
    keep = (f > 1e-3) & (f < 1 - 1e-3) & np.isfinite(f)  # skip (near-)representable values
    return f[keep], away[keep]


def test_fp16_weights_stochastic_rounding(dev):
    """stochastic_rounding=True: every result is one of the two fp16
    neighbours of the fp32 update, rounded away from zero with probability
    equal to its distance from the toward-zero neighbour (checked per decile
    over ~200k elements), and the same torch seed gives the same result."""
    print("[case] fp16 weights stochastic rounding", flush=True)
    rng = np.random.default_rng(43)
    inp = random_tbe(rng, 2, 1024, [128, 128], [1500, 1500], 30, empty_frac=0.0)
    torch.manual_seed(123)
    got, u, touched = _fp16_update(dev, inp, True, seed=5)
    f, away = _sr_statistics(got, u, touched)
    assert f.size > 100_000, f.size
    for lo_ in np.arange(0, 1, 0.1):
        sel = (f >= lo_) & (f < lo_ + 0.1)
        assert sel.sum() > 2000
        p = away[sel].mean()
        assert abs(p - f[sel].mean()) < 0.03, (lo_, p, f[sel].mean())
    torch.manual_seed(123)
    again, _, _ = _fp16_update(dev, inp, True, seed=5)
    assert np.array_equal(again.view(np.uint16), got.view(np.uint16))
    torch.manual_seed(124)
    other, _, _ = _fp16_update(dev, inp, True, seed=5)
    assert not np.array_equal(other.view(np.uint16), got.view(np.uint16))


@pytest.mark.parametrize("sr", [False, True])
def test_module_training_step_fp16(dev, sr):
    """fp16 weights through the module (weighted, per-sample-weight gradient):
    forward bit-exact vs the oracle on the widened weights; the update within
    the fp16 bracket of the oracle's fp32 update."""
    print(f"[case] module fp16 training step sr={sr}", flush=True)
    from mx_fbgemm import ComputeDevice, EmbeddingLocation, PoolingMode, SparseType
    from mx_fbgemm.split_table_batched_embeddings_ops_training import (
        SplitTableBatchedEmbeddingBagsCodegen,
    )

    specs = [(300, 64, EmbeddingLocation.DEVICE, ComputeDevice.CUDA),
             (200, 128, EmbeddingLocation.DEVICE, ComputeDevice.CUDA)]
    tbe = SplitTableBatchedEmbeddingBagsCodegen(
        specs, pooling_mode=PoolingMode.SUM, learning_rate=0.05, eps=1e-6, device=dev,
        weights_init=(-1.0, 1.0), weights_precision=SparseType.FP16, stochastic_rounding=sr)
    assert tbe.weights_dev.dtype == torch.float16
    rng = np.random.default_rng(17)
    inp = random_tbe(rng, 2, 40, [64, 128], [300, 200], 10)
    iw = rng.uniform(0.5, 1.5, inp.N).astype(np.float32)
    psw = torch.from_numpy(iw).to(dev).requires_grad_()
    W0 = tbe.weights_dev.detach().cpu().numpy().copy()
    out = tbe(torch.from_numpy(inp.indices).to(dev), torch.from_numpy(inp.offsets).to(dev), psw)
    exp = orc.tbe_forward_f32(W0, weight_offsets(inp), inp.D_offsets, inp.B, inp.indices,
                              inp.offsets, 0, iw)
    assert out.dtype == torch.float32 and np.array_equal(out.detach().cpu().numpy(), exp)
    gout = rng.normal(0, 1, size=out.shape).astype(np.float32)
    out.backward(torch.from_numpy(gout).to(dev))
    giw = orc.grad_indice_weights(gout, W0, weight_offsets(inp), inp.D_offsets, inp.B,
                                  inp.indices, inp.offsets, 0)
    mag = orc.grad_indice_weights(np.abs(gout), np.abs(W0).astype(np.float32),
                                  weight_offsets(inp), inp.D_offsets, inp.B, inp.indices,
                                  inp.offsets, 0)
    assert np.all(np.abs(psw.grad.cpu().numpy() - giw) <= 1e-5 * mag + 1e-30)
    u, m_exp = orc.backward_rowwise_adagrad(
        W0.astype(np.float32), weight_offsets(inp), inp.D_offsets, inp.B, inp.hash_size_cumsum,
        inp.total_hash_size_bits, inp.indices, inp.offsets, 0, gout, np.zeros(500, np.float32),
        np.array([0, 300], np.int64), 0.05, 1e-6, 0.0, 0, orc.info_B_num_bits(2, 40),
        indice_weights=iw)
    np.testing.assert_allclose(tbe.momentum1_dev.cpu().numpy(), m_exp, rtol=RTOL, atol=0)
    got = tbe.weights_dev.detach().cpu().numpy().astype(np.float32)
    lo, hi = _f16_bracket(u, W0)
    assert np.all((got >= lo.astype(np.float32)) & (got <= hi.astype(np.float32)))


def test_lookback_giveup_is_reported_and_leaves_outputs_alone(dev):
    """Forced from the host (a test hook makes every look-back wait give up at
    once; every kernel still exits normally): the transpose returns an empty
    run layout, the backward leaves weights and momentum alone, and the next
    call on the device raises."""
    print("[case] forced look-back give-up", flush=True)
    rng = np.random.default_rng(21)
    inp = random_tbe(rng, 3, 2048, [64] * 3, [5000, 300, 70000], 20)  # ~12 sort tiles
    nb = orc.info_B_num_bits(inp.T, inp.B)
    _check_transpose(dev, inp)  # registers the device's failure word
    W0 = rng.uniform(-0.01, 0.01, size=sum(E * D for E, D in zip(inp.E, inp.D))).astype(np.float32)
    W = torch.from_numpy(W0).to(dev)
    m1 = torch.zeros(sum(inp.E), device=dev)
    grad = torch.from_numpy(rng.normal(0, 1e-2, (inp.B, inp.total_D)).astype(np.float32)).to(dev)
    w_off = torch.from_numpy(weight_offsets(inp)).to(dev)
    m_off = torch.from_numpy(np.concatenate([[0], np.cumsum(inp.E)[:-1]]).astype(np.int64)).to(dev)
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(inp.T, dtype=torch.int32, device=dev)
    e32 = torch.zeros(0, dtype=torch.int32, device=dev)

    def backward():
        torch.ops.fbgemm.split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_cuda(
            grad, W, empty, empty, pl, w_off, torch.from_numpy(inp.D_offsets).to(dev),
            max(inp.D), torch.from_numpy(inp.hash_size_cumsum).to(dev),
            inp.total_hash_size_bits, torch.from_numpy(inp.indices).to(dev),
            torch.from_numpy(inp.offsets).to(dev), 0, e32, 0, 0, False, m1, empty, pl, m_off,
            1e-8, 0.05, 0.0, 0, 0.0)

    # A failed transpose returns an empty layout: no runs, every run length 0,
    # the whole cumsum 0 (not memory left as allocated).
    torch.ops.mx_fbgemm.test_force_lookback_giveup(True)
    try:
        _, _, _, _, lengths, num_runs, cum = _transpose_gpu(dev, inp, nb)
        torch.cuda.synchronize()
    finally:
        torch.ops.mx_fbgemm.test_force_lookback_giveup(False)
    assert int(num_runs.item()) == 0
    assert not lengths.any() and not cum.any(), "a failed transpose left a non-empty layout"
    with pytest.raises(RuntimeError, match="gave up a look-back wait"):
        _transpose_gpu(dev, inp, nb)
    _check_transpose(dev, inp)

    torch.ops.mx_fbgemm.test_force_lookback_giveup(True)
    try:
        backward()
        torch.cuda.synchronize()
    finally:
        torch.ops.mx_fbgemm.test_force_lookback_giveup(False)
    assert np.array_equal(W.cpu().numpy(), W0) and not m1.any(), "a failed call updated rows"
    with pytest.raises(RuntimeError, match="gave up a look-back wait"):
        _transpose_gpu(dev, inp, nb)
    # Reported once; the same calls then run normally.
    _check_transpose(dev, inp)
    backward()
    torch.cuda.synchronize()
    assert not np.array_equal(W.cpu().numpy(), W0)
    assert torch.ops.mx_fbgemm.pending_lookback_faults(0) == 0


def test_counter_region_matches_workspace_counters(dev):
    """Eager backward calls keep the sort's digit counters in a region of
    their stream that each call's last kernel clears for the next call.
    Batches of different shapes in turn (40 features, then 3, then one table
    with long runs, then 3 radix passes) give bit-identical weights with the
    region and with the counters cleared in the workspace by one more kernel
    (the graph-capture form), and both match the oracle."""
    rng = np.random.default_rng(77)
    cases = [
        random_tbe(rng, 40, 24, [16] * 40, [300] * 40, 12),
        random_tbe(rng, 3, 200, [4, 64, 256], [50, 2000, 40], 30),
        random_tbe(rng, 1, 300, [128], [7], 40, dup_heavy=True),
        random_tbe(rng, 5, 700, [4] * 5, [2 ** 20, 3, 100, 9, 2 ** 21], 10),
    ]
    for i, inp in enumerate(cases):
        print(f"[case] counter region, batch {i} (T={inp.T})", flush=True)
        got_region, _ = _backward_case(dev, inp, i % 2, seed=i)
        torch.ops.mx_fbgemm.test_force_workspace_counters(True)
        try:
            got_ws, _ = _backward_case(dev, inp, i % 2, seed=i)
        finally:
            torch.ops.mx_fbgemm.test_force_workspace_counters(False)
        assert np.array_equal(got_region, got_ws)


def test_counter_region_after_a_failed_call(dev):
    """A backward whose look-backs give up (forced from the host; every
    kernel still exits normally) has already added into its stream's counter
    region; its last kernel clears it all the same, so the next backward on
    the stream matches the oracle."""
    print("[case] counter region after a forced look-back give-up", flush=True)
    rng = np.random.default_rng(23)
    inp = random_tbe(rng, 3, 2048, [64] * 3, [5000, 300, 70000], 20)
    nb = orc.info_B_num_bits(inp.T, inp.B)
    _check_transpose(dev, inp)  # registers the device's failure word
    W = rng.uniform(-0.01, 0.01, size=sum(E * D for E, D in zip(inp.E, inp.D))).astype(np.float32)
    m1 = np.zeros(sum(inp.E), dtype=np.float32)
    m1_off = np.concatenate([[0], np.cumsum(inp.E)[:-1]]).astype(np.int64)
    grad = rng.normal(0, 1e-2, (inp.B, inp.total_D)).astype(np.float32)
    torch.ops.mx_fbgemm.test_force_lookback_giveup(True)
    try:
        Wg, mg = _backward_gpu(dev, inp, W, m1, m1_off, grad, 0, 0.01, 1e-8)
    finally:
        torch.ops.mx_fbgemm.test_force_lookback_giveup(False)
    assert np.array_equal(Wg, W) and not mg.any()
    with pytest.raises(RuntimeError, match="gave up a look-back wait"):
        _transpose_gpu(dev, inp, nb)
    _backward_case(dev, inp, 0, seed=5)
    _backward_case(dev, inp, 1, seed=6)
