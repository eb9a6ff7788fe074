"""GPU parity of the sparse-feature helpers against the oracle, bit-exact:
asynchronous_{exclusive,inclusive,complete}_cumsum (int32/int64, 1-D and
2-D, sizes around the 8192-element tile, wrap-around),
permute_2D_sparse_data / permute_1D_sparse_data (repeats, dropped and
out-of-range features, weights, with and without permuted_lengths_sum),
offsets_range and expand_into_jagged_permute."""

import numpy as np
import pytest
import torch

import oracle as orc

pytestmark = pytest.mark.gpu

OPS = {0: "asynchronous_exclusive_cumsum", 1: "asynchronous_inclusive_cumsum",
       2: "asynchronous_complete_cumsum"}


@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("dtype", [np.int32, np.int64])
@pytest.mark.parametrize("n", [0, 1, 5, 8191, 8192, 8193, 100_000, 3_000_000, 9_000_000])
def test_cumsum(dev, kind, dtype, n):
    print(f"[case] cumsum kind={kind} dtype={np.dtype(dtype).name} n={n}", flush=True)
    rng = np.random.default_rng(n + kind)
    x = rng.integers(0, 50, n).astype(dtype)
    got = getattr(torch.ops.fbgemm, OPS[kind])(torch.from_numpy(x).to(dev))
    np.testing.assert_array_equal(got.cpu().numpy(), orc.cumsum(x, kind))


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
def test_cumsum_wraps(dev, dtype):
    """Sums past the type's range wrap as its integer adds do (two's complement)."""
    print(f"[case] cumsum wrap {np.dtype(dtype).name}", flush=True)
    big = np.iinfo(dtype).max // 3
    rng = np.random.default_rng(1)
    x = (rng.integers(0, 2, 20_000) * big - rng.integers(0, 1000, 20_000)).astype(dtype)
    for kind in (0, 1, 2):
        got = getattr(torch.ops.fbgemm, OPS[kind])(torch.from_numpy(x).to(dev))
        np.testing.assert_array_equal(got.cpu().numpy(), orc.cumsum(x, kind))


@pytest.mark.parametrize("rows,n", [(1, 7), (3, 0), (100, 37), (5, 20_000), (2, 100_000)])
@pytest.mark.parametrize("dtype", [np.int32, np.int64])
def test_complete_cumsum_2d(dev, rows, n, dtype):
    print(f"[case] complete cumsum 2-D rows={rows} n={n}", flush=True)
    rng = np.random.default_rng(rows * 7 + n)
    x = rng.integers(-20, 50, (rows, n)).astype(dtype)
    got = torch.ops.fbgemm.asynchronous_complete_cumsum(torch.from_numpy(x).to(dev))
    assert got.shape == (rows, n + 1)
    np.testing.assert_array_equal(got.cpu().numpy(), orc.cumsum(x, 2))


@pytest.mark.parametrize("ldtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("idtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("given_sum", [False, True])
def test_permute_2d_sparse_data(dev, ldtype, idtype, weighted, given_sum):
    print(f"[case] permute_2D l={ldtype} i={idtype} w={weighted} sum={given_sum}", flush=True)
    rng = np.random.default_rng(int(weighted) + 2 * int(given_sum))
    T, B = 6, 300
    lengths = rng.integers(0, 30, (T, B))
    lengths[2] = 0  # an empty feature
    n = int(lengths.sum())
    idx = rng.integers(0, 10**6, n)
    w = rng.standard_normal(n).astype(np.float32) if weighted else None
    permute = np.array([3, 0, 5, 5, 1, 2, 4, 0], np.int32)  # repeats; every feature kept
    exp_l, exp_i, exp_w = orc.permute_2d_sparse_data(permute, lengths, idx, w)
    psum = int(exp_l.sum()) if given_sum else None
    pl, pi, pw = torch.ops.fbgemm.permute_2D_sparse_data(
        torch.from_numpy(permute).to(dev), torch.from_numpy(lengths).to(dev, ldtype),
        torch.from_numpy(idx).to(dev, idtype),
        None if w is None else torch.from_numpy(w).to(dev), psum)
    np.testing.assert_array_equal(pl.cpu().numpy(), exp_l)
    np.testing.assert_array_equal(pi.cpu().numpy(), exp_i)
    if weighted:
        np.testing.assert_array_equal(pw.cpu().numpy(), exp_w)
    else:
        assert pw is None


def test_permute_2d_sparse_data_subset(dev):
    """A permute that drops features, and one naming a feature past T (zero lengths)."""
    print("[case] permute_2D subset", flush=True)
    rng = np.random.default_rng(9)
    T, B = 5, 64
    lengths = rng.integers(0, 9, (T, B))
    idx = rng.integers(0, 500, int(lengths.sum()))
    permute = np.array([4, 1, 7], np.int32)
    exp_l, exp_i, _ = orc.permute_2d_sparse_data(permute, lengths, idx)
    pl, pi, pw = torch.ops.fbgemm.permute_2D_sparse_data(
        torch.from_numpy(permute).to(dev), torch.from_numpy(lengths).to(dev),
        torch.from_numpy(idx).to(dev))
    np.testing.assert_array_equal(pl.cpu().numpy(), exp_l)
    np.testing.assert_array_equal(pi.cpu().numpy(), exp_i)
    assert pw is None


@pytest.mark.parametrize("weighted", [False, True])
def test_permute_1d_sparse_data(dev, weighted):
    print(f"[case] permute_1D w={weighted}", flush=True)
    rng = np.random.default_rng(21)
    T = 40
    lengths = rng.integers(0, 50, T)
    idx = rng.integers(0, 10**6, int(lengths.sum()))
    w = rng.standard_normal(idx.size).astype(np.float32) if weighted else None
    permute = rng.permutation(T).astype(np.int32)[:30]
    exp_l, exp_i, exp_w = orc.permute_2d_sparse_data(permute, lengths[:, None], idx, w)
    pl, pi, pw = torch.ops.fbgemm.permute_1D_sparse_data(
        torch.from_numpy(permute).to(dev), torch.from_numpy(lengths).to(dev),
        torch.from_numpy(idx).to(dev), None if w is None else torch.from_numpy(w).to(dev))
    np.testing.assert_array_equal(pl.cpu().numpy(), exp_l.reshape(-1))
    np.testing.assert_array_equal(pi.cpu().numpy(), exp_i)
    if weighted:
        np.testing.assert_array_equal(pw.cpu().numpy(), exp_w)


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
def test_offsets_range(dev, dtype):
    print(f"[case] offsets_range {np.dtype(dtype).name}", flush=True)
    rng = np.random.default_rng(22)
    lengths = rng.integers(0, 100, 5000)
    lengths[::7] = 0
    off = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(dtype)
    n = int(lengths.sum())
    got = torch.ops.fbgemm.offsets_range(torch.from_numpy(off).to(dev), n)
    np.testing.assert_array_equal(got.cpu().numpy(), orc.offsets_range(off, n))


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
@pytest.mark.parametrize("with_end", [False, True])
def test_expand_into_jagged_permute(dev, dtype, with_end):
    print(f"[case] expand_into_jagged_permute {np.dtype(dtype).name} end={with_end}", flush=True)
    rng = np.random.default_rng(23)
    T = 300
    in_len = rng.integers(0, 40, T)
    in_off = np.concatenate([[0], np.cumsum(in_len)[:-1]]).astype(dtype)
    permute = rng.permutation(T).astype(np.int32)
    out_len = in_len[permute]
    out_off = np.concatenate([[0], np.cumsum(out_len)]).astype(dtype)
    size = int(out_len.sum())
    oo = out_off if with_end else out_off[:-1]
    got = torch.ops.fbgemm.expand_into_jagged_permute(
        torch.from_numpy(permute).to(dev), torch.from_numpy(in_off).to(dev),
        torch.from_numpy(oo).to(dev), size)
    np.testing.assert_array_equal(got.cpu().numpy(),
                                  orc.expand_into_jagged_permute(permute, in_off, oo, size))


@pytest.mark.parametrize("T,B,Tp", [(8, 8192, 8), (8, 8192, 9), (3, 30000, 3), (1, 70000, 2)])
@pytest.mark.parametrize("ldtype", [torch.int32, torch.int64])
def test_permute_2d_sparse_data_sizes(dev, T, B, Tp, ldtype):
    """Batches of 65,536 bags and more (cumsums over several 8192-element
    tiles), more output features than input ones, and one feature copied twice."""
    print(f"[case] permute_2D sizes T={T} B={B} Tp={Tp} l={ldtype}", flush=True)
    rng = np.random.default_rng(T * B + Tp)
    lengths = rng.integers(0, 6, (T, B))
    idx = rng.integers(0, 10**6, int(lengths.sum()))
    permute = rng.integers(0, T, Tp).astype(np.int32)
    exp_l, exp_i, _ = orc.permute_2d_sparse_data(permute, lengths, idx)
    pl, pi, pw = torch.ops.fbgemm.permute_2D_sparse_data(
        torch.from_numpy(permute).to(dev), torch.from_numpy(lengths).to(dev, ldtype),
        torch.from_numpy(idx).to(dev))
    np.testing.assert_array_equal(pl.cpu().numpy(), exp_l)
    np.testing.assert_array_equal(pi.cpu().numpy(), exp_i)
    assert pw is None
