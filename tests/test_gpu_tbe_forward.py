"""GPU parity of the TBE fp32 training forward against the C oracle.

Each output column is accumulated in index order on the GPU (one wave per
bag, lanes own columns), exactly like the oracle's sequential loop, so the
fp32 SUM/MEAN results are compared bit for bit -- stricter than the stated
fp32 tolerance (rtol 1e-5)."""

import numpy as np
import pytest
import torch

import oracle as orc
from mx_fbgemm import bench_inputs
from tbe_helpers import random_tbe, tbe_forward_gpu, weight_offsets

pytestmark = pytest.mark.gpu


def _exact(got: torch.Tensor, exp: np.ndarray):
    g = got.cpu().numpy()
    assert g.shape == exp.shape
    if not np.array_equal(g.view(np.uint32 if g.dtype == np.float32 else np.uint16),
                          exp.view(np.uint32 if exp.dtype == np.float32 else np.uint16)):
        bad = np.argwhere(g != exp)
        raise AssertionError(f"{bad.shape[0]} mismatches, first {bad[:3].tolist()}: "
                             f"got {g[tuple(bad[0])]}, expected {exp[tuple(bad[0])]}")


SHAPES = [
    # T, B, dims, rows, max_L
    (1, 1, [4], [3], 1),
    (3, 17, [8, 128, 36], [50, 100, 7], 9),
    (2, 64, [64, 64], [1000, 1000], 70),          # bags longer than 64 indices
    (4, 33, [256, 512, 1024, 132], [20, 20, 20, 20], 6),
    (2, 5, [128, 128], [10, 10], 0),              # all bags empty
]


@pytest.mark.parametrize("T,B,dims,rows,max_L", SHAPES)
@pytest.mark.parametrize("pooling", [0, 1])
@pytest.mark.parametrize("index_dtype", [torch.int64, torch.int32])
def test_forward_matches_oracle(dev, T, B, dims, rows, max_L, pooling, index_dtype):
    print(f"[case] tbe fwd T={T} B={B} dims={dims} pool={pooling} {index_dtype}", flush=True)
    rng = np.random.default_rng(10 + T * B)
    inp = random_tbe(rng, T, B, dims, rows, max_L)
    W = rng.uniform(-0.01, 0.01, size=sum(E * D for E, D in zip(rows, dims))).astype(np.float32)
    exp = orc.tbe_forward_f32(W, weight_offsets(inp), inp.D_offsets, B, inp.indices, inp.offsets,
                              pooling)
    got = tbe_forward_gpu(dev, torch.from_numpy(W).to(dev), inp, pooling, index_dtype)
    _exact(got, exp)


@pytest.mark.parametrize("T,B,dims,rows,max_L", SHAPES[1:4])
@pytest.mark.parametrize("pooling", [0, 1])
@pytest.mark.parametrize("weighted", [False, True])
def test_fp16_weights_match_oracle(dev, T, B, dims, rows, max_L, pooling, weighted):
    """fp16 weight rows, fp32 output: each weight widened to fp32, summed in
    index order -- bit-exact to the oracle (itself bit-exact to FBGEMM's
    fp16-input CPU kernel)."""
    print(f"[case] tbe fwd fp16 weights T={T} B={B} dims={dims} pool={pooling} w={weighted}",
          flush=True)
    rng = np.random.default_rng(20 + T * B)
    inp = random_tbe(rng, T, B, dims, rows, max_L)
    W16 = rng.uniform(-1, 1, size=sum(E * D for E, D in zip(rows, dims))).astype(np.float16)
    iw = rng.uniform(0, 2, size=inp.N).astype(np.float32) if weighted else None
    exp = orc.tbe_forward_f32(W16, weight_offsets(inp), inp.D_offsets, B, inp.indices,
                              inp.offsets, pooling, iw)
    got = tbe_forward_gpu(dev, torch.from_numpy(W16).to(dev), inp, pooling,
                          indice_weights=None if iw is None else torch.from_numpy(iw))
    _exact(got, exp)


@pytest.mark.parametrize("pooling", [0, 1])
def test_weighted_and_fp16_out(dev, pooling):
    print(f"[case] tbe fwd weighted + fp16 out pool={pooling}", flush=True)
    rng = np.random.default_rng(7)
    inp = random_tbe(rng, 3, 20, [32, 128, 64], [40, 40, 40], 12)
    W = rng.uniform(-1, 1, size=sum(E * D for E, D in zip(inp.E, inp.D))).astype(np.float32)
    iw = rng.uniform(0, 2, size=inp.N).astype(np.float32)
    exp = orc.tbe_forward_f32(W, weight_offsets(inp), inp.D_offsets, inp.B, inp.indices,
                              inp.offsets, pooling, iw)
    got = tbe_forward_gpu(dev, torch.from_numpy(W).to(dev), inp, pooling,
                          indice_weights=torch.from_numpy(iw))
    _exact(got, exp)
    got16 = tbe_forward_gpu(dev, torch.from_numpy(W).to(dev), inp, pooling, output_dtype=1)
    exp32 = orc.tbe_forward_f32(W, weight_offsets(inp), inp.D_offsets, inp.B, inp.indices,
                                inp.offsets, pooling)
    _exact(got16, exp32.astype(np.float16))


def test_duplicate_heavy_and_repeatable(dev):
    print("[case] tbe fwd duplicates, determinism", flush=True)
    rng = np.random.default_rng(8)
    inp = random_tbe(rng, 2, 100, [128, 128], [1000, 1000], 40, dup_heavy=True)
    W = rng.uniform(-0.01, 0.01, size=2 * 1000 * 128).astype(np.float32)
    Wd = torch.from_numpy(W).to(dev)
    a = tbe_forward_gpu(dev, Wd, inp, 0)
    b = tbe_forward_gpu(dev, Wd, inp, 0)
    assert torch.equal(a, b)
    _exact(a, orc.tbe_forward_f32(W, weight_offsets(inp), inp.D_offsets, inp.B, inp.indices,
                                  inp.offsets, 0))


@pytest.mark.parametrize("pooling", [0, 1])
def test_many_tables(dev, pooling):
    """700 tables (past the 512 whose metadata the kernels stage in LDS), mixed
    D and row counts, bit-exact."""
    print(f"[case] tbe fwd 700 tables pool={pooling}", flush=True)
    rng = np.random.default_rng(700 + pooling)
    T, B = 700, 6
    dims = [int(d) for d in rng.choice([4, 8, 16, 64, 128], T)]
    rows = [int(r) for r in rng.integers(1, 60, T)]
    inp = random_tbe(rng, T, B, dims, rows, 5)
    W = rng.uniform(-1, 1, size=sum(E * D for E, D in zip(rows, dims))).astype(np.float32)
    exp = orc.tbe_forward_f32(W, weight_offsets(inp), inp.D_offsets, B, inp.indices, inp.offsets,
                              pooling)
    _exact(tbe_forward_gpu(dev, torch.from_numpy(W).to(dev), inp, pooling), exp)


def test_config2_full(dev):
    """Config 2 at full size (8 x 1M x 128 fp32, B=4096, Zipf 1.05): every bag
    bit-exact against the oracle."""
    print("[case] config2 full size", flush=True)
    inp = bench_inputs.config2()
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    W = torch.empty(8 * 1_000_000 * 128, device=dev).uniform_(-0.01, 0.01, generator=g)
    got = tbe_forward_gpu(dev, W, inp, 0)
    Wh = W.cpu().numpy()
    exp = orc.tbe_forward_f32(Wh, weight_offsets(inp), inp.D_offsets, inp.B, inp.indices,
                              inp.offsets, 0)
    _exact(got, exp)
    # Size-independent property: the sum over the batch of table t's slice
    # equals the row-count-weighted sum of its rows (linearity).
    counts = np.bincount(inp.indices[: int(inp.offsets[inp.B])], minlength=1_000_000)
    t0 = Wh[: 1_000_000 * 128].reshape(1_000_000, 128).astype(np.float64)
    lin = counts.astype(np.float64) @ t0
    np.testing.assert_allclose(got[:, :128].double().sum(0).cpu().numpy(), lin, rtol=1e-4,
                               atol=1e-4)


def test_config2_full_mean_int32(dev):
    """Config 2's batch at full size with MEAN pooling and int32 indices and
    offsets: every bag bit-exact against the oracle (each column summed in
    index order, then scaled by 1/L)."""
    print("[case] config2 full size, MEAN, int32", flush=True)
    inp = bench_inputs.config2()
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    W = torch.empty(8 * 1_000_000 * 128, device=dev).uniform_(-0.01, 0.01, generator=g)
    got = tbe_forward_gpu(dev, W, inp, 1, torch.int32)
    exp = orc.tbe_forward_f32(W.cpu().numpy(), weight_offsets(inp), inp.D_offsets, inp.B,
                              inp.indices, inp.offsets, 1)
    _exact(got, exp)


def test_config2_full_fp16_weighted(dev):
    """Config 2's batch at full size with fp16 weight rows and per-sample
    weights (SUM): every bag bit-exact against the oracle."""
    print("[case] config2 full size, fp16 weights, weighted", flush=True)
    inp = bench_inputs.config2()
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    W = torch.empty(8 * 1_000_000 * 128, dtype=torch.float16, device=dev).uniform_(-1, 1, generator=g)
    iw = np.random.default_rng(3).uniform(0, 2, size=inp.N).astype(np.float32)
    got = tbe_forward_gpu(dev, W, inp, 0, indice_weights=torch.from_numpy(iw))
    exp = orc.tbe_forward_f32(W.cpu().numpy(), weight_offsets(inp), inp.D_offsets, inp.B,
                              inp.indices, inp.offsets, 0, iw)
    _exact(got, exp)


def test_unserved_arguments_raise(dev):
    """UVM storage and a populated LXU cache are refused, not ignored."""
    print("[case] tbe fwd unserved arguments", flush=True)
    rng = np.random.default_rng(3)
    inp = random_tbe(rng, 2, 4, [8, 8], [5, 5], 3)
    W = torch.zeros(80, device=dev)
    w_off = torch.from_numpy(weight_offsets(inp)).to(dev)
    D_off = torch.from_numpy(inp.D_offsets).to(dev)
    idx = torch.from_numpy(inp.indices).to(dev)
    off = torch.from_numpy(inp.offsets).to(dev)
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(2, dtype=torch.int32, device=dev)
    e32 = torch.zeros(0, dtype=torch.int32, device=dev)
    op = torch.ops.fbgemm.split_embedding_codegen_forward_unweighted_cuda
    with pytest.raises(RuntimeError, match="UVM"):
        op(W, torch.zeros(4, device=dev), empty, pl, w_off, D_off, 16, 8, idx, off, 0, e32, empty,
           0, False)
    with pytest.raises(RuntimeError, match="LXU cache"):
        op(W, empty, torch.zeros(3, 8, device=dev), pl, w_off, D_off, 16, 8, idx, off, 0, e32,
           empty, 0, False)
    op(W, empty, empty, pl, w_off, D_off, 16, 8, idx, off, 0, e32, empty, 0, False)


def test_metadata_arguments_checked(dev):
    """The small arrays the kernels read by pointer must be dense and on the
    weights' device: a strided view or a host tensor raises instead of being
    misread; strided indices are copied and served."""
    print("[case] tbe fwd metadata argument checks", flush=True)
    rng = np.random.default_rng(4)
    inp = random_tbe(rng, 2, 4, [8, 8], [5, 5], 3)
    W = torch.from_numpy(rng.uniform(-1, 1, 80).astype(np.float32)).to(dev)
    w_off = torch.from_numpy(weight_offsets(inp)).to(dev)
    D_off = torch.from_numpy(inp.D_offsets).to(dev)
    idx = torch.from_numpy(inp.indices).to(dev)
    off = torch.from_numpy(inp.offsets).to(dev)
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(2, dtype=torch.int32, device=dev)
    e32 = torch.zeros(0, dtype=torch.int32, device=dev)
    op = torch.ops.fbgemm.split_embedding_codegen_forward_unweighted_cuda
    strided = torch.stack([D_off, D_off], 1)[:, 0]
    assert not strided.is_contiguous()
    with pytest.raises(RuntimeError, match="D_offsets must be contiguous"):
        op(W, empty, empty, pl, w_off, strided, 16, 8, idx, off, 0, e32, empty, 0, False)
    with pytest.raises(RuntimeError, match="weights_offsets must be a GPU"):
        op(W, empty, empty, pl, w_off.cpu(), D_off, 16, 8, idx, off, 0, e32, empty, 0, False)
    ref = op(W, empty, empty, pl, w_off, D_off, 16, 8, idx, off, 0, e32, empty, 0, False)
    idx_strided = torch.stack([idx, idx], 1)[:, 1]
    got = op(W, empty, empty, pl, w_off, D_off, 16, 8, idx_strided, off, 0, e32, empty, 0, False)
    assert torch.equal(got, ref)


@pytest.mark.parametrize("wdtype,D", [(torch.float32, 128), (torch.float16, 256)])
def test_table_past_4gib(dev, wdtype, D):
    """A table of 8.99M rows x 512 bytes (4.6 GB) between two small ones.
    Rows ending at or below 4 GiB into their table are read through a buffer
    descriptor with 32-bit byte offsets, the rest through 64-bit addresses;
    bags lie wholly below the boundary, wholly above it, across it, and on the
    rows either side of it, in runs of 16 bags (whole waves of one kind) and
    interleaved (waves that switch path batch by batch).  The expected values
    come from the oracle on a compact copy of the rows looked up: the same
    rows summed in the same order, so the comparison is bit-exact."""
    print(f"[case] tbe fwd table past 4 GiB {wdtype} D={D}", flush=True)
    row_bytes = D * torch.finfo(wdtype).bits // 8
    bnd = (1 << 32) // row_bytes  # first row that ends past 4 GiB is bnd - 1
    E_big = bnd + 600_000
    rows, dims, B = [1000, E_big, 1000], [64, D, 32], 256
    rng = np.random.default_rng(4096 + D)
    lengths = rng.integers(0, 70, size=3 * B)
    off = bench_inputs.offsets_from_lengths(lengths)
    idx = np.empty(int(off[-1]), dtype=np.int64)
    for t in (0, 2):
        s, e = int(off[t * B]), int(off[(t + 1) * B])
        idx[s:e] = rng.integers(0, rows[t], size=e - s)
    for b in range(B):
        s, e = int(off[B + b]), int(off[B + b + 1])
        kind = (b // 16) % 4 if b < B // 2 else b % 4
        lo, hi = [(0, bnd - 1), (bnd, E_big), (0, E_big), (bnd - 3, bnd + 3)][kind]
        idx[s:e] = rng.integers(lo, hi, size=e - s)
    inp = bench_inputs.TbeInput(T=3, E=rows, D=dims, B=B, indices=idx, offsets=off)
    w_off = weight_offsets(inp)
    n_elem = int(w_off[2]) + rows[2] * dims[2]
    g = torch.Generator(device=dev)
    g.manual_seed(D)
    W = torch.empty(n_elem, dtype=wdtype, device=dev).uniform_(-1, 1, generator=g)

    big = idx[int(off[B]): int(off[2 * B])]
    used = np.unique(big)
    assert used[0] < bnd - 1 and used[-1] >= bnd
    rows_used = W[int(w_off[1]): int(w_off[2])].view(E_big, D)[torch.from_numpy(used).to(dev)]
    Wc = np.concatenate([W[: int(w_off[1])].cpu().numpy(), rows_used.cpu().numpy().ravel(),
                         W[int(w_off[2]):].cpu().numpy()])
    idx_c = idx.copy()
    idx_c[int(off[B]): int(off[2 * B])] = np.searchsorted(used, big)
    inp_c = bench_inputs.TbeInput(T=3, E=[rows[0], used.size, rows[2]], D=dims, B=B,
                                  indices=idx_c, offsets=off)
    iw = rng.uniform(0, 2, size=inp.N).astype(np.float32)
    for pooling, weights, index_dtype in [(0, None, torch.int64), (1, iw, torch.int32)]:
        exp = orc.tbe_forward_f32(Wc, weight_offsets(inp_c), inp.D_offsets, B, idx_c, off,
                                  pooling, weights)
        got = tbe_forward_gpu(dev, W, inp, pooling, index_dtype,
                              indice_weights=None if weights is None else torch.from_numpy(weights))
        _exact(got, exp)
    del W, rows_used
    torch.cuda.empty_cache()
