"""GPU parity of bounds_check_indices against the oracle: repaired indices,
offsets and the warning count are integers and must match exactly; FATAL
raises and repairs nothing."""

import numpy as np
import pytest
import torch

import oracle as orc

pytestmark = pytest.mark.gpu


def _case(rng, T, B, rows, bad_idx_frac, bad_offsets):
    lengths = rng.integers(0, 8, T * B)
    off = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    N = int(off[-1])
    idx = np.concatenate([rng.integers(0, rows[t], int(off[(t + 1) * B] - off[t * B]))
                          for t in range(T)]).astype(np.int64)
    if bad_idx_frac:
        sel = rng.random(N) < bad_idx_frac
        idx[sel] = rng.integers(-5, max(rows) + 5, sel.sum())
    if bad_offsets:
        pos = rng.integers(0, T * B + 1, 5)
        off[pos[:2]] = -rng.integers(1, 9, 2)
        off[pos[2:4]] = N + rng.integers(1, 9, 2)
        off[pos[4]] = max(int(off[pos[4]]) - 3, 0)  # a local decrease
    return idx, off


@pytest.mark.parametrize("mode", [1, 2, 3])
@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
@pytest.mark.parametrize("T,B,bad_offsets", [(3, 11, False), (3, 11, True), (4, 9000, True)])
def test_bounds_check_matches_oracle(dev, mode, dtype, T, B, bad_offsets):
    print(f"[case] bounds_check mode={mode} {dtype} T={T} B={B} bad_off={bad_offsets}", flush=True)
    rng = np.random.default_rng(T * B + mode)
    rows = rng.integers(1, 100, T)
    idx, off = _case(rng, T, B, rows, 0.05, bad_offsets)
    exp_idx, exp_off, exp_n = orc.bounds_check_indices(rows, idx, off, mode)
    gi = torch.from_numpy(idx).to(dev, dtype)
    go = torch.from_numpy(off).to(dev, dtype)
    warn = torch.full((1,), 7, dtype=torch.int64, device=dev)  # counts accumulate
    torch.ops.fbgemm.bounds_check_indices(torch.from_numpy(rows).to(dev), gi, go, mode, warn)
    np.testing.assert_array_equal(gi.cpu().numpy().astype(np.int64), exp_idx)
    np.testing.assert_array_equal(go.cpu().numpy().astype(np.int64), exp_off)
    assert int(warn.item()) == 7 + (exp_n if mode != 3 else 0)


@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
@pytest.mark.parametrize("T,B,maxlen,long_bags",
                         [(5, 60000, 8, False), (3, 700, 8, True), (2, 3000, 60, False)])
def test_bounds_check_large_batch_and_long_bags(dev, dtype, T, B, maxlen, long_bags):
    """Batches past 2^18 bags (multi-block tiles), mean bag lengths that give
    blocks of 256, 64 and 32 bags, and bags of thousands of indices (a
    block's positions span many passes); offsets broken at block and tile
    boundaries, where the carry from earlier bags decides the repair."""
    print(f"[case] bounds_check large {dtype} T={T} B={B} maxlen={maxlen} long={long_bags}",
          flush=True)
    rng = np.random.default_rng(T * B)
    rows = rng.integers(50, 5000, T)
    lengths = rng.integers(0, maxlen, T * B)
    if long_bags:
        lengths[rng.integers(0, T * B, 4)] = rng.integers(2000, 6000, 4)
    off = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    N = int(off[-1])
    idx = rng.integers(-3, int(rows.max()) + 3, N).astype(np.int64)
    nb = T * B
    for p in [64, 255, 256, 257, 1024, 4096, nb // 2, nb - 1]:
        if p < nb:
            off[p] = off[p] - rng.integers(1, 40) if rng.random() < 0.5 else -1
    p = nb // 3
    off[p] = off[min(p + 300, nb)]  # an overshoot: the next ~300 bags (past a block) repair to it
    off[nb] = N + 5  # the final offset, owned by the last block
    exp_idx, exp_off, exp_n = orc.bounds_check_indices(rows, idx, off, 1)
    gi = torch.from_numpy(idx).to(dev, dtype)
    go = torch.from_numpy(off).to(dev, dtype)
    warn = torch.zeros(1, dtype=torch.int64, device=dev)
    torch.ops.fbgemm.bounds_check_indices(torch.from_numpy(rows).to(dev), gi, go, 1, warn)
    np.testing.assert_array_equal(go.cpu().numpy().astype(np.int64), exp_off)
    np.testing.assert_array_equal(gi.cpu().numpy().astype(np.int64), exp_idx)
    assert int(warn.item()) == exp_n


def test_fatal_raises_and_repairs_nothing(dev):
    print("[case] bounds_check FATAL", flush=True)
    rng = np.random.default_rng(3)
    rows = np.array([5, 6])
    idx, off = _case(rng, 2, 20, rows, 0.2, False)
    gi = torch.from_numpy(idx).to(dev)
    go = torch.from_numpy(off).to(dev)
    warn = torch.zeros(1, dtype=torch.int64, device=dev)
    with pytest.raises(RuntimeError, match="out-of-range"):
        torch.ops.fbgemm.bounds_check_indices(torch.from_numpy(rows).to(dev), gi, go, 0, warn)
    assert np.array_equal(gi.cpu().numpy(), idx) and np.array_equal(go.cpu().numpy(), off)
    # clean input passes FATAL silently
    ci = np.clip(idx, 0, 4)
    torch.ops.fbgemm.bounds_check_indices(torch.from_numpy(rows).to(dev),
                                          torch.from_numpy(ci).to(dev), go, 0, warn)
    assert int(warn.item()) == 0


def test_repaired_batch_is_safe_for_lookup(dev):
    """After WARNING repair a TBE forward over the batch matches the oracle on
    the repaired arrays (no out-of-range gather)."""
    print("[case] bounds_check then forward", flush=True)
    from tbe_helpers import tbe_forward_gpu, weight_offsets
    from mx_fbgemm import bench_inputs

    rng = np.random.default_rng(11)
    T, B, E, D = 2, 50, 40, 16
    rows = np.array([E, E])
    idx, off = _case(rng, T, B, rows, 0.1, True)
    gi, go = torch.from_numpy(idx).to(dev), torch.from_numpy(off).to(dev)
    torch.ops.fbgemm.bounds_check_indices(torch.from_numpy(rows).to(dev), gi, go, 1,
                                          torch.zeros(1, dtype=torch.int64, device=dev))
    ri, ro = gi.cpu().numpy(), go.cpu().numpy()
    inp = bench_inputs.TbeInput(T=T, E=[E, E], D=[D, D], B=B, indices=ri, offsets=ro)
    W = rng.uniform(-1, 1, T * E * D).astype(np.float32)
    got = tbe_forward_gpu(dev, torch.from_numpy(W).to(dev), inp, 0)
    exp = orc.tbe_forward_f32(W, weight_offsets(inp), inp.D_offsets, B, ri, ro, 0)
    np.testing.assert_array_equal(got.cpu().numpy(), exp)
