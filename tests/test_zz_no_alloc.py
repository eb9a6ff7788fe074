"""The allocation-free bounds check, called through the C-ABI exactly as a
ctypes caller would: mx_bounds_check_indices_noalloc (scratch in a static
device array of the library) must repair indices and offsets and count
exactly as mx_bounds_check_indices (caller workspace) does, on two calls in
a row, the second with a smaller batch (the scratch keeps the first call's
contents), and both as the oracle does."""

import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as orc

pytestmark = pytest.mark.gpu

REPO = Path(__file__).resolve().parents[1]
LIB = REPO / "torchlib-xpu_amd" / "mx_fbgemm" / "lib" / "libmx_fbgemm_kernels.so"
P, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64


@pytest.fixture(scope="module")
def lib(dev):
    lib = ctypes.CDLL(str(LIB))
    lib.mx_bounds_check_workspace_bytes.argtypes = [i32, i64]
    lib.mx_bounds_check_workspace_bytes.restype = ctypes.c_size_t
    lib.mx_bounds_check_indices.argtypes = [P, i32, i64, P, P, i32, i64, i32, P, P,
                                            ctypes.c_size_t, P]
    lib.mx_bounds_check_indices.restype = ctypes.c_int
    lib.mx_bounds_check_indices_noalloc.argtypes = [P, i32, i64, P, P, i32, i64, i32, P, P]
    lib.mx_bounds_check_indices_noalloc.restype = ctypes.c_int
    lib.mx_last_error.restype = ctypes.c_char_p
    return lib


def _case(rng, T, B, rows, bad_idx_frac=0.05):
    lengths = rng.integers(0, 12, T * B)
    off = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    N = int(off[-1])
    idx = np.concatenate([rng.integers(0, rows[t], int(off[(t + 1) * B] - off[t * B]))
                          for t in range(T)]).astype(np.int64)
    sel = rng.random(N) < bad_idx_frac
    idx[sel] = rng.integers(-5, int(max(rows)) + 5, int(sel.sum()))
    pos = rng.integers(0, T * B + 1, 5)
    off[pos[:2]] = -rng.integers(1, 9, 2)
    off[pos[2:4]] = N + rng.integers(1, 9, 2)
    off[pos[4]] = max(int(off[pos[4]]) - 3, 0)
    return idx, off


def _run(lib, dev, rows, idx, off, T, B, mode, dtype, noalloc):
    gi = torch.from_numpy(idx).to(dev, dtype)
    go = torch.from_numpy(off).to(dev, dtype)
    r = torch.from_numpy(rows).to(dev)
    warn = torch.zeros(1, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    eb = 8 if dtype == torch.int64 else 4
    if noalloc:
        rc = lib.mx_bounds_check_indices_noalloc(r.data_ptr(), T, B, gi.data_ptr(), go.data_ptr(),
                                                 eb, idx.size, mode, warn.data_ptr(), stream)
    else:
        nbytes = lib.mx_bounds_check_workspace_bytes(T, B)
        ws = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)
        rc = lib.mx_bounds_check_indices(r.data_ptr(), T, B, gi.data_ptr(), go.data_ptr(), eb,
                                         idx.size, mode, warn.data_ptr(), ws.data_ptr(), nbytes,
                                         stream)
    assert rc == 0, lib.mx_last_error().decode()
    torch.cuda.synchronize()
    return gi.cpu().numpy().astype(np.int64), go.cpu().numpy().astype(np.int64), int(warn.item())


@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
def test_noalloc_bounds_check_matches_workspace_entry_point(dev, lib, dtype):
    rng = np.random.default_rng(77)
    # Call 1: 3 x 40000 bags (469 tiles of 256 bags); call 2: 2 x 300 bags.
    for T, B, mode in [(3, 40000, 1), (2, 300, 1), (2, 300, 0)]:
        print(f"[case] noalloc bounds check T={T} B={B} mode={mode} {dtype}", flush=True)
        rows = rng.integers(1, 1000, T).astype(np.int64)
        idx, off = _case(rng, T, B, rows)
        got = _run(lib, dev, rows, idx, off, T, B, mode, dtype, noalloc=True)
        ref = _run(lib, dev, rows, idx, off, T, B, mode, dtype, noalloc=False)
        np.testing.assert_array_equal(got[0], ref[0])
        np.testing.assert_array_equal(got[1], ref[1])
        assert got[2] == ref[2]
        exp_idx, exp_off, exp_n = orc.bounds_check_indices(rows, idx, off, mode)
        np.testing.assert_array_equal(got[0], exp_idx)
        np.testing.assert_array_equal(got[1], exp_off)
        assert got[2] == exp_n > 0
