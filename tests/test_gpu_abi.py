"""The C-ABI driven on the device exactly as the ctypes binding of the
integration guide shows it (no torch op in between): mx_tbe_forward on a
small batch, checked bit-exactly against the oracle, and an argument error
reported through the status code and mx_last_error()."""

import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as orc
from tbe_helpers import random_tbe, weight_offsets

pytestmark = pytest.mark.gpu

REPO = Path(__file__).resolve().parents[1]
LIB = REPO / "torchlib-xpu_amd" / "mx_fbgemm" / "lib" / "libmx_fbgemm_kernels.so"


@pytest.fixture(scope="module")
def lib(dev):
    lib = ctypes.CDLL(str(LIB))
    P, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    lib.mx_tbe_forward.argtypes = [P, i32, P, P, i32, i64, i32, P, P, i32, i32, P, P, i32, i64, P]
    lib.mx_tbe_forward.restype = ctypes.c_int
    lib.mx_last_error.restype = ctypes.c_char_p
    return lib


@pytest.mark.parametrize("pooling", [0, 1])
def test_tbe_forward_through_ctypes(dev, lib, pooling):
    print(f"[case] ctypes mx_tbe_forward pooling={pooling}", flush=True)
    rng = np.random.default_rng(31 + pooling)
    inp = random_tbe(rng, 3, 40, [16, 64, 128], [50, 700, 9], 12)
    W_h = rng.uniform(-0.01, 0.01, sum(E * D for E, D in zip(inp.E, inp.D))).astype(np.float32)
    W = torch.from_numpy(W_h).to(dev)
    w_off = torch.from_numpy(weight_offsets(inp)).to(dev)
    D_off = torch.from_numpy(inp.D_offsets).to(dev)
    idx = torch.from_numpy(inp.indices).to(dev)
    off = torch.from_numpy(inp.offsets).to(dev)
    out = torch.empty((inp.B, inp.total_D), device=dev)
    T, B, max_D, total_D = inp.T, inp.B, max(inp.D), inp.total_D

    stream = torch.cuda.current_stream().cuda_stream          # hipStream_t on ROCm
    rc = lib.mx_tbe_forward(W.data_ptr(), 0, w_off.data_ptr(), D_off.data_ptr(), T, B, max_D,
                            idx.data_ptr(), off.data_ptr(), 8, pooling, None, out.data_ptr(), 0,
                            total_D, stream)
    if rc != 0:
        raise RuntimeError(lib.mx_last_error().decode())
    torch.cuda.synchronize()
    exp = orc.tbe_forward_f32(W_h, weight_offsets(inp), inp.D_offsets, B, inp.indices,
                              inp.offsets, pooling)
    assert np.array_equal(out.cpu().numpy(), exp)


def test_argument_error_through_ctypes(dev, lib):
    print("[case] ctypes mx_tbe_forward bad pooling mode", flush=True)
    out = torch.empty((1, 4), device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    z64 = torch.zeros(2, dtype=torch.int64, device=dev)
    z32 = torch.tensor([0, 4], dtype=torch.int32, device=dev)
    rc = lib.mx_tbe_forward(out.data_ptr(), 0, z64.data_ptr(), z32.data_ptr(), 1, 1, 4,
                            z64.data_ptr(), z64.data_ptr(), 8, 7, None, out.data_ptr(), 0, 4,
                            stream)
    assert rc == -1  # MX_EINVAL
    assert b"pooling" in lib.mx_last_error().lower()
