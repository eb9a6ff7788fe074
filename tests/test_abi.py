"""The C-ABI library loads without a GPU, exports every function
include/mx_fbgemm.h declares, and its host-side argument checks and size
queries behave -- no compute call is made here."""

import ctypes
import re
from pathlib import Path

import pytest
import torch  # noqa: F401  (binds the HIP runtime torch ships before the library loads)

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "mx_fbgemm.h"
LIB = REPO / "torchlib-xpu_amd" / "mx_fbgemm" / "lib" / "libmx_fbgemm_kernels.so"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(mx_[a-z_0-9]+)\s*\(",
                                 text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        pytest.fail(f"{LIB} not built (run __graft_entry__.build())")
    return ctypes.CDLL(str(LIB))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for must in ("mx_jagged_to_padded_dense", "mx_dense_to_jagged", "mx_jagged_dense_elementwise_add",
                 "mx_tbe_forward", "mx_tbe_transpose_embedding_input",
                 "mx_tbe_backward_rowwise_adagrad", "mx_nbit_forward", "mx_last_error"):
        assert must in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_version_and_last_error(lib):
    # The library reports the version its header declares (0.2.0 changed the
    # backward's stochastic-rounding argument from a seed to mx_rng_state*;
    # 0.3.0 added the backward's per-stream counter region; 0.4.0 the FP8
    # arguments of mx_nbit_forward and the hfp8 codecs).
    hdr = re.search(r"#define MX_FBGEMM_VERSION (\d+)", HEADER.read_text())
    assert hdr and lib.mx_version() == int(hdr.group(1)) == 500
    lib.mx_last_error.restype = ctypes.c_char_p
    assert isinstance(lib.mx_last_error(), bytes)


def test_row_bytes(lib):
    f = lib.mx_nbit_row_bytes
    f.restype = ctypes.c_int64
    f.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
    assert f(2, 128, 16) == 144   # INT8: 128 + 4 -> 144
    assert f(3, 128, 16) == 80    # INT4: 64 + 4 -> 80
    assert f(4, 128, 16) == 48    # INT2: 32 + 4 -> 48
    assert f(1, 128, 16) == 256   # FP16
    assert f(0, 100, 16) == 400   # FP32
    assert f(2, 128, 1) == 132
    assert f(9, 128, 16) == -1


def test_info_bits(lib):
    f = lib.mx_tbe_info_B_num_bits
    f.restype = ctypes.c_int32
    f.argtypes = [ctypes.c_int32, ctypes.c_int64]
    assert f(8, 4096) == 26
    assert f(64, 1 << 26) == 26
    assert f(128, 1000) == 25      # 7 bits for t leave 25 for b
    assert f(1 << 20, 1 << 20) == -1


def test_workspace_sizes_grow(lib):
    f = lib.mx_tbe_backward_workspace_bytes
    f.restype = ctypes.c_size_t
    f.argtypes = [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32]
    a, b = f(1000, 23, 128), f(100000, 23, 128)
    assert 0 < a < b
    g = lib.mx_tbe_transpose_workspace_bytes
    g.restype = ctypes.c_size_t
    g.argtypes = [ctypes.c_int64, ctypes.c_int32]
    assert 0 < g(1000, 23) < a


def test_bad_arguments_rejected_before_any_launch(lib):
    lib.mx_last_error.restype = ctypes.c_char_p
    P = ctypes.c_void_p
    i32, i64, f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_float
    f = lib.mx_tbe_forward
    f.argtypes = [P, i32, P, P, i32, i64, i32, P, P, i32, i32, P, P, i32, i64, P]
    # index_bytes 3 is invalid
    assert f(None, 0, None, None, 1, 1, 128, None, None, 3, 0, None, None, 0, 128, None) == -1
    assert b"int32 or int64" in lib.mx_last_error()
    # max_D not a multiple of 4
    assert f(None, 0, None, None, 1, 1, 130, None, None, 8, 0, None, None, 0, 130, None) == -1
    assert b"multiple of 4" in lib.mx_last_error()
    # pooling NONE is not served
    assert f(None, 0, None, None, 1, 1, 128, None, None, 8, 2, None, None, 0, 128, None) == -1
    assert b"pooling_mode" in lib.mx_last_error()
    # bf16 weights are not served
    assert f(None, 5, None, None, 1, 1, 128, None, None, 8, 0, None, None, 0, 128, None) == -1
    assert b"weights type" in lib.mx_last_error()
    # empty problem: success without touching the device (fp32 and fp16 weights)
    assert f(None, 0, None, None, 0, 0, 128, None, None, 8, 0, None, None, 0, 128, None) == 0
    assert f(None, 1, None, None, 0, 0, 128, None, None, 8, 0, None, None, 0, 128, None) == 0
    g = lib.mx_nbit_forward
    g.argtypes = [P, P, P, P, i32, i64] + [i32] * 5 + \
        [P, P, i32, i32, P, i32, i32, i32, i32, i32, P, i64, P]
    assert g(None, None, None, None, 1, 1, 0, 0, 2048, 0, 0, None, None, 4, 0, None, 1, 16,
             0, -1, -1, None, 2048, None) == -1  # max D above 1024
    assert b"1024" in lib.mx_last_error()
    assert g(None, None, None, None, 1, 1, 0, 29, 0, 0, 0, None, None, 4, 0, None, 1, 16,
             0, -1, -1, None, 29, None) == -1  # odd INT4 D: codes would not fill whole bytes
    assert b"INT4 D must be even" in lib.mx_last_error()
    assert g(None, None, None, None, 1, 1, 6, 0, 0, 0, 0, None, None, 4, 0, None, 1, 16,
             0, -1, -1, None, 6, None) == -1  # INT2 D not a multiple of 4
    assert b"INT2 D a multiple of 4" in lib.mx_last_error()
    for ebits, bias in ((0, 7), (8, 7), (4, -1), (4, 121)):  # FP8 formats outside the served range
        assert g(None, None, None, None, 1, 1, 0, 0, 0, 0, 0, None, None, 4, 0, None, 1, 16,
                 64, ebits, bias, None, 64, None) == -1
        assert b"fp8_exponent_bits" in lib.mx_last_error()
    e = lib.mx_float_to_hfp8
    e.argtypes = [P, i64, i32, i32, f32, P, P]
    assert e(None, 8, 4, 7, 0.0, None, None) == -1 and b"max_pos" in lib.mx_last_error()
    assert e(None, 8, 9, 7, 240.0, None, None) == -1 and b"ebits" in lib.mx_last_error()
    assert e(None, 0, 4, 7, 240.0, None, None) == 0  # nothing to convert
    d = lib.mx_hfp8_to_float
    d.argtypes = [P, i64, i32, i32, P, P]
    assert d(None, 8, 4, 130, None, None) == -1 and b"exponent_bias" in lib.mx_last_error()
    h = lib.mx_tbe_backward_rowwise_adagrad
    h.restype = ctypes.c_int
    h.argtypes = [P, i32, P, P, i32, i64, i32, P, i32, P, P, i32, i64, i32, P, P, i64, P, P,
                  f32, f32, f32, i32, i32, ctypes.c_uint64, P, ctypes.c_size_t, P]
    args = [None, 0, None, None, 1, 4, 128, None, 23, None, None, 8, 10, 0, None, None, 128,
            None, None, 0.1, 1e-8, 0.0, 0, 0, 0, None, 0, None]
    bad_mode = list(args)
    bad_mode[22] = 7  # weight_decay_mode
    assert h(*bad_mode) == -1
    assert b"weight_decay_mode" in lib.mx_last_error()
    bad_ty = list(args)
    bad_ty[1] = 2  # INT8 training weights
    assert h(*bad_ty) == -1
    assert b"weights type" in lib.mx_last_error()
    empty = list(args)
    empty[12] = 0  # N = 0: nothing to do
    assert h(*empty) == 0
