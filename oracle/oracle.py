"""TEST INFRASTRUCTURE ONLY -- the CPU oracle of the mx_fbgemm operators.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg import this module, and only as the checker; the product never does.

* Jagged ops: numpy restatement of the semantics torch's own port of the
  fbgemm jagged ops states (torch/_inductor/jagged_lowerings.py:161-177:
  masked load, else padding; :231-249: jagged rows past the max length
  become 0) -- pinned against aten._jagged_to_padded_dense_forward /
  _padded_dense_to_jagged_forward on the CPU.
* TBE forward, nbit forward, transpose_embedding_input and the rowwise
  Adagrad backward: the C restatement in mx_oracle.c (ctypes), pinned
  against FBGEMM's CPU kernels (fbgemm_cpu.cpp), F.embedding_bag, torch
  autograd and brute force.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
BUILD_DIR = ORACLE_DIR / "_build"
ORACLE_LIB = BUILD_DIR / "libmx_oracle.so"
FBGEMM_LIB = BUILD_DIR / "libfbgemm_cpu.so"
ORACLE_MT_LIB = BUILD_DIR / "libmx_oracle_mt.so"

POOL_SUM, POOL_MEAN, POOL_NONE = 0, 1, 2
FP32, FP16, INT8, INT4, INT2, FP8 = 0, 1, 2, 3, 4, 6


def build(quiet: bool = True) -> None:
    """Compile the C checkers (make -C oracle)."""
    import sys

    subprocess.run(["make", "-C", str(ORACLE_DIR), f"PYTHON={sys.executable}"], check=True,
                   capture_output=quiet)


_lib = None
_fb = None
_mt = None


def _load(path: Path):
    if not path.exists():
        build()
    return ctypes.CDLL(str(path))


def lib():
    global _lib
    if _lib is None:
        _lib = _load(ORACLE_LIB)
        P = ctypes.c_void_p
        i32, i64, f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_float
        _lib.orc_tbe_forward_f32.argtypes = [P, P, P, i32, i64, P, P, i32, P, P, i64]
        _lib.orc_tbe_forward_f32.restype = None
        _lib.orc_nbit_forward.argtypes = [P, P, P, P, i32, i64, P, P, i32, P, i32, i32, P, i64,
                                          i32, i32]
        _lib.orc_nbit_forward.restype = ctypes.c_int
        _lib.orc_nbit_row_bytes.argtypes = [i32, i32, i32]
        _lib.orc_nbit_row_bytes.restype = i64
        _lib.orc_transpose.argtypes = [P, i32, i64, i32, i32, P, P, i64, P, P, P, P, P, P, P]
        _lib.orc_transpose.restype = ctypes.c_int
        _lib.orc_backward_rowwise_adagrad.argtypes = [
            P, P, P, i32, i64, P, i32, P, P, i64, i32, P, P, i64, P, P, f32, f32, f32, i32, i32]
        _lib.orc_backward_rowwise_adagrad.restype = ctypes.c_int
        _lib.orc_nbit_forward_nobag.argtypes = [P, P, P, i32, i32, i64, P, P, i32, i32, P, i32,
                                                i32]
        _lib.orc_nbit_forward_nobag.restype = ctypes.c_int
        _lib.orc_backward_rowwise_adagrad_nobag.argtypes = [
            P, P, i32, i32, i64, P, i32, P, P, i64, P, P, P, f32, f32, f32, i32, i32]
        _lib.orc_backward_rowwise_adagrad_nobag.restype = ctypes.c_int
        _lib.orc_grad_indice_weights.argtypes = [P, i64, P, P, P, i32, i64, P, P, i32, P, P]
        _lib.orc_grad_indice_weights.restype = None
        _lib.orc_bounds_check.argtypes = [P, i32, i64, P, P, i64, i32]
        _lib.orc_bounds_check.restype = i64
        for name in ("orc_quantize_8bit", "orc_dequantize_8bit"):
            getattr(_lib, name).argtypes = [P, i64, i64, P]
            getattr(_lib, name).restype = None
        for name in ("orc_quantize_nbit", "orc_dequantize_nbit"):
            getattr(_lib, name).argtypes = [P, i64, i64, i32, P]
            getattr(_lib, name).restype = None
        _lib.orc_half_to_float.argtypes = [ctypes.c_uint16]
        _lib.orc_half_to_float.restype = f32
        _lib.orc_float_to_half.argtypes = [f32]
        _lib.orc_float_to_half.restype = ctypes.c_uint16
        _lib.orc_hfp8_to_float.argtypes = [ctypes.c_uint8, i32, i32]
        _lib.orc_hfp8_to_float.restype = f32
        _lib.orc_float_to_hfp8.argtypes = [f32, i32, i32, f32]
        _lib.orc_float_to_hfp8.restype = ctypes.c_uint8
    return _lib


def lib_mt():
    """The multithreaded C++ restatement of the backward (backward_mt.cpp)."""
    global _mt
    if _mt is None:
        _mt = _load(ORACLE_MT_LIB)
        P = ctypes.c_void_p
        i32, i64, f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_float
        _mt.orc_backward_rowwise_adagrad_mt.argtypes = [
            P, P, P, i32, i64, P, i32, P, P, i64, i32, P, P, i64, P, P, f32, f32, f32, i32, i32]
        _mt.orc_backward_rowwise_adagrad_mt.restype = ctypes.c_int
    return _mt


def fbgemm():
    global _fb
    if _fb is None:
        import torch  # noqa: F401  (loads libtorch_cpu, which exports the kernels)

        _fb = _load(FBGEMM_LIB)
        P = ctypes.c_void_p
        i32, i64 = ctypes.c_int32, ctypes.c_int64
        _fb.fb_tbe_forward_f32.argtypes = [P, P, P, i32, i64, P, P, i32, P, P, i64, P, i32]
        _fb.fb_tbe_forward_f32.restype = ctypes.c_int
        _fb.fb_tbe_forward_f16w.argtypes = [P, P, P, i32, i64, P, P, i32, P, P, i64, P, i32]
        _fb.fb_tbe_forward_f16w.restype = ctypes.c_int
        _fb.fb_nbit_forward.argtypes = [P, P, P, P, i32, i64, P, P, i32, P, i32, i32, P, i64, P,
                                        i32, i32, i32]
        _fb.fb_nbit_forward.restype = ctypes.c_int
        _fb.fb_hfp8_to_float.argtypes = [ctypes.c_uint8, i32, i32]
        _fb.fb_hfp8_to_float.restype = ctypes.c_float
        _fb.fb_float_to_hfp8.argtypes = [ctypes.c_float, i32, i32]
        _fb.fb_float_to_hfp8.restype = ctypes.c_uint8
    return _fb


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------------------
# Jagged ops (numpy)
# ---------------------------------------------------------------------------


def dense_index_map(offsets: list[np.ndarray], max_lengths: list[int]) -> np.ndarray:
    """int64 array [B, *max_lengths]: the values row at each dense position, or -1."""
    offs = [np.asarray(o, dtype=np.int64) for o in offsets]
    B = offs[0].shape[0] - 1
    cur = np.arange(B, dtype=np.int64)
    valid = np.ones(B, dtype=bool)
    for k, o in enumerate(offs):
        safe = np.where(valid, cur, 0)
        begin = o[safe]
        length = o[safe + 1] - begin
        j = np.arange(max_lengths[k], dtype=np.int64)
        nvalid = valid[..., None] & (j < length[..., None])
        cur = np.where(nvalid, begin[..., None] + j, 0)
        valid = nvalid
    return np.where(valid, cur, -1)


def jagged_to_padded_dense(values: np.ndarray, offsets, max_lengths, padding_value=0.0):
    values = np.asarray(values)
    m = dense_index_map(offsets, list(max_lengths))
    inner = values.shape[1:]
    out = np.empty(m.shape + inner, dtype=values.dtype)
    out[...] = np.asarray(padding_value).astype(values.dtype)
    sel = m >= 0
    out[sel] = values[m[sel]]
    return out


def dense_to_jagged(dense: np.ndarray, offsets, total_L=None):
    dense = np.asarray(dense)
    nd = len(offsets)
    max_lengths = list(dense.shape[1:1 + nd])
    if total_L is None:
        total_L = int(np.asarray(offsets[-1])[-1])
    m = dense_index_map(offsets, max_lengths)
    inner = dense.shape[1 + nd:]
    out = np.zeros((total_L,) + inner, dtype=dense.dtype)
    sel = (m >= 0) & (m < total_L)
    out[m[sel]] = dense[sel]
    return out


def _bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    return (u16.astype(np.uint32) << 16).view(np.float32)


def _f32_to_bf16(f: np.ndarray) -> np.ndarray:
    u = f.astype(np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def jagged_dense_elementwise_add(x: np.ndarray, offsets, y: np.ndarray, dtype: str):
    """out[i] = x[i] + y[coord(i)] (x[i] + 0 outside y); f16/bf16 in fp32, RNE.

    ``dtype`` is one of "f32", "f64", "f16", "bf16"; bf16 arrays are passed
    as their uint16 bit patterns."""
    nd = len(offsets)
    yz = dense_to_jagged(y, offsets, total_L=x.shape[0])  # y at each jagged row, 0 elsewhere
    if dtype == "f32":
        return (x.astype(np.float32) + yz.astype(np.float32)).astype(np.float32)
    if dtype == "f64":
        return x.astype(np.float64) + yz.astype(np.float64)
    if dtype == "f16":
        return (x.astype(np.float32) + yz.astype(np.float32)).astype(np.float16)
    if dtype == "bf16":
        return _f32_to_bf16(_bf16_to_f32(x) + _bf16_to_f32(yz))
    raise ValueError(dtype)
    del nd


def jagged_dense_elementwise_mul(x: np.ndarray, offsets, y: np.ndarray, dtype: str):
    """out[i] = x[i] * y[coord(i)] (x[i] * 0 outside y); f16/bf16 in fp32 (the
    product of two such values is exact there), rounded once, RNE."""
    yz = dense_to_jagged(y, offsets, total_L=x.shape[0])
    if dtype == "f32":
        return (x.astype(np.float32) * yz.astype(np.float32)).astype(np.float32)
    if dtype == "f64":
        return x.astype(np.float64) * yz.astype(np.float64)
    if dtype == "f16":
        return (x.astype(np.float32) * yz.astype(np.float32)).astype(np.float16)
    if dtype == "bf16":
        return _f32_to_bf16(_bf16_to_f32(x) * _bf16_to_f32(yz))
    raise ValueError(dtype)


# ---------------------------------------------------------------------------
# TBE (C restatement)
# ---------------------------------------------------------------------------


def tbe_forward_f32(W, w_off, D_off, B, indices, offsets, pooling=POOL_SUM, indice_weights=None):
    W = _c(W, np.float32)
    w_off, D_off = _c(w_off, np.int64), _c(D_off, np.int32)
    indices, offsets = _c(indices, np.int64), _c(offsets, np.int64)
    iw = _c(indice_weights, np.float32)
    T = D_off.shape[0] - 1
    total_D = int(D_off[-1])
    out = np.zeros((B, total_D), dtype=np.float32)
    lib().orc_tbe_forward_f32(_p(W), _p(w_off), _p(D_off), T, B, _p(indices), _p(offsets),
                              pooling, _p(iw), _p(out), total_D)
    return out


def position_tables(offsets, T: int, B: int, N: int) -> np.ndarray:
    """Table of each of the N positions of a t-major batch (-1 outside every bag)."""
    offsets = np.asarray(offsets, np.int64)
    t_of = np.full(N, -1, np.int64)
    for t in range(T):
        t_of[max(offsets[t * B], 0): max(offsets[(t + 1) * B], 0)] = t
    return t_of


def tbe_forward_nobag(W, w_off, D: int, B: int, indices, offsets, N: int | None = None):
    """PoolingMode NONE training forward: out[l] = W_t[indices[l]] (fp16 rows
    widened to fp32); rows of positions outside every bag are 0."""
    W = np.asarray(W)
    w_off = np.asarray(w_off, np.int64)
    indices = np.asarray(indices, np.int64)
    T = w_off.shape[0]
    N = indices.shape[0] if N is None else N
    t_of = position_tables(offsets, T, B, N)
    out = np.zeros((N, D), np.float32)
    inb = np.nonzero(t_of >= 0)[0]
    if inb.size:
        start = w_off[t_of[inb]] + indices[inb] * D
        out[inb] = W[start[:, None] + np.arange(D)[None, :]].astype(np.float32)
    return out


def nbit_forward_nobag(W, w_off, tys, D: int, B: int, indices, offsets, row_align=16,
                       out_kind: int = 1, fp8_exponent_bits=4, fp8_exponent_bias=7):
    """PoolingMode NONE nbit lookup, out [N, D] (out_kind 0 fp32, 1 fp16, 2 bf16
    bits as uint16); rows of positions outside every bag are 0."""
    W = _c(W, np.uint8)
    w_off, tys = _c(w_off, np.int64), _c(tys, np.uint8)
    indices, offsets = _c(indices, np.int64), _c(offsets, np.int64)
    T = w_off.shape[0]
    N = indices.shape[0]
    out = np.zeros((N, D), dtype=(np.float32, np.float16, np.uint16)[out_kind])
    rc = lib().orc_nbit_forward_nobag(_p(W), _p(w_off), _p(tys), D, T, B, _p(indices),
                                      _p(offsets), row_align, out_kind, _p(out),
                                      fp8_exponent_bits, fp8_exponent_bias)
    assert rc == 0, f"orc_nbit_forward_nobag failed ({rc})"
    return out


def cumsum(x, kind: int) -> np.ndarray:
    """asynchronous_{exclusive,inclusive,complete}_cumsum (kind 0/1/2) in the
    input's integer type, wrapping as its adds do; a 2-D input (complete only)
    per row."""
    x = np.asarray(x)
    assert x.dtype in (np.int32, np.int64)
    inc = np.cumsum(x, axis=-1, dtype=x.dtype)
    zero = np.zeros(x.shape[:-1] + (1,), x.dtype)
    if kind == 1:
        return inc
    if kind == 0:
        return np.concatenate([zero, inc[..., :-1]], axis=-1)[..., :x.shape[-1]]
    return np.concatenate([zero, inc], axis=-1)


def permute_2d_sparse_data(permute, lengths, indices, weights=None):
    """permute_2D_sparse_data: output feature f is input feature permute[f]
    (lengths [T, B]); returns (permuted_lengths, permuted_indices,
    permuted_weights or None)."""
    permute = np.asarray(permute, np.int64)
    lengths = np.asarray(lengths)
    T, B = lengths.shape
    off = np.concatenate([[0], np.cumsum(lengths.reshape(-1), dtype=np.int64)])
    plen = np.zeros((permute.shape[0], B), lengths.dtype)
    segs_i, segs_w = [], []
    for f, src in enumerate(permute):
        if not 0 <= src < T:
            continue
        plen[f] = lengths[src]
        for b in range(B):
            s, e = off[src * B + b], off[src * B + b + 1]
            segs_i.append(indices[s:e])
            if weights is not None:
                segs_w.append(weights[s:e])
    cat_i = np.concatenate(segs_i) if segs_i else np.zeros(0, np.asarray(indices).dtype)
    cat_w = None
    if weights is not None:
        cat_w = np.concatenate(segs_w) if segs_w else np.zeros(0, np.float32)
    return plen, cat_i, cat_w


def offsets_range(offsets, range_size: int) -> np.ndarray:
    """out[j] = j - offsets[i] over segment i = [offsets[i], offsets[i+1]) (the
    last ends at range_size)."""
    offsets = np.asarray(offsets)
    out = np.zeros(range_size, offsets.dtype)
    ends = np.concatenate([offsets[1:], [range_size]]).astype(np.int64)
    for s, e in zip(offsets.astype(np.int64), ends):
        s, e = max(int(s), 0), min(int(e), range_size)
        out[s:e] = np.arange(e - s, dtype=offsets.dtype)
    return out


def expand_into_jagged_permute(permute, input_offsets, output_offsets, output_size: int):
    """out[output_offsets[t] + j] = input_offsets[permute[t]] + j over output
    feature t's length."""
    output_offsets = np.asarray(output_offsets)
    input_offsets = np.asarray(input_offsets)
    T = len(permute)
    ends = output_offsets[1:T + 1] if output_offsets.shape[0] == T + 1 else \
        np.concatenate([output_offsets[1:T], [output_size]])
    out = np.zeros(output_size, input_offsets.dtype)
    for t in range(T):
        d0, d1 = int(output_offsets[t]), min(int(ends[t]), output_size)
        out[d0:d1] = input_offsets[permute[t]] + np.arange(d1 - d0, dtype=input_offsets.dtype)
    return out


def hfp8_to_float(codes, ebits: int, ebias: int) -> np.ndarray:
    """Decodes hfp8 codes (uint8) to fp32 (the C restatement)."""
    f = lib().orc_hfp8_to_float
    c = np.asarray(codes, dtype=np.uint8)
    return np.array([f(int(v), ebits, ebias) for v in c.ravel()], np.float32).reshape(c.shape)


def float_to_hfp8(x, ebits: int, ebias: int, max_pos: float) -> np.ndarray:
    """Encodes fp32 values as hfp8 codes (the C restatement)."""
    f = lib().orc_float_to_hfp8
    a = np.asarray(x, dtype=np.float32)
    return np.array([f(float(v), ebits, ebias, max_pos) for v in a.ravel()],
                    np.uint8).reshape(a.shape)


def hfp8_max_pos(ebits: int, ebias: int) -> float:
    """The largest magnitude FBGEMM's hfp8 encoder produces: the top exponent
    field is left unused by encoding (decoding still defines it)."""
    m = 7 - ebits
    return float(np.ldexp(2.0 - 2.0 ** -m, (1 << ebits) - 2 - ebias))


def fbgemm_hfp8_to_float(codes, ebits: int, ebias: int) -> np.ndarray:
    """fbgemm::Float8ToFloat_ref on each code."""
    f = fbgemm().fb_hfp8_to_float
    c = np.asarray(codes, dtype=np.uint8)
    return np.array([f(int(v), ebits, ebias) for v in c.ravel()], np.float32).reshape(c.shape)


def fbgemm_float_to_hfp8(x, ebits: int, ebias: int) -> np.ndarray:
    """fbgemm::FloatToFloat8_ref on each value."""
    f = fbgemm().fb_float_to_hfp8
    a = np.asarray(x, dtype=np.float32)
    return np.array([f(float(v), ebits, ebias) for v in a.ravel()], np.uint8).reshape(a.shape)


def nbit_row_bytes(ty: int, D: int, row_align: int) -> int:
    return int(lib().orc_nbit_row_bytes(ty, D, row_align))


def nbit_forward(W, w_off, tys, D_off, B, indices, offsets, pooling=POOL_SUM,
                 indice_weights=None, row_align=16, out_f16=True, fp8_exponent_bits=4,
                 fp8_exponent_bias=7, out_bf16=False):
    """Pooled nbit lookup; output fp16 (out_f16), bf16 (out_bf16, returned as
    the uint16 bits) or fp32."""
    W = _c(W, np.uint8)
    w_off, tys, D_off = _c(w_off, np.int64), _c(tys, np.uint8), _c(D_off, np.int32)
    indices, offsets = _c(indices, np.int64), _c(offsets, np.int64)
    iw = _c(indice_weights, np.float32)
    T = D_off.shape[0] - 1
    total_D = int(D_off[-1])
    kind = 2 if out_bf16 else (1 if out_f16 else 0)
    out = np.zeros((B, total_D), dtype=(np.float32, np.float16, np.uint16)[kind])
    rc = lib().orc_nbit_forward(_p(W), _p(w_off), _p(tys), _p(D_off), T, B, _p(indices),
                                _p(offsets), pooling, _p(iw), row_align, kind, _p(out),
                                total_D, fp8_exponent_bits, fp8_exponent_bias)
    assert rc == 0, f"orc_nbit_forward failed ({rc})"
    return out


def transpose_embedding_input(hsc, B, info_B_num_bits, bits, indices, offsets):
    hsc = _c(hsc, np.int64)
    indices, offsets = _c(indices, np.int64), _c(offsets, np.int64)
    T = hsc.shape[0] - 1
    N = indices.shape[0]
    n = max(N, 1)
    linear = np.zeros(n, np.int64)
    srt = np.zeros(n, np.int64)
    infos = np.zeros(n, np.int32)
    run = np.zeros(n, np.int64)
    lengths = np.zeros(n, np.int32)
    cum = np.zeros(n + 1, np.int32)
    num_runs = np.zeros(1, np.int64)
    if N:
        rc = lib().orc_transpose(_p(hsc), T, B, info_B_num_bits, bits, _p(indices), _p(offsets),
                                 N, _p(linear), _p(srt), _p(infos), _p(run), _p(lengths),
                                 _p(num_runs), _p(cum))
        assert rc == 0
    r = int(num_runs[0])
    return dict(linear_indices=linear[:N], sorted_linear_indices=srt[:N], infos_sorted=infos[:N],
                run=run[:r], run_lengths=lengths[:r], num_runs=r, cumulative_run_lengths=cum[:r + 1],
                run_lengths_full=lengths[:N], cumulative_run_lengths_full=cum[:N + 1])


def backward_rowwise_adagrad(W, w_off, D_off, B, hsc, bits, indices, offsets, pooling, grad,
                             momentum1, m1_off, lr, eps, weight_decay=0.0, weight_decay_mode=0,
                             info_B_num_bits=26, indice_weights=None, inplace=False):
    """Updates copies of W and momentum1; returns (W_new, momentum1_new).
    ``indice_weights`` (fp32 [N]) makes it the weighted backward.  With
    ``inplace`` W and momentum1 (contiguous fp32) are updated where they lie
    (the CPU-baseline timing, which must not copy gigabytes per call)."""
    if inplace:
        assert W.dtype == np.float32 and W.flags["C_CONTIGUOUS"]
        assert momentum1.dtype == np.float32 and momentum1.flags["C_CONTIGUOUS"]
        m1 = momentum1
    else:
        W = np.array(W, dtype=np.float32, copy=True)
        m1 = np.array(momentum1, dtype=np.float32, copy=True)
    w_off, D_off = _c(w_off, np.int64), _c(D_off, np.int32)
    hsc, m1_off = _c(hsc, np.int64), _c(m1_off, np.int64)
    indices, offsets = _c(indices, np.int64), _c(offsets, np.int64)
    grad = _c(grad, np.float32)
    iw = None if indice_weights is None else _c(indice_weights, np.float32)
    assert iw is None or iw.shape[0] == indices.shape[0]
    T = D_off.shape[0] - 1
    rc = lib().orc_backward_rowwise_adagrad(
        _p(W), _p(w_off), _p(D_off), T, B, _p(hsc), bits, _p(indices), _p(offsets),
        indices.shape[0], pooling, None if iw is None else _p(iw), _p(grad), grad.shape[1],
        _p(m1), _p(m1_off), lr, eps, weight_decay, weight_decay_mode, info_B_num_bits)
    assert rc == 0, f"orc_backward_rowwise_adagrad failed ({rc})"
    return W, m1


def backward_rowwise_adagrad_nobag(W, w_off, D: int, B: int, hsc, bits, indices, offsets, grad,
                                   momentum1, m1_off, lr, eps, weight_decay=0.0,
                                   weight_decay_mode=0):
    """PoolingMode NONE backward (grad [N, D], row l the gradient of position
    l) on copies of W and momentum1; returns (W_new, momentum1_new)."""
    W = np.array(W, dtype=np.float32, copy=True)
    m1 = np.array(momentum1, dtype=np.float32, copy=True)
    w_off, hsc, m1_off = _c(w_off, np.int64), _c(hsc, np.int64), _c(m1_off, np.int64)
    indices, offsets = _c(indices, np.int64), _c(offsets, np.int64)
    grad = _c(grad, np.float32)
    T = w_off.shape[0]
    N = indices.shape[0]
    assert grad.shape == (N, D)
    rc = lib().orc_backward_rowwise_adagrad_nobag(
        _p(W), _p(w_off), D, T, B, _p(hsc), bits, _p(indices), _p(offsets), N, _p(grad),
        _p(m1), _p(m1_off), lr, eps, weight_decay, weight_decay_mode, info_B_num_bits(T, B))
    assert rc == 0, f"orc_backward_rowwise_adagrad_nobag failed ({rc})"
    return W, m1


def transpose_embedding_input_nobag(hsc, B, bits, indices, offsets):
    """transpose_embedding_input(nobag=True): keys hsc[t] + indices[l] stably
    sorted on their low ``bits`` bits, infos l * T + t (int64), runs as in the
    pooled transpose.  numpy (a stable argsort), no C."""
    hsc = np.asarray(hsc, np.int64)
    indices = np.asarray(indices, np.int64)
    T = hsc.shape[0] - 1
    N = indices.shape[0]
    t_of = position_tables(offsets, T, B, N)
    linear = hsc[t_of] + indices
    mask = (1 << bits) - 1 if bits < 63 else -1
    order = np.argsort(linear & mask, kind="stable")
    srt = linear[order]
    infos = order.astype(np.int64) * T + t_of[order]
    if N:
        heads = np.concatenate([[True], srt[1:] != srt[:-1]])
        starts = np.nonzero(heads)[0]
        run = srt[starts]
        lengths = np.diff(np.concatenate([starts, [N]])).astype(np.int32)
    else:
        run = np.zeros(0, np.int64)
        lengths = np.zeros(0, np.int32)
    r = run.shape[0]
    cum = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    return dict(linear_indices=linear, sorted_linear_indices=srt, infos_sorted=infos, run=run,
                run_lengths=lengths, num_runs=r, cumulative_run_lengths=cum)


def backward_rowwise_adagrad_mt(W, w_off, D_off, B, hsc, bits, indices, offsets, pooling, grad,
                                momentum1, m1_off, lr, eps, weight_decay=0.0,
                                weight_decay_mode=0, indice_weights=None, inplace=False,
                                nthreads=None):
    """backward_rowwise_adagrad on `nthreads` threads (default: this host's),
    split over key ranges; bit-identical to it.  Requires every key below
    2^bits."""
    if inplace:
        assert W.dtype == np.float32 and W.flags["C_CONTIGUOUS"]
        assert momentum1.dtype == np.float32 and momentum1.flags["C_CONTIGUOUS"]
        m1 = momentum1
    else:
        W = np.array(W, dtype=np.float32, copy=True)
        m1 = np.array(momentum1, dtype=np.float32, copy=True)
    w_off, D_off = _c(w_off, np.int64), _c(D_off, np.int32)
    hsc, m1_off = _c(hsc, np.int64), _c(m1_off, np.int64)
    indices, offsets = _c(indices, np.int64), _c(offsets, np.int64)
    grad = _c(grad, np.float32)
    iw = None if indice_weights is None else _c(indice_weights, np.float32)
    T = D_off.shape[0] - 1
    rc = lib_mt().orc_backward_rowwise_adagrad_mt(
        _p(W), _p(w_off), _p(D_off), T, B, _p(hsc), bits, _p(indices), _p(offsets),
        indices.shape[0], pooling, None if iw is None else _p(iw), _p(grad), grad.shape[1],
        _p(m1), _p(m1_off), lr, eps, weight_decay, weight_decay_mode,
        nthreads or host_threads())
    assert rc == 0, f"orc_backward_rowwise_adagrad_mt failed ({rc})"
    return W, m1


def grad_indice_weights(grad, W, w_off, D_off, B, indices, offsets, pooling=POOL_SUM,
                        feature_requires_grad=None):
    """fp32 [N]: d(out)/d(indice_weights[l]) contracted with grad_output."""
    grad, W = _c(grad, np.float32), _c(W, np.float32)
    w_off, D_off = _c(w_off, np.int64), _c(D_off, np.int32)
    indices, offsets = _c(indices, np.int64), _c(offsets, np.int64)
    frg = None if feature_requires_grad is None else _c(feature_requires_grad, np.int32)
    T = D_off.shape[0] - 1
    out = np.zeros(indices.shape[0], dtype=np.float32)
    lib().orc_grad_indice_weights(_p(grad), grad.shape[1], _p(W), _p(w_off), _p(D_off), T, B,
                                  _p(indices), _p(offsets), pooling,
                                  None if frg is None else _p(frg), _p(out))
    return out


def bounds_check_indices(rows_per_table, indices, offsets, mode):
    """Returns (indices', offsets', count) -- repaired copies and the number of
    out-of-range entries."""
    rows = _c(rows_per_table, np.int64)
    idx = np.array(indices, dtype=np.int64, copy=True)
    off = np.array(offsets, dtype=np.int64, copy=True)
    T = rows.shape[0]
    B = (off.shape[0] - 1) // T
    n = lib().orc_bounds_check(_p(rows), T, B, _p(idx), _p(off), idx.shape[0], mode)
    return idx, off, int(n)


def quantize_fused8bit(x):
    x = _c(x, np.float32)
    rows, D = x.shape
    out = np.zeros((rows, D + 8), np.uint8)
    lib().orc_quantize_8bit(_p(x), rows, D, _p(out))
    return out


def dequantize_fused8bit(q):
    q = _c(q, np.uint8)
    rows, D = q.shape[0], q.shape[1] - 8
    out = np.zeros((rows, D), np.float32)
    lib().orc_dequantize_8bit(_p(q), rows, D, _p(out))
    return out


def quantize_fused_nbit(x, bits):
    x = _c(x, np.float32)
    rows, D = x.shape
    per = 8 // bits
    out = np.zeros((rows, (D + per - 1) // per + 4), np.uint8)
    lib().orc_quantize_nbit(_p(x), rows, D, bits, _p(out))
    return out


def dequantize_fused_nbit(q, bits, D):
    q = _c(q, np.uint8)
    rows = q.shape[0]
    out = np.zeros((rows, D), np.float32)
    lib().orc_dequantize_nbit(_p(q), rows, D, bits, _p(out))
    return out


def info_B_num_bits(T: int, B: int) -> int:
    """Bits of b in an info word: 26 unless T or B need another split."""
    tb = max(0, int(T - 1).bit_length())
    bb = max(1, int(B - 1).bit_length())
    if tb + bb > 32:
        raise ValueError("T, B do not fit 32 bits")
    if bb <= 26 and tb <= 6:
        return 26
    return 32 - tb


# ---------------------------------------------------------------------------
# FBGEMM CPU kernels (pins and CPU baseline)
# ---------------------------------------------------------------------------


def fbgemm_tbe_forward_f32(W, w_off, D_off, rows_per_table, B, indices, offsets, pooling=POOL_SUM,
                           indice_weights=None, nthreads=1):
    """FBGEMM's CPU SpMDM, fp32 output; fp16 ``W`` uses the fp16-input kernel."""
    if np.asarray(W).dtype == np.float16:
        return _fbgemm_tbe_forward_f16w(W, w_off, D_off, rows_per_table, B, indices, offsets,
                                        pooling, indice_weights, nthreads)
    W = _c(W, np.float32)
    w_off, D_off = _c(w_off, np.int64), _c(D_off, np.int32)
    rows = _c(rows_per_table, np.int64)
    indices, offsets = _c(indices, np.int64), _c(offsets, np.int64)
    iw = _c(indice_weights, np.float32)
    T = D_off.shape[0] - 1
    total_D = int(D_off[-1])
    out = np.zeros((B, total_D), dtype=np.float32)
    rc = fbgemm().fb_tbe_forward_f32(_p(W), _p(w_off), _p(D_off), T, B, _p(indices), _p(offsets),
                                     pooling, _p(iw), _p(out), total_D, _p(rows), nthreads)
    assert rc == 0, f"FBGEMM SpMDM kernel reported failure ({rc})"
    return out


def _fbgemm_tbe_forward_f16w(W, w_off, D_off, rows_per_table, B, indices, offsets, pooling,
                             indice_weights, nthreads):
    W = _c(W, np.float16)
    w_off, D_off = _c(w_off, np.int64), _c(D_off, np.int32)
    rows = _c(rows_per_table, np.int64)
    indices, offsets = _c(indices, np.int64), _c(offsets, np.int64)
    iw = _c(indice_weights, np.float32)
    T = D_off.shape[0] - 1
    total_D = int(D_off[-1])
    out = np.zeros((B, total_D), dtype=np.float32)
    rc = fbgemm().fb_tbe_forward_f16w(_p(W), _p(w_off), _p(D_off), T, B, _p(indices), _p(offsets),
                                      pooling, _p(iw), _p(out), total_D, _p(rows), nthreads)
    assert rc == 0, f"FBGEMM SpMDM kernel reported failure ({rc})"
    return out


def fbgemm_nbit_forward(W, w_off, tys, D_off, rows_per_table, B, indices, offsets,
                        pooling=POOL_SUM, indice_weights=None, row_align=16, nthreads=1,
                        fp8_exponent_bits=4, fp8_exponent_bias=7, out_bf16=False):
    W = _c(W, np.uint8)
    w_off, tys, D_off = _c(w_off, np.int64), _c(tys, np.uint8), _c(D_off, np.int32)
    rows = _c(rows_per_table, np.int64)
    indices, offsets = _c(indices, np.int64), _c(offsets, np.int64)
    iw = _c(indice_weights, np.float32)
    T = D_off.shape[0] - 1
    total_D = int(D_off[-1])
    out = np.zeros((B, total_D), dtype=np.uint16 if out_bf16 else np.float16)
    rc = fbgemm().fb_nbit_forward(_p(W), _p(w_off), _p(tys), _p(D_off), T, B, _p(indices),
                                  _p(offsets), pooling, _p(iw), row_align, 2 if out_bf16 else 1,
                                  _p(out), total_D,
                                  _p(rows), nthreads, fp8_exponent_bits, fp8_exponent_bias)
    assert rc == 0, f"FBGEMM nbit kernel reported failure ({rc})"
    return out


def host_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1
