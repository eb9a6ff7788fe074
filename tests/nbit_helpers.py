"""Builders of nbit (quantized TBE) test inputs in the TBE row layout."""

from __future__ import annotations

import numpy as np
import torch

import oracle as orc


def build_weights(rng: np.random.Generator, tys, dims, rows, row_align: int = 16):
    """uint8 buffer with every table's padded rows, plus weights_offsets.

    Quantized rows: fp16 scale in [1e-3, 1e-2), fp16 bias in [-0.1, 0.1),
    uniform codes; FP16/FP32 rows: values in [-0.01, 0.01)."""
    strides = [orc.nbit_row_bytes(ty, D, row_align) for ty, D in zip(tys, dims)]
    sizes = [E * s for E, s in zip(rows, strides)]
    w_off = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    buf = np.zeros(int(sum(sizes)), dtype=np.uint8)
    for t, (ty, D, E, s) in enumerate(zip(tys, dims, rows, strides)):
        tab = buf[w_off[t]: w_off[t] + E * s].reshape(E, s)
        if ty in (orc.INT8, orc.INT4, orc.INT2):
            tab[:, 4:] = rng.integers(0, 256, size=(E, s - 4), dtype=np.uint8)
            sc = rng.uniform(1e-3, 1e-2, size=E).astype(np.float16)
            bi = rng.uniform(-0.1, 0.1, size=E).astype(np.float16)
            tab[:, 0:2] = sc.view(np.uint8).reshape(E, 2)
            tab[:, 2:4] = bi.view(np.uint8).reshape(E, 2)
        elif ty == orc.FP16:
            v = rng.uniform(-0.01, 0.01, size=(E, D)).astype(np.float16)
            tab[:, : 2 * D] = v.view(np.uint8).reshape(E, 2 * D)
        else:
            v = rng.uniform(-0.01, 0.01, size=(E, D)).astype(np.float32)
            tab[:, : 4 * D] = v.view(np.uint8).reshape(E, 4 * D)
    return buf, w_off


def max_dims(tys, dims):
    def m(ty):
        return max([D for t, D in zip(tys, dims) if t == ty], default=0)

    return m(orc.INT2), m(orc.INT4), m(orc.INT8), m(orc.FP16), m(orc.FP32)


def nbit_forward_gpu(dev, W: torch.Tensor, w_off, tys, dims, indices, offsets, pooling: int,
                     out_f16: bool = True, indice_weights=None, row_align: int = 16,
                     index_dtype=torch.int64):
    T = len(tys)
    D_off = np.concatenate([[0], np.cumsum(dims)]).astype(np.int32)
    m2, m4, m8, m16, m32 = max_dims(tys, dims)
    empty = torch.zeros(0, dtype=torch.uint8, device=dev)
    return torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function(
        W, empty, torch.zeros(T, dtype=torch.int32, device=dev),
        torch.as_tensor(w_off, device=dev), torch.as_tensor(np.asarray(tys, np.uint8), device=dev),
        torch.as_tensor(D_off, device=dev), int(D_off[-1]), m2, m4, m8, m16, m32,
        torch.as_tensor(indices).to(dev, index_dtype), torch.as_tensor(offsets).to(dev, index_dtype),
        pooling, None if indice_weights is None else torch.as_tensor(indice_weights).to(dev),
        1 if out_f16 else 0, None, None, row_align)
