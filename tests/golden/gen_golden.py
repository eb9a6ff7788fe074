"""Writes the golden fixtures of this directory from in-container reference
implementations (not from this build's oracle):

* jagged.npz    aten._jagged_to_padded_dense_forward / _padded_dense_to_jagged_forward
* tbe_fwd.npz   FBGEMM GenerateEmbeddingSpMDMWithStrides (CPU kernel exported by torch)
* nbit.npz      FBGEMM 8-bit / N-bit / fp16 SpMDM CPU kernels, TBE row layout
* transpose.npz numpy stable argsort + unique

Run from the repository root:  python tests/golden/gen_golden.py
"""

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path[:0] = [str(REPO / "tests"), str(REPO / "oracle"), str(REPO / "torchlib-xpu_amd")]

import oracle as orc  # noqa: E402  (FBGEMM harness lives beside the oracle)
from nbit_helpers import build_weights  # noqa: E402
from tbe_helpers import random_tbe, weight_offsets  # noqa: E402


def jagged():
    rng = np.random.default_rng(2024)
    lengths = np.array([3, 0, 7, 1, 4, 4, 0, 2])
    off = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    vals = rng.standard_normal((int(off[-1]), 6)).astype(np.float32)
    dense = torch.ops.aten._jagged_to_padded_dense_forward(
        torch.from_numpy(vals), [torch.from_numpy(off)], [5], -1.0).numpy()
    lengths2 = np.minimum(lengths, 5)
    off2 = np.concatenate([[0], np.cumsum(lengths2)]).astype(np.int64)
    dense2 = rng.standard_normal((8, 5, 6)).astype(np.float32)
    jag2 = torch.ops.aten._padded_dense_to_jagged_forward(
        torch.from_numpy(dense2), [torch.from_numpy(off2)], int(off2[-1])).numpy()
    np.savez_compressed(HERE / "jagged.npz", values=vals, offsets=off, max_L=5, pad=-1.0,
                        dense=dense, dense2=dense2, offsets2=off2, jagged2=jag2)


def tbe_fwd():
    rng = np.random.default_rng(2025)
    inp = random_tbe(rng, 3, 24, [8, 64, 128], [40, 90, 25], 11)
    W = rng.uniform(-1, 1, size=sum(E * D for E, D in zip(inp.E, inp.D))).astype(np.float32)
    iw = rng.uniform(0, 2, inp.N).astype(np.float32)
    outs = {}
    for pooling in (0, 1):
        outs[f"out_p{pooling}"] = orc.fbgemm_tbe_forward_f32(
            W, weight_offsets(inp), inp.D_offsets, inp.E, inp.B, inp.indices, inp.offsets, pooling)
        outs[f"out_w_p{pooling}"] = orc.fbgemm_tbe_forward_f32(
            W, weight_offsets(inp), inp.D_offsets, inp.E, inp.B, inp.indices, inp.offsets, pooling,
            iw)
    np.savez_compressed(HERE / "tbe_fwd.npz", W=W, w_off=weight_offsets(inp), D_off=inp.D_offsets,
                        E=np.array(inp.E), B=inp.B, indices=inp.indices, offsets=inp.offsets,
                        iw=iw, **outs)


def nbit():
    rng = np.random.default_rng(2026)
    tys = [orc.INT8, orc.INT4, orc.INT2, orc.FP16, orc.FP32]
    dims = [64, 32, 128, 16, 32]
    rows = [30, 60, 20, 45, 15]
    inp = random_tbe(rng, len(tys), 14, dims, rows, 13)
    buf, w_off = build_weights(rng, tys, dims, rows)
    outs = {f"out_p{p}": orc.fbgemm_nbit_forward(buf, w_off, tys, inp.D_offsets, rows, inp.B,
                                                 inp.indices, inp.offsets, p) for p in (0, 1)}
    np.savez_compressed(HERE / "nbit.npz", W=buf, w_off=w_off, tys=np.array(tys, np.uint8),
                        D_off=inp.D_offsets, E=np.array(rows), B=inp.B, indices=inp.indices,
                        offsets=inp.offsets, **outs)


def transpose():
    rng = np.random.default_rng(2027)
    T, B = 3, 40
    inp = random_tbe(rng, T, B, [4] * T, [7, 300, 3], 12, dup_heavy=False)
    nb = 26
    bag = np.repeat(np.arange(T * B), np.diff(inp.offsets))
    t, b = bag // B, bag % B
    lin = inp.hash_size_cumsum[t] + inp.indices
    info = ((t.astype(np.int64) << nb) | b).astype(np.int64)
    order = np.argsort(lin, kind="stable")
    u, first, counts = np.unique(lin[order], return_index=True, return_counts=True)
    np.savez_compressed(HERE / "transpose.npz", hsc=inp.hash_size_cumsum, B=B, nb=nb,
                        bits=inp.total_hash_size_bits, indices=inp.indices, offsets=inp.offsets,
                        linear=lin, sorted=lin[order], infos=info[order].astype(np.uint32).view(np.int32),
                        run=u, run_lengths=counts.astype(np.int32),
                        cum=np.append(first, lin.size).astype(np.int32))


if __name__ == "__main__":
    jagged()
    tbe_fwd()
    nbit()
    transpose()
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)
