"""Builders of small TBE test inputs and thin wrappers over the fbgemm ops."""

from __future__ import annotations

import numpy as np
import torch

from mx_fbgemm import bench_inputs


def random_tbe(rng: np.random.Generator, T: int, B: int, dims, rows, max_L: int,
               empty_frac: float = 0.2, dup_heavy: bool = False) -> bench_inputs.TbeInput:
    lengths = rng.integers(0, max_L + 1, size=T * B)
    lengths[rng.random(T * B) < empty_frac] = 0
    off = bench_inputs.offsets_from_lengths(lengths)
    idx = np.empty(int(off[-1]), dtype=np.int64)
    for t in range(T):
        s, e = int(off[t * B]), int(off[(t + 1) * B])
        hi = min(rows[t], 3) if dup_heavy else rows[t]
        idx[s:e] = rng.integers(0, hi, size=e - s)
    return bench_inputs.TbeInput(T=T, E=list(rows), D=list(dims), B=B, indices=idx, offsets=off)


def weight_offsets(inp: bench_inputs.TbeInput) -> np.ndarray:
    sizes = [E * D for E, D in zip(inp.E, inp.D)]
    return np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)


def tbe_forward_gpu(dev, W: torch.Tensor, inp: bench_inputs.TbeInput, pooling: int,
                    index_dtype=torch.int64, indice_weights=None, output_dtype: int = 0):
    w_off = torch.from_numpy(weight_offsets(inp)).to(dev)
    D_off = torch.from_numpy(inp.D_offsets).to(dev)
    idx = torch.from_numpy(inp.indices).to(dev, index_dtype)
    off = torch.from_numpy(inp.offsets).to(dev, index_dtype)
    empty = torch.zeros(0, device=dev)
    placements = torch.zeros(inp.T, dtype=torch.int32, device=dev)
    common = (W, empty, empty, placements, w_off, D_off, inp.total_D, max(inp.D), idx, off,
              pooling)
    tail = (torch.zeros(0, dtype=torch.int32, device=dev), torch.zeros(0, device=dev),
            output_dtype, False)
    if indice_weights is None:
        return torch.ops.fbgemm.split_embedding_codegen_forward_unweighted_cuda(*common, *tail)
    return torch.ops.fbgemm.split_embedding_codegen_forward_weighted_cuda(
        *common, indice_weights.to(dev), *tail)


class VbeCase:
    """A variable-batch-per-feature lookup and its dense equivalent.

    Table t has bs[t][r] bags on rank r; VBE bags are feature-major and
    rank-major within a feature.  The dense equivalent pads every table to
    max_B bags with empty bags: the index order and every per-row sum are the
    same, so the dense oracle gives the expected values.  The flat VBE output
    is rank-major then feature-major, bs[t][r] rows of D_t per block."""

    def __init__(self, rng: np.random.Generator, bs, dims, rows, max_L: int, empty_frac=0.15):
        self.bs = [list(r) for r in bs]
        self.T, self.R = len(bs), len(bs[0])
        self.dims, self.rows = list(dims), list(rows)
        self.B_t = [sum(r) for r in bs]
        self.max_B = max(1, max(self.B_t))
        self.B_offsets = np.concatenate([[0], np.cumsum(self.B_t)]).astype(np.int32)
        self.rpf = np.array([np.concatenate([[0], np.cumsum(r)]) for r in bs], dtype=np.int32)
        sizes = [bs[t][r] * dims[t] for r in range(self.R) for t in range(self.T)]
        self.out_ofr = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
        self.output_size = int(self.out_ofr[-1])
        self.total_B = int(self.B_offsets[-1])
        lengths = rng.integers(0, max_L + 1, size=self.total_B)
        lengths[rng.random(self.total_B) < empty_frac] = 0
        self.offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
        self.indices = np.empty(int(self.offsets[-1]), dtype=np.int64)
        for t in range(self.T):
            s, e = self.offsets[self.B_offsets[t]], self.offsets[self.B_offsets[t + 1]]
            self.indices[s:e] = rng.integers(0, rows[t], size=e - s)
        self.N = self.indices.size
        # dense padded equivalent
        dl = np.zeros(self.T * self.max_B, dtype=np.int64)
        for t in range(self.T):
            dl[t * self.max_B: t * self.max_B + self.B_t[t]] = \
                lengths[self.B_offsets[t]: self.B_offsets[t + 1]]
        self.dense = bench_inputs.TbeInput(T=self.T, E=list(rows), D=list(dims), B=self.max_B,
                                           indices=self.indices,
                                           offsets=bench_inputs.offsets_from_lengths(dl))
        # per-bag (t, feature-global b, row output offset), written out longhand
        self.bag_t, self.bag_b, self.row_out = [], [], []
        for t in range(self.T):
            for r in range(self.R):
                for br in range(bs[t][r]):
                    self.bag_t.append(t)
                    self.bag_b.append(int(self.rpf[t][r]) + br)
                    self.row_out.append(int(self.out_ofr[r * self.T + t]) + br * dims[t])
        self.bag_t, self.bag_b = np.array(self.bag_t), np.array(self.bag_b)
        self.row_out = np.array(self.row_out, dtype=np.int64)

    def b_t_map(self, nb: int) -> np.ndarray:
        return ((self.bag_t.astype(np.int64) << nb) | self.bag_b).astype(np.uint32).view(np.int32)

    def dense_to_flat(self, dense: np.ndarray) -> np.ndarray:
        """[max_B, total_D] (dense) -> flat VBE output."""
        out = np.zeros(self.output_size, dtype=dense.dtype)
        D_off = self.dense.D_offsets
        for i, (t, b, ro) in enumerate(zip(self.bag_t, self.bag_b, self.row_out)):
            out[ro: ro + self.dims[t]] = dense[b, D_off[t]: D_off[t + 1]]
        return out

    def flat_to_dense(self, flat: np.ndarray) -> np.ndarray:
        """flat VBE gradient -> [max_B, total_D] (padding bags get 0)."""
        D_off = self.dense.D_offsets
        out = np.zeros((self.max_B, int(D_off[-1])), dtype=flat.dtype)
        for t, b, ro in zip(self.bag_t, self.bag_b, self.row_out):
            out[b, D_off[t]: D_off[t + 1]] = flat[ro: ro + self.dims[t]]
        return out
