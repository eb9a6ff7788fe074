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
