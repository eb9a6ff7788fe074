"""Training TBE module: the caller that builds the arguments of
``torch.ops.fbgemm.split_embedding_codegen_lookup_rowwise_adagrad_function``.

Mirrors fbgemm_gpu's SplitTableBatchedEmbeddingBagsCodegen (upstream
fbgemm_gpu/split_table_batched_embeddings_ops_training.py, recalled) for the
path this build serves: DEVICE placement, fp32 or fp16 weights
(``weights_precision``; fp16 updates round stochastically by default, as
upstream), SUM/MEAN pooling and the EXACT_ROWWISE_ADAGRAD optimizer fused
into the backward.  Weights and the
per-row momentum live in one flat HBM buffer each; tables are laid out back
to back (weights_offsets, momentum1_offsets in elements).
"""

from __future__ import annotations

import itertools
from typing import Optional

import torch
from torch import nn

from . import load_mx_fbgemm_library
from .sparse_types import (
    BoundsCheckMode,
    ComputeDevice,
    EmbeddingLocation,
    EmbOptimType,
    PoolingMode,
    SparseType,
)

load_mx_fbgemm_library()


def _cumsum(xs: list[int]) -> list[int]:
    return [0] + list(itertools.accumulate(xs))


class SplitTableBatchedEmbeddingBagsCodegen(nn.Module):
    """T embedding tables looked up and pooled in one launch.

    ``embedding_specs`` holds ``(num_embeddings, embedding_dim, location,
    compute_device)`` per table; only EmbeddingLocation.DEVICE on a GPU is
    supported.  ``feature_table_map`` ([T] table index per feature, default
    one feature per table) lets features share a table: they look up the same
    rows, and the fused update sums every feature's gradient into each row
    once.  ``forward(indices, offsets)`` takes feature-major offsets of T*B+1
    entries (T features) and returns ``[B, sum of the features' D]``; ``loss.backward()`` updates the
    weights and momentum in place (the gradient itself is never materialised).
    Indices and offsets are first validated, and repaired in place, by
    ``torch.ops.fbgemm.bounds_check_indices`` (BoundsCheckMode.WARNING by
    default, as upstream); the count accumulates in ``bounds_check_warning``.
    ``per_sample_weights`` (fp32, one per index) make it a weighted lookup:
    each row is scaled by its weight before pooling, the fused update uses the
    weighted row gradient, and the weights themselves receive a gradient when
    they require one (``feature_requires_grad`` [T] masks tables out).

    ``batch_size_per_feature_per_rank`` ([T][R] ints) selects variable batch
    size per feature (VBE): table t has sum_r B[t][r] bags, offsets has
    sum_t sum_r B[t][r] + 1 entries (feature-major, rank-major within a
    feature), and the output is one flat tensor, rank-major then
    feature-major, holding B[t][r] rows of D_t per (rank, feature).

    PoolingMode.NONE (sequence lookups) needs every feature of one width D:
    ``forward`` returns ``[N, D]``, row l the row of index l, and the fused
    update sums each row's gradient rows (no per-sample weights, no VBE).
    """

    def __init__(
        self,
        embedding_specs: list[tuple[int, int, EmbeddingLocation, ComputeDevice]],
        feature_table_map: Optional[list[int]] = None,
        optimizer: EmbOptimType = EmbOptimType.EXACT_ROWWISE_ADAGRAD,
        pooling_mode: PoolingMode = PoolingMode.SUM,
        learning_rate: float = 0.01,
        eps: float = 1.0e-8,
        weight_decay: float = 0.0,
        weight_decay_mode: int = 0,
        output_dtype: SparseType = SparseType.FP32,
        device: Optional[torch.device] = None,
        weights_init: Optional[tuple[float, float]] = None,
        bounds_check_mode: BoundsCheckMode = BoundsCheckMode.WARNING,
        weights_precision: SparseType = SparseType.FP32,
        stochastic_rounding: bool = True,
    ) -> None:
        super().__init__()
        if optimizer != EmbOptimType.EXACT_ROWWISE_ADAGRAD:
            raise ValueError(f"optimizer {optimizer} is not supported")
        if pooling_mode not in (PoolingMode.SUM, PoolingMode.MEAN, PoolingMode.NONE):
            raise ValueError(f"pooling_mode {pooling_mode} is not supported")
        if output_dtype != SparseType.FP32:
            raise ValueError("the training lookup produces fp32 output")
        if weights_precision not in (SparseType.FP32, SparseType.FP16):
            raise ValueError("weights_precision must be FP32 or FP16")
        if not embedding_specs:
            raise ValueError("at least one table is required")
        for E, D, loc, cd in embedding_specs:
            if loc != EmbeddingLocation.DEVICE or cd != ComputeDevice.CUDA:
                raise ValueError("only EmbeddingLocation.DEVICE on the GPU is supported")
            if D <= 0 or D % 4 != 0 or D > 1024:
                raise ValueError(f"embedding_dim {D} must be a positive multiple of 4, <= 1024")
            if E <= 0:
                raise ValueError("num_embeddings must be positive")
        device = torch.device(device) if device is not None else torch.device(
            "cuda", torch.cuda.current_device())
        self.embedding_specs = embedding_specs
        self.pooling_mode = pooling_mode
        self.learning_rate = float(learning_rate)
        self.eps = float(eps)
        self.weight_decay = float(weight_decay)
        self.weight_decay_mode = int(weight_decay_mode)
        self.bounds_check_mode = BoundsCheckMode(bounds_check_mode)
        self.weights_precision = weights_precision
        # Only fp16 weights have a rounding step; fp32 updates ignore the flag.
        self.stochastic_rounding = bool(stochastic_rounding)
        rows = [E for E, _, _, _ in embedding_specs]
        dims = [D for _, D, _, _ in embedding_specs]
        # Features (the T of the batch) map onto tables; several features may
        # share one table, i.e. its rows, hash offset and momentum.
        ftm = list(range(len(embedding_specs))) if feature_table_map is None else \
            [int(t) for t in feature_table_map]
        if not ftm or any(t < 0 or t >= len(embedding_specs) for t in ftm):
            raise ValueError("feature_table_map must name tables of embedding_specs")
        self.feature_table_map = ftm
        self.T = len(ftm)
        f_rows = [rows[t] for t in ftm]
        f_dims = [dims[t] for t in ftm]
        if pooling_mode == PoolingMode.NONE and len(set(f_dims)) > 1:
            raise ValueError("PoolingMode.NONE needs every feature of one embedding_dim")
        self.total_D = sum(f_dims)
        self.max_D = max(f_dims)
        table_hash = _cumsum(rows)
        self.total_hash_size_bits = max(1, int(table_hash[-1] - 1).bit_length())
        if self.total_hash_size_bits > 32:
            raise ValueError("total hash size above 2^32 rows is not supported")
        w_elems = [E * D for E, D in zip(rows, dims)]
        table_w_off = _cumsum(w_elems)[:-1]
        i64 = dict(device=device, dtype=torch.int64)
        self.register_buffer("weights_offsets",
                             torch.tensor([table_w_off[t] for t in ftm], **i64))
        self.register_buffer("D_offsets", torch.tensor(_cumsum(f_dims), device=device,
                                                       dtype=torch.int32))
        self.register_buffer("hash_size_cumsum",
                             torch.tensor([table_hash[t] for t in ftm] + [table_hash[-1]], **i64))
        self.register_buffer("weights_placements",
                             torch.full((self.T,), int(EmbeddingLocation.DEVICE), device=device,
                                        dtype=torch.int32))
        self.register_buffer("momentum1_offsets",
                             torch.tensor([table_hash[t] for t in ftm], **i64))
        lo, hi = weights_init if weights_init is not None else (-0.01, 0.01)
        self.weights_dev = nn.Parameter(
            torch.empty(sum(w_elems), device=device, dtype=torch.float32).uniform_(lo, hi)
            .to(weights_precision.as_dtype()),
            requires_grad=False)
        self.register_buffer("momentum1_dev",
                             torch.zeros(sum(rows), device=device, dtype=torch.float32))
        empty_f = torch.zeros(0, device=device, dtype=torch.float32)
        self.register_buffer("weights_uvm", empty_f.clone(), persistent=False)
        self.register_buffer("lxu_cache_weights", empty_f.clone(), persistent=False)
        self.register_buffer("momentum1_uvm", empty_f.clone(), persistent=False)
        self.register_buffer("lxu_cache_locations",
                             torch.zeros(0, device=device, dtype=torch.int32), persistent=False)
        # A zero-element leaf that makes autograd record the lookup even
        # though the weights are updated by the fused backward, not by autograd.
        self.placeholder_autograd_tensor = nn.Parameter(
            torch.zeros(0, device=device, dtype=torch.float32))
        self.register_buffer("rows_per_table", torch.tensor(f_rows, **i64))
        self.register_buffer("bounds_check_warning", torch.zeros(1, **i64))
        self._rows = rows
        self._dims = dims
        self._f_dims = f_dims
        self._table_w_off = table_w_off
        self._table_m_off = table_hash[:-1]

    def _vbe_args(self, batch_size_per_feature_per_rank: list[list[int]], device):
        """B_offsets, output offsets per (rank, feature), batch offsets per
        feature and rank, max_B, max_B_feature_rank, output size."""
        bs = batch_size_per_feature_per_rank
        if len(bs) != self.T or len({len(r) for r in bs}) != 1:
            raise ValueError("batch_size_per_feature_per_rank must be [T][R]")
        R = len(bs[0])
        per_feature = [sum(r) for r in bs]
        B_offsets = _cumsum(per_feature)
        rpf = [_cumsum(r) for r in bs]
        out_sizes = [bs[t][r] * self._f_dims[t] for r in range(R) for t in range(self.T)]
        i32 = dict(device=device, dtype=torch.int32)
        return dict(
            B_offsets=torch.tensor(B_offsets, **i32),
            vbe_output_offsets_feature_rank=torch.tensor(_cumsum(out_sizes), device=device,
                                                         dtype=torch.int64),
            vbe_B_offsets_rank_per_feature=torch.tensor(rpf, **i32),
            max_B=max(per_feature), max_B_feature_rank=max(max(r) for r in bs),
            vbe_output_size=sum(out_sizes))

    def forward(self, indices: torch.Tensor, offsets: torch.Tensor,
                per_sample_weights: Optional[torch.Tensor] = None,
                feature_requires_grad: Optional[torch.Tensor] = None,
                batch_size_per_feature_per_rank: Optional[list[list[int]]] = None
                ) -> torch.Tensor:
        if per_sample_weights is not None:
            if per_sample_weights.dtype != torch.float32:
                raise ValueError("per_sample_weights must be fp32")
            if per_sample_weights.numel() != indices.numel():
                raise ValueError("per_sample_weights must have one entry per index")
        if self.pooling_mode == PoolingMode.NONE and (
                per_sample_weights is not None or batch_size_per_feature_per_rank is not None):
            raise ValueError("PoolingMode.NONE takes no per_sample_weights and no VBE batch")
        vbe = (self._vbe_args(batch_size_per_feature_per_rank, indices.device)
               if batch_size_per_feature_per_rank is not None else None)
        if vbe is not None:
            if offsets.numel() - 1 != int(vbe["B_offsets"][-1]):
                raise ValueError("offsets must have one entry per bag of every feature, plus one")
        elif (offsets.numel() - 1) % self.T:
            raise ValueError(f"offsets must have T*B+1 entries (T={self.T})")
        if indices.dtype != offsets.dtype:
            offsets = offsets.to(indices.dtype)
        if self.bounds_check_mode != BoundsCheckMode.NONE:
            torch.ops.fbgemm.bounds_check_indices(
                self.rows_per_table, indices, offsets, int(self.bounds_check_mode),
                self.bounds_check_warning, per_sample_weights,
                vbe["B_offsets"] if vbe is not None else None,
                vbe["max_B"] if vbe is not None else -1)
        return torch.ops.fbgemm.split_embedding_codegen_lookup_rowwise_adagrad_function(
            self.placeholder_autograd_tensor, self.weights_dev, self.weights_uvm,
            self.lxu_cache_weights, self.weights_placements, self.weights_offsets,
            self.D_offsets, self.total_D, self.max_D, self.hash_size_cumsum,
            self.total_hash_size_bits, indices, offsets, int(self.pooling_mode),
            per_sample_weights, feature_requires_grad,
            self.lxu_cache_locations, False, 0.0, self.stochastic_rounding, self.momentum1_dev,
            self.momentum1_uvm,
            self.weights_placements, self.momentum1_offsets, self.eps, self.learning_rate,
            self.weight_decay, self.weight_decay_mode, 0.0, int(SparseType.FP32.as_int()),
            **(vbe or {}))

    @torch.no_grad()
    def split_embedding_weights(self) -> list[torch.Tensor]:
        """Per-table ``[E_t, D_t]`` views of the flat weight buffer."""
        out = []
        for o, E, D in zip(self._table_w_off, self._rows, self._dims):
            out.append(self.weights_dev.detach()[o:o + E * D].view(E, D))
        return out

    def set_learning_rate(self, lr: float) -> None:
        """The rate the next backward's fused update uses."""
        self.learning_rate = float(lr)

    def get_learning_rate(self) -> float:
        return self.learning_rate

    @torch.no_grad()
    def init_embedding_weights_uniform(self, min_val: float, max_val: float) -> None:
        """Every row of every table drawn from U(min_val, max_val)."""
        w = torch.empty(self.weights_dev.numel(), device=self.weights_dev.device,
                        dtype=torch.float32).uniform_(min_val, max_val)
        self.weights_dev.copy_(w.to(self.weights_dev.dtype))

    @torch.no_grad()
    def split_optimizer_states(self) -> list[list[torch.Tensor]]:
        """Per-table ``[[momentum1 (E_t,)]]`` views."""
        return [[self.momentum1_dev[o:o + E]] for o, E in zip(self._table_m_off, self._rows)]
