"""Inference TBE module: the caller that builds the arguments of
``torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function``.

Mirrors fbgemm_gpu's IntNBitTableBatchedEmbeddingBagsCodegen (upstream
fbgemm_gpu/split_table_batched_embeddings_ops_inference.py, recalled) for
DEVICE placement: all tables live in one uint8 HBM buffer, each row padded
to ``row_alignment`` bytes; INT8/INT4/INT2 rows start with an fp16 scale and
an fp16 bias; FP8 rows are D hfp8 codes (``fp8_exponent_bits`` exponent bits,
bias ``fp8_exponent_bias``).  Also carries the rowwise quantizer that produces
that layout from fp32 rows.
"""

from __future__ import annotations

import itertools
from typing import Optional

import torch
from torch import nn

from . import load_mx_fbgemm_library
from .sparse_types import (
    BoundsCheckMode,
    EmbeddingLocation,
    PoolingMode,
    SparseType,
    padded_row_size_in_bytes,
    unpadded_row_size_in_bytes,
)

load_mx_fbgemm_library()


def hfp8_max_pos(exponent_bits: int, exponent_bias: int) -> float:
    """The largest magnitude FBGEMM's hfp8 encoder produces (it leaves the top
    exponent field unused): 2^(2^ebits - 2 - bias) * (2 - 2^-(7 - ebits))."""
    m = 7 - exponent_bits
    return (2.0 - 2.0 ** -m) * 2.0 ** ((1 << exponent_bits) - 2 - exponent_bias)


def quantize_rows(weights: torch.Tensor, weight_ty: SparseType, row_alignment: int = 16,
                  fp8_exponent_bits: int = 4, fp8_exponent_bias: int = 7) -> torch.Tensor:
    """fp32/fp16 ``[E, D]`` (on the GPU) -> uint8 ``[E, padded_row_bytes]`` in
    the TBE row layout.

    INT8/INT4/INT2 rows are quantized by
    ``torch.ops.fbgemm.FloatOrHalfToFusedNBitRowwiseQuantizedSBHalf`` (bit rate
    8/4/2: fp16 scale and bias) and the two fp16 qparams are moved from the
    row end to the row front, as the TBE layout wants; FP8 rows are encoded by
    ``torch.ops.fbgemm.FloatToHFP8Quantized`` (nearest code, clamped to
    ``hfp8_max_pos``); FP16/FP32 rows are stored as-is.  Padding bytes are
    zero."""
    if not weights.is_cuda:
        raise ValueError("quantize_rows runs on the GPU; move the weights to the device first")
    E, D = weights.shape
    stride = padded_row_size_in_bytes(D, weight_ty, row_alignment)
    out = torch.zeros((E, stride), dtype=torch.uint8, device=weights.device)
    if weight_ty == SparseType.FP32:
        out[:, : 4 * D] = weights.float().contiguous().view(torch.uint8).view(E, 4 * D)
        return out
    if weight_ty == SparseType.FP16:
        out[:, : 2 * D] = weights.half().contiguous().view(torch.uint8).view(E, 2 * D)
        return out
    if weight_ty == SparseType.FP8:
        out[:, :D] = torch.ops.fbgemm.FloatToHFP8Quantized(
            weights.float().contiguous(), fp8_exponent_bits, fp8_exponent_bias,
            hfp8_max_pos(fp8_exponent_bits, fp8_exponent_bias))
        return out
    q = torch.ops.fbgemm.FloatOrHalfToFusedNBitRowwiseQuantizedSBHalf(
        weights.contiguous(), weight_ty.bit_rate())
    nbytes = q.shape[1] - 4
    out[:, 0:4] = q[:, nbytes:]
    out[:, 4:4 + nbytes] = q[:, :nbytes]
    return out


class IntNBitTableBatchedEmbeddingBagsCodegen(nn.Module):
    """Quantized TBE for inference.

    ``embedding_specs`` holds ``(name, num_embeddings, embedding_dim,
    weight_ty, location)`` per table; only EmbeddingLocation.DEVICE is
    supported.  ``feature_table_map`` ([T] table index per feature, default
    one feature per table) lets several features look up one table.
    PoolingMode.NONE (sequence lookups) needs every table of one width D and
    returns ``[N, D]``, row l the dequantized row of index l."""

    def __init__(
        self,
        embedding_specs: list[tuple[str, int, int, SparseType, EmbeddingLocation]],
        feature_table_map: Optional[list[int]] = None,
        pooling_mode: PoolingMode = PoolingMode.SUM,
        output_dtype: SparseType = SparseType.FP16,
        row_alignment: int = 16,
        device: Optional[torch.device] = None,
        bounds_check_mode: BoundsCheckMode = BoundsCheckMode.WARNING,
        fp8_exponent_bits: Optional[int] = None,
        fp8_exponent_bias: Optional[int] = None,
    ) -> None:
        super().__init__()
        if pooling_mode not in (PoolingMode.SUM, PoolingMode.MEAN, PoolingMode.NONE):
            raise ValueError(f"pooling_mode {pooling_mode} is not supported")
        if pooling_mode == PoolingMode.NONE and len({D for _, _, D, _, _ in embedding_specs}) > 1:
            raise ValueError("PoolingMode.NONE needs every table of one embedding_dim")
        if output_dtype not in (SparseType.FP16, SparseType.FP32, SparseType.BF16):
            raise ValueError("output_dtype must be FP16, FP32 or BF16")
        for _, E, D, ty, loc in embedding_specs:
            if loc != EmbeddingLocation.DEVICE:
                raise ValueError("only EmbeddingLocation.DEVICE is supported")
            if ty not in (SparseType.FP32, SparseType.FP16, SparseType.INT8, SparseType.INT4,
                          SparseType.INT2, SparseType.FP8):
                raise ValueError(f"weight type {ty} is not supported")
            if D <= 0 or D > 1024 or D % 8:
                raise ValueError(f"embedding_dim {D} must be a positive multiple of 8, <= 1024")
            if row_alignment < 1 or padded_row_size_in_bytes(D, ty, row_alignment) % 4:
                # The kernels read codes and qparams in 4-byte words.
                raise ValueError(f"row_alignment {row_alignment} leaves {ty} rows of D={D} "
                                 f"off 4-byte boundaries")
        device = torch.device(device) if device is not None else torch.device(
            "cuda", torch.cuda.current_device())
        self.embedding_specs = embedding_specs
        self.pooling_mode = pooling_mode
        self.output_dtype = output_dtype
        self.row_alignment = row_alignment
        self.bounds_check_mode = BoundsCheckMode(bounds_check_mode)
        dims = [D for _, _, D, _, _ in embedding_specs]
        rows = [E for _, E, _, _, _ in embedding_specs]
        tys = [ty for _, _, _, ty, _ in embedding_specs]
        ftm = list(range(len(embedding_specs))) if feature_table_map is None else \
            [int(t) for t in feature_table_map]
        if not ftm or any(t < 0 or t >= len(embedding_specs) for t in ftm):
            raise ValueError("feature_table_map must name tables of embedding_specs")
        self.feature_table_map = ftm
        self.T = len(ftm)  # features
        self.total_D = sum(dims[t] for t in ftm)
        self.row_bytes = [padded_row_size_in_bytes(D, ty, row_alignment)
                          for D, ty in zip(dims, tys)]
        sizes = [E * rb for E, rb in zip(rows, self.row_bytes)]
        offs = [0] + list(itertools.accumulate(sizes))
        self._table_offsets = offs[:-1]
        self.register_buffer("weights_offsets", torch.tensor([offs[t] for t in ftm],
                                                             device=device, dtype=torch.int64))
        self.register_buffer("weights_tys", torch.tensor([tys[t].as_int() for t in ftm],
                                                         device=device, dtype=torch.uint8))
        self.register_buffer("D_offsets",
                             torch.tensor([0] + list(itertools.accumulate(dims[t] for t in ftm)),
                                          device=device, dtype=torch.int32))
        self.register_buffer("weights_placements",
                             torch.full((self.T,), int(EmbeddingLocation.DEVICE), device=device,
                                        dtype=torch.int32))
        self.register_buffer("weights_dev", torch.zeros(offs[-1], device=device,
                                                        dtype=torch.uint8))
        self.register_buffer("weights_uvm", torch.zeros(0, device=device, dtype=torch.uint8),
                             persistent=False)

        def max_d(*kinds):
            return max([D for D, ty in zip(dims, tys) if ty in kinds], default=0)

        self.max_int2_D = max_d(SparseType.INT2)
        self.max_int4_D = max_d(SparseType.INT4)
        self.max_int8_D = max_d(SparseType.INT8)
        self.max_float16_D = max_d(SparseType.FP16)
        self.max_float32_D = max_d(SparseType.FP32)
        self.max_float8_D = max_d(SparseType.FP8)
        # hfp8 format of the FP8 tables (e4m3 with bias 7 unless given); -1 without them.
        self.fp8_exponent_bits = -1
        self.fp8_exponent_bias = -1
        if self.max_float8_D > 0:
            self.fp8_exponent_bits = 4 if fp8_exponent_bits is None else int(fp8_exponent_bits)
            self.fp8_exponent_bias = 7 if fp8_exponent_bias is None else int(fp8_exponent_bias)
            if not (1 <= self.fp8_exponent_bits <= 7 and 0 <= self.fp8_exponent_bias <= 120):
                raise ValueError("FP8 tables need 1 <= fp8_exponent_bits <= 7 and "
                                 "0 <= fp8_exponent_bias <= 120")
        self.register_buffer("rows_per_table", torch.tensor([rows[t] for t in ftm],
                                                            device=device, dtype=torch.int64))
        self.register_buffer("bounds_check_warning", torch.zeros(1, device=device,
                                                                 dtype=torch.int64))
        self._rows, self._dims, self._tys = rows, dims, tys
        for D, ty in zip(dims, tys):
            unpadded_row_size_in_bytes(D, ty)  # validates the type

    def forward(self, indices: torch.Tensor, offsets: torch.Tensor,
                per_sample_weights: Optional[torch.Tensor] = None) -> torch.Tensor:
        if (offsets.numel() - 1) % self.T:
            raise ValueError(f"offsets must have T*B+1 entries (T={self.T})")
        if self.pooling_mode == PoolingMode.NONE and per_sample_weights is not None:
            raise ValueError("PoolingMode.NONE takes no per_sample_weights")
        if indices.dtype != offsets.dtype:
            offsets = offsets.to(indices.dtype)
        if self.bounds_check_mode != BoundsCheckMode.NONE:
            torch.ops.fbgemm.bounds_check_indices(self.rows_per_table, indices, offsets,
                                                  int(self.bounds_check_mode),
                                                  self.bounds_check_warning, per_sample_weights)
        return torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function(
            self.weights_dev, self.weights_uvm, self.weights_placements, self.weights_offsets,
            self.weights_tys, self.D_offsets, self.total_D, self.max_int2_D, self.max_int4_D,
            self.max_int8_D, self.max_float16_D, self.max_float32_D, indices, offsets,
            int(self.pooling_mode), per_sample_weights, self.output_dtype.as_int(), None, None,
            self.row_alignment, self.max_float8_D, self.fp8_exponent_bits, self.fp8_exponent_bias)

    @torch.no_grad()
    def split_embedding_weights(self) -> list[torch.Tensor]:
        """Per-table uint8 ``[E_t, row_bytes_t]`` views (qparams included)."""
        out = []
        for o, E, rb in zip(self._table_offsets, self._rows, self.row_bytes):
            out.append(self.weights_dev[o:o + E * rb].view(E, rb))
        return out

    @torch.no_grad()
    def assign_embedding_weights(self, weights: list[torch.Tensor]) -> None:
        """Quantize fp32 ``[E_t, D_t]`` tables into the device buffer."""
        for t, (w, dst) in enumerate(zip(weights, self.split_embedding_weights())):
            dst.copy_(quantize_rows(w.to(dst.device), self._tys[t], self.row_alignment,
                                    self.fp8_exponent_bits, self.fp8_exponent_bias))

    @torch.no_grad()
    def fill_random_weights(self, seed: int = 0) -> None:
        """Random codes (FP8 rows: random hfp8 codes), fp16 scale in
        [1e-3, 1e-2), bias in [-0.1, 0.1)."""
        g = torch.Generator(device=self.weights_dev.device)
        g.manual_seed(seed)
        for t, dst in enumerate(self.split_embedding_weights()):
            dst.copy_(torch.randint(0, 256, dst.shape, generator=g, device=dst.device,
                                    dtype=torch.int32).to(torch.uint8))
            ty = self._tys[t]
            if ty.is_rowwise_quantized():
                E = dst.shape[0]
                sc = (torch.rand(E, generator=g, device=dst.device) * 9e-3 + 1e-3).half()
                bi = (torch.rand(E, generator=g, device=dst.device) * 0.2 - 0.1).half()
                dst[:, 0:2] = sc.view(torch.uint8).view(E, 2)
                dst[:, 2:4] = bi.view(torch.uint8).view(E, 2)
            elif ty == SparseType.FP16:
                E, rb = dst.shape
                D = self._dims[t]
                v = (torch.rand((E, D), generator=g, device=dst.device) * 0.02 - 0.01).half()
                dst[:, : 2 * D] = v.view(torch.uint8).view(E, 2 * D)
            elif ty == SparseType.FP32:
                E, rb = dst.shape
                D = self._dims[t]
                v = torch.rand((E, D), generator=g, device=dst.device) * 0.02 - 0.01
                dst[:, : 4 * D] = v.view(torch.uint8).view(E, 4 * D)
