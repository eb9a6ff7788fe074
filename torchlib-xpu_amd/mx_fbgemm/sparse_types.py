"""Enums and row-layout helpers of the TBE operators.

The integer values are the ones fbgemm_gpu passes through its op schemas
(upstream fbgemm_gpu/split_embedding_configs.py and
split_table_batched_embeddings_ops_common.py, recalled): SparseType for
``weights_tys``/``output_dtype``, PoolingMode for ``pooling_mode`` and
EmbeddingLocation for ``weights_placements``.
"""

from __future__ import annotations

import enum

import torch


class SparseType(enum.Enum):
    FP32 = "fp32"
    FP16 = "fp16"
    INT8 = "int8"
    INT4 = "int4"
    INT2 = "int2"
    BF16 = "bf16"
    FP8 = "fp8"

    def as_int(self) -> int:
        return {"fp32": 0, "fp16": 1, "int8": 2, "int4": 3, "int2": 4, "bf16": 5,
                "fp8": 6}[self.value]

    @staticmethod
    def from_int(ty: int) -> "SparseType":
        for s in SparseType:
            if s.as_int() == ty:
                return s
        raise ValueError(f"unknown SparseType value {ty}")

    def bit_rate(self) -> int:
        return {"fp32": 32, "fp16": 16, "int8": 8, "int4": 4, "int2": 2, "bf16": 16,
                "fp8": 8}[self.value]

    def as_dtype(self) -> torch.dtype:
        return {
            "fp32": torch.float32,
            "fp16": torch.float16,
            "bf16": torch.bfloat16,
            "int8": torch.uint8,
            "int4": torch.quint4x2,
            "int2": torch.quint2x4,
            "fp8": torch.uint8,
        }[self.value]

    def is_rowwise_quantized(self) -> bool:
        return self in (SparseType.INT8, SparseType.INT4, SparseType.INT2)


class PoolingMode(enum.IntEnum):
    SUM = 0
    MEAN = 1
    NONE = 2


class EmbeddingLocation(enum.IntEnum):
    DEVICE = 0
    MANAGED = 1
    MANAGED_CACHING = 2
    HOST = 3


class BoundsCheckMode(enum.IntEnum):
    FATAL = 0
    WARNING = 1
    IGNORE = 2
    NONE = 3


class ComputeDevice(enum.IntEnum):
    CPU = 0
    CUDA = 1


class EmbOptimType(enum.Enum):
    EXACT_ROWWISE_ADAGRAD = "exact_row_wise_adagrad"


# Bytes of the fp16 scale + fp16 bias at the front of each quantized row.
QPARAM_BYTES = 4


def unpadded_row_size_in_bytes(dim: int, weight_ty: SparseType) -> int:
    """Bytes of one row before alignment padding."""
    if weight_ty == SparseType.FP32:
        return dim * 4
    if weight_ty in (SparseType.FP16, SparseType.BF16):
        return dim * 2
    if weight_ty == SparseType.FP8:
        return dim
    if weight_ty == SparseType.INT8:
        return dim + QPARAM_BYTES
    if weight_ty == SparseType.INT4:
        return dim // 2 + QPARAM_BYTES
    if weight_ty == SparseType.INT2:
        return dim // 4 + QPARAM_BYTES
    raise ValueError(f"unsupported weight type {weight_ty}")


def padded_row_size_in_bytes(dim: int, weight_ty: SparseType, row_alignment: int = 16) -> int:
    """Row stride: the unpadded size rounded up to ``row_alignment`` bytes."""
    r = unpadded_row_size_in_bytes(dim, weight_ty)
    return (r + row_alignment - 1) // row_alignment * row_alignment
