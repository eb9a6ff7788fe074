"""Host-side logic without a GPU: enums, row sizes, the TBE modules' argument
builders (constructed on the CPU device; no op is called) and the rowwise
quantizer's TBE row layout (checked by decoding it with the oracle)."""

import numpy as np
import pytest
import torch

import oracle as orc
from mx_fbgemm import ComputeDevice, EmbeddingLocation, PoolingMode, SparseType, bench_inputs
from mx_fbgemm.sparse_types import padded_row_size_in_bytes, unpadded_row_size_in_bytes
from mx_fbgemm.split_table_batched_embeddings_ops_inference import (
    IntNBitTableBatchedEmbeddingBagsCodegen,
    quantize_rows,
)
from mx_fbgemm.split_table_batched_embeddings_ops_training import (
    SplitTableBatchedEmbeddingBagsCodegen,
)


def test_enums_match_fbgemm_values():
    assert [s.as_int() for s in (SparseType.FP32, SparseType.FP16, SparseType.INT8, SparseType.INT4,
                                 SparseType.INT2, SparseType.BF16, SparseType.FP8)] == \
        [0, 1, 2, 3, 4, 5, 6]
    assert SparseType.from_int(6) == SparseType.FP8
    assert (PoolingMode.SUM, PoolingMode.MEAN, PoolingMode.NONE) == (0, 1, 2)
    assert EmbeddingLocation.DEVICE == 0 and EmbeddingLocation.HOST == 3
    assert SparseType.from_int(3) == SparseType.INT4


@pytest.mark.parametrize("ty,D,unpadded,padded", [(SparseType.INT8, 128, 132, 144),
                                                  (SparseType.INT4, 128, 68, 80),
                                                  (SparseType.INT2, 64, 20, 32),
                                                  (SparseType.FP16, 36, 72, 80),
                                                  (SparseType.FP32, 8, 32, 32)])
def test_row_sizes(ty, D, unpadded, padded):
    assert unpadded_row_size_in_bytes(D, ty) == unpadded
    assert padded_row_size_in_bytes(D, ty, 16) == padded
    assert orc.nbit_row_bytes(ty.as_int(), D, 16) == padded


def test_training_module_arguments():
    specs = [(100, 64, EmbeddingLocation.DEVICE, ComputeDevice.CUDA),
             (7, 128, EmbeddingLocation.DEVICE, ComputeDevice.CUDA),
             (2 ** 20, 4, EmbeddingLocation.DEVICE, ComputeDevice.CUDA)]
    m = SplitTableBatchedEmbeddingBagsCodegen(specs, device="cpu")
    assert m.weights_offsets.tolist() == [0, 6400, 6400 + 896]
    assert m.D_offsets.tolist() == [0, 64, 192, 196]
    assert m.hash_size_cumsum.tolist() == [0, 100, 107, 107 + 2 ** 20]
    assert m.total_hash_size_bits == 21
    assert m.momentum1_offsets.tolist() == [0, 100, 107]
    assert m.weights_dev.numel() == 6400 + 896 + 4 * 2 ** 20
    assert m.total_D == 196 and m.max_D == 128
    w = m.split_embedding_weights()
    assert [tuple(x.shape) for x in w] == [(100, 64), (7, 128), (2 ** 20, 4)]
    assert float(m.weights_dev.abs().max()) <= 0.01


def test_training_module_feature_table_map():
    """Features 0 and 2 share table 0: per-feature offsets point at its rows,
    hash range and momentum; the output has one column block per feature."""
    specs = [(100, 64, EmbeddingLocation.DEVICE, ComputeDevice.CUDA),
             (7, 128, EmbeddingLocation.DEVICE, ComputeDevice.CUDA)]
    m = SplitTableBatchedEmbeddingBagsCodegen(specs, [0, 1, 0], device="cpu")
    assert m.T == 3
    assert m.weights_offsets.tolist() == [0, 6400, 0]
    assert m.D_offsets.tolist() == [0, 64, 192, 256]
    assert m.hash_size_cumsum.tolist() == [0, 100, 0, 107]
    assert m.momentum1_offsets.tolist() == [0, 100, 0]
    assert m.rows_per_table.tolist() == [100, 7, 100]
    assert m.total_D == 256 and m.max_D == 128 and m.total_hash_size_bits == 7
    assert m.weights_dev.numel() == 6400 + 896 and m.momentum1_dev.numel() == 107
    assert [tuple(x.shape) for x in m.split_embedding_weights()] == [(100, 64), (7, 128)]
    with pytest.raises(ValueError):
        SplitTableBatchedEmbeddingBagsCodegen(specs, [0, 2], device="cpu")


def test_training_module_learning_rate_and_init():
    m = SplitTableBatchedEmbeddingBagsCodegen(
        [(10, 8, EmbeddingLocation.DEVICE, ComputeDevice.CUDA)], learning_rate=0.1, device="cpu")
    assert m.get_learning_rate() == 0.1
    m.set_learning_rate(0.02)
    assert m.get_learning_rate() == 0.02
    m.init_embedding_weights_uniform(2.0, 3.0)
    w = m.split_embedding_weights()[0]
    assert float(w.min()) >= 2.0 and float(w.max()) <= 3.0


def test_training_module_rejects_unsupported():
    with pytest.raises(ValueError):
        SplitTableBatchedEmbeddingBagsCodegen(
            [(10, 6, EmbeddingLocation.DEVICE, ComputeDevice.CUDA)], device="cpu")  # D % 4
    with pytest.raises(ValueError):
        SplitTableBatchedEmbeddingBagsCodegen(
            [(10, 8, EmbeddingLocation.MANAGED, ComputeDevice.CUDA)], device="cpu")
    with pytest.raises(ValueError, match="one embedding_dim"):  # NONE: one width for all
        SplitTableBatchedEmbeddingBagsCodegen(
            [(10, 8, EmbeddingLocation.DEVICE, ComputeDevice.CUDA),
             (10, 16, EmbeddingLocation.DEVICE, ComputeDevice.CUDA)],
            pooling_mode=PoolingMode.NONE, device="cpu")
    m = SplitTableBatchedEmbeddingBagsCodegen(
        [(10, 8, EmbeddingLocation.DEVICE, ComputeDevice.CUDA)] * 2, pooling_mode=PoolingMode.NONE,
        device="cpu")
    with pytest.raises(ValueError, match="PoolingMode.NONE takes no"):
        m(torch.zeros(2, dtype=torch.int64), torch.tensor([0, 1, 2]),
          per_sample_weights=torch.ones(2))


def test_inference_module_nobag_arguments():
    with pytest.raises(ValueError, match="one embedding_dim"):
        IntNBitTableBatchedEmbeddingBagsCodegen(
            [("a", 10, 16, SparseType.INT8, EmbeddingLocation.DEVICE),
             ("b", 10, 32, SparseType.INT8, EmbeddingLocation.DEVICE)],
            pooling_mode=PoolingMode.NONE, device="cpu")
    m = IntNBitTableBatchedEmbeddingBagsCodegen(
        [("a", 10, 16, SparseType.INT8, EmbeddingLocation.DEVICE),
         ("b", 10, 16, SparseType.FP16, EmbeddingLocation.DEVICE)],
        pooling_mode=PoolingMode.NONE, device="cpu")
    with pytest.raises(ValueError, match="PoolingMode.NONE takes no"):
        m(torch.zeros(2, dtype=torch.int64), torch.tensor([0, 1, 2]),
          per_sample_weights=torch.ones(2))


def test_inference_module_arguments():
    specs = [("a", 10, 128, SparseType.INT8, EmbeddingLocation.DEVICE),
             ("b", 20, 64, SparseType.INT4, EmbeddingLocation.DEVICE),
             ("c", 5, 32, SparseType.FP16, EmbeddingLocation.DEVICE)]
    m = IntNBitTableBatchedEmbeddingBagsCodegen(specs, device="cpu")
    assert m.row_bytes == [144, 48, 64]
    assert m.weights_offsets.tolist() == [0, 1440, 1440 + 960]
    assert m.weights_tys.tolist() == [2, 3, 1]
    assert (m.max_int8_D, m.max_int4_D, m.max_float16_D, m.max_int2_D, m.max_float32_D) == \
        (128, 64, 32, 0, 0)
    assert m.weights_dev.numel() == 1440 + 960 + 320
    # INT2 rows of D = 8 are 6 bytes: row_alignment 1 or 2 would leave them off
    # 4-byte boundaries, which the kernels cannot read.
    int2 = [("d", 10, 8, SparseType.INT2, EmbeddingLocation.DEVICE)]
    m4 = IntNBitTableBatchedEmbeddingBagsCodegen(int2, row_alignment=4, device="cpu")
    assert m4.row_bytes == [8]
    for bad in (0, 1, 2):
        with pytest.raises(ValueError):
            IntNBitTableBatchedEmbeddingBagsCodegen(int2, row_alignment=bad, device="cpu")


def test_quantize_rows_needs_gpu():
    with pytest.raises(ValueError):
        quantize_rows(torch.zeros(3, 8), SparseType.INT8)


def test_bench_inputs_shapes():
    c2 = bench_inputs.config2(E=1000, B=64)
    assert c2.offsets.size == 8 * 64 + 1 and c2.indices.min() >= 0 and c2.indices.max() < 1000
    lengths = np.diff(c2.offsets)
    assert lengths.min() >= 1 and lengths.max() <= 40
    c4 = bench_inputs.config4(E=100, B=16)
    assert c4.tys == [2] * 16 + [3] * 16 and np.all(np.diff(c4.offsets) == 20)
    c5 = bench_inputs.config5(T=8, B=200, e_hi=1e5)
    assert c5.D == [32, 64, 128, 256] * 2 and (np.diff(c5.offsets) == 0).mean() > 0.05


def test_config2_batches_share_hot_rows():
    """Batch 0 is config2 itself; later batches draw afresh over the same
    per-table permutations, so each table's hottest row is the same row."""
    bs = bench_inputs.config2_batches(3, T=3, E=5000, B=300)
    c2 = bench_inputs.config2(T=3, E=5000, B=300)
    assert np.array_equal(bs[0].indices, c2.indices) and np.array_equal(bs[0].offsets, c2.offsets)
    assert not np.array_equal(bs[1].offsets, bs[2].offsets)
    for t in range(3):
        tops = {int(np.bincount(b.indices[b.offsets[t * 300]:b.offsets[(t + 1) * 300]],
                                minlength=5000).argmax()) for b in bs}
        assert len(tops) == 1


def test_inference_module_feature_table_map():
    specs = [("a", 10, 128, SparseType.INT8, EmbeddingLocation.DEVICE),
             ("b", 20, 64, SparseType.INT4, EmbeddingLocation.DEVICE)]
    m = IntNBitTableBatchedEmbeddingBagsCodegen(specs, [1, 0, 1], device="cpu")
    assert m.T == 3 and m.total_D == 256
    assert m.weights_offsets.tolist() == [1440, 0, 1440]
    assert m.weights_tys.tolist() == [3, 2, 3]
    assert m.D_offsets.tolist() == [0, 64, 192, 256]
    assert m.rows_per_table.tolist() == [20, 10, 20]
    assert m.weights_dev.numel() == 1440 + 960
    assert [tuple(x.shape) for x in m.split_embedding_weights()] == [(10, 144), (20, 48)]
