"""GPU parity of the rowwise quantization codecs: bit-exact against the C
oracle, which is itself pinned bit-exactly to torch's
quantized::embedding_bag_{byte,4bit,2bit}_prepack/unpack (FBGEMM's CPU codecs)
in test_oracle_pins.py; plus the TBE-layout packer feeding the nbit lookup."""

import numpy as np
import pytest
import torch

import oracle as orc

pytestmark = pytest.mark.gpu


def _rows(rng, n, D):
    x = (rng.standard_normal((n, D)) * rng.uniform(1e-3, 10, (n, 1))).astype(np.float32)
    x[0] = 0.25            # constant row
    x[1, :] = np.linspace(-1, 1, D)
    return x


@pytest.mark.parametrize("D", [1, 7, 16, 64, 128, 200])
def test_fused8bit_round_trip_bits(dev, D):
    print(f"[case] fused8bit D={D}", flush=True)
    x = _rows(np.random.default_rng(D), 300, D)
    q = torch.ops.fbgemm.FloatToFused8BitRowwiseQuantized(torch.from_numpy(x).to(dev))
    np.testing.assert_array_equal(q.cpu().numpy(), orc.quantize_fused8bit(x))
    d = torch.ops.fbgemm.Fused8BitRowwiseQuantizedToFloat(q)
    np.testing.assert_array_equal(d.cpu().numpy(), orc.dequantize_fused8bit(q.cpu().numpy()))
    h = torch.ops.fbgemm.Fused8BitRowwiseQuantizedToHalf(q)
    np.testing.assert_array_equal(h.cpu().numpy(), d.cpu().numpy().astype(np.float16))
    xh = torch.from_numpy(x).half()
    qh = torch.ops.fbgemm.HalfToFused8BitRowwiseQuantized(xh.to(dev))
    np.testing.assert_array_equal(qh.cpu().numpy(), orc.quantize_fused8bit(xh.float().numpy()))


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("D", [7, 8, 13, 16, 36, 128, 256])
def test_fused_nbit_round_trip_bits(dev, bits, D):
    """D not a multiple of the codes per byte (7, 13): the last byte is
    partly padding and the dequantized rows come back padded to whole bytes,
    as FBGEMM's fused N-bit format has it (torch's CPU prepack refuses such D,
    so there they are checked against the oracle only)."""
    print(f"[case] fused nbit bits={bits} D={D}", flush=True)
    x = _rows(np.random.default_rng(D * bits), 300, D)
    q = torch.ops.fbgemm.FloatToFusedNBitRowwiseQuantizedSBHalf(torch.from_numpy(x).to(dev), bits)
    np.testing.assert_array_equal(q.cpu().numpy(), orc.quantize_fused_nbit(x, bits))
    d = torch.ops.fbgemm.FusedNBitRowwiseQuantizedSBHalfToFloat(q, bits)
    d_out = (q.shape[1] - 4) * (8 // bits)
    assert d.shape[1] == d_out >= D
    np.testing.assert_array_equal(d.cpu().numpy(),
                                  orc.dequantize_fused_nbit(q.cpu().numpy(), bits, d_out))
    xh = torch.from_numpy(x).half()
    qh = torch.ops.fbgemm.HalfToFusedNBitRowwiseQuantizedSBHalf(xh.to(dev), bits)
    np.testing.assert_array_equal(qh.cpu().numpy(), orc.quantize_fused_nbit(xh.float().numpy(), bits))


@pytest.mark.parametrize("ebits,ebias", [(4, 7), (5, 15), (3, 3), (2, 1), (7, 0), (1, 0)])
def test_hfp8_codecs(dev, ebits, ebias):
    """fbgemm::HFP8QuantizedToFloat on all 256 codes and FloatToHFP8Quantized on
    the encoder probe values (ties, ulps around them, subnormal range, zeros,
    values past the clamp), bit-exact to the oracle (itself bit-exact to
    FBGEMM's Float8ToFloat_ref / FloatToFloat8_ref)."""
    from nbit_helpers import hfp8_probe_values

    print(f"[case] hfp8 codecs ebits={ebits} bias={ebias}", flush=True)
    codes = np.arange(256, dtype=np.uint8).reshape(16, 16)
    dec = torch.ops.fbgemm.HFP8QuantizedToFloat(torch.from_numpy(codes).to(dev), ebits, ebias)
    assert dec.dtype == torch.float32 and dec.shape == (16, 16)
    np.testing.assert_array_equal(dec.cpu().numpy().view(np.uint32),
                                  orc.hfp8_to_float(codes, ebits, ebias).view(np.uint32))
    x = hfp8_probe_values(np.random.default_rng(ebits * 31 + ebias), ebits, ebias)
    mx = orc.hfp8_max_pos(ebits, ebias)
    enc = torch.ops.fbgemm.FloatToHFP8Quantized(torch.from_numpy(x).to(dev), ebits, ebias, mx)
    assert enc.dtype == torch.uint8
    np.testing.assert_array_equal(enc.cpu().numpy(), orc.float_to_hfp8(x, ebits, ebias, mx))


@pytest.mark.parametrize("ty", ["INT8", "INT4", "INT2", "FP16", "FP8"])
def test_inference_module_assign_and_lookup(dev, ty):
    """quantize_rows' TBE layout decodes (through the nbit lookup) to the
    codec's own dequantization, and the module matches the oracle."""
    print(f"[case] inference module {ty}", flush=True)
    from mx_fbgemm import EmbeddingLocation, PoolingMode, SparseType
    from mx_fbgemm.split_table_batched_embeddings_ops_inference import (
        IntNBitTableBatchedEmbeddingBagsCodegen,
    )
    from tbe_helpers import random_tbe

    sty = SparseType[ty]
    E, D, B = 60, 32, 12
    m = IntNBitTableBatchedEmbeddingBagsCodegen(
        [("a", E, D, sty, EmbeddingLocation.DEVICE), ("b", E, 2 * D, sty, EmbeddingLocation.DEVICE)],
        pooling_mode=PoolingMode.SUM, output_dtype=SparseType.FP32, device=dev)
    rng = np.random.default_rng(7)
    ws = [torch.from_numpy(rng.uniform(-1, 1, (E, d)).astype(np.float32)) for d in (D, 2 * D)]
    m.assign_embedding_weights([w.to(dev) for w in ws])
    # one-row bags decode each row exactly once
    idx = np.tile(np.arange(E), 2).astype(np.int64)
    off = np.arange(2 * E + 1, dtype=np.int64)
    got = m(torch.from_numpy(idx).to(dev), torch.from_numpy(off).to(dev)).cpu().numpy()
    for t, w in enumerate(ws):
        d = w.shape[1]
        if sty == SparseType.FP16:
            exp = w.half().float().numpy()
        elif sty == SparseType.FP8:  # the module's default format, e4m3 with bias 7
            exp = orc.hfp8_to_float(orc.float_to_hfp8(w.numpy(), 4, 7, orc.hfp8_max_pos(4, 7)), 4, 7)
        else:
            q = orc.quantize_fused_nbit(w.numpy(), sty.bit_rate())
            exp = orc.dequantize_fused_nbit(q, sty.bit_rate(), d)
        cols = slice(0, D) if t == 0 else slice(D, 3 * D)
        np.testing.assert_allclose(got[:, cols], exp, rtol=1e-6, atol=1e-6)
    # pooled lookup vs the oracle on the packed buffer
    inp = random_tbe(rng, 2, B, [D, 2 * D], [E, E], 9)
    res = m(torch.from_numpy(inp.indices).to(dev), torch.from_numpy(inp.offsets).to(dev))
    buf = m.weights_dev.cpu().numpy()
    exp = orc.nbit_forward(buf, m.weights_offsets.cpu().numpy(), [sty.as_int()] * 2,
                           inp.D_offsets, B, inp.indices, inp.offsets, 0, out_f16=False)
    np.testing.assert_allclose(res.cpu().numpy(), exp, rtol=1e-5, atol=1e-5)


def test_inference_module_shared_tables(dev):
    """IntNBitTableBatchedEmbeddingBagsCodegen with feature_table_map [1, 0, 1]:
    the lookup equals the oracle's on the per-feature arrays."""
    print("[case] nbit module shared tables", flush=True)
    from mx_fbgemm import EmbeddingLocation, PoolingMode, SparseType
    from mx_fbgemm.split_table_batched_embeddings_ops_inference import (
        IntNBitTableBatchedEmbeddingBagsCodegen,
    )
    from tbe_helpers import random_tbe

    ftm = [1, 0, 1]
    m = IntNBitTableBatchedEmbeddingBagsCodegen(
        [("a", 40, 64, SparseType.INT8, EmbeddingLocation.DEVICE),
         ("b", 30, 32, SparseType.INT4, EmbeddingLocation.DEVICE)], ftm,
        pooling_mode=PoolingMode.MEAN, output_dtype=SparseType.FP32, device=dev)
    m.fill_random_weights(3)
    rng = np.random.default_rng(13)
    rows, dims = [40, 30], [64, 32]
    inp = random_tbe(rng, 3, 20, [dims[t] for t in ftm], [rows[t] for t in ftm], 9)
    got = m(torch.from_numpy(inp.indices).to(dev), torch.from_numpy(inp.offsets).to(dev))
    exp = orc.nbit_forward(m.weights_dev.cpu().numpy(), m.weights_offsets.cpu().numpy(),
                           m.weights_tys.cpu().numpy(), inp.D_offsets, inp.B, inp.indices,
                           inp.offsets, 1, out_f16=False)
    np.testing.assert_allclose(got.cpu().numpy(), exp, rtol=1e-2, atol=1e-3)
