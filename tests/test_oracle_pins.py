"""CPU pins of the oracle (no GPU): every oracle function is checked against
an independent in-container implementation, brute force or a closed form,
chosen so that a dropped term, a wrong index or a transposed operand fails.

* jagged: aten._jagged_to_padded_dense_forward / _padded_dense_to_jagged_forward
  (torch's port of the fbgemm jagged ops), bit-exact;
* TBE forward: FBGEMM's exported CPU SpMDM kernel (the CPU kernel fbgemm_gpu's
  CPU TBE op wraps), bit-exact; F.embedding_bag within fp32 rounding;
* nbit: FBGEMM's exported 8-bit / N-bit / fp16 / FP8 CPU kernels with the TBE
  row layout (scale_bias_last=false), fp16 output; the hfp8 decode and encode
  against FBGEMM's Float8ToFloat_ref / FloatToFloat8_ref;
* transpose: numpy stable argsort + unique (brute force), bit-exact;
* rowwise Adagrad: torch autograd of embedding_bag for the row gradient and
  the update rule evaluated with torch fp32 ops.
"""

import numpy as np
import pytest
import torch

import oracle as orc
from mx_fbgemm import bench_inputs
from nbit_helpers import build_weights, hfp8_probe_values
from tbe_helpers import random_tbe, weight_offsets


# ---- jagged -----------------------------------------------------------------

@pytest.mark.parametrize("lengths,max_L", [([3, 0, 5, 1], 4), ([0], 2), ([2, 2], 2),
                                           ([9, 1, 0, 4, 7], 6)])
def test_jagged_to_padded_dense_vs_aten(lengths, max_L):
    rng = np.random.default_rng(0)
    off = bench_inputs.offsets_from_lengths(np.array(lengths))
    vals = rng.standard_normal((int(off[-1]), 5)).astype(np.float32)
    exp = torch.ops.aten._jagged_to_padded_dense_forward(
        torch.from_numpy(vals), [torch.from_numpy(off)], [max_L], 1.25).numpy()
    got = orc.jagged_to_padded_dense(vals, [off], [max_L], 1.25)
    assert got.tobytes() == exp.tobytes()


@pytest.mark.parametrize("lengths,max_L", [([3, 0, 4, 1], 4), ([2, 2], 2), ([0, 0], 3)])
def test_dense_to_jagged_vs_aten(lengths, max_L):
    rng = np.random.default_rng(1)
    off = bench_inputs.offsets_from_lengths(np.array(lengths))
    dense = rng.standard_normal((len(lengths), max_L, 3)).astype(np.float32)
    exp = torch.ops.aten._padded_dense_to_jagged_forward(
        torch.from_numpy(dense), [torch.from_numpy(off)], int(off[-1])).numpy()
    got = orc.dense_to_jagged(dense, [off])
    assert got.tobytes() == exp.tobytes()


def test_dense_to_jagged_truncated_rows_are_zero():
    # A row longer than max_L: positions past max_L have no dense source -> 0
    # (torch/_inductor/jagged_lowerings.py:248).  aten raises here, so the pin
    # is the closed form.
    off = np.array([0, 5], np.int64)
    dense = np.arange(1 * 3 * 2, dtype=np.float32).reshape(1, 3, 2) + 1
    got = orc.dense_to_jagged(dense, [off])
    np.testing.assert_array_equal(got[:3], dense[0])
    np.testing.assert_array_equal(got[3:], 0)


def test_jagged_add_closed_form_and_rounding():
    off = np.array([0, 2, 5], np.int64)
    x = np.arange(10, dtype=np.float32).reshape(5, 2)
    y = np.full((2, 2, 2), 0.5, np.float32)
    got = orc.jagged_dense_elementwise_add(x, [off], y, "f32")
    exp = x.copy()
    exp[[0, 1, 2, 3]] += 0.5  # row 4 (j=2 of bag 1) lies past max_L=2 -> x + 0
    np.testing.assert_array_equal(got, exp)
    # f16: computed in fp32 then rounded once (2049 + 1 = 2050 exactly; 2048+1 ties to even)
    xh = np.array([[2048.0]], np.float16)
    yh = np.array([[[1.0]]], np.float16)
    r = orc.jagged_dense_elementwise_add(xh, [np.array([0, 1])], yh, "f16")
    assert r[0, 0] == np.float16(2048.0)
    # bf16 round-to-nearest-even of 1 + 2^-8 (a tie) stays 1.0
    xb = np.array([[0x3F80]], np.uint16)
    yb = np.array([[[0x3B80]]], np.uint16)  # 2^-8
    rb = orc.jagged_dense_elementwise_add(xb, [np.array([0, 1])], yb, "bf16")
    assert rb[0, 0] == 0x3F80


def test_two_level_index_map_brute_force():
    off0 = np.array([0, 2, 2, 5])
    off1 = np.array([0, 1, 5, 5, 7, 10])
    m = orc.dense_index_map([off0, off1], [2, 3])
    for b in range(3):
        for j0 in range(2):
            for j1 in range(3):
                exp = -1
                if j0 < off0[b + 1] - off0[b]:
                    r = off0[b] + j0
                    if j1 < off1[r + 1] - off1[r]:
                        exp = off1[r] + j1
                assert m[b, j0, j1] == exp


# ---- TBE forward ------------------------------------------------------------

def _tbe_case(seed, T=3, B=20, dims=(8, 128, 36), rows=(50, 70, 9), max_L=12):
    rng = np.random.default_rng(seed)
    inp = random_tbe(rng, T, B, list(dims), list(rows), max_L)
    W = rng.uniform(-1, 1, size=sum(E * D for E, D in zip(rows, dims))).astype(np.float32)
    return inp, W


@pytest.mark.parametrize("pooling", [0, 1])
@pytest.mark.parametrize("weighted", [False, True])
def test_tbe_forward_vs_fbgemm_cpu(pooling, weighted):
    inp, W = _tbe_case(3)
    iw = np.random.default_rng(4).uniform(0, 2, inp.N).astype(np.float32) if weighted else None
    got = orc.tbe_forward_f32(W, weight_offsets(inp), inp.D_offsets, inp.B, inp.indices,
                              inp.offsets, pooling, iw)
    exp = orc.fbgemm_tbe_forward_f32(W, weight_offsets(inp), inp.D_offsets, inp.E, inp.B,
                                     inp.indices, inp.offsets, pooling, iw, nthreads=2)
    np.testing.assert_array_equal(got, exp)  # bit-exact


@pytest.mark.parametrize("pooling", [0, 1])
@pytest.mark.parametrize("weighted", [False, True])
def test_tbe_forward_fp16_weights_vs_fbgemm_cpu(pooling, weighted):
    """fp16 weight rows: the oracle widens each weight to fp32 and sums in
    index order; FBGEMM's fp16-input SpMDM kernel (fp32 output) must agree
    bit for bit."""
    inp, W = _tbe_case(7)
    W16 = W.astype(np.float16)
    iw = np.random.default_rng(8).uniform(0, 2, inp.N).astype(np.float32) if weighted else None
    got = orc.tbe_forward_f32(W16, weight_offsets(inp), inp.D_offsets, inp.B, inp.indices,
                              inp.offsets, pooling, iw)
    exp = orc.fbgemm_tbe_forward_f32(W16, weight_offsets(inp), inp.D_offsets, inp.E, inp.B,
                                     inp.indices, inp.offsets, pooling, iw, nthreads=2)
    np.testing.assert_array_equal(got, exp)


@pytest.mark.parametrize("pooling", [0, 1])
def test_tbe_forward_vs_embedding_bag(pooling):
    inp, W = _tbe_case(5)
    got = orc.tbe_forward_f32(W, weight_offsets(inp), inp.D_offsets, inp.B, inp.indices,
                              inp.offsets, pooling)
    w_off = weight_offsets(inp)
    for t in range(inp.T):
        Wt = torch.from_numpy(W[w_off[t]: w_off[t] + inp.E[t] * inp.D[t]].reshape(inp.E[t], -1))
        o = inp.offsets[t * inp.B:(t + 1) * inp.B + 1]
        ref = torch.nn.functional.embedding_bag(
            torch.from_numpy(inp.indices[o[0]:o[-1]]), Wt, torch.from_numpy(o[:-1] - o[0]),
            mode="sum" if pooling == 0 else "mean")
        d0, d1 = inp.D_offsets[t], inp.D_offsets[t + 1]
        np.testing.assert_allclose(got[:, d0:d1], ref.numpy(), rtol=1e-5, atol=1e-6)


def test_tbe_forward_closed_form():
    # Two tables, bag sums written by hand.
    W = np.arange(2 * 4 + 3 * 4, dtype=np.float32)
    w_off = np.array([0, 8], np.int64)
    D_off = np.array([0, 4, 8], np.int32)
    idx = np.array([1, 1, 0, 2, 0], np.int64)
    off = np.array([0, 2, 3, 5], np.int64)  # T=2? -> 3 bags: needs T*B+1; use B=1? see below
    # T=2, B=1 would need 3 offsets; use bags (t0,b0)=[1,1], (t1,b0)=[0]  and check
    off = np.array([0, 2, 3], np.int64)
    out = orc.tbe_forward_f32(W, w_off, D_off, 1, idx[:3], off, 0)
    np.testing.assert_array_equal(out[0, :4], 2 * W[4:8])
    np.testing.assert_array_equal(out[0, 4:], W[8:12])
    out = orc.tbe_forward_f32(W, w_off, D_off, 1, idx[:3], off, 1)
    np.testing.assert_array_equal(out[0, :4], W[4:8])  # mean of a repeated row


# ---- nbit -------------------------------------------------------------------

@pytest.mark.parametrize("ty", [orc.INT8, orc.INT4, orc.INT2, orc.FP16, orc.FP32])
@pytest.mark.parametrize("pooling", [0, 1])
def test_nbit_vs_fbgemm_cpu(ty, pooling):
    rng = np.random.default_rng(ty * 10 + pooling)
    dims = [32, 64]
    rows = [40, 70]
    inp = random_tbe(rng, 2, 15, dims, rows, 20)
    buf, w_off = build_weights(rng, [ty, ty], dims, rows)
    got = orc.nbit_forward(buf, w_off, [ty, ty], inp.D_offsets, inp.B, inp.indices, inp.offsets,
                           pooling)
    exp = orc.fbgemm_nbit_forward(buf, w_off, [ty, ty], inp.D_offsets, rows, inp.B, inp.indices,
                                  inp.offsets, pooling, nthreads=2)
    # Same terms, same order, same fp32 fma steps: bit-exact fp16 output.
    np.testing.assert_array_equal(got.view(np.uint16), exp.view(np.uint16))


HFP8_CONFIGS = [(4, 7), (5, 15), (3, 3), (4, 8), (2, 1), (5, 20)]  # (exponent bits, bias)


@pytest.mark.parametrize("ebits,ebias", HFP8_CONFIGS)
def test_hfp8_decode_vs_fbgemm(ebits, ebias):
    """Every one of the 256 codes decodes to FBGEMM's Float8ToFloat_ref value, bit for bit."""
    codes = np.arange(256, dtype=np.uint8)
    got = orc.hfp8_to_float(codes, ebits, ebias)
    exp = orc.fbgemm_hfp8_to_float(codes, ebits, ebias)
    np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))


@pytest.mark.parametrize("ebits,ebias", HFP8_CONFIGS)
def test_hfp8_encode_vs_fbgemm(ebits, ebias):
    """The encoder gives FBGEMM's FloatToFloat8_ref code on every code's value,
    on the midpoints between neighbouring codes (ties to even) and one fp32
    ulp either side of them, on normal and log-uniform samples from 1e-12 to
    past the largest code, on subnormal-range values, signed zeros and values
    past the clamp."""
    rng = np.random.default_rng(ebits * 100 + ebias)
    x = hfp8_probe_values(rng, ebits, ebias)
    np.testing.assert_array_equal(orc.float_to_hfp8(x, ebits, ebias, orc.hfp8_max_pos(ebits, ebias)),
                                  orc.fbgemm_float_to_hfp8(x, ebits, ebias))


@pytest.mark.parametrize("ebits,ebias", [(4, 7), (5, 15)])
@pytest.mark.parametrize("pooling", [0, 1])
@pytest.mark.parametrize("weighted", [False, True])
def test_nbit_fp8_vs_fbgemm_cpu(ebits, ebias, pooling, weighted):
    """FP8 tables: FBGEMM's GenerateEmbeddingSpMDMFP8WithStrides, bit-exact fp16 output."""
    rng = np.random.default_rng(ebits + 10 * pooling + 100 * weighted)
    dims, rows = [32, 64], [40, 70]
    inp = random_tbe(rng, 2, 15, dims, rows, 20)
    buf, w_off = build_weights(rng, [orc.FP8] * 2, dims, rows, fp8_exponent_bits=ebits,
                               fp8_exponent_bias=ebias)
    iw = rng.uniform(-1, 1, inp.N).astype(np.float32) if weighted else None
    got = orc.nbit_forward(buf, w_off, [orc.FP8] * 2, inp.D_offsets, inp.B, inp.indices,
                           inp.offsets, pooling, indice_weights=iw, fp8_exponent_bits=ebits,
                           fp8_exponent_bias=ebias)
    exp = orc.fbgemm_nbit_forward(buf, w_off, [orc.FP8] * 2, inp.D_offsets, rows, inp.B,
                                  inp.indices, inp.offsets, pooling, indice_weights=iw,
                                  nthreads=2, fp8_exponent_bits=ebits, fp8_exponent_bias=ebias)
    np.testing.assert_array_equal(got.view(np.uint16), exp.view(np.uint16))


@pytest.mark.parametrize("ty", [orc.INT8, orc.INT4, orc.INT2, orc.FP16, orc.FP32, orc.FP8])
@pytest.mark.parametrize("pooling", [0, 1])
@pytest.mark.parametrize("weighted", [False, True])
def test_nbit_bf16_out_vs_fbgemm_cpu(ty, pooling, weighted):
    """bf16 output (FBGEMM's is_bf16_out), bit-exact.  Weights in steps of 1/4
    keep many sums exactly halfway between two bf16 values, where FBGEMM
    rounds away from zero: the oracle must follow it on every tie."""
    rng = np.random.default_rng(ty * 7 + 3 * weighted + pooling)
    dims, rows = [32, 64], [40, 70]
    inp = random_tbe(rng, 2, 40, dims, rows, 20)
    buf, w_off = build_weights(rng, [ty] * 2, dims, rows)
    iw = (rng.integers(-4, 5, inp.N) / 4).astype(np.float32) if weighted else None
    got = orc.nbit_forward(buf, w_off, [ty] * 2, inp.D_offsets, inp.B, inp.indices,
                           inp.offsets, pooling, indice_weights=iw, out_bf16=True)
    exp = orc.fbgemm_nbit_forward(buf, w_off, [ty] * 2, inp.D_offsets, rows, inp.B,
                                  inp.indices, inp.offsets, pooling, indice_weights=iw,
                                  nthreads=2, out_bf16=True)
    np.testing.assert_array_equal(got, exp)


def test_nbit_int8_vs_quantized_embedding_bag_byte():
    # torch's byte rowwise op keeps fp32 scale/bias at the row end; move ours there.
    rng = np.random.default_rng(12)
    E, D, B = 60, 16, 9
    inp = random_tbe(rng, 1, B, [D], [E], 7)
    buf, w_off = build_weights(rng, [orc.INT8], [D], [E])
    stride = orc.nbit_row_bytes(orc.INT8, D, 16)
    tab = buf.reshape(E, stride)
    sc = tab[:, 0:2].copy().view(np.float16).astype(np.float32)
    bi = tab[:, 2:4].copy().view(np.float16).astype(np.float32)
    packed = np.concatenate([tab[:, 4:4 + D], sc.view(np.uint8).reshape(E, 4),
                             bi.view(np.uint8).reshape(E, 4)], axis=1)
    ref = torch.ops.quantized.embedding_bag_byte_rowwise_offsets(
        torch.from_numpy(packed), torch.from_numpy(inp.indices), torch.from_numpy(inp.offsets),
        False, 0, False, None, None, True).numpy()
    got = orc.nbit_forward(buf, w_off, [orc.INT8], inp.D_offsets, B, inp.indices, inp.offsets, 0,
                           out_f16=False)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_fp16_conversion_matches_numpy():
    lib = orc.lib()
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000),
                         np.array([65504, 65519.99, 65520, 6e-8, 3e-8, 2.98e-8, -0.0, np.inf,
                                   -np.inf, 5.96e-8], np.float32)]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = xs.astype(np.float16).view(np.uint16)
    got = np.array([lib.orc_float_to_half(float(x)) for x in xs], np.uint16)
    np.testing.assert_array_equal(got, ref)
    h = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    back = np.array([lib.orc_half_to_float(int(v)) for v in h[::7]], np.float32)
    hv = h[::7].view(np.float16).astype(np.float32)
    finite = np.isfinite(hv)
    np.testing.assert_array_equal(back[finite], hv[finite])


# ---- transpose + backward ---------------------------------------------------

@pytest.mark.parametrize("seed,T,B,rows,dup", [(0, 3, 40, [10, 1000, 7], False),
                                                (1, 2, 100, [4, 4], True),
                                                (2, 1, 1, [1], False)])
def test_transpose_vs_numpy(seed, T, B, rows, dup):
    rng = np.random.default_rng(seed)
    inp = random_tbe(rng, T, B, [4] * T, rows, 15, dup_heavy=dup)
    nb = orc.info_B_num_bits(T, B)
    got = orc.transpose_embedding_input(inp.hash_size_cumsum, B, nb, inp.total_hash_size_bits,
                                        inp.indices, inp.offsets)
    bag = np.repeat(np.arange(T * B), np.diff(inp.offsets))
    t, b = bag // B, bag % B
    lin = inp.hash_size_cumsum[t] + inp.indices
    info = (t.astype(np.int64) << nb) | b
    order = np.argsort(lin, kind="stable")
    np.testing.assert_array_equal(got["linear_indices"], lin)
    np.testing.assert_array_equal(got["sorted_linear_indices"], lin[order])
    np.testing.assert_array_equal(got["infos_sorted"].astype(np.int64) & 0xFFFFFFFF, info[order])
    u, first, counts = np.unique(lin[order], return_index=True, return_counts=True)
    np.testing.assert_array_equal(got["run"], u)
    np.testing.assert_array_equal(got["run_lengths"], counts)
    np.testing.assert_array_equal(got["cumulative_run_lengths"], np.append(first, lin.size))
    assert got["run_lengths"].sum() == inp.N


def _torch_bag(Wt, idx, starts, pooling, psw):
    """torch autograd graph of one table's pooled lookup.  Weighted MEAN is
    written as SUM with per-sample weights psw / L (torch's embedding_bag takes
    per-sample weights under mode='sum' only), which has the same value and
    derivatives as (sum_l psw_l W[i_l]) / L."""
    if psw is None:
        return torch.nn.functional.embedding_bag(idx, Wt, starts,
                                                 mode="sum" if pooling == 0 else "mean")
    if pooling == 1:
        lens = torch.diff(torch.cat([starts, torch.tensor([idx.numel()])]))
        psw = psw / torch.repeat_interleave(lens.to(psw.dtype), lens)
    return torch.nn.functional.embedding_bag(idx, Wt, starts, mode="sum", per_sample_weights=psw)


@pytest.mark.parametrize("pooling", [0, 1])
@pytest.mark.parametrize("wd_mode,wd", [(0, 0.0), (1, 0.1), (2, 0.05)])
@pytest.mark.parametrize("weighted", [False, True])
def test_adagrad_vs_torch_autograd(pooling, wd_mode, wd, weighted):
    rng = np.random.default_rng(21)
    dims, rows = [8, 16], [30, 20]
    inp = random_tbe(rng, 2, 12, dims, rows, 9, empty_frac=0.1)
    W = rng.uniform(-0.5, 0.5, size=sum(E * D for E, D in zip(rows, dims))).astype(np.float32)
    m1 = rng.uniform(0, 0.01, size=sum(rows)).astype(np.float32)
    m1_off = np.array([0, rows[0]], np.int64)
    grad = rng.normal(0, 1, size=(inp.B, inp.total_D)).astype(np.float32)
    iw = rng.uniform(-1.5, 1.5, inp.N).astype(np.float32) if weighted else None
    lr, eps = 0.1, 1e-6
    W_new, m_new = orc.backward_rowwise_adagrad(
        W, weight_offsets(inp), inp.D_offsets, inp.B, inp.hash_size_cumsum,
        inp.total_hash_size_bits, inp.indices, inp.offsets, pooling, grad, m1, m1_off, lr, eps,
        wd, wd_mode, orc.info_B_num_bits(2, inp.B), indice_weights=iw)
    w_off = weight_offsets(inp)
    for t in range(2):
        E, D = rows[t], dims[t]
        Wt = torch.tensor(W[w_off[t]: w_off[t] + E * D].reshape(E, D), requires_grad=True)
        o = inp.offsets[t * inp.B:(t + 1) * inp.B + 1]
        psw = None if iw is None else torch.from_numpy(iw[o[0]:o[-1]])
        out = _torch_bag(Wt, torch.from_numpy(inp.indices[o[0]:o[-1]]),
                         torch.from_numpy(o[:-1] - o[0]), pooling, psw)
        d0, d1 = inp.D_offsets[t], inp.D_offsets[t + 1]
        (out * torch.from_numpy(grad[:, d0:d1])).sum().backward()
        g = Wt.grad.detach()
        w = Wt.detach()
        touched = torch.from_numpy(np.isin(np.arange(E), inp.indices[o[0]:o[-1]]))
        s = g + wd * w if wd_mode == 1 else g
        h = torch.from_numpy(m1[m1_off[t]: m1_off[t] + E]) + (s * s).sum(1) / D
        m = lr / (h.sqrt() + eps)
        c = torch.ones_like(m)
        if wd_mode == 1:
            c = 1 - m * wd
        elif wd_mode == 2:
            c = torch.full_like(m, 1 - lr * wd)
        w_ref = torch.where(touched[:, None], c[:, None] * w - m[:, None] * g, w)
        h_ref = torch.where(touched, h, torch.from_numpy(m1[m1_off[t]: m1_off[t] + E]))
        np.testing.assert_allclose(W_new[w_off[t]: w_off[t] + E * D].reshape(E, D), w_ref.numpy(),
                                   rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(m_new[m1_off[t]: m1_off[t] + E], h_ref.numpy(), rtol=1e-5,
                                   atol=1e-7)


@pytest.mark.parametrize("pooling", [0, 1])
@pytest.mark.parametrize("weighted", [False, True])
def test_adagrad_shared_tables_vs_torch_autograd(pooling, weighted):
    """Features sharing a table (fbgemm's feature_table_map = [0, 1, 0]): the
    per-feature arrays point features 0 and 2 at table 0's rows, hash offset
    and momentum, so a row looked up by both is one run whose gradient sums
    each occurrence's slice from its own feature's columns."""
    rng = np.random.default_rng(31 + pooling + 2 * weighted)
    ftm, rows, dims = [0, 1, 0], [30, 20], [16, 8]
    fr, fd = [rows[t] for t in ftm], [dims[t] for t in ftm]
    inp = random_tbe(rng, 3, 10, fd, fr, 7, empty_frac=0.1)
    t_off = np.array([0, rows[0] * dims[0]], np.int64)
    t_hsc = np.array([0, rows[0]], np.int64)
    w_off = t_off[ftm]
    hsc = np.concatenate([t_hsc[ftm], [sum(rows)]]).astype(np.int64)
    m1_off = t_hsc[ftm]
    W = rng.uniform(-0.5, 0.5, size=sum(E * D for E, D in zip(rows, dims))).astype(np.float32)
    m1 = rng.uniform(0, 0.01, size=sum(rows)).astype(np.float32)
    grad = rng.normal(0, 1, size=(inp.B, inp.total_D)).astype(np.float32)
    iw = rng.uniform(-1.5, 1.5, inp.N).astype(np.float32) if weighted else None
    lr, eps = 0.1, 1e-6
    W_new, m_new = orc.backward_rowwise_adagrad(
        W, w_off, inp.D_offsets, inp.B, hsc, 6, inp.indices, inp.offsets, pooling, grad, m1,
        m1_off, lr, eps, 0.0, 0, orc.info_B_num_bits(3, inp.B), indice_weights=iw)
    Wt = [torch.tensor(W[t_off[t]: t_off[t] + rows[t] * dims[t]].reshape(rows[t], dims[t]),
                       requires_grad=True) for t in range(2)]
    loss = 0
    for f, t in enumerate(ftm):
        o = inp.offsets[f * inp.B:(f + 1) * inp.B + 1]
        psw = None if iw is None else torch.from_numpy(iw[o[0]:o[-1]])
        out = _torch_bag(Wt[t], torch.from_numpy(inp.indices[o[0]:o[-1]]),
                         torch.from_numpy(o[:-1] - o[0]), pooling, psw)
        d0, d1 = inp.D_offsets[f], inp.D_offsets[f + 1]
        loss = loss + (out * torch.from_numpy(grad[:, d0:d1])).sum()
    loss.backward()
    for t in range(2):
        E, D = rows[t], dims[t]
        g, w = Wt[t].grad.detach(), Wt[t].detach()
        seen = np.concatenate([inp.indices[inp.offsets[f * inp.B]: inp.offsets[(f + 1) * inp.B]]
                               for f in range(3) if ftm[f] == t])
        touched = torch.from_numpy(np.isin(np.arange(E), seen))
        h0 = torch.from_numpy(m1[t_hsc[t]: t_hsc[t] + E])
        h = h0 + (g * g).sum(1) / D
        m = lr / (h.sqrt() + eps)
        w_ref = torch.where(touched[:, None], w - m[:, None] * g, w)
        np.testing.assert_allclose(W_new[t_off[t]: t_off[t] + E * D].reshape(E, D), w_ref.numpy(),
                                   rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(m_new[t_hsc[t]: t_hsc[t] + E],
                                   torch.where(touched, h, h0).numpy(), rtol=1e-5, atol=1e-7)


def test_adagrad_zero_grad_changes_nothing():
    rng = np.random.default_rng(2)
    inp = random_tbe(rng, 1, 10, [8], [20], 5)
    W = rng.uniform(-1, 1, 160).astype(np.float32)
    m1 = rng.uniform(0.1, 1, 20).astype(np.float32)
    W2, m2 = orc.backward_rowwise_adagrad(W, np.array([0]), inp.D_offsets, 10,
                                          inp.hash_size_cumsum, inp.total_hash_size_bits,
                                          inp.indices, inp.offsets, 0,
                                          np.zeros((10, 8), np.float32), m1, np.array([0]), 0.1,
                                          1e-8)
    np.testing.assert_array_equal(W2, W)
    np.testing.assert_array_equal(m2, m1)


@pytest.mark.parametrize("pooling", [0, 1])
def test_grad_indice_weights_vs_torch_autograd(pooling):
    rng = np.random.default_rng(23)
    dims, rows = [8, 36, 128], [40, 25, 30]
    inp = random_tbe(rng, 3, 10, dims, rows, 11, empty_frac=0.1)
    W = rng.uniform(-0.5, 0.5, size=sum(E * D for E, D in zip(rows, dims))).astype(np.float32)
    grad = rng.normal(0, 1, size=(inp.B, inp.total_D)).astype(np.float32)
    iw = rng.uniform(0.2, 2.0, inp.N).astype(np.float32)
    w_off = weight_offsets(inp)
    frg = np.array([1, 0, 1], np.int32)
    got = orc.grad_indice_weights(grad, W, w_off, inp.D_offsets, inp.B, inp.indices,
                                  inp.offsets, pooling, frg)
    all_on = orc.grad_indice_weights(grad, W, w_off, inp.D_offsets, inp.B, inp.indices,
                                     inp.offsets, pooling)
    for t in range(3):
        E, D = rows[t], dims[t]
        Wt = torch.tensor(W[w_off[t]: w_off[t] + E * D].reshape(E, D))
        o = inp.offsets[t * inp.B:(t + 1) * inp.B + 1]
        psw = torch.tensor(iw[o[0]:o[-1]], requires_grad=True)
        out = _torch_bag(Wt, torch.from_numpy(inp.indices[o[0]:o[-1]]),
                         torch.from_numpy(o[:-1] - o[0]), pooling, psw)
        d0, d1 = inp.D_offsets[t], inp.D_offsets[t + 1]
        (out * torch.from_numpy(grad[:, d0:d1])).sum().backward()
        np.testing.assert_allclose(all_on[o[0]:o[-1]], psw.grad.numpy(), rtol=1e-5, atol=1e-5)
        if frg[t]:
            np.testing.assert_array_equal(got[o[0]:o[-1]], all_on[o[0]:o[-1]])
        else:
            assert not got[o[0]:o[-1]].any()


# ---- bounds_check_indices ---------------------------------------------------

def _bounds_brute(rows, idx, off, mode):
    """Straight restatement with Python ints (independent of the C loops)."""
    idx, off = [int(x) for x in idx], [int(x) for x in off]
    T = len(rows)
    B = (len(off) - 1) // T
    N = len(idx)
    if mode == 3:
        return idx, off, 0
    rep, run = [], 0
    for o in off:
        run = max(run, min(max(o, 0), N))
        rep.append(run)
    bad = 0
    out_idx = list(idx)
    for bag in range(T * B):
        for l in range(rep[bag], rep[bag + 1]):
            if not (0 <= idx[l] < rows[bag // B]):
                bad += 1
                if mode != 0:
                    out_idx[l] = 0
    bad += sum(1 for a, b in zip(rep, off) if a != b)
    return (out_idx if mode != 0 else idx), (rep if mode != 0 else off), bad


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
@pytest.mark.parametrize("case", ["clean", "bad_indices", "bad_offsets"])
def test_bounds_check_vs_python(mode, case):
    rng = np.random.default_rng(5)
    T, B = 3, 7
    rows = np.array([10, 3, 50])
    lengths = rng.integers(0, 6, T * B)
    off = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    N = int(off[-1])
    idx = np.concatenate([rng.integers(0, rows[t], int(off[(t + 1) * B] - off[t * B]))
                          for t in range(T)]).astype(np.int64)
    if case == "bad_indices":
        idx[::5] = rng.integers(-3, 60, idx[::5].size)
    if case == "bad_offsets":
        off[4] = -2
        off[9] = N + 5  # also makes offsets non-monotone
    got_idx, got_off, n = orc.bounds_check_indices(rows, idx, off, mode)
    exp_idx, exp_off, bad = _bounds_brute(rows, idx, off, mode)
    assert n == bad
    np.testing.assert_array_equal(got_idx, exp_idx)
    np.testing.assert_array_equal(got_off, exp_off)
    if case == "clean":
        assert n == 0
    if mode in (1, 2):  # repaired arrays are safe to look up
        assert np.all(np.diff(got_off) >= 0) and got_off[0] >= 0 and got_off[-1] <= N
        for bag in range(T * B):
            seg = got_idx[got_off[bag]:got_off[bag + 1]]
            assert np.all((seg >= 0) & (seg < rows[bag // B]))


# ---- rowwise quantization codecs -------------------------------------------

@pytest.mark.parametrize("D", [1, 7, 16, 36, 128])
def test_codecs_vs_torch_quantized_prepack(D):
    rng = np.random.default_rng(D)
    x = (rng.standard_normal((100, D)) * rng.uniform(1e-3, 10, (100, 1))).astype(np.float32)
    x[0] = 0.5
    xt = torch.from_numpy(x)
    q8 = orc.quantize_fused8bit(x)
    np.testing.assert_array_equal(q8, torch.ops.quantized.embedding_bag_byte_prepack(xt).numpy())
    np.testing.assert_array_equal(
        orc.dequantize_fused8bit(q8),
        torch.ops.quantized.embedding_bag_byte_unpack(torch.from_numpy(q8)).numpy())
    for bits, pack, unpack in ((4, torch.ops.quantized.embedding_bag_4bit_prepack,
                                torch.ops.quantized.embedding_bag_4bit_unpack),
                               (2, torch.ops.quantized.embedding_bag_2bit_prepack,
                                torch.ops.quantized.embedding_bag_2bit_unpack)):
        if D % (8 // bits):
            continue
        q = orc.quantize_fused_nbit(x, bits)
        np.testing.assert_array_equal(q, pack(xt).numpy())
        np.testing.assert_array_equal(orc.dequantize_fused_nbit(q, bits, D),
                                      unpack(torch.from_numpy(q)).numpy())


# ---- sequence lookups (PoolingMode NONE) --------------------------------------

def _nobag_case(seed, T=3, B=14, D=16, rows=(40, 9, 70), max_L=7):
    rng = np.random.default_rng(seed)
    inp = random_tbe(rng, T, B, [D] * T, list(rows), max_L, empty_frac=0.2)
    return rng, inp


@pytest.mark.parametrize("wdtype", [np.float32, np.float16])
def test_tbe_forward_nobag_vs_embedding(wdtype):
    """out[l] = F.embedding(indices of table t, W_t)[l], bit for bit (fp16 rows widened)."""
    rng, inp = _nobag_case(5)
    D = 16
    W = rng.uniform(-1, 1, size=sum(E * D for E in (40, 9, 70))).astype(wdtype)
    w_off = weight_offsets(inp)
    got = orc.tbe_forward_nobag(W, w_off, D, inp.B, inp.indices, inp.offsets)
    for t, E in enumerate((40, 9, 70)):
        o0, o1 = inp.offsets[t * inp.B], inp.offsets[(t + 1) * inp.B]
        Wt = torch.from_numpy(W[w_off[t]: w_off[t] + E * D].reshape(E, D))
        ref = torch.nn.functional.embedding(torch.from_numpy(inp.indices[o0:o1]), Wt).float()
        np.testing.assert_array_equal(got[o0:o1], ref.numpy())


def _bf16_bits_to_f32(u16):
    return (np.asarray(u16, np.uint32) << 16).view(np.float32)


def _nbit_rows_f32(buf, w_off, ty, D, idx):
    """Closed form of dequantized rows in fp32: fma(scale, q, bias) is the
    float64 value of scale*q + bias rounded once to fp32 (both exact in
    float64 for fp16 qparams and codes below 256); other types as stored."""
    stride = orc.nbit_row_bytes(ty, D, 16)
    rows = np.stack([buf[w_off + i * stride: w_off + (i + 1) * stride] for i in idx])
    if ty in (orc.INT8, orc.INT4, orc.INT2):
        bits = {orc.INT8: 8, orc.INT4: 4, orc.INT2: 2}[ty]
        sc = rows[:, 0:2].copy().view(np.float16).astype(np.float64)
        bi = rows[:, 2:4].copy().view(np.float16).astype(np.float64)
        codes = rows[:, 4:]
        per = 8 // bits
        q = np.stack([(codes[:, d // per] >> ((d % per) * bits)) & ((1 << bits) - 1)
                      for d in range(D)], axis=1).astype(np.float64)
        return (sc * q + bi).astype(np.float32)
    if ty == orc.FP16:
        return rows[:, :2 * D].copy().view(np.float16).astype(np.float32)
    if ty == orc.FP8:
        return orc.hfp8_to_float(rows[:, :D], 4, 7)
    return rows[:, :4 * D].copy().view(np.float32)


@pytest.mark.parametrize("ty", [orc.INT8, orc.INT4, orc.INT2, orc.FP16, orc.FP32, orc.FP8])
@pytest.mark.parametrize("out_kind", [0, 1, 2])
def test_nbit_nobag_vs_fbgemm_cpu(ty, out_kind):
    """fp16 / bf16 out: each position's row equals FBGEMM's CPU kernel on a bag
    holding that row alone (a table's positions as bags of length one), as
    values (FBGEMM's first row adds to +0.0, so a stored -0.0 is +0.0 there
    and -0.0 here).  fp32 out: the closed form, bit for bit."""
    rng, inp = _nobag_case(ty * 3 + out_kind, D=32)
    D, rows = 32, [40, 9, 70]
    tys = [ty] * 3
    buf, w_off = build_weights(rng, tys, [D] * 3, rows)
    got = orc.nbit_forward_nobag(buf, w_off, tys, D, inp.B, inp.indices, inp.offsets,
                                 out_kind=out_kind)
    for t in range(3):
        o0, o1 = int(inp.offsets[t * inp.B]), int(inp.offsets[(t + 1) * inp.B])
        n = o1 - o0
        if n == 0:
            continue
        g = got[o0:o1]
        if out_kind == 0:
            exp = _nbit_rows_f32(buf, int(w_off[t]), ty, D, inp.indices[o0:o1])
            np.testing.assert_array_equal(g.view(np.uint32), exp.view(np.uint32))
            continue
        exp = orc.fbgemm_nbit_forward(buf, np.array([w_off[t]]), [ty], np.array([0, D], np.int32),
                                      [rows[t]], n, inp.indices[o0:o1],
                                      np.arange(n + 1, dtype=np.int64), 0, nthreads=1,
                                      out_bf16=out_kind == 2)
        if out_kind == 2:
            np.testing.assert_array_equal(_bf16_bits_to_f32(g), _bf16_bits_to_f32(exp))
        else:
            np.testing.assert_array_equal(g.astype(np.float32), exp.astype(np.float32))


@pytest.mark.parametrize("wd_mode,wd", [(0, 0.0), (1, 0.1), (2, 0.05)])
def test_adagrad_nobag_vs_torch_autograd(wd_mode, wd):
    """The nobag row gradient is torch autograd of F.embedding (the sum of the
    positions' gradient rows per row), then the rule in torch fp32."""
    rng, inp = _nobag_case(77, D=8, rows=(30, 6, 25))
    D, rows = 8, (30, 6, 25)
    W = rng.uniform(-0.5, 0.5, size=sum(E * D for E in rows)).astype(np.float32)
    m1 = rng.uniform(0, 0.01, size=sum(rows)).astype(np.float32)
    m1_off = np.array([0, rows[0], rows[0] + rows[1]], np.int64)
    grad = rng.normal(0, 1, size=(inp.N, D)).astype(np.float32)
    lr, eps = 0.1, 1e-6
    w_off = weight_offsets(inp)
    W_new, m_new = orc.backward_rowwise_adagrad_nobag(
        W, w_off, D, inp.B, inp.hash_size_cumsum, inp.total_hash_size_bits, inp.indices,
        inp.offsets, grad, m1, m1_off, lr, eps, wd, wd_mode)
    for t, E in enumerate(rows):
        o0, o1 = inp.offsets[t * inp.B], inp.offsets[(t + 1) * inp.B]
        Wt = torch.tensor(W[w_off[t]: w_off[t] + E * D].reshape(E, D), requires_grad=True)
        out = torch.nn.functional.embedding(torch.from_numpy(inp.indices[o0:o1]), Wt)
        (out * torch.from_numpy(grad[o0:o1])).sum().backward()
        g, w = Wt.grad.detach(), Wt.detach()
        touched = torch.from_numpy(np.isin(np.arange(E), inp.indices[o0:o1]))
        s = g + wd * w if wd_mode == 1 else g
        h0 = torch.from_numpy(m1[m1_off[t]: m1_off[t] + E])
        h = h0 + (s * s).sum(1) / D
        m = lr / (h.sqrt() + eps)
        c = 1 - m * wd if wd_mode == 1 else torch.full_like(m, 1 - lr * wd if wd_mode == 2 else 1)
        w_ref = torch.where(touched[:, None], c[:, None] * w - m[:, None] * g, w)
        np.testing.assert_allclose(W_new[w_off[t]: w_off[t] + E * D].reshape(E, D), w_ref.numpy(),
                                   rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(m_new[m1_off[t]: m1_off[t] + E],
                                   torch.where(touched, h, h0).numpy(), rtol=1e-5, atol=1e-7)


def test_transpose_nobag_vs_pooled_transpose():
    """The numpy nobag transpose against the C pooled one on the same batch:
    identical keys and runs, and each nobag info l*T + t names the table and,
    through offsets, the bag of the pooled info at the same sorted place."""
    _, inp = _nobag_case(9, rows=(40, 9, 70), max_L=9)
    T = 3
    nb = orc.info_B_num_bits(T, inp.B)
    a = orc.transpose_embedding_input_nobag(inp.hash_size_cumsum, inp.B, inp.total_hash_size_bits,
                                            inp.indices, inp.offsets)
    b = orc.transpose_embedding_input(inp.hash_size_cumsum, inp.B, nb, inp.total_hash_size_bits,
                                      inp.indices, inp.offsets)
    for k in ("sorted_linear_indices", "run", "run_lengths", "cumulative_run_lengths"):
        np.testing.assert_array_equal(a[k], b[k])
    l, t = a["infos_sorted"] // T, a["infos_sorted"] % T
    bag = np.searchsorted(inp.offsets, l, side="right") - 1
    np.testing.assert_array_equal(t, b["infos_sorted"] >> nb)
    np.testing.assert_array_equal(bag - t * inp.B, b["infos_sorted"] & ((1 << nb) - 1))
    np.testing.assert_array_equal(a["linear_indices"], b["linear_indices"])


# ---- sparse-feature helpers ----------------------------------------------------

@pytest.mark.parametrize("dtype", [np.int32, np.int64])
@pytest.mark.parametrize("kind", [0, 1, 2])
def test_cumsum_vs_python_loop(dtype, kind):
    """A running sum in Python integers, reduced to the type's two's complement,
    on values that wrap the int32 range."""
    rng = np.random.default_rng(kind)
    big = np.iinfo(dtype).max // 3
    for x in (np.zeros(0, dtype), np.array([5], dtype), rng.integers(-100, 100, 37).astype(dtype),
              np.array([big, big, big, big, -7, big], dtype)):
        bits = np.dtype(dtype).itemsize * 8
        acc, inc = 0, []
        for v in x.tolist():
            acc = (acc + v + (1 << (bits - 1))) % (1 << bits) - (1 << (bits - 1))
            inc.append(acc)
        exp = {1: inc, 0: [0] + inc[:-1] if inc else [], 2: [0] + inc}[kind]
        np.testing.assert_array_equal(orc.cumsum(x, kind), np.array(exp, dtype))
    m = rng.integers(0, 9, (4, 6)).astype(dtype)
    if kind == 2:  # 2-D: per row
        np.testing.assert_array_equal(orc.cumsum(m, 2), np.stack([orc.cumsum(r, 2) for r in m]))


def test_permute_2d_sparse_data_vs_bag_lists():
    """Against lists of bags: output bag (f, b) is input bag (permute[f], b);
    repeats and a feature outside the range (zero lengths) included."""
    rng = np.random.default_rng(3)
    T, B = 4, 5
    lengths = rng.integers(0, 4, (T, B)).astype(np.int64)
    n = int(lengths.sum())
    idx = rng.integers(0, 1000, n).astype(np.int64)
    w = rng.standard_normal(n).astype(np.float32)
    bags, p = [], 0
    for t in range(T):
        row = []
        for b in range(B):
            row.append((idx[p:p + lengths[t, b]], w[p:p + lengths[t, b]]))
            p += lengths[t, b]
        bags.append(row)
    permute = [2, 0, 2, 3, 9]
    pl, pi, pw = orc.permute_2d_sparse_data(permute, lengths, idx, w)
    exp_i = [bags[s][b][0] for s in permute if s < T for b in range(B)]
    exp_w = [bags[s][b][1] for s in permute if s < T for b in range(B)]
    np.testing.assert_array_equal(pi, np.concatenate(exp_i))
    np.testing.assert_array_equal(pw, np.concatenate(exp_w))
    np.testing.assert_array_equal(pl[:4], lengths[[2, 0, 2, 3]])
    assert np.all(pl[4] == 0)


def test_jagged_mul_vs_torch_composition():
    """x * y at the jagged coordinates: torch's own padded-dense-to-jagged
    gather of y, times x, in each dtype (f16/bf16 through fp32, as torch's
    half and bfloat16 mul compute); rows past max_L give x * 0 (signed zero)."""
    rng = np.random.default_rng(4)
    off = np.array([0, 3, 3, 9, 10], np.int64)  # bag 2 has 6 rows, max_L 4: two past it
    for dt, tdt in (("f32", torch.float32), ("f64", torch.float64), ("f16", torch.float16),
                    ("bf16", torch.bfloat16)):
        x = torch.from_numpy(rng.standard_normal((10, 3))).to(tdt)
        y = torch.from_numpy(rng.standard_normal((4, 4, 3))).to(tdt)
        yg = torch.zeros_like(x)
        for b in range(4):
            n = min(off[b + 1] - off[b], 4)
            yg[off[b]:off[b] + n] = y[b, :n]
        exp = x * yg
        as_np = (lambda t: t.view(torch.int16).numpy().view(np.uint16)) if dt == "bf16" else \
            (lambda t: t.numpy())
        got = orc.jagged_dense_elementwise_mul(as_np(x), [off], as_np(y), dt)
        if dt == "bf16":
            np.testing.assert_array_equal(got, as_np(exp))
        else:
            np.testing.assert_array_equal(np.signbit(got), np.signbit(exp.numpy()))
            np.testing.assert_array_equal(got, exp.numpy())


def test_offsets_range_and_expand_permute_vs_python():
    """Element by element in Python: offsets_range's positions within their
    segments, and expand_into_jagged_permute's source positions."""
    off = np.array([0, 3, 3, 7], np.int64)
    exp = []
    bounds = [0, 3, 3, 7, 10]
    for i in range(4):
        exp += list(range(bounds[i + 1] - bounds[i]))
    np.testing.assert_array_equal(orc.offsets_range(off, 10), np.array(exp, np.int64))
    in_len = [2, 5, 0, 3]
    in_off = np.array([0, 2, 7, 7], np.int64)
    permute = [3, 1, 0, 1]
    out_len = [in_len[p] for p in permute]
    out_off = np.array([0, 3, 8, 10, 15], np.int64)
    exp = [in_off[p] + j for p in permute for j in range(in_len[p])]
    np.testing.assert_array_equal(orc.expand_into_jagged_permute(permute, in_off, out_off, 15),
                                  np.array(exp, np.int64))
    np.testing.assert_array_equal(orc.expand_into_jagged_permute(permute, in_off, out_off[:4], 15),
                                  np.array(exp, np.int64))
    assert sum(out_len) == 15
