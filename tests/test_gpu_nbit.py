"""GPU parity of the nbit (quantized) inference lookup against the C oracle
and, at full size, FBGEMM's CPU kernels (pinned bit-exact to the oracle).

Tolerance: the operator contract states rtol 1e-2 for fp16/quantized
outputs (atol 1e-3 near zero), and that is checked; on top, every fp16
output must lie within one fp16 ulp of the oracle's.  The GPU accumulates
sum(scale*q) and sum(bias) separately while the oracle follows FBGEMM's
fma(scale, q, acc + bias); both are fp32 sums of the same terms, so at most
the last fp16 bit differs.  fp32 outputs: rtol 1e-5, atol 1e-5."""

import numpy as np
import pytest
import torch

import oracle as orc
from mx_fbgemm import bench_inputs
from nbit_helpers import (assert_nbit_close, bf16_ulp_distance, build_weights, build_weights_gpu, max_dims,
                          nbit_forward_gpu)
from tbe_helpers import random_tbe

pytestmark = pytest.mark.gpu


def _check(got: torch.Tensor, exp: np.ndarray):
    assert_nbit_close(got, exp)


TYPES = [orc.FP32, orc.FP16, orc.INT8, orc.INT4, orc.INT2]


@pytest.mark.parametrize("ty", TYPES)
@pytest.mark.parametrize("D", [8, 16, 32, 64, 128, 256, 24, 96])
def test_single_type(dev, ty, D):
    print(f"[case] nbit ty={ty} D={D}", flush=True)
    rng = np.random.default_rng(100 + ty * 1000 + D)
    T, B = 2, 19
    inp = random_tbe(rng, T, B, [D] * T, [37, 5], 25)
    tys = [ty] * T
    buf, w_off = build_weights(rng, tys, inp.D, inp.E)
    for pooling in (0, 1):
        exp = orc.nbit_forward(buf, w_off, tys, inp.D_offsets, B, inp.indices, inp.offsets,
                               pooling)
        got = nbit_forward_gpu(dev, torch.from_numpy(buf).to(dev), w_off, tys, inp.D,
                               inp.indices, inp.offsets, pooling)
        _check(got, exp)


@pytest.mark.parametrize("ebits,ebias", [(4, 7), (5, 15), (3, 3)])
@pytest.mark.parametrize("D", [8, 16, 24, 32, 96, 128, 256, 520])
def test_fp8_tables(dev, ebits, ebias, D):
    """FP8 (hfp8) tables: every code decodes exactly and the rows add in index
    order, as in the oracle (bit-exact to FBGEMM's FP8 CPU kernel), so SUM and
    MEAN, weighted or not, fp16 or fp32 out, match bit for bit; D = 24 and
    520 take the general path."""
    print(f"[case] nbit fp8 ebits={ebits} bias={ebias} D={D}", flush=True)
    rng = np.random.default_rng(ebits * 1000 + D)
    inp = random_tbe(rng, 2, 19, [D, D], [37, 5], 25)
    tys = [orc.FP8, orc.FP8]
    buf, w_off = build_weights(rng, tys, inp.D, inp.E, fp8_exponent_bits=ebits,
                               fp8_exponent_bias=ebias)
    iw = rng.uniform(-1, 1, size=inp.N).astype(np.float32)
    for pooling, weights, out_f16 in ((0, None, True), (1, None, True), (0, iw, False),
                                      (1, iw, True)):
        exp = orc.nbit_forward(buf, w_off, tys, inp.D_offsets, inp.B, inp.indices, inp.offsets,
                               pooling, indice_weights=weights, out_f16=out_f16,
                               fp8_exponent_bits=ebits, fp8_exponent_bias=ebias)
        got = nbit_forward_gpu(dev, torch.from_numpy(buf).to(dev), w_off, tys, inp.D,
                               inp.indices, inp.offsets, pooling, out_f16=out_f16,
                               indice_weights=weights, fp8_exponent_bits=ebits,
                               fp8_exponent_bias=ebias).cpu().numpy()
        view = np.uint16 if out_f16 else np.uint32
        np.testing.assert_array_equal(got.view(view), exp.view(view))


@pytest.mark.parametrize("ty", TYPES + [orc.FP8])
@pytest.mark.parametrize("pooling", [0, 1])
@pytest.mark.parametrize("weighted", [False, True])
def test_bf16_output(dev, ty, pooling, weighted):
    """bf16 output, rounded to nearest with ties away from zero as FBGEMM's CPU
    kernels do (the oracle matches them bit for bit).  Weights in steps of 1/4
    put many sums exactly between two bf16 values.  FP32/FP16/FP8 rows add in
    the oracle's order: bit-exact; quantized rows group scale*q and bias
    differently: within one bf16 place, at least 90 % exact."""
    print(f"[case] nbit bf16 out ty={ty} pool={pooling} weighted={weighted}", flush=True)
    rng = np.random.default_rng(ty * 7 + 3 * weighted + pooling)
    dims, rows = [32, 64, 24], [40, 70, 30]
    inp = random_tbe(rng, 3, 40, dims, rows, 20)
    tys = [ty] * 3
    buf, w_off = build_weights(rng, tys, dims, rows)
    iw = (rng.integers(-4, 5, inp.N) / 4).astype(np.float32) if weighted else None
    exp = orc.nbit_forward(buf, w_off, tys, inp.D_offsets, inp.B, inp.indices, inp.offsets,
                           pooling, indice_weights=iw, out_bf16=True)
    got = nbit_forward_gpu(dev, torch.from_numpy(buf).to(dev), w_off, tys, dims, inp.indices,
                           inp.offsets, pooling, indice_weights=iw, out_bf16=True)
    assert got.dtype == torch.bfloat16
    g = got.cpu().view(torch.int16).numpy().view(np.uint16)
    if ty in (orc.INT8, orc.INT4, orc.INT2):
        d = bf16_ulp_distance(g, exp)
        assert d.max() <= 1 and (d == 0).mean() >= 0.9, (d.max(), (d == 0).mean())
    else:
        np.testing.assert_array_equal(g, exp)


def test_mixed_types_weighted_fp32_out(dev):
    print("[case] nbit mixed types, weighted, fp32 out, int32 indices", flush=True)
    rng = np.random.default_rng(5)
    tys = [orc.INT8, orc.INT4, orc.FP16, orc.INT2, orc.FP32, orc.INT4, orc.FP8]
    dims = [128, 64, 32, 256, 16, 512, 64]
    rows = [100, 200, 50, 10, 30, 40, 60]
    inp = random_tbe(rng, len(tys), 33, dims, rows, 30)
    buf, w_off = build_weights(rng, tys, dims, rows)
    iw = rng.uniform(0, 1, size=inp.N).astype(np.float32)
    for pooling in (0, 1):
        exp = orc.nbit_forward(buf, w_off, tys, inp.D_offsets, inp.B, inp.indices, inp.offsets,
                               pooling, indice_weights=iw, out_f16=False)
        got = nbit_forward_gpu(dev, torch.from_numpy(buf).to(dev), w_off, tys, dims, inp.indices,
                               inp.offsets, pooling, out_f16=False, indice_weights=iw,
                               index_dtype=torch.int32)
        _check(got, exp)


def test_config4_reduced_batch(dev):
    """Config 4 tables (16 INT8 + 16 INT4, E=1e6, D=128, MEAN, fp16 out) with
    the batch cut to B=1024 so the C oracle checks every bag; the full-size
    batch is checked against FBGEMM's kernels below."""
    print("[case] config4 B=1024", flush=True)
    cfg = bench_inputs.config4(B=1024)
    rng = np.random.default_rng(44)
    buf, w_off = build_weights(rng, cfg.tys, cfg.D, cfg.E)
    exp = orc.nbit_forward(buf, w_off, cfg.tys, cfg.D_offsets, cfg.B, cfg.indices, cfg.offsets, 1)
    got = nbit_forward_gpu(dev, torch.from_numpy(buf).to(dev), w_off, cfg.tys, cfg.D, cfg.indices,
                           cfg.offsets, 1, index_dtype=torch.int32)
    _check(got, exp)


def test_config5_reduced_batch(dev):
    """Config 5 shapes (64 mixed FP16/INT4 tables, D 32..256, Poisson bags, 10%
    empty) with a reduced batch."""
    print("[case] config5 B=256", flush=True)
    cfg = bench_inputs.config5(B=256, e_hi=2e5)
    rng = np.random.default_rng(55)
    buf, w_off = build_weights(rng, cfg.tys, cfg.D, cfg.E)
    exp = orc.nbit_forward(buf, w_off, cfg.tys, cfg.D_offsets, cfg.B, cfg.indices, cfg.offsets, 0)
    got = nbit_forward_gpu(dev, torch.from_numpy(buf).to(dev), w_off, cfg.tys, cfg.D, cfg.indices,
                           cfg.offsets, 0, index_dtype=torch.int32)
    _check(got, exp)
    empty = (np.diff(cfg.offsets) == 0).reshape(cfg.T, cfg.B)
    g = got.float().cpu().numpy()
    for t in range(cfg.T):
        d0, d1 = int(cfg.D_offsets[t]), int(cfg.D_offsets[t + 1])
        assert np.all(g[empty[t], d0:d1] == 0.0)


@pytest.mark.parametrize("config", [4, 5])
def test_full_size_every_bag(dev, config):
    """Configs 4 and 5 at full size (the bench's tables, batch and indices):
    every bag of the whole [B, total_D] output is checked against FBGEMM's
    CPU nbit kernels on all host threads (bit-exact to the C oracle, see the
    oracle pins); config 5's empty bags are exactly zero."""
    print(f"[case] config{config} full size, every bag", flush=True)
    cfg = bench_inputs.config4() if config == 4 else bench_inputs.config5()
    pooling = 1 if config == 4 else 0
    W, w_off = build_weights_gpu(dev, cfg.tys, cfg.D, cfg.E, seed=config)
    got = nbit_forward_gpu(dev, W, w_off, cfg.tys, cfg.D, cfg.indices, cfg.offsets, pooling,
                           index_dtype=torch.int32)
    torch.cuda.synchronize()
    buf = W.cpu().numpy()
    del W
    exp = orc.fbgemm_nbit_forward(buf, w_off, cfg.tys, cfg.D_offsets, cfg.E, cfg.B, cfg.indices,
                                  cfg.offsets, pooling, nthreads=orc.host_threads())
    del buf
    g = got.cpu().numpy()
    del got
    assert g.shape == exp.shape == (cfg.B, cfg.total_D)
    assert_nbit_close(g, exp)
    if config == 5:
        empty = (np.diff(cfg.offsets) == 0).reshape(cfg.T, cfg.B)
        for t in range(cfg.T):
            d0, d1 = int(cfg.D_offsets[t]), int(cfg.D_offsets[t + 1])
            assert np.all(g[empty[t], d0:d1].view(np.uint16) == 0)


def _raw_nbit(dev, W, w_off, ty_bytes, dims, indices, offsets, maxima, pooling=0, iw=None):
    """The op called with maxima chosen by the test (not derived from the tables)."""
    T = len(ty_bytes)
    D_off = np.concatenate([[0], np.cumsum(dims)]).astype(np.int32)
    m2, m4, m8, m16, m32 = maxima
    return torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function(
        W, torch.zeros(0, dtype=torch.uint8, device=dev),
        torch.zeros(T, dtype=torch.int32, device=dev), torch.as_tensor(w_off, device=dev),
        torch.as_tensor(np.asarray(ty_bytes, np.uint8), device=dev),
        torch.as_tensor(D_off, device=dev), int(D_off[-1]), m2, m4, m8, m16, m32,
        torch.as_tensor(indices, device=dev), torch.as_tensor(offsets, device=dev), pooling,
        None if iw is None else torch.as_tensor(iw, device=dev), 1, None, None, 16)


def test_short_indice_weights_raise(dev):
    print("[case] nbit indice_weights shorter than indices", flush=True)
    rng = np.random.default_rng(61)
    tys, dims = [orc.INT8, orc.INT4], [32, 64]
    inp = random_tbe(rng, 2, 8, dims, [20, 30], 6, empty_frac=0.0)
    buf, w_off = build_weights(rng, tys, dims, inp.E)
    iw = np.ones(inp.N - 1, np.float32)
    with pytest.raises(RuntimeError, match="one entry per index"):
        _raw_nbit(dev, torch.from_numpy(buf).to(dev), w_off, tys, dims, inp.indices,
                  inp.offsets, max_dims(tys, dims), iw=iw)


# (bad table's type byte, its D, the type its bytes are built as, maxima override,
#  bytes the bad table's rows are moved by in the weights buffer)
BAD_TABLES = {
    "bf16_type_byte": (5, 32, orc.FP16, None, 0),           # BF16: no nbit launch serves it
    "odd_int4_D": (orc.INT4, 7, orc.INT4, None, 0),          # 7 codes leave half a byte
    "int2_D_not_multiple_of_4": (orc.INT2, 6, orc.INT2, None, 0),
    "type_with_zero_max_D": (orc.INT2, 16, orc.INT2, 0, 0),  # max_int2_D = 0: not launched
    "rows_not_4_byte_aligned": (orc.INT8, 32, orc.INT8, None, 2),  # weights_offsets[t] % 4 == 2
}


@pytest.mark.parametrize("case", sorted(BAD_TABLES))
def test_unservable_table_is_zeroed_and_reported(dev, case):
    """A table no launch of the call can serve has its output columns written
    as zeros (not left as allocated); the other tables match the oracle, and
    the next nbit call on the device raises, once."""
    print(f"[case] nbit unservable table: {case}", flush=True)
    bad_ty, bad_D, build_ty, bad_max, shift = BAD_TABLES[case]
    rng = np.random.default_rng(62)
    ty_bytes = [orc.INT8, bad_ty, orc.FP16, orc.INT4]
    dims = [32, bad_D, 64, 16]
    build_tys = [orc.INT8, build_ty, orc.FP16, orc.INT4]
    inp = random_tbe(rng, 4, 37, dims, [50, 40, 30, 20], 9)
    buf, w_off = build_weights(rng, build_tys, dims, inp.E)
    good = [0, 2, 3]
    maxima = list(max_dims([ty_bytes[t] for t in good], [dims[t] for t in good]))
    if bad_max is not None:
        maxima[0] = bad_max  # the INT2 slot
    elif bad_ty == orc.INT2:
        # INT2 is launched, with a maximum the host check accepts (a multiple
        # of 4), so the device check is the one that finds the table.  (The
        # INT4 case keeps the served INT4 table's maximum, 16.)
        maxima[0] = 8
    if shift:  # the bad table's bytes move by `shift`, the next tables' by 4 (aligned again)
        w_off_k = w_off + np.array([0, shift, 4, 4], np.int64)
        gap = np.zeros(shift, np.uint8)
        buf_k = np.concatenate([buf[:w_off[1]], gap, buf[w_off[1]:w_off[2]],
                                np.zeros(4 - shift, np.uint8), buf[w_off[2]:]])
    else:
        w_off_k, buf_k = w_off, buf
    W = torch.from_numpy(buf_k).to(dev)
    # The output reuses a freed block full of NaN, so unwritten columns would show.
    junk = torch.full((inp.B, inp.total_D), float("nan"), dtype=torch.float16, device=dev)
    del junk
    got = _raw_nbit(dev, W, w_off_k, ty_bytes, dims, inp.indices, inp.offsets, maxima)
    torch.cuda.synchronize()
    g = got.cpu().numpy()
    d0 = int(inp.D_offsets[1])
    assert np.all(g[:, d0:d0 + bad_D].view(np.uint16) == 0), "unservable columns not zeroed"
    # The served tables: the oracle on the same lookup restricted to them.
    lens = np.diff(inp.offsets).reshape(inp.T, inp.B)
    sub_idx = np.concatenate([inp.indices[inp.offsets[t * inp.B]:inp.offsets[(t + 1) * inp.B]]
                              for t in good])
    sub_off = bench_inputs.offsets_from_lengths(lens[good].reshape(-1))
    sub_D_off = np.concatenate([[0], np.cumsum([dims[t] for t in good])]).astype(np.int32)
    exp = orc.nbit_forward(buf, w_off[good], [ty_bytes[t] for t in good], sub_D_off, inp.B,
                           sub_idx, sub_off, 0)
    cols = np.concatenate([np.arange(inp.D_offsets[t], inp.D_offsets[t + 1]) for t in good])
    assert_nbit_close(g[:, cols], exp)
    with pytest.raises(RuntimeError, match="cannot serve"):
        _raw_nbit(dev, W, w_off_k, ty_bytes, dims, inp.indices, inp.offsets, maxima)
    # Reported once: a valid call then runs normally.
    ok = _raw_nbit(dev, W, w_off_k[good], [ty_bytes[t] for t in good], [dims[t] for t in good],
                   sub_idx, sub_off, maxima)
    assert_nbit_close(ok, exp)
