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
from nbit_helpers import assert_nbit_close, build_weights, build_weights_gpu, nbit_forward_gpu
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


def test_mixed_types_weighted_fp32_out(dev):
    print("[case] nbit mixed types, weighted, fp32 out, int32 indices", flush=True)
    rng = np.random.default_rng(5)
    tys = [orc.INT8, orc.INT4, orc.FP16, orc.INT2, orc.FP32, orc.INT4]
    dims = [128, 64, 32, 256, 16, 512]
    rows = [100, 200, 50, 10, 30, 40]
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
