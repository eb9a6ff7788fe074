"""GPU parity of the nbit (quantized) inference lookup against the C oracle.

Tolerance (stated by the operator contract): fp16/quantized outputs within
rtol 1e-2.  The GPU accumulates sum(scale*q) and sum(bias) separately while
the oracle follows FBGEMM's fma(scale, q, acc + bias); both are fp32 sums of
the same terms, so the only visible difference is the last fp16 bit.  An
absolute floor of 1e-3 covers outputs within rounding distance of zero."""

import numpy as np
import pytest
import torch

import oracle as orc
from mx_fbgemm import bench_inputs
from nbit_helpers import build_weights, nbit_forward_gpu
from tbe_helpers import random_tbe

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3


def _check(got: torch.Tensor, exp: np.ndarray):
    g = got.float().cpu().numpy()
    np.testing.assert_allclose(g, exp.astype(np.float32), rtol=RTOL, atol=ATOL)


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
    the batch cut to B=1024 so the oracle stays quick; the full-size run is
    checked against the same oracle on a sample of bags in the bench tests."""
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
