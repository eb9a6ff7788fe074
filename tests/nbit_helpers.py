"""Builders of nbit (quantized TBE) test inputs in the TBE row layout."""

from __future__ import annotations

import numpy as np
import torch

import oracle as orc


def build_weights(rng: np.random.Generator, tys, dims, rows, row_align: int = 16,
                  fp8_exponent_bits: int = 4, fp8_exponent_bias: int = 7):
    """uint8 buffer with every table's padded rows, plus weights_offsets.

    Quantized rows: fp16 scale in [1e-3, 1e-2), fp16 bias in [-0.1, 0.1),
    uniform codes; FP16/FP32 rows: values in [-0.01, 0.01); FP8 rows: values
    in [-0.5, 0.5) rounded to the nearest hfp8 code."""
    strides = [orc.nbit_row_bytes(ty, D, row_align) for ty, D in zip(tys, dims)]
    sizes = [E * s for E, s in zip(rows, strides)]
    w_off = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    buf = np.zeros(int(sum(sizes)), dtype=np.uint8)
    for t, (ty, D, E, s) in enumerate(zip(tys, dims, rows, strides)):
        tab = buf[w_off[t]: w_off[t] + E * s].reshape(E, s)
        if ty in (orc.INT8, orc.INT4, orc.INT2):
            tab[:, 4:] = rng.integers(0, 256, size=(E, s - 4), dtype=np.uint8)
            sc = rng.uniform(1e-3, 1e-2, size=E).astype(np.float16)
            bi = rng.uniform(-0.1, 0.1, size=E).astype(np.float16)
            tab[:, 0:2] = sc.view(np.uint8).reshape(E, 2)
            tab[:, 2:4] = bi.view(np.uint8).reshape(E, 2)
        elif ty == orc.FP16:
            v = rng.uniform(-0.01, 0.01, size=(E, D)).astype(np.float16)
            tab[:, : 2 * D] = v.view(np.uint8).reshape(E, 2 * D)
        elif ty == orc.FP8:
            v = rng.uniform(-0.5, 0.5, size=(E, D)).astype(np.float32)
            tab[:, :D] = orc.float_to_hfp8(v, fp8_exponent_bits, fp8_exponent_bias,
                                           orc.hfp8_max_pos(fp8_exponent_bits, fp8_exponent_bias))
        else:
            v = rng.uniform(-0.01, 0.01, size=(E, D)).astype(np.float32)
            tab[:, : 4 * D] = v.view(np.uint8).reshape(E, 4 * D)
    return buf, w_off


def max_dims(tys, dims):
    def m(ty):
        return max([D for t, D in zip(tys, dims) if t == ty], default=0)

    return m(orc.INT2), m(orc.INT4), m(orc.INT8), m(orc.FP16), m(orc.FP32)


def nbit_forward_gpu(dev, W: torch.Tensor, w_off, tys, dims, indices, offsets, pooling: int,
                     out_f16: bool = True, indice_weights=None, row_align: int = 16,
                     index_dtype=torch.int64, fp8_exponent_bits: int = 4,
                     fp8_exponent_bias: int = 7, out_bf16: bool = False):
    T = len(tys)
    D_off = np.concatenate([[0], np.cumsum(dims)]).astype(np.int32)
    m2, m4, m8, m16, m32 = max_dims(tys, dims)
    empty = torch.zeros(0, dtype=torch.uint8, device=dev)
    return torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function(
        W, empty, torch.zeros(T, dtype=torch.int32, device=dev),
        torch.as_tensor(w_off, device=dev), torch.as_tensor(np.asarray(tys, np.uint8), device=dev),
        torch.as_tensor(D_off, device=dev), int(D_off[-1]), m2, m4, m8, m16, m32,
        torch.as_tensor(indices).to(dev, index_dtype), torch.as_tensor(offsets).to(dev, index_dtype),
        pooling, None if indice_weights is None else torch.as_tensor(indice_weights).to(dev),
        5 if out_bf16 else (1 if out_f16 else 0), None, None, row_align,
        max([D for t, D in zip(tys, dims) if t == orc.FP8], default=0), fp8_exponent_bits,
        fp8_exponent_bias)


def build_weights_gpu(dev, tys, dims, rows, seed: int, row_align: int = 16):
    """build_weights' layout and value ranges, generated on the device (the
    full-size configs hold gigabytes of rows)."""
    strides = [orc.nbit_row_bytes(ty, D, row_align) for ty, D in zip(tys, dims)]
    sizes = [E * s for E, s in zip(rows, strides)]
    w_off = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    W = torch.randint(0, 256, (int(sum(sizes)),), generator=g, device=dev, dtype=torch.uint8)
    for t, (ty, D, E, s) in enumerate(zip(tys, dims, rows, strides)):
        tab = W[int(w_off[t]): int(w_off[t]) + E * s].view(E, s)
        if ty in (orc.INT8, orc.INT4, orc.INT2):
            sc = (torch.rand(E, generator=g, device=dev) * 9e-3 + 1e-3).half()
            bi = (torch.rand(E, generator=g, device=dev) * 0.2 - 0.1).half()
            tab[:, 0:2] = sc.view(torch.uint8).view(-1, 2)
            tab[:, 2:4] = bi.view(torch.uint8).view(-1, 2)
        elif ty == orc.FP16:
            v = (torch.rand((E, D), generator=g, device=dev) * 0.02 - 0.01).half()
            tab[:, : 2 * D] = v.view(torch.uint8).view(E, -1)
        else:
            v = torch.rand((E, D), generator=g, device=dev) * 0.02 - 0.01
            tab[:, : 4 * D] = v.view(torch.uint8).view(E, -1)
    return W, w_off


def fp16_ulp_distance(a, b) -> np.ndarray:
    """Distance in fp16 units in the last place between two fp16 arrays: the
    difference of their bit patterns mapped to a monotonic integer scale
    (+0 and -0 are the same point)."""
    def ordinal(x):
        h = np.ascontiguousarray(x, dtype=np.float16).view(np.uint16).astype(np.int32)
        mag = h & 0x7FFF
        return np.where(h & 0x8000, -mag, mag)

    return np.abs(ordinal(a) - ordinal(b))


def bf16_ulp_distance(a_bits, b_bits) -> np.ndarray:
    """Distance in bf16 units in the last place between two arrays of bf16 bit
    patterns (uint16), on the same monotonic scale as fp16_ulp_distance."""
    def ordinal(x):
        h = np.ascontiguousarray(x, dtype=np.uint16).astype(np.int32)
        mag = h & 0x7FFF
        return np.where(h & 0x8000, -mag, mag)

    return np.abs(ordinal(a_bits) - ordinal(b_bits))


def assert_nbit_close(got, exp, max_ulps: int = 1, min_exact: float = 0.9):
    """The nbit parity check.  Stated contract: rtol 1e-2 (atol 1e-3 near
    zero).  What the kernels achieve, and what is asserted on top: fp16
    outputs within `max_ulps` fp16 place of the oracle (both are fp32 sums of
    the same terms, grouped differently, rounded once to fp16), and at least
    `min_exact` of them equal to it (the two fp32 sums land on different
    sides of an fp16 rounding boundary only rarely, while a wrong rounding
    mode moves about half of all outputs by one place); fp32 outputs within
    rtol 1e-5 / atol 1e-5."""
    g = got.cpu().numpy() if hasattr(got, "cpu") else np.asarray(got)
    e = np.asarray(exp)
    np.testing.assert_allclose(g.astype(np.float32), e.astype(np.float32), rtol=1e-2, atol=1e-3)
    if g.dtype == np.float16:
        d = fp16_ulp_distance(g, e.astype(np.float16))
        assert d.max(initial=0) <= max_ulps, (
            f"{int((d > max_ulps).sum())} outputs differ by more than {max_ulps} fp16 ulp "
            f"(max {int(d.max())})")
        if d.size:
            exact = float((d == 0).mean())
            assert exact >= min_exact, (
                f"only {exact:.3f} of the fp16 outputs equal the oracle's (at least {min_exact})")
    else:
        np.testing.assert_allclose(g.astype(np.float32), e.astype(np.float32), rtol=1e-5,
                                   atol=1e-5)


def hfp8_probe_values(rng: np.random.Generator, ebits: int, ebias: int) -> np.ndarray:
    """fp32 values that exercise an hfp8 encoder: every code's value, the
    midpoints between neighbouring codes (ties) and one fp32 ulp either side
    of them, normal and log-uniform samples from 1e-12 to past the largest
    code, signed zeros, fp32 subnormals and values past the clamp."""
    mx = orc.hfp8_max_pos(ebits, ebias)
    vals = orc.hfp8_to_float(np.arange(256, dtype=np.uint8), ebits, ebias)
    pos = np.unique(np.abs(vals))
    mids = ((pos[:-1].astype(np.float64) + pos[1:]) / 2).astype(np.float32)
    around = np.concatenate([np.nextafter(mids, np.float32(np.inf)),
                             np.nextafter(mids, np.float32(0))])
    normal = (rng.standard_normal(5000) * mx / 3).astype(np.float32)
    logs = np.exp(rng.uniform(np.log(1e-12), np.log(min(mx * 4, 1e38)), 5000))
    logs = (logs * rng.choice([-1, 1], logs.size)).astype(np.float32)
    edge = np.array([0.0, -0.0, mx, -mx, mx * 1.01, 1e30, -1e30, 1e-40, -1e-40], np.float32)
    return np.concatenate([vals, mids, -mids, around, -around, normal, logs, edge])
