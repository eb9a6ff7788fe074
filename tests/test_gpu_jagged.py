"""GPU parity of the jagged ops against the oracle: bit-exact (pure data
movement, and one correctly rounded add per element)."""

import numpy as np
import pytest
import torch

import oracle as orc
from mx_fbgemm import bench_inputs

pytestmark = pytest.mark.gpu


def _offsets(lengths):
    return bench_inputs.offsets_from_lengths(np.asarray(lengths, dtype=np.int64))


def _bits_equal(a: torch.Tensor, b: np.ndarray):
    a = a.detach().cpu().contiguous()
    if a.dtype == torch.bfloat16:
        a = a.view(torch.int16)
        b = np.asarray(b).view(np.int16)
    an = a.numpy()
    assert an.shape == b.shape, (an.shape, b.shape)
    assert an.tobytes() == np.ascontiguousarray(b).astype(an.dtype).tobytes()


CASES = [
    # (lengths, max_L, D)
    ([3, 0, 5, 1], 4, 8),          # truncation (len 5 > max_L 4) and an empty row
    ([0, 0, 0], 3, 16),            # all empty
    ([7], 7, 3),                   # odd inner size -> 4-byte path
    ([1, 2, 3, 4, 5, 6], 6, 128),  # 16-byte path
    ([2, 9, 0, 4], 3, 1),          # inner 1
]


@pytest.mark.parametrize("lengths,max_L,D", CASES)
@pytest.mark.parametrize("offset_dtype", [torch.int64, torch.int32])
def test_jagged_to_padded_dense(dev, lengths, max_L, D, offset_dtype):
    print(f"[case] j2pd lengths={lengths} max_L={max_L} D={D} {offset_dtype}", flush=True)
    rng = np.random.default_rng(1)
    off = _offsets(lengths)
    vals = rng.standard_normal((int(off[-1]), D)).astype(np.float32)
    exp = orc.jagged_to_padded_dense(vals, [off], [max_L], padding_value=-7.5)
    got = torch.ops.fbgemm.jagged_to_padded_dense(
        torch.from_numpy(vals).to(dev), [torch.from_numpy(off).to(dev, offset_dtype)], [max_L],
        -7.5)
    _bits_equal(got, exp)


@pytest.mark.parametrize("lengths,max_L,D", CASES)
def test_dense_to_jagged(dev, lengths, max_L, D):
    print(f"[case] d2j lengths={lengths} max_L={max_L} D={D}", flush=True)
    rng = np.random.default_rng(2)
    off = _offsets(lengths)
    dense = rng.standard_normal((len(lengths), max_L, D)).astype(np.float32)
    exp = orc.dense_to_jagged(dense, [off])
    got, got_off = torch.ops.fbgemm.dense_to_jagged(torch.from_numpy(dense).to(dev),
                                                     [torch.from_numpy(off).to(dev)])
    _bits_equal(got, exp)
    assert torch.equal(got_off[0].cpu(), torch.from_numpy(off))


@pytest.mark.parametrize("dtype", ["f32", "f64", "f16", "bf16"])
@pytest.mark.parametrize("lengths,max_L,D", CASES[:4])
def test_jagged_dense_add(dev, dtype, lengths, max_L, D):
    print(f"[case] add {dtype} lengths={lengths} max_L={max_L} D={D}", flush=True)
    rng = np.random.default_rng(3)
    off = _offsets(lengths)
    x = rng.standard_normal((int(off[-1]), D)).astype(np.float32)
    y = rng.standard_normal((len(lengths), max_L, D)).astype(np.float32)
    tdt = {"f32": torch.float32, "f64": torch.float64, "f16": torch.float16,
           "bf16": torch.bfloat16}[dtype]
    xt = torch.from_numpy(x).to(tdt)
    yt = torch.from_numpy(y).to(tdt)
    if dtype == "bf16":
        xn, yn = xt.view(torch.int16).numpy().view(np.uint16), yt.view(torch.int16).numpy().view(np.uint16)
    else:
        xn, yn = xt.numpy(), yt.numpy()
    exp = orc.jagged_dense_elementwise_add(xn, [off], yn, dtype)
    got, _ = torch.ops.fbgemm.jagged_dense_elementwise_add_jagged_output(
        xt.to(dev), [torch.from_numpy(off).to(dev)], yt.to(dev))
    _bits_equal(got, exp)


def test_two_jagged_dims(dev):
    print("[case] j2pd/d2j two jagged dims", flush=True)
    rng = np.random.default_rng(4)
    off0 = _offsets([2, 0, 3])          # 5 level-1 rows
    off1 = _offsets([1, 4, 0, 2, 3])    # 10 values rows
    vals = rng.standard_normal((10, 6)).astype(np.float32)
    exp = orc.jagged_to_padded_dense(vals, [off0, off1], [2, 3], 0.0)
    offs = [torch.from_numpy(off0).to(dev), torch.from_numpy(off1).to(dev)]
    got = torch.ops.fbgemm.jagged_to_padded_dense(torch.from_numpy(vals).to(dev), offs, [2, 3])
    _bits_equal(got, exp)
    back = torch.ops.fbgemm.dense_to_jagged_forward(got, offs)
    _bits_equal(back, orc.dense_to_jagged(exp, [off0, off1]))


def test_config1_round_trip(dev):
    """Config 1: j2pd then d2j returns the values bit for bit (all len <= max_L)."""
    print("[case] config1 round trip B=512 D=128 max_L=64", flush=True)
    cfg = bench_inputs.config1()
    v = torch.from_numpy(cfg.values).to(dev)
    off = torch.from_numpy(cfg.offsets).to(dev)
    dense = torch.ops.fbgemm.jagged_to_padded_dense(v, [off], [cfg.max_L], 0.0)
    _bits_equal(dense, orc.jagged_to_padded_dense(cfg.values, [cfg.offsets], [cfg.max_L], 0.0))
    back, _ = torch.ops.fbgemm.dense_to_jagged(dense, [off])
    assert torch.equal(back, v)


def test_autograd(dev):
    print("[case] jagged autograd", flush=True)
    rng = np.random.default_rng(5)
    off = _offsets([2, 5, 0, 3])
    vals = torch.from_numpy(rng.standard_normal((10, 4)).astype(np.float32)).to(dev)
    vals.requires_grad_(True)
    offt = torch.from_numpy(off).to(dev)
    dense = torch.ops.fbgemm.jagged_to_padded_dense(vals, [offt], [4], 0.0)
    g = torch.from_numpy(rng.standard_normal((4, 4, 4)).astype(np.float32)).to(dev)
    (dense * g).sum().backward()
    exp = orc.dense_to_jagged(g.cpu().numpy(), [off], total_L=10)  # truncated rows get 0
    _bits_equal(vals.grad, exp)

    y = torch.from_numpy(rng.standard_normal((4, 4, 4)).astype(np.float32)).to(dev)
    y.requires_grad_(True)
    x = vals.detach().clone().requires_grad_(True)
    out, _ = torch.ops.fbgemm.jagged_dense_elementwise_add_jagged_output(x, [offt], y)
    gout = torch.from_numpy(rng.standard_normal((10, 4)).astype(np.float32)).to(dev)
    (out * gout).sum().backward()
    _bits_equal(x.grad, gout.cpu().numpy())
    _bits_equal(y.grad, orc.jagged_to_padded_dense(gout.cpu().numpy(), [off], [4], 0.0))


def test_autograd_two_jagged_dims(dev):
    """Backward of the 2-level jagged ops: d(j2pd) = d2j of the upstream
    gradient (truncated/padded positions get 0), d(d2j) = j2pd with pad 0."""
    print("[case] jagged autograd, two jagged dims", flush=True)
    rng = np.random.default_rng(6)
    off0 = _offsets([2, 0, 3])
    off1 = _offsets([1, 4, 0, 2, 3])
    offs = [torch.from_numpy(off0).to(dev), torch.from_numpy(off1).to(dev)]
    vals = torch.from_numpy(rng.standard_normal((10, 3)).astype(np.float32)).to(dev).requires_grad_()
    dense = torch.ops.fbgemm.jagged_to_padded_dense(vals, offs, [2, 3], 0.0)
    g = rng.standard_normal(tuple(dense.shape)).astype(np.float32)
    (dense * torch.from_numpy(g).to(dev)).sum().backward()
    _bits_equal(vals.grad, orc.dense_to_jagged(g, [off0, off1], total_L=10))
    d = torch.from_numpy(rng.standard_normal((3, 2, 3, 3)).astype(np.float32)).to(dev).requires_grad_()
    jv, _ = torch.ops.fbgemm.dense_to_jagged(d, offs)
    gj = rng.standard_normal(tuple(jv.shape)).astype(np.float32)
    (jv * torch.from_numpy(gj).to(dev)).sum().backward()
    _bits_equal(d.grad, orc.jagged_to_padded_dense(gj, [off0, off1], [2, 3], 0.0))


def test_jagged_to_padded_dense_backward_op(dev):
    print("[case] jagged_to_padded_dense_backward op", flush=True)
    rng = np.random.default_rng(8)
    off = _offsets([3, 0, 6, 2])
    g = rng.standard_normal((4, 4, 5)).astype(np.float32)
    got = torch.ops.fbgemm.jagged_to_padded_dense_backward(
        torch.from_numpy(g).to(dev), [torch.from_numpy(off).to(dev)], 11)
    _bits_equal(got, orc.dense_to_jagged(g, [off], total_L=11))


@pytest.mark.parametrize("dtype", ["f32", "f64", "f16", "bf16"])
@pytest.mark.parametrize("lengths,max_L,D", CASES)
def test_jagged_dense_mul(dev, dtype, lengths, max_L, D):
    """x * y at the jagged coordinates (x * 0 past max_L), bit for bit."""
    print(f"[case] mul {dtype} lengths={lengths} max_L={max_L} D={D}", flush=True)
    rng = np.random.default_rng(13)
    off = _offsets(lengths)
    tdt = {"f32": torch.float32, "f64": torch.float64, "f16": torch.float16,
           "bf16": torch.bfloat16}[dtype]
    xt = torch.from_numpy(rng.standard_normal((int(off[-1]), D))).to(tdt)
    yt = torch.from_numpy(rng.standard_normal((len(lengths), max_L, D))).to(tdt)
    if dtype == "bf16":
        xn, yn = xt.view(torch.int16).numpy().view(np.uint16), yt.view(torch.int16).numpy().view(np.uint16)
    else:
        xn, yn = xt.numpy(), yt.numpy()
    exp = orc.jagged_dense_elementwise_mul(xn, [off], yn, dtype)
    got = torch.ops.fbgemm.jagged_dense_elementwise_mul(xt.to(dev), [torch.from_numpy(off).to(dev)],
                                                        yt.to(dev))
    _bits_equal(got, exp)


def test_jagged_dense_mul_two_dims_and_autograd(dev):
    """Two jagged dims; d/dx = grad * y at the coordinates, d/dy = the padded
    dense of grad * x, both against the oracle's gather / scatter, bit for bit."""
    print("[case] mul two jagged dims + autograd", flush=True)
    rng = np.random.default_rng(14)
    off0 = _offsets([2, 0, 3])
    off1 = _offsets([1, 4, 0, 2, 3])
    offs = [torch.from_numpy(off0).to(dev), torch.from_numpy(off1).to(dev)]
    x = rng.standard_normal((10, 3)).astype(np.float32)
    y = rng.standard_normal((3, 2, 3, 3)).astype(np.float32)
    xt = torch.from_numpy(x).to(dev).requires_grad_()
    yt = torch.from_numpy(y).to(dev).requires_grad_()
    out = torch.ops.fbgemm.jagged_dense_elementwise_mul(xt, offs, yt)
    _bits_equal(out, orc.jagged_dense_elementwise_mul(x, [off0, off1], y, "f32"))
    g = rng.standard_normal((10, 3)).astype(np.float32)
    (out * torch.from_numpy(g).to(dev)).sum().backward()
    _bits_equal(xt.grad, orc.jagged_dense_elementwise_mul(g, [off0, off1], y, "f32"))
    _bits_equal(yt.grad, orc.jagged_to_padded_dense((g * x).astype(np.float32), [off0, off1],
                                                    [2, 3], 0.0))


@pytest.mark.parametrize("lengths,max_L,D", CASES)
def test_jagged_2d_to_dense(dev, lengths, max_L, D):
    print(f"[case] jagged_2d_to_dense lengths={lengths} max_L={max_L} D={D}", flush=True)
    rng = np.random.default_rng(15)
    off = _offsets(lengths)
    v = rng.standard_normal((int(off[-1]), D)).astype(np.float32)
    vt = torch.from_numpy(v).to(dev).requires_grad_()
    got = torch.ops.fbgemm.jagged_2d_to_dense(vt, torch.from_numpy(off).to(dev), max_L)
    _bits_equal(got, orc.jagged_to_padded_dense(v, [off], [max_L], 0.0))
    g = rng.standard_normal(tuple(got.shape)).astype(np.float32)
    (got * torch.from_numpy(g).to(dev)).sum().backward()
    _bits_equal(vt.grad, orc.dense_to_jagged(g, [off], total_L=int(off[-1])))


@pytest.mark.parametrize("dtype,pad", [(np.int64, -1), (np.int64, (1 << 62) + 3),
                                       (np.int32, 7), (np.float32, -2)])
def test_jagged_1d_to_dense(dev, dtype, pad):
    """Integer padding keeps every bit of an int64 (2^62 + 3 is not a double)."""
    print(f"[case] jagged_1d_to_dense {np.dtype(dtype).name} pad={pad}", flush=True)
    rng = np.random.default_rng(16)
    lengths = [3, 0, 6, 1, 2]
    off = _offsets(lengths)
    v = rng.integers(-1000, 1000, int(off[-1])).astype(dtype)
    got = torch.ops.fbgemm.jagged_1d_to_dense(torch.from_numpy(v).to(dev),
                                              torch.from_numpy(off).to(dev), 4, pad)
    exp = np.full((len(lengths), 4), pad, dtype)
    for b, n in enumerate(lengths):
        k = min(n, 4)
        exp[b, :k] = v[off[b]:off[b] + k]
    _bits_equal(got, exp)


def test_jagged_dense_add_autograd_two_dims(dev):
    """The add's backward with two jagged dims: grad_x = grad, grad_y = the
    padded dense of grad (the offsets list is one argument of the node)."""
    print("[case] add autograd two jagged dims", flush=True)
    rng = np.random.default_rng(17)
    off0 = _offsets([2, 0, 3])
    off1 = _offsets([1, 4, 0, 2, 3])
    offs = [torch.from_numpy(off0).to(dev), torch.from_numpy(off1).to(dev)]
    xt = torch.from_numpy(rng.standard_normal((10, 3)).astype(np.float32)).to(dev).requires_grad_()
    yt = torch.from_numpy(rng.standard_normal((3, 2, 3, 3)).astype(np.float32)).to(dev).requires_grad_()
    out, _ = torch.ops.fbgemm.jagged_dense_elementwise_add_jagged_output(xt, offs, yt)
    g = rng.standard_normal((10, 3)).astype(np.float32)
    (out * torch.from_numpy(g).to(dev)).sum().backward()
    _bits_equal(xt.grad, g)
    _bits_equal(yt.grad, orc.jagged_to_padded_dense(g, [off0, off1], [2, 3], 0.0))
