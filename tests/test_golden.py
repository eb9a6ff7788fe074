"""Committed golden fixtures (tests/golden/*.npz, written by gen_golden.py from
aten's jagged ops, FBGEMM's exported CPU kernels and numpy brute force):
the C oracle must reproduce them on the CPU, and the HIP kernels on the GPU."""

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as orc

GOLD = Path(__file__).resolve().parent / "golden"


def load(name):
    return dict(np.load(GOLD / f"{name}.npz", allow_pickle=False))


def test_oracle_reproduces_jagged_fixture():
    g = load("jagged")
    d = orc.jagged_to_padded_dense(g["values"], [g["offsets"]], [int(g["max_L"])], float(g["pad"]))
    assert d.tobytes() == g["dense"].tobytes()
    j = orc.dense_to_jagged(g["dense2"], [g["offsets2"]])
    assert j.tobytes() == g["jagged2"].tobytes()


@pytest.mark.parametrize("pooling", [0, 1])
def test_oracle_reproduces_tbe_fixture(pooling):
    g = load("tbe_fwd")
    B = int(g["B"])
    out = orc.tbe_forward_f32(g["W"], g["w_off"], g["D_off"], B, g["indices"], g["offsets"], pooling)
    np.testing.assert_array_equal(out, g[f"out_p{pooling}"])
    out = orc.tbe_forward_f32(g["W"], g["w_off"], g["D_off"], B, g["indices"], g["offsets"], pooling,
                              g["iw"])
    np.testing.assert_array_equal(out, g[f"out_w_p{pooling}"])


@pytest.mark.parametrize("pooling", [0, 1])
def test_oracle_reproduces_nbit_fixture(pooling):
    g = load("nbit")
    out = orc.nbit_forward(g["W"], g["w_off"], g["tys"], g["D_off"], int(g["B"]), g["indices"],
                           g["offsets"], pooling)
    np.testing.assert_array_equal(out.view(np.uint16), g[f"out_p{pooling}"].view(np.uint16))


def test_oracle_reproduces_transpose_fixture():
    g = load("transpose")
    r = orc.transpose_embedding_input(g["hsc"], int(g["B"]), int(g["nb"]), int(g["bits"]),
                                      g["indices"], g["offsets"])
    np.testing.assert_array_equal(r["linear_indices"], g["linear"])
    np.testing.assert_array_equal(r["sorted_linear_indices"], g["sorted"])
    np.testing.assert_array_equal(r["infos_sorted"], g["infos"])
    np.testing.assert_array_equal(r["run"], g["run"])
    np.testing.assert_array_equal(r["run_lengths"], g["run_lengths"])
    np.testing.assert_array_equal(r["cumulative_run_lengths"], g["cum"])


# ---- the HIP kernels against the same fixtures -------------------------------

@pytest.mark.gpu
def test_gpu_jagged_fixture(dev):
    g = load("jagged")
    d = torch.ops.fbgemm.jagged_to_padded_dense(
        torch.from_numpy(g["values"]).to(dev), [torch.from_numpy(g["offsets"]).to(dev)],
        [int(g["max_L"])], float(g["pad"]))
    assert d.cpu().numpy().tobytes() == g["dense"].tobytes()
    j, _ = torch.ops.fbgemm.dense_to_jagged(torch.from_numpy(g["dense2"]).to(dev),
                                            [torch.from_numpy(g["offsets2"]).to(dev)])
    assert j.cpu().numpy().tobytes() == g["jagged2"].tobytes()


@pytest.mark.gpu
@pytest.mark.parametrize("pooling", [0, 1])
def test_gpu_tbe_fixture(dev, pooling):
    g = load("tbe_fwd")
    T = g["D_off"].size - 1
    args = (torch.from_numpy(g["W"]).to(dev), torch.zeros(0, device=dev), torch.zeros(0, device=dev),
            torch.zeros(T, dtype=torch.int32, device=dev), torch.from_numpy(g["w_off"]).to(dev),
            torch.from_numpy(g["D_off"]).to(dev), int(g["D_off"][-1]), int(np.diff(g["D_off"]).max()),
            torch.from_numpy(g["indices"]).to(dev), torch.from_numpy(g["offsets"]).to(dev), pooling)
    tail = (torch.zeros(0, dtype=torch.int32, device=dev), torch.zeros(0, device=dev), 0, False)
    out = torch.ops.fbgemm.split_embedding_codegen_forward_unweighted_cuda(*args, *tail)
    np.testing.assert_array_equal(out.cpu().numpy(), g[f"out_p{pooling}"])
    out = torch.ops.fbgemm.split_embedding_codegen_forward_weighted_cuda(
        *args, torch.from_numpy(g["iw"]).to(dev), *tail)
    np.testing.assert_array_equal(out.cpu().numpy(), g[f"out_w_p{pooling}"])


@pytest.mark.gpu
@pytest.mark.parametrize("pooling", [0, 1])
def test_gpu_nbit_fixture(dev, pooling):
    from nbit_helpers import assert_nbit_close, nbit_forward_gpu

    g = load("nbit")
    dims = list(np.diff(g["D_off"]))
    out = nbit_forward_gpu(dev, torch.from_numpy(g["W"]).to(dev), g["w_off"], list(g["tys"]), dims,
                           g["indices"], g["offsets"], pooling)
    assert_nbit_close(out, g[f"out_p{pooling}"])  # rtol 1e-2 contract and <= 1 fp16 ulp


@pytest.mark.gpu
def test_gpu_transpose_fixture(dev):
    g = load("transpose")
    lin, srt, infos, run, lengths, num_runs, cum = torch.ops.fbgemm.transpose_embedding_input(
        torch.from_numpy(g["hsc"]).to(dev), int(g["bits"]), torch.from_numpy(g["indices"]).to(dev),
        torch.from_numpy(g["offsets"]).to(dev), False, None, int(g["nb"]))
    r = int(num_runs.item())
    np.testing.assert_array_equal(lin.cpu().numpy(), g["linear"])
    np.testing.assert_array_equal(srt.cpu().numpy(), g["sorted"])
    np.testing.assert_array_equal(infos.cpu().numpy(), g["infos"])
    np.testing.assert_array_equal(run.cpu().numpy()[:r], g["run"])
    np.testing.assert_array_equal(lengths.cpu().numpy()[:r], g["run_lengths"])
    np.testing.assert_array_equal(cum.cpu().numpy()[:r + 1], g["cum"])
