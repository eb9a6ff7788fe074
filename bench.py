#!/usr/bin/env python3
"""Benchmark of the TBE hot path on one MI355X.

Default workload (config 2): TBE fp32 forward, SUM pooling, T=8 tables of
E=1,000,000 x D=128, B=4096 bags per table, pooling factor U{1..40}, int64
indices Zipf(1.05) with a per-table permutation (seeded synthetic data; the
weights are generated on the device).  One step = one
torch.ops.fbgemm.split_embedding_codegen_forward_unweighted_cuda call over
the batch, inputs resident in HBM.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config {1,2,3,4,5}]
                    [--op {lookup,bounds-check}]

Prints one JSON line: lookups/s (whole job), the roofline of the dominant
kernel (algorithmic bytes per launch / HIP-event-timed launch duration vs
8 TB/s) and the CPU baseline (FBGEMM's CPU kernel on this host's cores).
--config 1/3/4/5 print the same line for the jagged round trip, the backward,
the nbit lookup and the mixed nbit workload; --op bounds-check times
bounds_check_indices over the config-2 batch.
"""

from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "torchlib-xpu_amd"))

PEAK_HBM_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5],
                    help="workload; 2 (default) is the headline")
    ap.add_argument("--op", default="lookup", choices=["lookup", "bounds-check"],
                    help="config 2 only: time bounds_check_indices (WARNING) on the batch "
                         "instead of the lookup")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 1 GiB device copy (PMC byte-counter calibration)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="bound on the CPU baseline's timed work")
    return ap.parse_args()


def traffic_from_profile(name: str):
    """HBM bytes per launch recorded by the rocprofv3 PMC summary, if present."""
    p = REPO / "profiles" / f"{name}.md"
    if not p.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", p.read_text())
    return float(m.group(1)) if m else None


def time_launches(fn, steps: int, warmup: int):
    """Runs `warmup` untimed steps, then times exactly `steps` steps back to
    back, synchronised on both sides.  Returns (wall seconds, mean step
    duration in ms from one pair of HIP events recorded around the steps on
    the current stream -- the stream the ops launch on).  No event sits
    between steps: an event record between launches costs ~7 us of GPU time
    per step here, which is not part of the op."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, start.elapsed_time(end) / steps


def cpu_time(fn, budget_s: float, min_runs: int = 3, warm: int = 1):
    for _ in range(warm):
        fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < min_runs or (time.perf_counter() - t_start < budget_s and len(times) < 10):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s and len(times) >= 1:
            break
    return statistics.median(times), len(times)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---------------------------------------------------------------------------


def bench_jagged(args, dev):
    """Config 1: jagged_to_padded_dense then dense_to_jagged (one round trip
    per step) on B=512 rows of up to 64 x 128 fp32."""
    import torch

    from mx_fbgemm import bench_inputs

    cfg = bench_inputs.config1()
    v = torch.from_numpy(cfg.values).to(dev)
    off = torch.from_numpy(cfg.offsets).to(dev)
    B, D, L, total = cfg.offsets.size - 1, cfg.values.shape[1], cfg.max_L, cfg.values.shape[0]
    j2pd = torch.ops.fbgemm.jagged_to_padded_dense
    d2j = torch.ops.fbgemm.dense_to_jagged

    def step():
        dense = j2pd(v, [off], [L], 0.0)
        return d2j(dense, [off], total)

    wall, mean_ms = time_launches(step, args.steps, args.warmup)
    # j2pd reads the values and writes the padded dense; d2j reads the dense at
    # the jagged positions and writes the values; both read the offsets.
    alg = total * D * 4 + B * L * D * 4 + 2 * total * D * 4 + 2 * (B + 1) * 8
    res = dict(
        metric="jagged round trip (jagged_to_padded_dense + dense_to_jagged) bytes/s, 1 MI355X",
        value=alg * args.steps / wall / 1e9, unit="GB/s", ms_per_step=wall / args.steps * 1e3,
        dtype="fp32",
        config={"workload": "config1: jagged round trip, B=512 D=128 max_L=64, len~U{0..64}",
                "B": B, "D": D, "max_L": L, "total_L": total},
        kernel="j2pd_kernel + d2j_kernel (one step)", alg_bytes=alg, kernel_ms_mean=mean_ms)
    cpu = None
    if not args.no_cpu_baseline:
        vc, oc = v.cpu(), off.cpu()

        def cpu_step():
            dense = torch.ops.aten._jagged_to_padded_dense_forward(vc, [oc], [L], 0.0)
            return torch.ops.aten._padded_dense_to_jagged_forward(dense, [oc], total)

        med, runs = cpu_time(cpu_step, args.cpu_seconds)
        cpu = dict(value=alg / med / 1e9, unit="GB/s", cores=torch.get_num_threads(),
                   kind="reference",
                   sample=(f"full config-1 round trip, median of {runs} runs; torch's CPU "
                           f"aten._jagged_to_padded_dense_forward / _padded_dense_to_jagged_forward "
                           f"(its port of the fbgemm jagged ops) on {torch.get_num_threads()} "
                           f"threads; host CPU: {cpu_model()}"))
    return res, traffic_from_profile("jagged_config1"), cpu


def bench_tbe_forward(args, dev):
    import numpy as np
    import torch

    from mx_fbgemm import bench_inputs

    log("generating config 2 indices")
    inp = bench_inputs.config2()
    T, E, D, B = inp.T, inp.E[0], inp.D[0], inp.B
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    W = torch.empty(T * E * D, device=dev).uniform_(-0.01, 0.01, generator=g)
    w_off = torch.arange(T, device=dev, dtype=torch.int64) * (E * D)
    D_off = torch.from_numpy(inp.D_offsets).to(dev)
    idx = torch.from_numpy(inp.indices).to(dev)
    off = torch.from_numpy(inp.offsets).to(dev)
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(T, dtype=torch.int32, device=dev)
    e32 = torch.zeros(0, dtype=torch.int32, device=dev)
    op = torch.ops.fbgemm.split_embedding_codegen_forward_unweighted_cuda

    def step():
        return op(W, empty, empty, pl, w_off, D_off, inp.total_D, D, idx, off, 0, e32, empty, 0,
                  False)

    log(f"timing N={inp.N} lookups, {args.steps} steps")
    wall, mean_ms = time_launches(step, args.steps, args.warmup)
    N = inp.N
    alg_bytes = N * (D * 4 + 8) + T * B * (8 + D * 4)

    # Cold cache: overwrite a 1 GiB buffer before each timed launch.
    flush = torch.empty(1 << 28, device=dev, dtype=torch.float32)
    cold = []
    for _ in range(5):
        flush.fill_(1.0)
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        step()
        e.record()
        torch.cuda.synchronize()
        cold.append(s.elapsed_time(e))
    del flush

    # Successive batches of one model: 8 batches with the same hot rows and
    # fresh draws, launched in rotation (each batch's tail rows are new to
    # the caches, as in training); reported beside the repeated-batch figure.
    log("generating 7 more config-2 batches of the same tables")
    batches = [(torch.from_numpy(b.indices).to(dev), torch.from_numpy(b.offsets).to(dev), b.N)
               for b in bench_inputs.config2_batches(8)]
    turn = [0]

    def fresh_step():
        bi, bo, _ = batches[turn[0] % len(batches)]
        turn[0] += 1
        return op(W, empty, empty, pl, w_off, D_off, inp.total_D, D, bi, bo, 0, e32, empty, 0,
                  False)

    # Compulsory bytes: every distinct row once (the Zipf heads repeat).
    t_of = np.repeat(np.arange(T * B) // B, np.diff(inp.offsets))
    uniq = int(np.unique(t_of * E + inp.indices).size)
    compulsory = uniq * D * 4 + N * 8 + (T * B + 1) * 8 + T * B * D * 4

    fresh_steps = 8 * max(1, args.steps // 8)
    _, fresh_ms = time_launches(fresh_step, fresh_steps, len(batches))
    fresh_n = sum(b[2] for b in batches) / len(batches)

    res = dict(
        metric="TBE fwd lookups/sec + achieved HBM GB/s (% of peak), 1 MI355X",
        value=N * args.steps / wall,
        unit="lookups/s",
        ms_per_step=wall / args.steps * 1e3,
        dtype="fp32",
        config={"workload": "config2: TBE fp32 forward SUM, T=8 E=1e6 D=128 B=4096 "
                            "L~U{1..40} Zipf(1.05) int64 indices",
                "T": T, "E": E, "D": D, "B": B, "N": N, "indices": "int64"},
        kernel="tbe_fwd_group_kernel",
        alg_bytes=alg_bytes,
        kernel_ms_mean=mean_ms,
        cold_kernel_ms_median=statistics.median(cold),
        fresh_batches=dict(batches=len(batches), launch_ms_mean=fresh_ms,
                           lookups_per_s=fresh_n / (fresh_ms * 1e-3)),
        compulsory_bytes=compulsory, unique_rows=uniq,
    )
    traffic = traffic_from_profile("tbe_fwd_config2")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_tbe(args, inp, W)
    return res, traffic, cpu


def bench_bounds_check(args, dev):
    """bounds_check_indices (WARNING) over the config-2 batch: every offset and
    index is read and checked; the batch is valid, so nothing is rewritten."""
    import numpy as np
    import torch

    from mx_fbgemm import bench_inputs

    log("generating config 2 batch")
    inp = bench_inputs.config2()
    rows = torch.tensor(inp.E, dtype=torch.int64, device=dev)
    idx = torch.from_numpy(inp.indices).to(dev)
    off = torch.from_numpy(inp.offsets).to(dev)
    warn = torch.zeros(1, dtype=torch.int64, device=dev)
    op = torch.ops.fbgemm.bounds_check_indices

    def step():
        op(rows, idx, off, 1, warn)

    wall, mean_ms = time_launches(step, args.steps, args.warmup)
    assert int(warn.item()) == 0, "the config-2 batch is valid"
    alg = inp.N * 8 + (inp.T * inp.B + 1) * 8
    res = dict(
        metric="bounds_check_indices lookups/sec, 1 MI355X", value=inp.N * args.steps / wall,
        unit="lookups/s", ms_per_step=wall / args.steps * 1e3, dtype="int64",
        config={"workload": "config2 batch: bounds_check_indices, WARNING mode", "T": inp.T,
                "B": inp.B, "N": inp.N},
        kernel="tile_max_kernel + bounds_main_kernel", alg_bytes=alg, kernel_ms_mean=mean_ms,
    )
    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, str(REPO / "oracle"))
        import oracle as orc

        rows_h = np.asarray(inp.E, dtype=np.int64)
        fn = lambda: orc.bounds_check_indices(rows_h, inp.indices, inp.offsets, 1)  # noqa: E731
        log("CPU baseline: C restatement of the bounds check, 1 thread")
        med, runs = cpu_time(fn, args.cpu_seconds)
        cpu = dict(value=inp.N / med, unit="lookups/s", cores=1, kind="port",
                   sample=(f"full config-2 batch (N={inp.N}), median of {runs} runs; the "
                           f"oracle's C restatement, one thread, including its copies of "
                           f"indices and offsets; host CPU: {cpu_model()}"))
    return res, traffic_from_profile("bounds_check_config2"), cpu


def cpu_baseline_tbe(args, inp, W):
    import numpy as np

    sys.path.insert(0, str(REPO / "oracle"))
    import oracle as orc

    log("CPU baseline: copying weights to host")
    Wh = W.cpu().numpy()
    w_off = (np.arange(inp.T) * inp.E[0] * inp.D[0]).astype(np.int64)
    nthreads = orc.host_threads()
    fn = lambda: orc.fbgemm_tbe_forward_f32(Wh, w_off, inp.D_offsets, inp.E, inp.B, inp.indices,  # noqa: E731
                                            inp.offsets, 0, nthreads=nthreads)
    log(f"CPU baseline: FBGEMM SpMDM on {nthreads} threads")
    med, runs = cpu_time(fn, args.cpu_seconds)
    fn1 = lambda: orc.fbgemm_tbe_forward_f32(Wh, w_off, inp.D_offsets, inp.E, inp.B, inp.indices,  # noqa: E731
                                             inp.offsets, 0, nthreads=1)
    med1, runs1 = cpu_time(fn1, args.cpu_seconds / 3, min_runs=1, warm=0)
    return dict(
        value=inp.N / med, unit="lookups/s", cores=nthreads, kind="reference",
        sample=(f"full config-2 batch (N={inp.N} lookups), median of {runs} runs; FBGEMM "
                f"GenerateEmbeddingSpMDMWithStrides<float,int64,int64,float> from the installed "
                f"torch (the CPU kernel fbgemm_gpu's CPU TBE forward wraps), {nthreads} threads "
                f"over (table, 256-bag chunks); 1 thread: {inp.N / med1:.4g} lookups/s "
                f"({runs1} runs); host CPU: {cpu_model()}"),
    )


def bench_nbit(args, dev, config: int):
    import numpy as np
    import torch

    from mx_fbgemm import bench_inputs
    from mx_fbgemm.sparse_types import SparseType, padded_row_size_in_bytes

    log(f"generating config {config} indices")
    inp = bench_inputs.config4() if config == 4 else bench_inputs.config5()
    tys = [SparseType.from_int(t) for t in inp.tys]
    strides = [padded_row_size_in_bytes(D, ty, 16) for D, ty in zip(inp.D, tys)]
    sizes = [E * s for E, s in zip(inp.E, strides)]
    w_off_np = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    W = torch.randint(0, 256, (int(sum(sizes)),), generator=g, device=dev, dtype=torch.uint8)
    for t, ty in enumerate(tys):
        tab = W[w_off_np[t]: w_off_np[t] + sizes[t]].view(inp.E[t], strides[t])
        if ty.is_rowwise_quantized():
            sc = (torch.rand(inp.E[t], generator=g, device=dev) * 9e-3 + 1e-3).half()
            bi = (torch.rand(inp.E[t], generator=g, device=dev) * 0.2 - 0.1).half()
            tab[:, 0:2] = sc.view(torch.uint8).view(-1, 2)
            tab[:, 2:4] = bi.view(torch.uint8).view(-1, 2)
        else:
            v = (torch.rand((inp.E[t], inp.D[t]), generator=g, device=dev) * 0.02 - 0.01).half()
            tab[:, : 2 * inp.D[t]] = v.view(torch.uint8).view(inp.E[t], -1)
    idx = torch.from_numpy(inp.indices).to(dev, torch.int32)
    off = torch.from_numpy(inp.offsets).to(dev, torch.int32)

    def mx(kind):
        return max([D for D, ty in zip(inp.D, tys) if ty == kind], default=0)

    args_ = (W, torch.zeros(0, dtype=torch.uint8, device=dev),
             torch.zeros(inp.T, dtype=torch.int32, device=dev),
             torch.from_numpy(w_off_np).to(dev),
             torch.tensor(inp.tys, dtype=torch.uint8, device=dev),
             torch.from_numpy(inp.D_offsets).to(dev), inp.total_D, mx(SparseType.INT2),
             mx(SparseType.INT4), mx(SparseType.INT8), mx(SparseType.FP16), mx(SparseType.FP32),
             idx, off, 1 if config == 4 else 0, None, 1, None, None, 16)
    op = torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function

    def step():
        return op(*args_)

    wall, mean_ms = time_launches(step, args.steps, args.warmup)
    N = inp.N
    unpadded = [strides_u for strides_u in
                [(D + 4) if ty == SparseType.INT8 else (D // 2 + 4) if ty == SparseType.INT4
                 else 2 * D for D, ty in zip(inp.D, tys)]]
    lens = np.diff(inp.offsets).reshape(inp.T, inp.B).sum(1)
    alg_bytes = int(sum(int(lens[t]) * (unpadded[t] + 4) for t in range(inp.T))
                    + inp.B * sum(4 + 2 * D for D in inp.D))
    # Compulsory bytes: every distinct row once, plus indices, offsets and output.
    uniq = [int(np.count_nonzero(np.bincount(
        inp.indices[inp.offsets[t * inp.B]: inp.offsets[(t + 1) * inp.B]], minlength=inp.E[t])))
        for t in range(inp.T)]
    compulsory = int(sum(u * r for u, r in zip(uniq, unpadded)) + N * 4
                     + inp.B * sum(4 + 2 * D for D in inp.D))
    res = dict(
        metric="nbit TBE fwd lookups/sec + achieved HBM GB/s (% of peak), 1 MI355X",
        value=N * args.steps / wall, unit="lookups/s", ms_per_step=wall / args.steps * 1e3,
        dtype="int8/int4 codes, fp32 accumulate, fp16 out" if config == 4 else
        "fp16/int4 codes, fp32 accumulate, fp16 out",
        config={"workload": (f"config{config}: " + (
            "nbit MEAN fp16 out, 16 INT8 + 16 INT4 tables E=1e6 D=128 B=16384 L=20"
            if config == 4 else "mixed nbit SUM fp16 out, 64 tables FP16/INT4 D 32..256 "
            "B=65536 L~Poisson(15) 10% empty Zipf(1.1)")), "T": inp.T, "B": inp.B, "N": N},
        kernel="nbit_fwd_kernel", alg_bytes=alg_bytes, kernel_ms_mean=mean_ms,
        compulsory_bytes=compulsory, unique_rows=int(sum(uniq)),
    )
    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, str(REPO / "oracle"))
        import oracle as orc

        # Bounded sample: the first B_s bags of every table.
        Bs = min(inp.B, 2048)
        sel_off = np.concatenate([inp.offsets[t * inp.B: t * inp.B + Bs] for t in range(inp.T)]
                                 + [[0]])
        idx_parts = [inp.indices[inp.offsets[t * inp.B]: inp.offsets[t * inp.B + Bs]]
                     for t in range(inp.T)]
        sidx = np.concatenate(idx_parts).astype(np.int64)
        lens_s = np.concatenate([np.diff(inp.offsets[t * inp.B: t * inp.B + Bs + 1])
                                 for t in range(inp.T)])
        soff = bench_inputs.offsets_from_lengths(lens_s)
        del sel_off
        log("CPU baseline: copying nbit weights to host")
        Wh = W.cpu().numpy()
        nthreads = orc.host_threads()
        fn = lambda: orc.fbgemm_nbit_forward(Wh, w_off_np, inp.tys, inp.D_offsets, inp.E, Bs,  # noqa: E731
                                             sidx, soff, 1 if config == 4 else 0,
                                             nthreads=nthreads)
        med, runs = cpu_time(fn, args.cpu_seconds)
        cpu = dict(value=sidx.size / med, unit="lookups/s", cores=nthreads, kind="reference",
                   sample=(f"first {Bs} bags of every table ({sidx.size} lookups), median of "
                           f"{runs} runs; FBGEMM 8-bit/N-bit/fp16 SpMDM CPU kernels "
                           f"(scale_bias_last=false) from the installed torch, {nthreads} "
                           f"threads; host CPU: {cpu_model()}"))
    return res, traffic_from_profile(f"nbit_fwd_config{config}"), cpu


def bench_backward(args, dev):
    import numpy as np
    import torch

    from mx_fbgemm import bench_inputs

    log("generating config 3 (config-2 indices)")
    inp = bench_inputs.config2()
    T, E, D, B = inp.T, inp.E[0], inp.D[0], inp.B
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    W = torch.empty(T * E * D, device=dev).uniform_(-0.01, 0.01, generator=g)
    m1 = torch.zeros(T * E, device=dev)
    grad = torch.randn((B, inp.total_D), generator=g, device=dev) * 1e-2
    w_off = torch.arange(T, device=dev, dtype=torch.int64) * (E * D)
    m_off = torch.arange(T, device=dev, dtype=torch.int64) * E
    D_off = torch.from_numpy(inp.D_offsets).to(dev)
    hsc = torch.from_numpy(inp.hash_size_cumsum).to(dev)
    idx = torch.from_numpy(inp.indices).to(dev)
    off = torch.from_numpy(inp.offsets).to(dev)
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(T, dtype=torch.int32, device=dev)
    e32 = torch.zeros(0, dtype=torch.int32, device=dev)
    op = torch.ops.fbgemm.split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_cuda

    def step():
        op(grad, W, empty, empty, pl, w_off, D_off, D, hsc, inp.total_hash_size_bits, idx, off, 0,
           e32, 0, 0, False, m1, empty, pl, m_off, 1e-8, 0.01, 0.0, 0, 0.0)

    wall, mean_ms = time_launches(step, args.steps, args.warmup)
    U = int(np.unique(inp.hash_size_cumsum[np.repeat(np.arange(T), np.diff(inp.offsets[::B]))]
                      + inp.indices).size)
    alg = inp.N * 8 + (T * B + 1) * 8 + B * inp.total_D * 4 + U * (2 * D * 4 + 2 * 4)
    res = dict(
        metric="TBE backward + exact rowwise Adagrad lookups/sec, 1 MI355X",
        value=inp.N * args.steps / wall, unit="lookups/s", ms_per_step=wall / args.steps * 1e3,
        dtype="fp32",
        config={"workload": "config3: TBE backward + exact rowwise Adagrad on config-2 shapes",
                "T": T, "E": E, "D": D, "B": B, "N": inp.N, "unique_rows": U},
        kernel="whole backward (transpose + segment reduce + update)", alg_bytes=alg,
        kernel_ms_mean=mean_ms,
    )
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_backward(args, inp, W, grad)
    return res, traffic_from_profile("tbe_bwd_config3"), cpu


def cpu_baseline_backward(args, inp, W, grad):
    """The C restatement of the backward (stable merge sort of the linearized
    keys, per-row sum in sorted order, rowwise Adagrad), one thread, in place
    on host copies of the weights and gradient."""
    import numpy as np

    sys.path.insert(0, str(REPO / "oracle"))
    import oracle as orc

    log("CPU baseline: copying weights and gradient to host")
    T, E, D = inp.T, inp.E[0], inp.D[0]
    Wh = W.cpu().numpy()
    gh = grad.cpu().numpy()
    m1h = np.zeros(T * E, dtype=np.float32)
    w_off = (np.arange(T) * E * D).astype(np.int64)
    m_off = (np.arange(T) * E).astype(np.int64)
    fn = lambda: orc.backward_rowwise_adagrad(  # noqa: E731
        Wh, w_off, inp.D_offsets, inp.B, inp.hash_size_cumsum, inp.total_hash_size_bits,
        inp.indices, inp.offsets, 0, gh, m1h, m_off, 0.01, 1e-8, inplace=True)
    log("CPU baseline: C restatement of the backward, 1 thread")
    med, runs = cpu_time(fn, args.cpu_seconds)
    return dict(
        value=inp.N / med, unit="lookups/s", cores=1, kind="port",
        sample=(f"full config-3 batch (N={inp.N} lookups), median of {runs} runs; the oracle's C "
                f"restatement (stable merge sort + segment sum + rowwise Adagrad), one thread, "
                f"in place; host CPU: {cpu_model()}"),
    )


def main():
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (the TBE would "
              "shard table-wise over RCCL all-to-all; see the design notes). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    import torch

    import mx_fbgemm  # noqa: F401

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    if args.copy_calibration:
        src = torch.ones(1 << 28, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel() * 4, "copy_bytes_written": dst.numel() * 4,
                          "launches": args.steps}))
        return
    if args.config == 1:
        res, traffic, cpu = bench_jagged(args, dev)
    elif args.config == 2 and args.op == "bounds-check":
        res, traffic, cpu = bench_bounds_check(args, dev)
    elif args.config == 2:
        res, traffic, cpu = bench_tbe_forward(args, dev)
    elif args.config == 3:
        res, traffic, cpu = bench_backward(args, dev)
    else:
        res, traffic, cpu = bench_nbit(args, dev, args.config)
    achieved = res["alg_bytes"] / (res["kernel_ms_mean"] * 1e-3) / 1e9
    line = dict(
        metric=res["metric"], value=res["value"], unit=res["unit"], n_gpus=1, steps=args.steps,
        warmup=args.warmup, ms_per_step=res["ms_per_step"], higher_is_better=True,
        scaling="weak", vs_baseline=None, dtype=res["dtype"], data="synthetic",
        config=res["config"],
        roofline=dict(bound="hbm", achieved=achieved, peak=PEAK_HBM_GBS, unit="GB/s",
                      frac=achieved / PEAK_HBM_GBS, traffic=traffic,
                      kernel=res["kernel"], alg_bytes_per_launch=res["alg_bytes"],
                      launch_ms_mean=res["kernel_ms_mean"]),
        cpu_baseline=cpu,
    )
    if "cold_kernel_ms_median" in res:
        line["roofline"]["cold_launch_ms_median"] = res["cold_kernel_ms_median"]
    if "fresh_batches" in res:
        line["roofline"]["fresh_batches"] = res["fresh_batches"]
    if "compulsory_bytes" in res:
        # The same launch against only the bytes no cache can serve: each
        # distinct row once, plus indices, offsets and output.
        comp = res["compulsory_bytes"] / (res["kernel_ms_mean"] * 1e-3) / 1e9
        line["roofline"].update(compulsory_bytes=res["compulsory_bytes"],
                                unique_rows=res["unique_rows"], compulsory_GBps=comp,
                                compulsory_frac=comp / PEAK_HBM_GBS)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
