#!/usr/bin/env python3
"""Benchmark of the TBE hot path on one MI355X.

Default workload (config 2): TBE fp32 forward, SUM pooling, T=8 tables of
E=1,000,000 x D=128, B=4096 bags per table, pooling factor U{1..40}, int64
indices Zipf(1.05) with a per-table permutation (seeded synthetic data; the
weights are generated on the device).  One step = one
torch.ops.fbgemm.split_embedding_codegen_forward_unweighted_cuda call over
one batch, inputs resident in HBM; the timed steps walk a rotation of 8
batches of the same tables (the same hot rows, fresh draws), as successive
training batches do.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config {1,2,3,4,5}]
                    [--op {lookup,bounds-check}] [--regime {all,steps,warm,cold}]

Prints one JSON line.  `value` is lookups/s over the K timed steps.  The
roofline of the dominant kernel is taken from COLD-cache launches: before
each of `--cold-launches` groups a 1 GiB buffer is written and read (well
past the 256 MB Infinity Cache and the L2s), then `--cold-copies` launches of
batch 0, each over its own copy of the inputs, run back to back inside one
pair of HIP events on the stream they run on; `achieved` = the bytes a
launch must move from HBM / the median per-launch time (group time / group
size), so it is an HBM figure: the
algorithmic bytes (per-unit figure x units), except for Zipf batches (configs
2 and 5), whose per-lookup count re-reads the hot rows that the L2 serves
within a launch even from cold; there it is the compulsory bytes (each
distinct row once + indices, offsets, output).  The per-lookup rate, repeated
launches of one batch ("warm") and the rotation ("steps") are reported as
effective rates: caches serve part of them, so they are no HBM bandwidth.  The CPU
baseline is FBGEMM's CPU kernel (or the C restatement) on this host's cores.
The default run also carries a `config4` record (nbit INT8/INT4 lookup) with
its own roofline and CPU baseline, and `config1`, `config3` and `config5`
records (jagged round trip, backward + rowwise Adagrad, mixed nbit lookup),
each measured the same way in the same process.

--regime runs one regime only (for profiling: every launch of the kernel in
the process then belongs to it): `steps` the rotation, `warm` batch 0
repeated, `cold` flushed launches of batch 0.
"""

from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable, Optional

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "torchlib-xpu_amd"))

PEAK_HBM_GBS = 8000.0
FLUSH_BYTES = 1 << 30


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 200 steps: the wall clock's fixed start and synchronisation latency
    # (~50 us) stays under 1 % of the timed region even for config 2's ~34 us steps.
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5],
                    help="workload; 2 (default) is the headline")
    ap.add_argument("--op", default="lookup", choices=["lookup", "bounds-check", "nobag", "permute"],
                    help="bounds-check (config 2): time bounds_check_indices (WARNING) on the "
                         "batch instead of the lookup; nobag (config 2 / 3): the PoolingMode NONE "
                         "forward / backward on the same batch (not the headline)")
    ap.add_argument("--regime", default="all", choices=["all", "steps", "warm", "cold"])
    ap.add_argument("--cold-launches", type=int, default=25,
                    help="flushes (groups of --cold-copies launches) whose median launch "
                         "time gives the roofline")
    ap.add_argument("--warm-groups", type=int, default=100,
                    help="groups of --cold-copies launches of batch 0 whose median gives the "
                         "warm launch time")
    ap.add_argument("--cold-copies", type=int, default=4,
                    help="launches timed back to back after each flush, each over its own "
                         "copy of the inputs")
    ap.add_argument("--no-config4", action="store_true",
                    help="config 2 only: leave out the config-4, -1, -3 and -5 records "
                         "(only the --config line)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 1 GiB device copy (PMC byte-counter calibration)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="bound on each CPU baseline's timed work")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# provenance and committed profile figures


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def provenance() -> dict:
    import torch

    return dict(torch_version=torch.__version__, torch_git=torch.version.git_version,
                hip=torch.version.hip, host_cpu=cpu_model(), host_nproc=os.cpu_count(),
                host_affinity=len(os.sched_getaffinity(0)))


def traffic_from_profile(name: str) -> tuple[Optional[float], Optional[str]]:
    """HBM bytes per cold launch recorded by the committed rocprofv3 PMC
    summary (FETCH_SIZE and WRITE_SIZE runs of `bench.py --regime cold`)."""
    p = REPO / "profiles" / f"{name}.md"
    if not p.exists():
        return None, None
    m = re.search(r"traffic_bytes_per_launch_cold:\s*([0-9.eE+]+)", p.read_text())
    if not m:
        return None, None
    return float(m.group(1)), (f"profiles/{name}.md: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE "
                               f"runs of bench.py --regime cold, calibrated by a 1 GiB copy")


# ---------------------------------------------------------------------------
# timing


def time_steps(fns: list[Callable], steps: int, warmup: int):
    """Calls fns[i % len(fns)] for `warmup` untimed steps, then times exactly
    `steps` steps back to back, synchronised on both sides.  Returns (wall
    seconds, mean step in ms from one pair of HIP events around the steps on
    the current stream, which the ops launch on).  No event sits between
    steps: an event record between launches adds GPU time that is not the
    op's."""
    import torch

    for i in range(warmup):
        fns[i % len(fns)]()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for i in range(steps):
        fns[i % len(fns)]()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, start.elapsed_time(end) / steps


def time_groups(fn: Callable, groups: int, per_group: int, warmup: int) -> list[float]:
    """Warm launches: `groups` groups of `per_group` launches of fn back to
    back, one pair of HIP events per group on the current stream, no
    synchronisation between groups.  Returns per-launch durations in ms (group
    time / per_group), one per group."""
    import torch

    for _ in range(warmup):
        fn()
    evs = []
    for _ in range(groups):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(per_group):
            fn()
        e.record()
        evs.append((s, e))
    torch.cuda.synchronize()
    return [s.elapsed_time(e) / per_group for s, e in evs]


def time_cold(fns: list[Callable], launches: int, warmup: int, dev) -> list[float]:
    """Cold launches: a write and then a read of a 1 GiB buffer empty the L2s
    and the 256 MB Infinity Cache of the inputs and leave only clean lines (a
    write-only flush leaves dirty lines whose write-back would land inside the
    timed launches); then the len(fns) launches, each over its own copy of the
    inputs, so each finds none of its inputs in any cache, run back to back
    inside one HIP event pair on the current stream (one pair per launch would
    also time the dispatch gap after the flush).  Returns `launches` per-launch
    durations in ms, each the mean over one such group."""
    import torch

    flush = torch.empty(FLUSH_BYTES // 4, device=dev, dtype=torch.float32)
    evs = []
    for i in range(warmup + launches):
        flush.fill_(float(i))
        flush.sum()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for fn in fns:
            fn()
        e.record()
        if i >= warmup:
            evs.append((s, e))
    torch.cuda.synchronize()
    del flush
    return [s.elapsed_time(e) / len(fns) for s, e in evs]


def cpu_time(fn, budget_s: float, min_runs: int = 3, warm: int = 1):
    """Median of at least `min_runs` (up to 10) runs within about `budget_s`."""
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


# ---------------------------------------------------------------------------
# workloads


@dataclass
class Workload:
    metric: str
    unit: str                       # what `value` counts per second
    steps: list[Callable]           # one callable per batch of the rotation
    units: list[float]              # the unit count of each batch (lookups, or bytes)
    alg_bytes: list[float]          # algorithmic bytes of each batch
    dtype: str
    config: dict
    kernel: str                     # the dominant kernel(s) one step launches
    profile: str                    # profiles/<profile>.md
    cpu: Optional[Callable] = None  # -> cpu_baseline dict
    extra: dict = field(default_factory=dict)
    # Bytes of batch 0 the roofline divides by the cold launch time, when not
    # alg_bytes[0]: for Zipf batches, the compulsory bytes (each distinct row
    # once, plus indices, offsets and output).  The per-lookup count re-reads
    # the Zipf head, which the L2 serves within a launch even from cold, so it
    # is no HBM quantity.
    roof_bytes: Optional[float] = None
    roof_bytes_kind: str = "algorithmic bytes per launch (per-unit figure x units)"
    # Launches of batch 0 over disjoint copies of its inputs (the cold regime
    # times them back to back after each flush); defaults to steps[0] alone.
    cold_steps: Optional[list[Callable]] = None


def run_workload(args, wl: Workload, dev) -> dict:
    """Times the regimes `args.regime` asks for; returns the bench record."""
    regimes = ["steps", "warm", "cold"] if args.regime == "all" else [args.regime]
    rec: dict = {}
    eff: dict = {}
    n_b = len(wl.steps)
    if "steps" in regimes:
        log(f"timing {args.steps} steps over {n_b} batch(es) in rotation")
        wall, ev_ms = time_steps(wl.steps, args.steps, args.warmup)
        units = sum(wl.units[i % n_b] for i in range(args.steps))
        alg = sum(wl.alg_bytes[i % n_b] for i in range(args.steps)) / args.steps
        rec.update(value=units / wall, ms_per_step=wall / args.steps * 1e3)
        eff["steps"] = dict(batches=n_b, launch_ms_mean=ev_ms,
                            effective_GBps=alg / (ev_ms * 1e-3) / 1e9,
                            note="HIP events around the K timed steps (the batch rotation); "
                                 "caches serve repeated rows, so not an HBM figure")
    if "warm" in regimes:
        log("timing batch 0 repeated (warm caches)")
        _, warm_ms = time_steps(wl.steps[:1], args.steps, args.warmup)
        per = args.cold_copies
        warm = sorted(time_groups(wl.steps[0], args.warm_groups, per, args.warmup))
        wmed = statistics.median(warm)
        eff["warm"] = dict(launch_ms_mean=warm_ms, launch_ms_median=wmed,
                           launch_ms_p10=warm[len(warm) // 10],
                           launch_ms_p90=warm[(len(warm) * 9) // 10],
                           groups=len(warm), launches_per_group=per,
                           effective_GBps=wl.alg_bytes[0] / (wmed * 1e-3) / 1e9,
                           units_per_s=wl.units[0] / (wmed * 1e-3),
                           note="batch 0 launched back to back: its distinct rows stay in the "
                                "L2s and the Infinity Cache, so not an HBM figure; median over "
                                "groups, mean over the K steps")
        if "value" not in rec:
            rec.update(value=wl.units[0] / (warm_ms * 1e-3), ms_per_step=warm_ms)
    roof = None
    if "cold" in regimes:
        cold_fns = wl.cold_steps or wl.steps[:1]
        log(f"timing {args.cold_launches} x {len(cold_fns)} cold-cache launches of batch 0")
        cold = time_cold(cold_fns, args.cold_launches, min(args.warmup, 3), dev)
        med = statistics.median(cold)
        nbytes = wl.roof_bytes if wl.roof_bytes is not None else wl.alg_bytes[0]
        achieved = nbytes / (med * 1e-3) / 1e9
        traffic, src = traffic_from_profile(wl.profile)
        roof = dict(bound="hbm", achieved=achieved, peak=PEAK_HBM_GBS, unit="GB/s",
                    frac=achieved / PEAK_HBM_GBS, traffic=traffic, traffic_source=src,
                    kernel=wl.kernel, alg_bytes_per_launch=nbytes,
                    alg_bytes_kind=wl.roof_bytes_kind,
                    launch_ms=med, launch_ms_min=min(cold), launch_ms_max=max(cold),
                    regime=(f"cold: median over {len(cold)} groups of {len(cold_fns)} launches of "
                            f"batch 0, each over its own copy of the inputs, back to back after "
                            f"a 1 GiB buffer is written and read; one HIP event pair per "
                            f"group"))
        if wl.roof_bytes is not None:
            eff["cold_per_lookup_bytes"] = dict(
                bytes=wl.alg_bytes[0], effective_GBps=wl.alg_bytes[0] / (med * 1e-3) / 1e9,
                note="every lookup's row counted once per lookup, over the cold launch time: "
                     "the Zipf head is re-read from the L2 within the launch, so this can pass "
                     "the HBM peak and is not an HBM figure")
        if "value" not in rec:
            rec.update(value=wl.units[0] / (med * 1e-3), ms_per_step=med)
    rec.update(roofline=roof, effective=eff)
    rec.update(wl.extra)
    return rec


def make_line(args, wl: Workload, rec: dict, cpu) -> dict:
    return dict(
        metric=wl.metric, value=rec["value"], unit=wl.unit, n_gpus=1, steps=args.steps,
        warmup=args.warmup, ms_per_step=rec["ms_per_step"], higher_is_better=True,
        scaling="weak", vs_baseline=None, dtype=wl.dtype, data="synthetic",
        config=wl.config, roofline=rec["roofline"], effective=rec["effective"],
        **{k: v for k, v in rec.items()
           if k not in ("value", "ms_per_step", "roofline", "effective")},
        cpu_baseline=cpu,
    )


def cpu_record(value, unit, cores, kind, sample) -> dict:
    return dict(value=value, unit=unit, cores=cores, kind=kind, sample=sample, **provenance())


# -- config 1 ----------------------------------------------------------------


def wl_jagged(args, dev) -> Workload:
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

    def make_step(vv, oo):
        return lambda: d2j(j2pd(vv, [oo], [L], 0.0), [oo], total)

    step = make_step(v, off)
    cold = [make_step(v.clone(), off.clone()) for _ in range(args.cold_copies)]
    # j2pd reads the values and writes the padded dense; d2j reads the dense at
    # the jagged positions and writes the values; both read the offsets.
    alg = total * D * 4 + B * L * D * 4 + 2 * total * D * 4 + 2 * (B + 1) * 8

    def cpu():
        vc, oc = v.cpu(), off.cpu()

        def cpu_step():
            dense = torch.ops.aten._jagged_to_padded_dense_forward(vc, [oc], [L], 0.0)
            return torch.ops.aten._padded_dense_to_jagged_forward(dense, [oc], total)

        med, runs = cpu_time(cpu_step, args.cpu_seconds)
        n = torch.get_num_threads()
        return cpu_record(alg / med / 1e9, "GB/s", n, "reference",
                          f"full config-1 round trip, median of {runs} runs; torch's CPU "
                          f"aten._jagged_to_padded_dense_forward / _padded_dense_to_jagged_forward "
                          f"(its port of the fbgemm jagged ops) on {n} threads")

    return Workload(
        metric="jagged round trip (jagged_to_padded_dense + dense_to_jagged) bytes/s, 1 MI355X",
        unit="GB/s", steps=[step], units=[alg / 1e9], alg_bytes=[alg], dtype="fp32",
        config={"workload": "config1: jagged round trip, B=512 D=128 max_L=64, len~U{0..64}",
                "B": B, "D": D, "max_L": L, "total_L": total},
        kernel="j2pd1_kernel + jagged_out1_kernel (one round trip)", profile="jagged_config1",
        cpu=cpu, cold_steps=cold)


# -- config 2 ----------------------------------------------------------------


def wl_tbe_forward(args, dev) -> Workload:
    import numpy as np
    import torch

    from mx_fbgemm import bench_inputs

    log("generating 8 config-2 batches (batch 0 is the seed-0 config)")
    batches = bench_inputs.config2_batches(8)
    inp = batches[0]
    T, E, D, B = inp.T, inp.E[0], inp.D[0], inp.B
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    W = torch.empty(T * E * D, device=dev).uniform_(-0.01, 0.01, generator=g)
    w_off = torch.arange(T, device=dev, dtype=torch.int64) * (E * D)
    D_off = torch.from_numpy(inp.D_offsets).to(dev)
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(T, dtype=torch.int32, device=dev)
    e32 = torch.zeros(0, dtype=torch.int32, device=dev)
    op = torch.ops.fbgemm.split_embedding_codegen_forward_unweighted_cuda

    def make_step(b, Wc):
        idx = torch.from_numpy(b.indices).to(dev)
        off = torch.from_numpy(b.offsets).to(dev)
        return lambda: op(Wc, empty, empty, pl, w_off, D_off, inp.total_D, D, idx, off, 0, e32,
                          empty, 0, False)

    steps = [make_step(b, W) for b in batches]
    cold = [make_step(inp, W.clone()) for _ in range(args.cold_copies)]
    # Per lookup: the row and its index; per bag: its offset and output row.
    alg = [b.N * (D * 4 + 8) + T * B * (8 + D * 4) for b in batches]
    # Compulsory bytes of batch 0: every distinct row once (the Zipf heads repeat).
    t_of = np.repeat(np.arange(T * B) // B, np.diff(inp.offsets))
    uniq = int(np.unique(t_of * E + inp.indices).size)
    compulsory = uniq * D * 4 + inp.N * 8 + (T * B + 1) * 8 + T * B * D * 4

    def cpu():
        sys.path.insert(0, str(REPO / "oracle"))
        import oracle as orc

        log("CPU baseline: copying weights to host")
        Wh = W.cpu().numpy()
        w_off_h = (np.arange(T) * E * D).astype(np.int64)
        nthreads = orc.host_threads()
        fn = lambda: orc.fbgemm_tbe_forward_f32(Wh, w_off_h, inp.D_offsets, inp.E, B,  # noqa: E731
                                                inp.indices, inp.offsets, 0, nthreads=nthreads)
        log(f"CPU baseline: FBGEMM SpMDM on {nthreads} threads")
        med, runs = cpu_time(fn, args.cpu_seconds)
        fn1 = lambda: orc.fbgemm_tbe_forward_f32(Wh, w_off_h, inp.D_offsets, inp.E, B,  # noqa: E731
                                                 inp.indices, inp.offsets, 0, nthreads=1)
        med1, runs1 = cpu_time(fn1, args.cpu_seconds / 3, min_runs=1, warm=0)
        return cpu_record(
            inp.N / med, "lookups/s", nthreads, "reference",
            f"full config-2 batch 0 (N={inp.N} lookups), median of {runs} runs; FBGEMM "
            f"GenerateEmbeddingSpMDMWithStrides<float,int64,int64,float> from the installed "
            f"torch (the CPU kernel fbgemm_gpu's CPU TBE forward wraps), {nthreads} threads "
            f"over (table, 256-bag chunks); 1 thread: {inp.N / med1:.4g} lookups/s ({runs1} runs)")

    return Workload(
        metric="TBE fwd lookups/sec + achieved HBM GB/s (% of peak), 1 MI355X",
        unit="lookups/s", steps=steps, units=[b.N for b in batches], alg_bytes=alg,
        dtype="fp32",
        config={"workload": "config2: TBE fp32 forward SUM, T=8 E=1e6 D=128 B=4096 "
                            "L~U{1..40} Zipf(1.05) int64 indices; timed steps rotate over 8 "
                            "batches of the same tables (same hot rows, fresh draws)",
                "T": T, "E": E, "D": D, "B": B, "N_batch0": inp.N,
                "N_mean": sum(b.N for b in batches) / len(batches), "indices": "int64"},
        kernel="tbe_fwd_group_kernel", profile="tbe_fwd_config2", cpu=cpu, cold_steps=cold,
        roof_bytes=compulsory,
        roof_bytes_kind=("compulsory bytes of batch 0: its distinct rows once (D*4 each) + "
                         "indices (8 B) + offsets (8 B per bag) + output (D*4 per bag)"),
        extra=dict(compulsory=dict(bytes=compulsory, unique_rows=uniq)))


def wl_bounds_check(args, dev) -> Workload:
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

    def make_cold(ic, oc):
        return lambda: op(rows, ic, oc, 1, warn)

    cold = [make_cold(idx.clone(), off.clone()) for _ in range(args.cold_copies)]

    def cpu():
        sys.path.insert(0, str(REPO / "oracle"))
        import oracle as orc

        assert int(warn.item()) == 0, "the config-2 batch is valid"
        rows_h = np.asarray(inp.E, dtype=np.int64)
        fn = lambda: orc.bounds_check_indices(rows_h, inp.indices, inp.offsets, 1)  # noqa: E731
        log("CPU baseline: C restatement of the bounds check, 1 thread")
        med, runs = cpu_time(fn, args.cpu_seconds)
        return cpu_record(inp.N / med, "lookups/s", 1, "port",
                          f"full config-2 batch (N={inp.N}), median of {runs} runs; the "
                          f"oracle's C restatement, one thread, including its copies of "
                          f"indices and offsets")

    return Workload(
        metric="bounds_check_indices lookups/sec, 1 MI355X", unit="lookups/s", steps=[step],
        units=[inp.N], alg_bytes=[inp.N * 8 + (inp.T * inp.B + 1) * 8], dtype="int64",
        config={"workload": "config2 batch: bounds_check_indices, WARNING mode", "T": inp.T,
                "B": inp.B, "N": inp.N},
        kernel="tile_max_kernel + bounds_main_kernel", profile="bounds_check_config2", cpu=cpu,
        cold_steps=cold)


def wl_nobag_forward(args, dev) -> Workload:
    """PoolingMode NONE forward on the config-2 batch: every position's row
    copied to its own output row ([N, 128] fp32)."""
    import numpy as np
    import torch

    from mx_fbgemm import bench_inputs

    log("generating config 2 batch")
    inp = bench_inputs.config2()
    T, E, D, B = inp.T, inp.E[0], inp.D[0], inp.B
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    W = torch.empty(T * E * D, device=dev).uniform_(-0.01, 0.01, generator=g)
    w_off = torch.arange(T, device=dev, dtype=torch.int64) * (E * D)
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(T, dtype=torch.int32, device=dev)
    e32 = torch.zeros(0, dtype=torch.int32, device=dev)
    op = torch.ops.fbgemm.split_embedding_nobag_codegen_forward_unweighted_cuda

    def make_step(Wc, ic, oc):
        return lambda: op(Wc, empty, empty, pl, w_off, D, ic, oc, e32, empty, 0, False)

    idx = torch.from_numpy(inp.indices).to(dev)
    off = torch.from_numpy(inp.offsets).to(dev)
    step = make_step(W, idx, off)
    cold = [make_step(W.clone(), idx.clone(), off.clone()) for _ in range(args.cold_copies)]
    alg = inp.N * (D * 4 + 8 + D * 4)
    t_of = np.repeat(np.arange(T * B) // B, np.diff(inp.offsets))
    uniq = int(np.unique(t_of * E + inp.indices).size)
    compulsory = uniq * D * 4 + inp.N * 8 + (T * B + 1) * 8 + inp.N * D * 4

    def cpu():
        sys.path.insert(0, str(REPO / "oracle"))
        import oracle as orc

        Wh = W.cpu().numpy()
        w_off_h = (np.arange(T) * E * D).astype(np.int64)
        fn = lambda: orc.tbe_forward_nobag(Wh, w_off_h, D, B, inp.indices, inp.offsets)  # noqa: E731
        log("CPU baseline: numpy gather of the nobag oracle, 1 process")
        med, runs = cpu_time(fn, args.cpu_seconds)
        return cpu_record(inp.N / med, "lookups/s", 1, "port",
                          f"full config-2 batch (N={inp.N}), median of {runs} runs; the "
                          f"oracle's numpy gather (one process)")

    return Workload(
        metric="TBE nobag fwd lookups/sec, 1 MI355X", unit="lookups/s", steps=[step],
        units=[inp.N], alg_bytes=[alg], dtype="fp32",
        config={"workload": "config2 batch, PoolingMode NONE forward: out [N, 128] fp32",
                "T": T, "E": E, "D": D, "B": B, "N": inp.N},
        kernel="tbe_fwd_nobag_kernel", profile="tbe_fwd_nobag_config2", cpu=cpu,
        cold_steps=cold, roof_bytes=compulsory,
        roof_bytes_kind=("compulsory bytes: distinct rows once (D*4) + indices + offsets + "
                         "one output row (D*4) per position"),
        extra=dict(compulsory=dict(bytes=compulsory, unique_rows=uniq)))


def wl_permute(args, dev) -> Workload:
    """permute_2D_sparse_data on the config-2 batch (lengths [8, 4096] int64,
    668k int64 indices, no weights): the features in reverse order, with
    permuted_lengths_sum given (no host sync), as a caller reorders a batch's
    features into its tables' order before the lookup."""
    import numpy as np
    import torch

    from mx_fbgemm import bench_inputs

    log("generating config 2 batch")
    inp = bench_inputs.config2()
    T, B, N = inp.T, inp.B, inp.N
    lengths_h = np.diff(inp.offsets).reshape(T, B)
    perm_h = np.arange(T - 1, -1, -1, dtype=np.int32)
    op = torch.ops.fbgemm.permute_2D_sparse_data

    def make_step(pc, lc, ic):
        return lambda: op(pc, lc, ic, None, N)

    perm = torch.from_numpy(perm_h).to(dev)
    lengths = torch.from_numpy(lengths_h).to(dev)
    idx = torch.from_numpy(inp.indices).to(dev)
    step = make_step(perm, lengths, idx)
    cold = [make_step(perm.clone(), lengths.clone(), idx.clone()) for _ in range(args.cold_copies)]
    # indices read and written once, lengths read and written once
    compulsory = 2 * N * 8 + 2 * T * B * 8

    def cpu():
        sys.path.insert(0, str(REPO / "oracle"))
        import oracle as orc

        fn = lambda: orc.permute_2d_sparse_data(perm_h, lengths_h, inp.indices)  # noqa: E731
        log("CPU baseline: numpy feature permute of the oracle, 1 process")
        med, runs = cpu_time(fn, args.cpu_seconds)
        return cpu_record(N / med, "indices/s", 1, "port",
                          f"full config-2 batch (N={N}), median of {runs} runs; the oracle's "
                          f"numpy permute (one process)")

    return Workload(
        metric="permute_2D_sparse_data indices/sec, 1 MI355X", unit="indices/s", steps=[step],
        units=[N], alg_bytes=[compulsory], dtype="int64",
        config={"workload": "config2 batch, permute_2D_sparse_data (features reversed, "
                            "int64 lengths and indices, no weights)", "T": T, "B": B, "N": N},
        kernel="whole op (permuted lengths, two complete cumsums, the copy)",
        profile="permute_2d_config2", cpu=cpu, cold_steps=cold, roof_bytes=compulsory,
        roof_bytes_kind="compulsory bytes: indices and lengths each read and written once")


# -- config 3 ----------------------------------------------------------------


def wl_backward(args, dev) -> Workload:
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

    def make_step(Wc, mc, gc, ic, oc):
        return lambda: op(gc, Wc, empty, empty, pl, w_off, D_off, D, hsc, inp.total_hash_size_bits,
                          ic, oc, 0, e32, 0, 0, False, mc, empty, pl, m_off, 1e-8, 0.01, 0.0, 0,
                          0.0)

    step = make_step(W, m1, grad, idx, off)
    cold = [make_step(W.clone(), m1.clone(), grad.clone(), idx.clone(), off.clone())
            for _ in range(args.cold_copies)]

    U = int(np.unique(inp.hash_size_cumsum[np.repeat(np.arange(T), np.diff(inp.offsets[::B]))]
                      + inp.indices).size)
    alg = inp.N * 8 + (T * B + 1) * 8 + B * inp.total_D * 4 + U * (2 * D * 4 + 2 * 4)

    def cpu():
        """The multithreaded C++ restatement of the backward (key ranges split
        over the host's threads; per range a sort of (key, position), then
        each run's sum in position order and its rowwise-Adagrad update), in
        place on host copies of the weights and gradient; bit-identical to the
        single-threaded C restatement, which is timed beside it."""
        sys.path.insert(0, str(REPO / "oracle"))
        import oracle as orc

        log("CPU baseline: copying weights and gradient to host")
        Wh = W.cpu().numpy()
        gh = grad.cpu().numpy()
        m1h = np.zeros(T * E, dtype=np.float32)
        w_off_h = (np.arange(T) * E * D).astype(np.int64)
        m_off_h = (np.arange(T) * E).astype(np.int64)
        nthreads = orc.host_threads()
        fn = lambda: orc.backward_rowwise_adagrad_mt(  # noqa: E731
            Wh, w_off_h, inp.D_offsets, B, inp.hash_size_cumsum, inp.total_hash_size_bits,
            inp.indices, inp.offsets, 0, gh, m1h, m_off_h, 0.01, 1e-8, inplace=True,
            nthreads=nthreads)
        log(f"CPU baseline: C++ restatement of the backward, {nthreads} threads")
        med, runs = cpu_time(fn, args.cpu_seconds)
        fn1 = lambda: orc.backward_rowwise_adagrad(  # noqa: E731
            Wh, w_off_h, inp.D_offsets, B, inp.hash_size_cumsum, inp.total_hash_size_bits,
            inp.indices, inp.offsets, 0, gh, m1h, m_off_h, 0.01, 1e-8, inplace=True)
        log("CPU baseline: C restatement of the backward, 1 thread")
        med1, runs1 = cpu_time(fn1, args.cpu_seconds / 3, min_runs=1, warm=0)
        return cpu_record(inp.N / med, "lookups/s", nthreads, "port",
                          f"full config-3 batch (N={inp.N} lookups), median of {runs} runs; the "
                          f"multithreaded C++ restatement (oracle/backward_mt.cpp: key ranges "
                          f"over {nthreads} threads, sort, per-run sum in position order, "
                          f"rowwise Adagrad; bit-identical to the C restatement), in place; "
                          f"1 thread (the C restatement: stable merge sort + segment sum + "
                          f"update): {inp.N / med1:.4g} lookups/s ({runs1} runs)")

    return Workload(
        metric="TBE backward + exact rowwise Adagrad lookups/sec, 1 MI355X", unit="lookups/s",
        steps=[step], units=[inp.N], alg_bytes=[alg], dtype="fp32",
        config={"workload": "config3: TBE backward + exact rowwise Adagrad on config-2 shapes",
                "T": T, "E": E, "D": D, "B": B, "N": inp.N, "unique_rows": U},
        kernel="whole backward (transpose + segment reduce + update)",
        profile="tbe_bwd_config3", cpu=cpu, cold_steps=cold)


def wl_nobag_backward(args, dev) -> Workload:
    """PoolingMode NONE backward + exact rowwise Adagrad on the config-3
    batch: one gradient row per position ([N, 128] fp32)."""
    import numpy as np
    import torch

    from mx_fbgemm import bench_inputs

    log("generating config 3 batch")
    inp = bench_inputs.config2()
    T, E, D, B = inp.T, inp.E[0], inp.D[0], inp.B
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    W = torch.empty(T * E * D, device=dev).uniform_(-0.01, 0.01, generator=g)
    m1 = torch.zeros(T * E, device=dev)
    grad = torch.randn((inp.N, D), generator=g, device=dev) * 1e-2
    w_off = torch.arange(T, device=dev, dtype=torch.int64) * (E * D)
    m_off = torch.arange(T, device=dev, dtype=torch.int64) * E
    hsc = torch.from_numpy(inp.hash_size_cumsum).to(dev)
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(T, dtype=torch.int32, device=dev)
    e32 = torch.zeros(0, dtype=torch.int32, device=dev)
    op = torch.ops.fbgemm.split_embedding_nobag_backward_codegen_rowwise_adagrad_unweighted_exact_cuda

    def make_step(Wc, mc, gc, ic, oc):
        return lambda: op(gc, Wc, empty, empty, pl, w_off, D, hsc, inp.total_hash_size_bits, ic,
                          oc, e32, 0, 0, False, mc, empty, pl, m_off, 1e-8, 0.01, 0.0, 0, 0.0)

    idx = torch.from_numpy(inp.indices).to(dev)
    off = torch.from_numpy(inp.offsets).to(dev)
    step = make_step(W, m1, grad, idx, off)
    cold = [make_step(W.clone(), m1.clone(), grad.clone(), idx.clone(), off.clone())
            for _ in range(args.cold_copies)]
    U = int(np.unique(inp.hash_size_cumsum[np.repeat(np.arange(T), np.diff(inp.offsets[::B]))]
                      + inp.indices).size)
    alg = inp.N * 8 + (T * B + 1) * 8 + inp.N * D * 4 + U * (2 * D * 4 + 2 * 4)

    def cpu():
        sys.path.insert(0, str(REPO / "oracle"))
        import oracle as orc

        Wh = W.cpu().numpy()
        gh = grad.cpu().numpy()
        w_off_h = (np.arange(T) * E * D).astype(np.int64)
        m_off_h = (np.arange(T) * E).astype(np.int64)
        m1h = np.zeros(T * E, dtype=np.float32)
        fn = lambda: orc.backward_rowwise_adagrad_nobag(  # noqa: E731
            Wh, w_off_h, D, B, inp.hash_size_cumsum, inp.total_hash_size_bits, inp.indices,
            inp.offsets, gh, m1h, m_off_h, 0.01, 1e-8)
        log("CPU baseline: C restatement of the nobag backward, 1 thread")
        med, runs = cpu_time(fn, args.cpu_seconds)
        return cpu_record(inp.N / med, "lookups/s", 1, "port",
                          f"full config-3 batch (N={inp.N}), median of {runs} runs; the "
                          f"oracle's C restatement, one thread, on copies of the weights")

    return Workload(
        metric="TBE nobag backward + exact rowwise Adagrad lookups/sec, 1 MI355X",
        unit="lookups/s", steps=[step], units=[inp.N], alg_bytes=[alg], dtype="fp32",
        config={"workload": "config3 batch, PoolingMode NONE backward: grad_output [N, 128]",
                "T": T, "E": E, "D": D, "B": B, "N": inp.N, "unique_rows": U},
        kernel="whole nobag backward (layout + transpose + segment reduce + update)",
        profile="tbe_bwd_nobag_config3", cpu=cpu, cold_steps=cold)


# -- configs 4 and 5 ---------------------------------------------------------


def wl_nbit(args, dev, config: int) -> Workload:
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

    pooling = 1 if config == 4 else 0
    args_ = (W, torch.zeros(0, dtype=torch.uint8, device=dev),
             torch.zeros(inp.T, dtype=torch.int32, device=dev),
             torch.from_numpy(w_off_np).to(dev),
             torch.tensor(inp.tys, dtype=torch.uint8, device=dev),
             torch.from_numpy(inp.D_offsets).to(dev), inp.total_D, mx(SparseType.INT2),
             mx(SparseType.INT4), mx(SparseType.INT8), mx(SparseType.FP16), mx(SparseType.FP32),
             idx, off, pooling, None, 1, None, None, 16)
    op = torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function

    def step():
        return op(*args_)

    def make_cold(Wc, ic, oc):
        a = (Wc,) + args_[1:12] + (ic, oc) + args_[14:]
        return lambda: op(*a)

    cold = [make_cold(W.clone(), idx.clone(), off.clone()) for _ in range(args.cold_copies)]

    N = inp.N
    unpadded = [(D + 4) if ty == SparseType.INT8 else (D // 2 + 4) if ty == SparseType.INT4
                else 2 * D for D, ty in zip(inp.D, tys)]
    lens = np.diff(inp.offsets).reshape(inp.T, inp.B).sum(1)
    # Per lookup: the unpadded row and its int32 index; per bag: offset + fp16 output row.
    alg = int(sum(int(lens[t]) * (unpadded[t] + 4) for t in range(inp.T))
              + inp.B * sum(4 + 2 * D for D in inp.D))
    uniq = [int(np.count_nonzero(np.bincount(
        inp.indices[inp.offsets[t * inp.B]: inp.offsets[(t + 1) * inp.B]], minlength=inp.E[t])))
        for t in range(inp.T)]
    compulsory = int(sum(u * r for u, r in zip(uniq, unpadded)) + N * 4
                     + inp.B * sum(4 + 2 * D for D in inp.D))
    # What 128-byte line fills make of the rows: each row's lines once per lookup.
    line_bytes = 0
    for t in range(inp.T):
        s = strides[t]
        starts = (np.arange(128 // np.gcd(s, 128)) * s) % 128
        lines = ((starts + unpadded[t] + 127) // 128).mean()
        line_bytes += int(lens[t]) * lines * 128
    line_bytes = int(line_bytes + N * 4 + inp.B * sum(4 + 2 * D for D in inp.D))

    def cpu():
        sys.path.insert(0, str(REPO / "oracle"))
        import oracle as orc

        # Bounded sample: the first Bs bags of every table.
        Bs = min(inp.B, 2048)
        idx_parts = [inp.indices[inp.offsets[t * inp.B]: inp.offsets[t * inp.B + Bs]]
                     for t in range(inp.T)]
        sidx = np.concatenate(idx_parts).astype(np.int64)
        lens_s = np.concatenate([np.diff(inp.offsets[t * inp.B: t * inp.B + Bs + 1])
                                 for t in range(inp.T)])
        soff = bench_inputs.offsets_from_lengths(lens_s)
        log("CPU baseline: copying nbit weights to host")
        Wh = W.cpu().numpy()
        nthreads = orc.host_threads()
        fn = lambda: orc.fbgemm_nbit_forward(Wh, w_off_np, inp.tys, inp.D_offsets, inp.E, Bs,  # noqa: E731
                                             sidx, soff, pooling, nthreads=nthreads)
        log(f"CPU baseline: FBGEMM nbit kernels on {nthreads} threads")
        med, runs = cpu_time(fn, args.cpu_seconds)
        return cpu_record(sidx.size / med, "lookups/s", nthreads, "reference",
                          f"first {Bs} bags of every table ({sidx.size} lookups), median of "
                          f"{runs} runs; FBGEMM 8-bit/N-bit/fp16 SpMDM CPU kernels "
                          f"(scale_bias_last=false) from the installed torch, {nthreads} "
                          f"threads")

    workload = (f"config{config}: " + (
        "nbit MEAN fp16 out, 16 INT8 + 16 INT4 tables E=1e6 D=128 B=16384 L=20 uniform int32 "
        "indices" if config == 4 else "mixed nbit SUM fp16 out, 64 tables FP16/INT4 D 32..256 "
        "B=65536 L~Poisson(15) 10% empty Zipf(1.1)"))
    return Workload(
        metric="nbit TBE fwd lookups/sec + achieved HBM GB/s (% of peak), 1 MI355X",
        unit="lookups/s", steps=[step], units=[N], alg_bytes=[alg],
        dtype="int8/int4 codes, fp32 accumulate, fp16 out" if config == 4 else
        "fp16/int4 codes, fp32 accumulate, fp16 out",
        config={"workload": workload, "T": inp.T, "B": inp.B, "N": N},
        kernel="nbit_fwd_kernel (one launch per table type present)",
        profile=f"nbit_fwd_config{config}", cpu=cpu, cold_steps=cold,
        # Config 5 draws Zipf indices (the per-lookup count re-reads the hot
        # rows); config 4's are uniform over 3.6 GB of rows, where a repeated
        # row is long evicted when it comes again, so every lookup is HBM traffic.
        roof_bytes=compulsory if config == 5 else None,
        roof_bytes_kind=("compulsory bytes: distinct rows once (unpadded) + int32 indices + "
                         "offsets + fp16 output" if config == 5 else
                         "algorithmic bytes: every lookup's unpadded row + its int32 index, "
                         "per bag its offset + fp16 output row"),
        extra=dict(compulsory=dict(bytes=compulsory, unique_rows=int(sum(uniq))),
                   line_fill=dict(bytes=line_bytes,
                                  frac_at_peak_alg=alg / line_bytes,
                                  note="rows fetched as whole 128-B lines, once per lookup: "
                                       "the algorithmic fraction of peak this traffic allows")))


# ---------------------------------------------------------------------------


def measure(args, config: int, dev) -> dict:
    import torch

    if config == 1:
        wl = wl_jagged(args, dev)
    elif config == 2 and args.op == "bounds-check":
        wl = wl_bounds_check(args, dev)
    elif config == 2 and args.op == "nobag":
        wl = wl_nobag_forward(args, dev)
    elif config == 2 and args.op == "permute":
        wl = wl_permute(args, dev)
    elif config == 3 and args.op == "nobag":
        wl = wl_nobag_backward(args, dev)
    elif config == 2:
        wl = wl_tbe_forward(args, dev)
    elif config == 3:
        wl = wl_backward(args, dev)
    else:
        wl = wl_nbit(args, dev, config)
    rec = run_workload(args, wl, dev)
    cpu = None
    if not args.no_cpu_baseline and wl.cpu is not None:
        cpu = wl.cpu()
    line = make_line(args, wl, rec, cpu)
    del wl
    torch.cuda.empty_cache()
    return line


def summary(line: dict) -> dict:
    """Per configuration, the figures the targets are read from, compactly:
    value and ms per step (the timed steps), the cold launch time and its
    fraction of peak HBM, measured traffic over the roofline bytes, and the CPU
    baseline."""
    out = {}
    for c in (1, 2, 3, 4, 5):
        r = line if c == 2 else line.get(f"config{c}")
        if not r:
            continue
        roof = r.get("roofline") or {}
        cpu = r.get("cpu_baseline") or {}
        traffic, nbytes = roof.get("traffic"), roof.get("alg_bytes_per_launch")
        out[f"config{c}"] = dict(
            value=r["value"], unit=r["unit"], ms_per_step=r["ms_per_step"],
            launch_ms_cold=roof.get("launch_ms"), frac=roof.get("frac"),
            traffic_over_roof_bytes=(traffic / nbytes) if traffic and nbytes else None,
            cpu_baseline=cpu.get("value"), cpu_unit=cpu.get("unit"), cpu_cores=cpu.get("cores"))
    return out


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
        src = torch.ones(FLUSH_BYTES // 4, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel() * 4, "copy_bytes_written": dst.numel() * 4,
                          "launches": args.steps}))
        return
    line = measure(args, args.config, dev)
    if args.config == 2 and args.op == "lookup" and not args.no_config4:
        # The second headline target: nbit INT8/INT4 lookup at >= 60 % of HBM.
        c4 = measure(args, 4, dev)
        line["config4"] = {k: c4[k] for k in ("metric", "value", "unit", "ms_per_step", "dtype",
                                              "config", "roofline", "effective", "compulsory",
                                              "line_fill", "cpu_baseline")}
        # The other configurations' records, so that one run observes every target.
        for c in (1, 3, 5):
            rc = measure(args, c, dev)
            line[f"config{c}"] = {k: rc[k] for k in ("metric", "value", "unit", "ms_per_step",
                                                     "dtype", "config", "roofline", "effective",
                                                     "cpu_baseline") if k in rc}
        line["summary"] = summary(line)  # last: a reader of the line's tail sees every config
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
