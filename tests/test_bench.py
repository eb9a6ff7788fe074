"""bench.py's host side (no GPU): it refuses more than one GPU with a
message, and every workload's roofline finds its HBM traffic in the committed
profile summary it names."""

import importlib.util
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PROFILES = ["tbe_fwd_config2", "nbit_fwd_config4", "nbit_fwd_config5", "jagged_config1",
            "tbe_bwd_config3", "bounds_check_config2"]


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("mx_bench", REPO / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules["mx_bench"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.parametrize("gpus", ["2", "8"])
def test_more_than_one_gpu_is_refused(gpus):
    out = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", gpus],
                         capture_output=True, text=True, timeout=120)
    assert out.returncode == 2
    assert "one MI355X" in out.stderr and out.stdout == ""


@pytest.mark.parametrize("name", PROFILES)
def test_profiles_carry_cold_traffic(bench, name):
    traffic, src = bench.traffic_from_profile(name)
    assert traffic is not None and traffic > 0
    assert src.startswith(f"profiles/{name}.md")
    text = (REPO / "profiles" / f"{name}.md").read_text()
    assert "rocprofv3 --pmc FETCH_SIZE" in text and "rocprofv3 --pmc WRITE_SIZE" in text
    assert "rocprofv3 --kernel-trace --stats" in text


def test_missing_profile_gives_no_traffic(bench):
    assert bench.traffic_from_profile("no_such_profile") == (None, None)


def test_summary_holds_every_config(bench):
    """The summary (printed as the line's last key) carries each config's
    value, step time, cold launch, fraction of peak, traffic ratio and CPU
    baseline."""
    def rec(v):
        return dict(value=v, unit="u", ms_per_step=v / 10,
                    roofline=dict(launch_ms=v / 20, frac=0.5, traffic=150.0,
                                  alg_bytes_per_launch=100.0),
                    cpu_baseline=dict(value=v / 100, unit="u", cores=16))
    line = rec(2.0)
    for c in (1, 3, 4, 5):
        line[f"config{c}"] = rec(float(c))
    line["summary"] = bench.summary(line)
    assert list(line)[-1] == "summary"
    s = line["summary"]
    assert sorted(s) == [f"config{c}" for c in (1, 2, 3, 4, 5)]
    assert s["config4"]["ms_per_step"] == 0.4 and s["config4"]["frac"] == 0.5
    assert s["config3"]["cpu_cores"] == 16 and s["config2"]["traffic_over_roof_bytes"] == 1.5
