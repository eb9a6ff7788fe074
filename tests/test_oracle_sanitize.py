"""The C restatement (oracle/mx_oracle.c) under AddressSanitizer and
UndefinedBehaviorSanitizer: oracle/san_driver.c runs every oracle function on
seeded random and edge-case batches (empty bags, no indices, no bags) with
recovery off, so any out-of-bounds access, leak or undefined behaviour in the
checker fails this test."""

import subprocess
import sys
from pathlib import Path

ORACLE = Path(__file__).resolve().parents[1] / "oracle"


def test_oracle_clean_under_asan_and_ubsan():
    subprocess.run(["make", "-C", str(ORACLE), "san", f"PYTHON={sys.executable}"], check=True,
                   capture_output=True)
    proc = subprocess.run([str(ORACLE / "_build" / "san_driver")], capture_output=True, text=True,
                          timeout=600)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "san_driver: ok" in proc.stdout
    assert "runtime error" not in proc.stderr
