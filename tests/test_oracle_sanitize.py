"""The C restatement under AddressSanitizer + UndefinedBehaviorSanitizer and,
separately, ThreadSanitizer (oracle/Makefile `sanitize`): every entry point,
the spin pool started, resized and shut down, results independent of the
thread count.  Host code only."""

import shutil
import subprocess
from pathlib import Path

import pytest

ORACLE = Path(__file__).resolve().parents[1] / "oracle"


@pytest.mark.parametrize("target", ["sanitize-asan", "sanitize-tsan"])
def test_oracle_under_sanitizers(target):
    if not shutil.which("gcc") or not shutil.which("make"):
        pytest.skip("gcc/make not available")
    res = subprocess.run(["make", "-s", "-C", str(ORACLE), target], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-4000:]
    assert "all checks passed" in res.stdout
