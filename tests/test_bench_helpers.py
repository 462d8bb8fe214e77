"""bench.py's host-side arithmetic, on the CPU: the error metrics its parity
entries report, the per-call percentiles, the block's algorithmic bytes and
the refusal of more than one GPU (before anything touches a GPU)."""

import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_normwise_is_per_token_max_over_token_max():
    ref = np.array([[1.0, -4.0, 2.0], [0.5, 0.25, -0.125]], np.float32)
    out = ref.copy()
    out[0, 2] += 0.004          # token 0: 0.004 / 4
    out[1, 0] -= 0.0005         # token 1: 0.0005 / 0.5
    assert bench.normwise(out, ref) == pytest.approx(1e-3, rel=1e-4)
    out[1, 0] = ref[1, 0]
    assert bench.normwise(out, ref) == pytest.approx(1e-3, rel=1e-4)
    out[0, 2] = ref[0, 2]
    assert bench.normwise(out, ref) == 0.0
    # a token that is all zeros divides by 1, not by 0
    z = np.zeros((1, 3), np.float32)
    assert bench.normwise(z + 1e-6, z) == pytest.approx(1e-6, rel=1e-3)


def test_elementwise_p99_keeps_outputs_above_a_thousandth_of_the_token_max():
    rng = np.random.default_rng(0)
    ref = rng.uniform(1.0, 2.0, (4, 1000)).astype(np.float32)
    out = ref * (1 + np.linspace(0, 1e-2, ref.size, dtype=np.float64).reshape(ref.shape)).astype(np.float32)
    want = np.percentile(np.abs(out.astype(np.float64) - ref) / np.abs(ref), 99)
    assert bench.elementwise_p99(out, ref) == pytest.approx(want, rel=1e-6)
    # outputs below 1e-3 of their token's largest are left out, whatever
    # their relative error
    ref2 = ref.copy()
    ref2[:, :5] = 1e-7
    out2 = out.copy()
    out2[:, :5] = 1.0
    assert bench.elementwise_p99(out2, ref2) < 2e-2
    assert bench.elementwise_p99(ref, ref) == 0.0


def test_percentiles_in_microseconds():
    r = bench.percentiles_us([0.001 * v for v in range(1, 101)])    # 1 .. 100 us
    assert r["calls"] == 100
    assert r["median"] == pytest.approx(50.5)
    assert r["p10"] == pytest.approx(10.9)
    assert r["p90"] == pytest.approx(90.1)


def test_block_bytes_count_each_routed_expert_once():
    from joule_amd.moe import QWEN3

    stages = {"route": 0.01, "gateup": 0.02, "down": 0.012}
    U = [50, 52]                                   # routed experts of the two rotated layers
    r = bench.block_numbers(QWEN3, 64, 8, 0.042, stages, U, steps=4, n_layers=2, router_bytes=2)
    # Qwen3 Q4 G64 records: gate/up 835,584 bytes each, down 835,584
    per_expert = 3 * 835_584
    assert r["experts_routed_avg"] == 51
    assert r["gateup_bytes"] == pytest.approx(51 * 2 * 835_584)
    assert r["down_bytes"] == pytest.approx(51 * 835_584)
    # plus the router table (bf16), x in and out
    router = 128 * 2048 * 2
    xio = 2 * 8 * 2048 * 4
    assert r["bytes_alg"] == pytest.approx(51 * per_expert + router + xio, rel=1e-3)
    assert r["block_frac"] == pytest.approx(r["bytes_alg"] / 42e-6 / 8e12, rel=1e-9)


def test_monotone_stats_reports_the_largest_inversion():
    assert bench.monotone_stats([1.0, 2.0, 2.0, 5.0]) == (True, 0.0)
    ok, inv = bench.monotone_stats([5.0, 6.0, 5.5, 7.0, 5.8])
    assert not ok and inv == pytest.approx(1.2)       # 7.0 against the later 5.8 (6.0 / 5.5: 0.5)
    assert bench.monotone_stats([3.0]) == (True, 0.0)
    assert bench.monotone_stats([]) == (True, 0.0)


def test_more_than_one_gpu_is_refused_before_the_gpu_is_touched():
    p = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=str(ROOT))
    assert p.returncode == 2
    assert "one GPU only" in p.stderr
    assert p.stdout == ""
