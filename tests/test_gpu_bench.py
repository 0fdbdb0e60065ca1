"""The bench line at the driver's exact command (bench.py --gpus 1 --steps 20
--warmup 5), run as a child process: one JSON line with the contract's
fields, a roofline whose figures agree with one another, and the
repetitions the value is the median of."""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


def test_driver_command_bench_line():
    print("bench --gpus 1 --steps 20 --warmup 5", flush=True)
    done = subprocess.run(
        [sys.executable, str(ROOT / "bench.py"), "--gpus", "1", "--steps", "20", "--warmup", "5",
         "--no-cpu-baseline", "--eager-steps", "0"],
        cwd=ROOT, capture_output=True, text=True, timeout=240)
    assert done.returncode == 0, done.stderr[-2000:]
    lines = [l for l in done.stdout.splitlines() if l.strip().startswith("{")]
    assert len(lines) == 1
    d = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline"):
        assert key in d, key
    assert (d["n_gpus"], d["steps"], d["warmup"]) == (1, 20, 5)
    assert d["unit"] == "tokens/s" and d["higher_is_better"] is True
    assert d["value"] > 0
    # value = batch * steps / the median repetition's seconds
    assert d["value"] == pytest.approx(64 * 20 / (d["ms_per_step"] * 20 / 1000.0), rel=1e-3)
    assert sorted(d["repeat_tokens_per_s"])[2] == pytest.approx(d["value"], rel=1e-6)
    r = d["roofline"]
    assert r["bound"] == "hbm" and r["unit"] == "GB/s" and r["peak"] == 8000.0
    assert r["frac"] == pytest.approx(r["achieved"] / r["peak"], abs=1e-3)
    assert r["achieved"] == pytest.approx(
        r["algorithmic_bytes_per_launch"] / (r["kernel_us"] * 1e-6) / 1e9, rel=1e-3)
    assert r["steps_per_launch"] == 20
    assert r["traffic"] is None or r["traffic"] > 0
    assert len(d["repeat_kernel_us"]) == 5 and all(x > 0 for x in d["repeat_kernel_us"])
    assert d["dense_control"]["state_max_abs_diff"] == 0.0
    # the reference's memory figures for the decoded state
    m = d["memory"]
    assert 0 < m["live_row_fraction"] <= m["physical_capacity_fraction"]
    assert 0 < m["packed_over_dense_live_bytes"] <= m["packed_over_dense_reserved_bytes"]
    assert m["logical_rows"] == 7 * 64 * 256
