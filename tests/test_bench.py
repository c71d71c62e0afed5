"""bench.py's command-line contract: the one-GPU refusal (CPU) and the JSON line (GPU)."""

from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def test_bench_refuses_more_than_one_gpu():
    """--gpus N > 1 exits with status 2 and says why, before touching a device."""

    done = subprocess.run([sys.executable, BENCH, "--gpus", "2"], capture_output=True, text=True, timeout=120)
    assert done.returncode == 2, done.stderr
    assert "one GPU" in done.stderr and "--gpus 2" in done.stderr
    assert done.stdout == ""


@pytest.mark.gpu
@pytest.mark.timeout(300)
def test_bench_prints_one_json_line_with_the_contract_keys():
    """One short run prints exactly one JSON line on stdout carrying the driver's keys and the
    roofline object for the greedy loop's LM-head kernel."""

    done = subprocess.run([sys.executable, "-u", BENCH, "--steps", "1", "--warmup", "1", "--no-cpu-baseline",
                           "--no-kernels"], capture_output=True, text=True, timeout=280, cwd=ROOT)
    assert done.returncode == 0, done.stderr[-2000:]
    lines = [line for line in done.stdout.splitlines() if line.strip()]
    assert len(lines) == 1, done.stdout
    line = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "prefill_tok_s"):
        assert key in line, key
    assert line["n_gpus"] == 1 and line["steps"] == 1 and line["warmup"] == 1
    assert line["unit"] == "tok/s" and line["higher_is_better"] is True and line["value"] > 0
    assert "workload" in line["config"]
    roof = line["roofline"]
    assert roof["bound"] == "hbm" and roof["unit"] == "GB/s" and roof["peak"] == 8000.0
    assert 0 < roof["frac"] < 1 and abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    assert line["decode_graph"] == "captured" and line["prefill_graph"] == "captured"
