"""The bench.py contract the driver depends on: one JSON line with the
required keys, `--gpus N` > 1 refused with a message (CPU), and a short GPU
run of a small configuration (GPU)."""

import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REQUIRED = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
            "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline")


def _run(args, timeout):
    return subprocess.run([sys.executable, "-u", os.path.join(ROOT, "bench.py")] + args, capture_output=True,
                          text=True, timeout=timeout, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = _run(["--gpus", "2"], 120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr) or "single" in (r.stdout + r.stderr).lower()


@pytest.mark.gpu
def test_bench_line_on_the_toy_config():
    r = _run(["--config", "toy", "--steps", "3", "--warmup", "1"], 600)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
    assert len(lines) == 1
    d = json.loads(lines[0])
    for k in REQUIRED:
        assert k in d, k
    assert d["n_gpus"] == 1 and d["steps"] == 3 and d["warmup"] == 1 and d["value"] > 0
    assert d["roofline"]["peak"] > 0 and 0 < d["roofline"]["frac"] < 1
    assert d["cpu_baseline"]["value"] and d["cpu_baseline"]["kind"] == "port"
    assert "toy" in d["config"]["workload"]
