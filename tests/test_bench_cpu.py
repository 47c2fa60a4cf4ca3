"""bench.py's contract on the CPU: the default configuration is the one BASELINE.json's
metric is quoted on, with that metric string, and a request for more than one GPU exits
with a message (status 2) before touching a GPU."""
from __future__ import annotations

import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_default_config_carries_the_baseline_metric():
    sys.path.insert(0, ROOT)
    import bench

    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        metric = json.load(f)["metric"]
    old = sys.argv
    try:
        sys.argv = ["bench.py"]
        args = bench.parse()
    finally:
        sys.argv = old
    assert args.gpus == 1
    assert bench.CONFIGS[args.config]["metric"] == metric


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""
