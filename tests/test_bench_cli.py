"""bench.py's command line on the CPU (no GPU is touched): more than one GPU
is refused with a message, and every path the measurement notes name is
offered."""
from __future__ import annotations

import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), *args],
                          capture_output=True, text=True, timeout=300)


def test_more_than_one_gpu_is_refused():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in (r.stdout + r.stderr)


def test_paths_and_step_configs_are_offered():
    r = _run("--help")
    assert r.returncode == 0
    for name in ("c1", "c3", "c4", "c5", "step", "logprobs", "top2", "commit", "verify", "masks"):
        assert name in r.stdout, name
    assert "--step-config {c2,c3,c4}" in r.stdout
