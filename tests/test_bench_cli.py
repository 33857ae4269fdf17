"""bench.py's command-line contract on the CPU: it runs on one GPU only, and a
request for more exits with status 2 and says why before touching a device."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def run_bench(*args, env=None):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True,
                          text=True, timeout=120, env=env)


def test_more_than_one_gpu_is_refused():
    r = run_bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_a_multi_rank_launch_is_refused():
    env = dict(os.environ, WORLD_SIZE="8")
    r = run_bench(env=env)
    assert r.returncode == 2
    assert "--gpus must be 1" in r.stderr
