"""Concurrent callers on one GPU: threads of one fresh process quantize at
once, each on a stream of its own, with no qs_init, so the first calls of
each IQ grid race to upload its tables (built once per process, uploaded once
per device under the library's lock). Every output must equal the oracle's."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent

SCRIPT = r"""
import importlib, sys, threading
import numpy as np
import torch
sys.path.insert(0, ROOT)
sys.path.insert(0, ROOT + "/tests")
qs = importlib.import_module("quant-studio_amd")
import oracle
from golden_data import TYPES

dev = torch.device("cuda:0")
types = ["iq2_xs", "iq3_s", "iq2_s", "iq3_xxs", "iq2_xxs", "q4_k", "q2_k", "iq4_xs"]
rng = np.random.default_rng(11)
rows, k = 96, 1024
inputs = {}
for t in types:
    a = (rng.standard_normal((rows, k)) * 0.02 * np.exp(0.3 * rng.standard_normal((rows, 1)))).astype(np.float32)
    xb = torch.from_numpy(a).to(torch.bfloat16)
    inputs[t] = (xb, xb.float().numpy(), rng.lognormal(0.0, 1.0, k).astype(np.float32))
start = threading.Barrier(len(types))
results, errors = {}, []

def work(t):
    try:
        xb, _, qw = inputs[t]
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            x, q = xb.to(dev, non_blocking=False), torch.from_numpy(qw).to(dev)
            s.synchronize()
            start.wait(timeout=120)
            outs = [qs.quantize(TYPES[t][0], x, q) for _ in range(3)]
            s.synchronize()
        results[t] = [o.cpu().numpy() for o in outs]
    except Exception as e:
        errors.append(f"{t}: {e!r}")
        start.abort()          # release the threads waiting at the barrier

threads = [threading.Thread(target=work, args=(t,)) for t in types]
for th in threads:
    th.start()
for th in threads:
    th.join()
assert not errors, errors
for t in types:
    _, xf, qw = inputs[t]
    ref = oracle.quantize(t, xf, qw)
    for i, got in enumerate(results[t]):
        assert np.array_equal(got, ref), f"{t} call {i}: differs from the oracle"
    print(f"{t}: 3 concurrent calls identical to the oracle", flush=True)
"""


def test_threads_on_their_own_streams_race_for_first_use():
    print("concurrency: 8 types x 3 calls, 8 threads, fresh process", flush=True)
    r = subprocess.run([sys.executable, "-c", f"ROOT = {str(ROOT)!r}\n" + SCRIPT],
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-3000:] + r.stdout[-2000:]
    assert r.stdout.count("identical to the oracle") == 8, r.stdout
