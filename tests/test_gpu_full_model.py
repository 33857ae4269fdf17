"""GPU end to end at full size: the command line on the synthetic 4B-class
bf16 model (36 layers, hidden 2560, ffn 9728, vocab 151936, tied embeddings,
per-tensor log-normal imatrix), for every whole-model run the reference
publishes (README.md:28-49: each scheme with the imatrix, Q4_0 without;
:62-64: Q4_0 and Q4_K --pure, IQ2_XXS --pure) and IQ3_XXS / IQ2_S with a Q4_0
token embedding. Each run's output must hold every tensor of the plan
(`--dry-run`) with its type and size, passthroughs unchanged, and for every
quantized tensor three rows (first, middle, last) byte-identical to the
oracle."""

from __future__ import annotations

import importlib
import subprocess
import sys
import tempfile
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from cli_models import io

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
IGNORE_IMATRIX = {"q4_0", "q4_1", "q5_0", "q5_1", "q8_0"}


@pytest.fixture(scope="module")
def model():
    bench = importlib.import_module("bench")
    base = Path("/dev/shm") if Path("/dev/shm").is_dir() else Path(tempfile.gettempdir())
    with tempfile.TemporaryDirectory(dir=base) as d:
        src, im = Path(d) / "m.gguf", Path(d) / "im.gguf"
        print("writing the synthetic 4B model", flush=True)
        bench.synth_model(torch, torch.device("cuda:0"), src, im)
        yield Path(d), src, im


def run_cli(*args):
    print("cli:", *args, flush=True)
    r = subprocess.run([sys.executable, str(ROOT / "quant-studio.py"), *map(str, args)],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr + r.stdout
    return r


# the C5 runs (IQ3_XXS and IQ2_S schemes with a Q4_0 token embedding) and the
# reference's published runs (README.md:28-49, :62-64; bench.E2E_PUBLISHED:
# every scheme with the imatrix, Q4_0 without, and three --pure runs)
RUNS = ["IQ3_XXS --token-embedding-type q4_0", "IQ2_S --token-embedding-type q4_0"] + \
    importlib.import_module("bench").E2E_PUBLISHED


@pytest.mark.parametrize("run", RUNS)
def test_full_model(model, run):
    d, src, im = model
    scheme, *extra = run.split()
    use_im = "--no-imatrix" not in extra
    extra = [a for a in extra if a != "--no-imatrix"]
    im_args = ["--imatrix", im] if use_im else []
    out = d / f"{scheme}.gguf"
    plan = run_cli(src, out, scheme, *im_args, "--dry-run", *extra).stdout
    want = {}
    for ln in plan.splitlines():
        p = ln.split()
        if len(p) >= 4 and p[2] == "->":
            want[p[0]] = p[3]
    run_cli(src, out, scheme, *im_args, *extra)
    imat = io.load_imatrix(im)
    names = {v: k for k, v in oracle.TYPE_IDS.items()}
    r_in, r_out = io.GGUFReader(src), io.GGUFReader(out)
    tin = {t.name: t for t in r_in.tensors}
    assert {t.name for t in r_out.tensors} == set(tin)
    n_checked = 0
    for t in r_out.tensors:
        s = tin[t.name]
        assert t.ne == s.ne
        assert t.ggml_type.name == want[t.name], (t.name, t.ggml_type.name, want[t.name])
        if t.ggml_type == s.ggml_type:
            assert np.array_equal(t.data, s.data), t.name
            continue
        name = names[int(t.ggml_type)]
        x = s.array().reshape(-1, s.ne[0])
        rows = sorted({0, x.shape[0] // 2, x.shape[0] - 1})
        xs = np.ascontiguousarray(x[rows])
        xs = (xs.astype(np.uint32) << 16).view(np.float32) if xs.dtype == np.uint16 else xs.astype(np.float32)
        qw = None if name in IGNORE_IMATRIX or not use_im else imat[t.name][: s.ne[0]].astype(np.float32)
        ref = oracle.quantize(name, xs, qw)
        got = t.rows()[rows]
        assert np.array_equal(got, ref), f"{t.name} ({name}) rows {rows} differ from the oracle"
        n_checked += 1
    r_in.close()
    r_out.close()
    out.unlink()
    assert n_checked >= 250
