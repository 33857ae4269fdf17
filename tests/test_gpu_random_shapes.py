"""Seeded random cases against the oracle, byte for byte: every type, ragged
row counts (tails of the 8- or 4-superblock waves and of the 256-block
workgroups), row lengths from one block up, f32 / f16 / bf16 sources, with and
without an imatrix, value scales from 1e-6 to 1e3, and rows of zeros or of
one repeated value mixed in."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

TYPE_BLOCK = {"q4_0": 32, "q4_1": 32, "q5_0": 32, "q5_1": 32, "q8_0": 32, "iq4_nl": 32,
              "q2_k": 256, "q3_k": 256, "q4_k": 256, "q5_k": 256, "q6_k": 256, "iq4_xs": 256,
              "iq2_xxs": 256, "iq2_xs": 256, "iq2_s": 256, "iq3_xxs": 256, "iq3_s": 256}
NEEDS_IMATRIX = {"iq2_xxs", "iq2_xs", "iq2_s"}     # IQ3_XXS runs without one (iq3_xxs.py:41-42)
IGNORES_IMATRIX = {"q4_0", "q4_1", "q5_0", "q5_1", "q8_0"}
SOURCES = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def make_case(qtype: str, i: int):
    rng = np.random.default_rng(1000 * list(TYPE_BLOCK).index(qtype) + i)
    blk = TYPE_BLOCK[qtype]
    rows = int(rng.integers(1, 70))
    k = blk * int(rng.integers(1, 13 if blk == 256 else 97))
    src = ("f32", "f16", "bf16")[i % 3]
    scale = float(10.0 ** rng.uniform(-6, 3))    # f16: tiny scales give subnormal and zero inputs
    a = rng.standard_normal((rows, k)) * scale * np.exp(0.5 * rng.standard_normal((rows, 1)))
    if rows > 2:
        a[int(rng.integers(rows))] = 0.0
        a[int(rng.integers(rows))] = scale
    imat = qtype in NEEDS_IMATRIX or (qtype not in IGNORES_IMATRIX and i % 2 == 0)
    qw = rng.lognormal(0.0, 1.0, k).astype(np.float32) if imat else None
    t = torch.from_numpy(a.astype(np.float32)).to(SOURCES[src])
    return rows, k, src, scale, t, qw


@pytest.mark.parametrize("qtype", list(TYPE_BLOCK))
def test_random_shapes_sources_and_scales(qs, qtype):
    dev = torch.device("cuda:0")
    spec = qs.QUANT_TYPES[qtype]
    for i in range(6):
        rows, k, src, scale, t, qw = make_case(qtype, i)
        print(f"{qtype} case {i}: {rows}x{k} {src} scale {scale:.3g} imatrix={qw is not None}", flush=True)
        q = None if qw is None else torch.from_numpy(qw).to(dev)
        got = qs.quantize(int(spec.ggml_type), t.to(dev), q).cpu().numpy()
        ref = oracle.quantize(qtype, t.float().numpy(), None if qtype in IGNORES_IMATRIX else qw)
        assert got.shape == ref.shape
        bad = np.flatnonzero((got != ref).any(1))
        assert bad.size == 0, f"{qtype} case {i}: rows {bad[:8].tolist()} differ"
