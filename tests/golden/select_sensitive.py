#!/usr/bin/env python3
"""Pick golden INPUT rows on which plausible restatement slips change the output.

Random data rarely exercises some conventions (e.g. torch's reciprocal-multiply
for `python_float / tensor` differs from IEEE division in the last ulp, which
changes a quantized block only about once in a few hundred superblocks). This
script draws many random superblocks and keeps, per type and imatrix mode, a
few for which the CPU oracle with one planted mistake (qso_set_mutation)
disagrees with the faithful oracle. Only the inputs are written
(sensitive.npz); gen_golden.py then runs the reference on them, so the
expected outputs still come from the reference alone.

Usage: python tests/golden/select_sensitive.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
import oracle  # noqa: E402

TYPES = ["q2_k", "q3_k", "q4_k", "q5_k", "q6_k", "iq4_xs"]
MUTANTS = [1, 2, 3, 4, 5, 6]
PER_COMBO = 2
K = 256


def bf16(a: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def main() -> None:
    rng = np.random.default_rng(777)
    imat = rng.lognormal(0.0, 1.0, K).astype(np.float32)
    n = 8192
    x = rng.standard_normal((n, K)) * 0.02 * np.exp(0.5 * rng.standard_normal((n, 1)))
    heavy = rng.standard_t(4, (n, K)) * 0.02
    x[n // 2:] = heavy[n // 2:]
    xb = bf16(x)
    xf = (xb.astype(np.uint32) << 16).view(np.float32)
    L = oracle.lib()
    keep: list[int] = []
    for t in TYPES:
        for qw in (None, imat):
            L.qso_set_mutation(0)
            base = oracle.quantize(t, xf, qw)
            for m in MUTANTS:
                L.qso_set_mutation(m)
                mut = oracle.quantize(t, xf, qw)
                L.qso_set_mutation(0)
                diff = np.nonzero((base != mut).any(1))[0]
                picked = [int(i) for i in diff if int(i) not in keep][:PER_COMBO]
                keep.extend(picked)
    keep = sorted(set(keep))
    np.savez_compressed(HERE / "sensitive.npz", x=xb[keep], imat=imat)
    print(f"kept {len(keep)} rows of {K}")


if __name__ == "__main__":
    main()
