"""Access to the golden vectors written by tests/golden/gen_golden.py from the
reference's eager CPU quantizers (inputs.npz + one <type>.npz per type)."""

from __future__ import annotations

from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"

# type name -> ggml id, block size, block bytes (BLOCK_BYTES in each reference module)
TYPES = {
    "q4_0": (2, 32, 18), "q2_k": (10, 256, 84), "q3_k": (11, 256, 110), "q4_k": (12, 256, 144),
    "q5_k": (13, 256, 176), "q6_k": (14, 256, 210), "iq4_xs": (23, 256, 136),
    "iq2_xxs": (16, 256, 66), "iq2_xs": (17, 256, 74), "iq2_s": (22, 256, 82),
    "iq3_xxs": (18, 256, 98), "iq3_s": (21, 256, 110),
}
ORACLE_TYPES = ["q4_0", "q2_k", "q3_k", "q4_k", "q5_k", "q6_k", "iq4_xs",
                "iq2_xxs", "iq2_xs", "iq2_s", "iq3_xxs", "iq3_s"]

_inputs = None


def inputs():
    global _inputs
    if _inputs is None:
        _inputs = dict(np.load(GOLDEN / "inputs.npz"))
    return _inputs


def cases(qtype: str):
    """[(key, x (bf16 bits as uint16, or f32), imatrix or None, expected uint8)]"""
    g = np.load(GOLDEN / f"{qtype}.npz")
    inp = inputs()
    out = []
    for key in sorted(g.files):
        if key.count(".") != 1:
            continue                      # intermediate records (e.g. search results)
        case, mode = key.split(".")
        qw = inp[f"{case}.imat"] if mode == "imat" else None
        out.append((key, inp[f"{case}.x"], qw, g[key]))
    return out


def as_f32(x: np.ndarray) -> np.ndarray:
    return (x.astype(np.uint32) << 16).view(np.float32) if x.dtype == np.uint16 else x


def block_identical(a: np.ndarray, b: np.ndarray, qtype: str) -> np.ndarray:
    bb = TYPES[qtype][2]
    return (a.reshape(-1, bb) == b.reshape(-1, bb)).all(1)


_zero = None


def zero_imatrix_cases(qtype: str):
    """[(case, x bf16 bits, imatrix with zero entries, expected uint8)] from
    zero_imat.npz, written by the reference's eager quantizers
    (gen_golden.py --zero-imatrix); empty for a type without an imatrix mode."""
    global _zero
    if _zero is None:
        _zero = dict(np.load(GOLDEN / "zero_imat.npz"))
    out = []
    for key in sorted(_zero):
        t, _, case = key.partition(".")
        if t == qtype:
            out.append((case, _zero[f"{case}.x"], _zero[f"{case}.imat"], _zero[key]))
    return out


def nonfinite_case():
    """(x f32 with NaN / +-Inf / +-1e38 values, imatrix, {"<type>.<mode>": the
    reference's bytes}) from nonfinite.npz (gen_golden.py --nonfinite); types
    whose reference quantizer raised on the input (Q3_K, Q6_K, IQ2_XXS) have
    no entry."""
    z = np.load(GOLDEN / "nonfinite.npz")
    ref = {k.split(".", 1)[0] + "." + k.rsplit(".", 1)[1]: z[k] for k in z.files if k.count(".") == 2}
    return z["nonfinite.x"], z["nonfinite.imat"], ref


def clean_blocks(x: np.ndarray, block: int, limit: float = 1e18) -> np.ndarray:
    """Per output block (row-major), True where every value is finite and small
    enough that its square stays finite in f32."""
    xb = x.reshape(x.shape[0], -1, block)
    return (np.isfinite(xb) & (np.abs(xb) < limit)).all(-1).reshape(-1)
