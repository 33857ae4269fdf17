#!/usr/bin/env python3
"""Write the golden input/output vectors for every quant type.

Runs ONLY in the build container, where the reference checkout is mounted at
/root/reference. It imports the reference's per-type modules (kernels/*.py) and
calls their eager CPU quantizers (the path `--device cpu` takes:
quant-studio.py:216-232 -> quant_fn) on seeded synthetic inputs, then stores
inputs and outputs as small .npz fixtures next to this script. Nothing from the
reference is stored except its outputs.

The reference imports gguf-py only for enum names (kernels/common.py:6-7,
kernels/q4_0.py:6-7, ...). gguf-py is not installed here, so this script
provides a minimal stand-in module exposing those names with the public GGUF
enum values; no arithmetic depends on it.

Usage: python tests/golden/gen_golden.py [--ref /root/reference] [--only TYPE ...]
       python tests/golden/gen_golden.py --zero-imatrix   (writes zero_imat.npz only)
"""

from __future__ import annotations

import argparse
import enum
import sys
import types
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent

# public ggml type ids and llama file types (GGUF spec); names only matter here
GGML_TYPES = dict(F32=0, F16=1, Q4_0=2, Q4_1=3, Q5_0=6, Q5_1=7, Q8_0=8, Q8_1=9, Q2_K=10,
                  Q3_K=11, Q4_K=12, Q5_K=13, Q6_K=14, Q8_K=15, IQ2_XXS=16, IQ2_XS=17,
                  IQ3_XXS=18, IQ1_S=19, IQ4_NL=20, IQ3_S=21, IQ2_S=22, IQ4_XS=23, I8=24,
                  I16=25, I32=26, I64=27, F64=28, IQ1_M=29, BF16=30, TQ1_0=34, TQ2_0=35,
                  MXFP4=39)
FILE_TYPES = dict(ALL_F32=0, MOSTLY_F16=1, MOSTLY_Q4_0=2, MOSTLY_Q4_1=3, MOSTLY_Q8_0=7,
                  MOSTLY_Q5_0=8, MOSTLY_Q5_1=9, MOSTLY_Q2_K=10, MOSTLY_Q3_K_S=11,
                  MOSTLY_Q3_K_M=12, MOSTLY_Q3_K_L=13, MOSTLY_Q4_K_S=14, MOSTLY_Q4_K_M=15,
                  MOSTLY_Q5_K_S=16, MOSTLY_Q5_K_M=17, MOSTLY_Q6_K=18, MOSTLY_IQ2_XXS=19,
                  MOSTLY_IQ2_XS=20, MOSTLY_Q2_K_S=21, MOSTLY_IQ3_XS=22, MOSTLY_IQ3_XXS=23,
                  MOSTLY_IQ1_S=24, MOSTLY_IQ4_NL=25, MOSTLY_IQ3_S=26, MOSTLY_IQ3_M=27,
                  MOSTLY_IQ2_S=28, MOSTLY_IQ2_M=29, MOSTLY_IQ4_XS=30, MOSTLY_IQ1_M=31,
                  MOSTLY_BF16=32, MOSTLY_TQ1_0=36, MOSTLY_TQ2_0=37, MOSTLY_MXFP4_MOE=38)


def install_enum_module() -> None:
    g = types.ModuleType("gguf")
    c = types.ModuleType("gguf.constants")
    g.GGMLQuantizationType = enum.IntEnum("GGMLQuantizationType", GGML_TYPES)
    c.LlamaFileType = enum.IntEnum("LlamaFileType", FILE_TYPES)
    g.LlamaFileType = c.LlamaFileType
    g.GGML_QUANT_VERSION = 2
    g.constants = c
    sys.modules["gguf"] = g
    sys.modules["gguf.constants"] = c


# (type name, reference module, function, imatrix modes)
TYPES = [
    ("q4_0", "q4_0", "quantize_q4_0", ("none",)),
    ("q2_k", "q2_k", "quantize_q2_k", ("none", "imat")),
    ("q3_k", "q3_k", "quantize_q3_k", ("none", "imat")),
    ("q4_k", "q4_k", "quantize_q4_k", ("none", "imat")),
    ("q5_k", "q5_k", "quantize_q5_k", ("none", "imat")),
    ("q6_k", "q6_k", "quantize_q6_k", ("none", "imat")),
    ("iq4_xs", "iq4_xs", "quantize_iq4_xs", ("none", "imat")),
    ("iq2_xxs", "iq2", "quantize_iq2_xxs", ("imat",)),
    ("iq2_xs", "iq2_xs", "quantize_iq2_xs", ("imat",)),
    ("iq2_s", "iq2_s", "quantize_iq2_s", ("imat",)),
    # the function takes None (weights x^2, iq3_xxs.py:41-42) although the
    # type's QuantSpec requires an imatrix (the command line refuses it)
    ("iq3_xxs", "iq3_xxs", "quantize_iq3_xxs", ("none", "imat")),
    ("iq3_s", "iq3_s", "quantize_iq3_s", ("none", "imat")),
]


def bf16_round(a: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit patterns (round to nearest even), as uint16."""
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def make_cases() -> dict[str, dict[str, np.ndarray]]:
    """Seeded inputs. bf16 cases store bf16 bits; the f32 case stores raw f32."""
    cases = {}
    rng = np.random.default_rng(20261201)

    # adversarial rows modelled on the reference's synthetic model (zeros, constants,
    # an outlier over tiny values, half-constant, one-signed rows) plus scale extremes
    k = 1024
    a = rng.standard_normal((16, k)) * 0.05 * (0.2 + rng.random((16, 1)) * 3.0)
    a[0, :] = 0.0
    a[1, :] = 0.5
    a[2, :] = -0.5
    a[3, :] = 1e-6
    a[3, 7] = 8.0
    a[4, :128] = 0.25
    a[5, :] = np.abs(a[5, :])
    a[6, :] = -np.abs(a[6, :])
    a[7, :] = rng.standard_normal(k) * 1e-17          # below the 1e-15 dead-group threshold
    a[8, :] = rng.standard_normal(k) * 1e-9           # between 1e-15 and 1e-8
    a[9, :] = rng.standard_normal(k) * 300.0
    a[10, ::2] = 0.0                                  # sparse row
    a[11, :] = np.round(rng.standard_normal(k) * 4) / 64.0   # coarse lattice values: many ties
    a[12, :256] = 0.0
    a[12, 3] = -1e-3
    a[13, :] = np.where(rng.random(k) < 0.5, 0.02, -0.02)
    cases["synth"] = dict(x=bf16_round(a), imat=rng.lognormal(0.0, 1.0, k).astype(np.float32))

    # ffn-like: N(0, 0.02) with log-normal per-row std jitter, 0.1% outliers x20
    rows, k = 64, 512
    a = rng.standard_normal((rows, k)) * 0.02 * np.exp(0.3 * rng.standard_normal((rows, 1)))
    idx = rng.choice(rows * k, rows * k // 1000, replace=False)
    a.reshape(-1)[idx] *= 20.0
    cases["normal"] = dict(x=bf16_round(a), imat=rng.lognormal(0.0, 1.0, k).astype(np.float32))

    # heavy-tailed: Student-t df=5 scaled to std 0.02
    rows, k = 32, 512
    a = rng.standard_t(5, (rows, k)) * 0.02 / np.sqrt(5.0 / 3.0)
    cases["student"] = dict(x=bf16_round(a), imat=rng.lognormal(0.0, 1.0, k).astype(np.float32))

    # raw f32 input (not bf16-representable) for the F32 source path
    rows, k = 8, 512
    a = (rng.standard_normal((rows, k)) * 0.05).astype(np.float32)
    cases["f32"] = dict(x=a, imat=rng.lognormal(0.0, 1.0, k).astype(np.float32))

    # superblocks on which plausible restatement slips change the output
    # (chosen by select_sensitive.py; inputs only)
    sens = HERE / "sensitive.npz"
    if sens.exists():
        z = np.load(sens)
        cases["sensitive"] = dict(x=z["x"], imat=z["imat"])
    return cases


def make_zero_cases() -> dict[str, dict[str, np.ndarray]]:
    """Imatrix vectors with zero entries, as real imatrix files give them: the
    reference's loader writes 0 wherever a column's count is not positive
    (quant-studio.py:80-85), and a 3-D expert tensor gets expert 0's first k
    values (quant-studio.py:455), all zero when that expert was never routed.
    The zeros then reach every weight formula (qw*sqrt(sigma2+x^2),
    q4_k.py:49-51; sqrt(w) in the IQ searches, iq2.py:429-436)."""
    cases = {}
    rng = np.random.default_rng(20261202)

    def rows_with_adversarial(rows, k, std):
        a = rng.standard_normal((rows, k)) * std * np.exp(0.3 * rng.standard_normal((rows, 1)))
        a[0, :] = 0.0
        a[1, :] = 0.5
        a[2, :] = rng.standard_normal(k) * 1e-17
        a[3, :] = np.abs(a[3, :])
        a[4, :] = np.round(rng.standard_normal(k) * 4) / 64.0
        return a

    # scattered zeros: about a quarter of the columns never fired
    k = 1024
    a = rows_with_adversarial(24, k, 0.02)
    qw = rng.lognormal(0.0, 1.0, k).astype(np.float32)
    qw[rng.random(k) < 0.25] = 0.0
    cases["zscatter"] = dict(x=bf16_round(a), imat=qw)

    # whole zero groups: 16- and 32-value groups, a 256-value superblock, half a
    # superblock, every other 16-group of one superblock, and 8-value subgroups
    k = 1024
    a = rows_with_adversarial(16, k, 0.02)
    qw = rng.lognormal(0.0, 1.0, k).astype(np.float32)
    qw[0:16] = 0.0
    qw[48:64] = 0.0
    qw[64:96] = 0.0
    qw[136:144] = 0.0
    qw[200:204] = 0.0
    qw[256:512] = 0.0
    qw[512:640] = 0.0
    for g in range(8):
        qw[768 + 32 * g: 768 + 32 * g + 16] = 0.0
    cases["zgroups"] = dict(x=bf16_round(a), imat=qw)

    # heavy-tailed rows, half of the 8-value subgroups' columns zero
    k = 512
    a = rng.standard_t(5, (16, k)) * 0.02 / np.sqrt(5.0 / 3.0)
    qw = rng.lognormal(0.0, 1.0, k).astype(np.float32)
    qw[np.repeat(rng.random(k // 8) < 0.5, 8)] = 0.0
    cases["zsub8"] = dict(x=bf16_round(a), imat=qw)

    # an all-zero vector: an expert that was never routed
    k = 512
    a = rows_with_adversarial(8, k, 0.02)
    cases["zall"] = dict(x=bf16_round(a), imat=np.zeros(k, np.float32))
    return cases


def make_nonfinite_cases() -> dict[str, dict[str, np.ndarray]]:
    """Rows holding NaN and +-Inf among ordinary values: one value per block,
    a whole block, the first and the last value of a 32/256-value group."""
    rng = np.random.default_rng(20261203)
    k = 512
    a = rng.standard_normal((12, k)) * 0.02
    a[0, 5] = np.nan
    a[1, 5] = np.inf
    a[2, 5] = -np.inf
    a[3, :32] = np.nan
    a[4, 0] = np.nan
    a[5, 255] = np.inf
    a[6, 31] = -np.inf
    a[7, 100:104] = [np.nan, np.inf, -np.inf, np.nan]
    a[8, ::64] = np.nan
    a[9, 300] = 1e38
    a[10, 7] = -1e38
    qw = rng.lognormal(0.0, 1.0, k).astype(np.float32)
    return {"nonfinite": dict(x=a.astype(np.float32), imat=qw)}


def write_nonfinite(out: Path, only) -> None:
    """nonfinite.npz: make_nonfinite_cases and the reference's bytes for every
    type and imatrix mode (keys <case>.x, <case>.imat, <type>.<case>.<mode>);
    a type whose quantizer raises on the input is left out."""
    import importlib
    cases = make_nonfinite_cases()
    rec = {}
    for cname, c in cases.items():
        rec[f"{cname}.x"] = c["x"]
        rec[f"{cname}.imat"] = c["imat"]
    for tname, mod, fn, modes in TYPES:
        if only and tname not in only:
            continue
        f = getattr(importlib.import_module(f"kernels.{mod}"), fn)
        for cname, c in cases.items():
            for mode in modes:
                x = torch.from_numpy(c["x"].copy())
                qw = torch.from_numpy(c["imat"].copy()) if mode == "imat" else None
                try:
                    y = f(x) if tname == "q4_0" else f(x, qw)
                except Exception as e:          # recorded as absent
                    print(f"{tname} {mode}: {type(e).__name__}: {e}", flush=True)
                    continue
                rec[f"{tname}.{cname}.{mode}"] = y.numpy().astype(np.uint8)
        print(f"{tname}: non-finite cases written", flush=True)
    np.savez_compressed(out / "nonfinite.npz", **rec)


def write_zero_imatrix(out: Path, only) -> None:
    """zero_imat.npz: the cases of make_zero_cases and the reference's bytes for
    every type that uses an imatrix (keys <case>.x, <case>.imat, <type>.<case>)."""
    import importlib
    cases = make_zero_cases()
    rec = {}
    for cname, c in cases.items():
        rec[f"{cname}.x"] = c["x"]
        rec[f"{cname}.imat"] = c["imat"]
    for tname, mod, fn, modes in TYPES:
        if "imat" not in modes or (only and tname not in only):
            continue
        f = getattr(importlib.import_module(f"kernels.{mod}"), fn)
        for cname, c in cases.items():
            y = f(torch.from_numpy(case_f32(c).copy()), torch.from_numpy(c["imat"].copy()))
            rec[f"{tname}.{cname}"] = y.numpy().astype(np.uint8)
        print(f"{tname}: zero-imatrix cases {', '.join(cases)}", flush=True)
    np.savez_compressed(out / "zero_imat.npz", **rec)


def case_f32(case: dict[str, np.ndarray]) -> np.ndarray:
    x = case["x"]
    return bf16_to_f32(x) if x.dtype == np.uint16 else x


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    ap.add_argument("--out", default=str(HERE))
    ap.add_argument("--only", nargs="*", help="write only these types' files (inputs.npz is left as is)")
    ap.add_argument("--zero-imatrix", action="store_true",
                    help="write only zero_imat.npz (imatrix vectors with zero entries)")
    ap.add_argument("--nonfinite", action="store_true",
                    help="write only nonfinite.npz (rows holding NaN and +-Inf)")
    args = ap.parse_args()

    install_enum_module()
    sys.path.insert(0, args.ref)
    import importlib

    torch.set_num_threads(1)
    if args.zero_imatrix:
        write_zero_imatrix(Path(args.out), args.only)
        return
    if args.nonfinite:
        write_nonfinite(Path(args.out), args.only)
        return
    cases = make_cases()
    inputs = {}
    for cname, c in cases.items():
        inputs[f"{cname}.x"] = c["x"]
        inputs[f"{cname}.imat"] = c["imat"]
    if not args.only:
        np.savez_compressed(Path(args.out) / "inputs.npz", **inputs)

    # per-group results of the shared IQ2_XS / IQ2_S search (iq2xs_common.scale_search),
    # recorded by wrapping the function the quantizers call
    xs_common = importlib.import_module("kernels.iq2xs_common")
    recorded: list = []

    def recording(fn):
        def wrapper(*a, **kw):
            scale, win = fn(*a, **kw)
            recorded.append((scale.clone(), win.clone()))
            return scale, win
        return wrapper

    # and the sweep's batched projection (the first search_codes call of each
    # scale_search): tentative codes, winning grid indices, kmap-hit flags
    sweeps: list = []
    reprojs: list = []
    orig_search_codes = xs_common.search_codes

    def recording_search(u_all, *a, **kw):
        win, og = orig_search_codes(u_all, *a, **kw)
        if kw.get("sel") is None and len(a) < 5:
            sweeps.append((u_all.clone(), win.clone(), og.clone()))
        else:
            reprojs.append((u_all.clone(), kw["sel"].clone(), win.clone()))
        return win, og

    xs_common.search_codes = recording_search

    for tname, mod, fn, modes in TYPES:
        if args.only and tname not in args.only:
            continue
        m = importlib.import_module(f"kernels.{mod}")
        f = getattr(m, fn)
        if tname in ("iq2_xs", "iq2_s"):
            m.scale_search = recording(xs_common.scale_search)
        outs = {}
        for cname, c in cases.items():
            x = torch.from_numpy(case_f32(c).copy())
            for mode in modes:
                qw = torch.from_numpy(c["imat"].copy()) if mode == "imat" else None
                recorded.clear()
                sweeps.clear()
                reprojs.clear()
                y = f(x) if tname == "q4_0" else f(x, qw)
                outs[f"{cname}.{mode}"] = y.numpy().astype(np.uint8)
                if recorded:
                    outs[f"{cname}.{mode}.search_scale"] = recorded[0][0].numpy()
                    outs[f"{cname}.{mode}.search_win"] = recorded[0][1].numpy().astype(np.int16)
                if sweeps:
                    u_all, win, og = sweeps[0]
                    outs[f"{cname}.{mode}.sweep_code"] = u_all.numpy().astype(np.uint16)
                    outs[f"{cname}.{mode}.sweep_win"] = win.numpy().astype(np.int16)
                    outs[f"{cname}.{mode}.sweep_on"] = og.numpy().astype(np.uint8)
                if reprojs:
                    u2, sel, win2 = reprojs[0]
                    outs[f"{cname}.{mode}.reproj_code"] = u2.numpy().astype(np.uint16)
                    outs[f"{cname}.{mode}.reproj_sel"] = sel.numpy().astype(np.uint8)
                    outs[f"{cname}.{mode}.reproj_win"] = win2.numpy().astype(np.int16)
        np.savez_compressed(Path(args.out) / f"{tname}.npz", **outs)
        print(f"{tname}: {', '.join(f'{k}={v.shape}' for k, v in outs.items())}", flush=True)


if __name__ == "__main__":
    main()
