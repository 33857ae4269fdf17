"""Build the gfx950 quantizer library (libqs_hip.so) in-tree with hipcc.

Flags that matter for bit-exact parity with the reference's eager torch path:
  -ffp-contract=off                         no FMA contraction (torch rounds a*b and +c separately)
  -fhip-fp32-correctly-rounded-divide-sqrt  IEEE `/` and sqrtf
  no -ffast-math, no denormal flushing
and, for every HIP source, packed FP32 instructions are disabled
(-Xclang -target-feature -Xclang -packed-fp32-ops).
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "_build" / "libqs_hip.so"
CALIB_OUT = PKG / "_build" / "libqs_calib.so"       # measurement aid for bench.py

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]
SOURCES = ["qs_api.hip", "qs_pipeline.cpp"]


def build(verbose: bool = False) -> Path:
    # the AMD-host square-root map is embedded in the library (.incbin)
    _compile(OUT, SOURCES, verbose, [f'-DQS_SQRT_AMD_BIN="{CSRC / "qs_sqrt_amd.bin"}"'], ["-lz"])
    _compile(CALIB_OUT, ["qs_calib.hip"], verbose)
    return OUT


def _compile(out: Path, sources: list[str], verbose: bool, defines: list[str] | None = None,
             libs: list[str] | None = None) -> None:
    out.parent.mkdir(parents=True, exist_ok=True)
    tmp = out.with_name(out.name + ".tmp")
    cmd = [HIPCC, *FLAGS, *(defines or []), f"-I{ROOT / 'include'}", f"-I{CSRC}", "-o", str(tmp),
           *[str(CSRC / s) for s in sources], *(libs or [])]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature flag; that warning is expected
    noise = [ln for ln in (r.stderr or "").splitlines() if ln.strip() and "packed-fp32-ops" not in ln]
    if r.returncode != 0:
        sys.stderr.write("\n".join(noise) + "\n")
        raise RuntimeError(f"hipcc failed ({r.returncode})")
    if noise and verbose:
        sys.stderr.write("\n".join(noise) + "\n")
    os.replace(tmp, out)


if __name__ == "__main__":
    print(build(verbose=True))
