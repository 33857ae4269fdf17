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
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "_build" / "libqs_hip.so"
CALIB_OUT = PKG / "_build" / "libqs_calib.so"       # measurement aid for bench.py

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]
# (source, extra defines): qs_launch.hip is built once per source element type
# (qs::SRC_F32 = 0, SRC_F16 = 1, SRC_BF16 = 30) so the kernel instantiations
# compile in parallel
UNITS = [
    ("qs_api.hip", [f'-DQS_SQRT_AMD_BIN="{CSRC / "qs_sqrt_amd.bin"}"']),   # embeds the AMD-host map
    ("qs_pipeline.cpp", []),
    ("qs_launch.hip", ["-DQS_LAUNCH_SRC=0"]),
    ("qs_launch.hip", ["-DQS_LAUNCH_SRC=1"]),
    ("qs_launch.hip", ["-DQS_LAUNCH_SRC=30"]),
]


def build(verbose: bool = False) -> Path:
    objs = OUT.parent / "obj"
    objs.mkdir(parents=True, exist_ok=True)
    jobs = []
    for i, (src, defs) in enumerate(UNITS):
        obj = objs / f"{i}_{Path(src).stem}.o"
        jobs.append(([HIPCC, *FLAGS, "-c", *defs, *_includes(), "-o", str(obj), str(CSRC / src)], obj))
    with ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 1)) as ex:
        list(ex.map(lambda j: _run(j[0], verbose), jobs))
    _link(OUT, [o for _, o in jobs], ["-lz"], verbose)
    _link(CALIB_OUT, [CSRC / "qs_calib.hip"], [], verbose, compile_flags=True)
    return OUT


def _includes() -> list[str]:
    return [f"-I{ROOT / 'include'}", f"-I{CSRC}"]


def _link(out: Path, inputs: list[Path], libs: list[str], verbose: bool, compile_flags: bool = False) -> None:
    out.parent.mkdir(parents=True, exist_ok=True)
    tmp = out.with_name(out.name + ".tmp")
    cmd = [HIPCC, *(FLAGS if compile_flags else ["--offload-arch=gfx950", "-fPIC"]), "-shared",
           *(_includes() if compile_flags else []), "-o", str(tmp), *[str(i) for i in inputs], *libs]
    _run(cmd, verbose)
    os.replace(tmp, out)


def _run(cmd: list[str], verbose: bool) -> None:
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


if __name__ == "__main__":
    print(build(verbose=True))
