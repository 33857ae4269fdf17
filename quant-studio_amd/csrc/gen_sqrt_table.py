#!/usr/bin/env python3
"""Generate qs_sqrt_table.h: the float32 inputs on which the reference's
square root is one ulp below the correctly rounded root.

Every weight of the reference's quantizers goes through `torch.sqrt` on a CPU
tensor (e.g. kernels/q4_k.py:34, :51; iq2.py:431, :436; iq3_xxs.py:45, :47),
which torch evaluates with MKL's vectorised square root. That routine is not
correctly rounded: for about 0.6% of inputs it returns the float just below
the IEEE root. Measured on this build (torch 2.10.0, MKL, x86-64):
  - the result is always the IEEE root or one ulp below it;
  - whether it is one below depends only on the 23 mantissa bits and the
    parity of the unbiased exponent (sqrt(x * 4^k) = sqrt(x) * 2^k), also for
    subnormal inputs after scaling by an even power of two;
  - the set is the same under ATEN_CPU_CAPABILITY default / avx2 / avx512.
So the 2^24 representatives in [1, 4) list every case. The header stores the
sorted keys (parity << 23 | mantissa) as deltas; the library expands them into
a 2 MiB bitmap on each device, and `sqrt_ref` in qs_device.h applies it. The
oracle uses the same table, and tests/test_oracle.py re-checks it against
torch.sqrt on random normal, subnormal and special inputs.

The rounding is a property of the host's MKL, not of torch: on an AMD EPYC
host (an MI355X machine's) the same torch build returns the IEEE root on 82.9%
of the keys, one ulp below on 7.4% and one ulp above on 9.8%, again a
function of the key alone and the same under every ATEN_CPU_CAPABILITY. That
host's rounding is kept as a 2-bit map per key (`--write-map`: 0 = IEEE root,
1 = one ulp below, 2 = one ulp above; key 4i + j in bits 2j..2j+1 of byte i;
zlib-compressed) in qs_sqrt_amd.bin, which the library embeds.

usage: python quant-studio_amd/csrc/gen_sqrt_table.py           (CPU torch required)
       python quant-studio_amd/csrc/gen_sqrt_table.py --write-map PATH   this host's
           rounding as a compressed 2-bit map (run on the host whose torch.sqrt it records)
       python quant-studio_amd/csrc/gen_sqrt_table.py --check   recompute the set on this
           host and compare it with the committed header (prints the host CPU, torch and
           MKL versions, the key count and both SHA-256 digests; exit 1 if they differ)
"""

from __future__ import annotations

import hashlib
import re
import sys
import zlib
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "qs_sqrt_table.h"
AMD_MAP = Path(__file__).resolve().parent / "qs_sqrt_amd.bin"


def down_keys() -> np.ndarray:
    m = np.arange(1 << 23, dtype=np.uint32)
    bits = np.concatenate([(127 << 23) | m, (128 << 23) | m])     # [1, 2) then [2, 4)
    x = bits.view(np.float32)
    got = torch.sqrt(torch.from_numpy(x)).numpy().view(np.int32)
    ieee = np.sqrt(x.astype(np.float64)).astype(np.float32).view(np.int32)
    d = got - ieee
    if not np.isin(d, (0, -1)).all():
        raise SystemExit("torch.sqrt differs from the IEEE root by more than one ulp below")
    return np.nonzero(d == -1)[0].astype(np.uint32)                 # index = parity << 23 | mantissa


def rounding_census() -> dict:
    """How torch.sqrt on this host differs from the IEEE root over the 2^24
    representatives in [1, 4): counts per difference in ulps, and the keys
    (parity << 23 | mantissa) of each non-zero difference."""
    m = np.arange(1 << 23, dtype=np.uint32)
    bits = np.concatenate([(127 << 23) | m, (128 << 23) | m])
    x = bits.view(np.float32)
    got = torch.sqrt(torch.from_numpy(x)).numpy().view(np.int32)
    ieee = np.sqrt(x.astype(np.float64)).astype(np.float32).view(np.int32)
    d = (got - ieee).astype(np.int64)
    vals, counts = np.unique(d, return_counts=True)
    return {"counts": {int(v): int(c) for v, c in zip(vals, counts)},
            "keys": {int(v): np.nonzero(d == v)[0].astype(np.uint32) for v in vals if v != 0}}


def encode_map(diff: np.ndarray) -> bytes:
    """Per-key ulp offsets (-1, 0, +1; 2^24 of them) as the compressed 2-bit map."""
    code = np.where(diff == -1, 1, np.where(diff == 1, 2, 0)).astype(np.uint8)
    packed = code[0::4] | (code[1::4] << 2) | (code[2::4] << 4) | (code[3::4] << 6)
    return zlib.compress(packed.astype(np.uint8).tobytes(), 9)


def decode_map(blob: bytes) -> np.ndarray:
    """The compressed 2-bit map back as 2^24 int8 ulp offsets."""
    packed = np.frombuffer(zlib.decompress(blob), dtype=np.uint8)
    code = np.stack([(packed >> (2 * j)) & 3 for j in range(4)], axis=1).reshape(-1)
    if code.size != 1 << 24 or (code == 3).any():
        raise ValueError("not a 2-bit square-root map of 2^24 keys")
    return np.where(code == 1, -1, np.where(code == 2, 1, 0)).astype(np.int8)


def header_keys() -> np.ndarray:
    """The keys stored in the committed header (gaps summed back)."""
    text = OUT.read_text()
    body = text[text.index("= {") + 3: text.index("};")]
    gaps = np.array([int(v) for v in re.findall(r"\d+", body)], dtype=np.int64)
    return np.cumsum(gaps).astype(np.uint32)


def host_cpu() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def check() -> int:
    census = rounding_census()
    here = census["keys"].get(-1, np.zeros(0, np.uint32))
    diff = np.zeros(1 << 24, np.int8)
    for v, k in census["keys"].items():
        diff[k] = v
    amd = decode_map(AMD_MAP.read_bytes()) if AMD_MAP.exists() else None
    committed = header_keys()
    same = set(census["counts"]) <= {0, -1} and here.size == committed.size and \
        bool((here == committed).all())
    mkl = [ln.strip() for ln in torch.__config__.show().splitlines() if "Math Kernel Library" in ln]
    print(f"cpu: {host_cpu()}")
    print(f"torch: {torch.__version__}; mkl available: {torch.backends.mkl.is_available()}; "
          f"{mkl[0] if mkl else 'no MKL line in torch config'}")
    print(f"cpu capability: {torch.backends.cpu.get_cpu_capability()}")
    print("torch.sqrt - IEEE root, in ulps, over the 2^24 keys: "
          + ", ".join(f"{v:+d}: {c}" for v, c in sorted(census["counts"].items())))
    for v, k in sorted(census["keys"].items()):
        print(f"  keys at {v:+d} ulp: {k.size}, sha256 {hashlib.sha256(k.tobytes()).hexdigest()}")
    print(f"this host: {here.size} keys one ulp below, sha256 {hashlib.sha256(here.tobytes()).hexdigest()}")
    print(f"header:    {committed.size} keys, sha256 {hashlib.sha256(committed.tobytes()).hexdigest()}")
    if not same:
        only_here = np.setdiff1d(here, committed).size
        only_hdr = np.setdiff1d(committed, here).size
        print(f"DIFFERENT: one ulp below on {only_here} keys only on this host, {only_hdr} only "
              f"in the header; other differences: "
              f"{sum(c for v, c in census['counts'].items() if v not in (0, -1))} keys")
    else:
        print("identical")
    if amd is not None:
        same_amd = bool((amd == diff).all())
        print(f"{AMD_MAP.name}: {'identical to' if same_amd else 'differs from'} this host's rounding "
              f"({int((amd != diff).sum())} keys differ)")
        same = same or same_amd
    return 0 if same else 1


def main() -> None:
    if "--check" in sys.argv[1:]:
        sys.exit(check())
    if "--write-map" in sys.argv[1:]:
        path = Path(sys.argv[sys.argv.index("--write-map") + 1])
        census = rounding_census()
        diff = np.zeros(1 << 24, np.int8)
        for v, k in census["keys"].items():
            diff[k] = v
        if not set(census["counts"]) <= {-1, 0, 1}:
            raise SystemExit("torch.sqrt differs from the IEEE root by more than one ulp")
        blob = encode_map(diff)
        path.write_bytes(blob)
        print(f"{path}: {len(blob)} bytes; host {host_cpu()}; "
              + ", ".join(f"{v:+d}: {c}" for v, c in sorted(census["counts"].items())))
        return
    keys = down_keys()
    deltas = np.diff(np.concatenate([[0], keys])).astype(np.int64)
    if (deltas >= 1 << 16).any():
        raise SystemExit("a key gap does not fit in 16 bits")
    digest = hashlib.sha256(keys.tobytes()).hexdigest()
    lines = [
        "// Generated by gen_sqrt_table.py; do not edit.",
        "// Float32 square roots that the reference's torch.sqrt (CPU, MKL) returns one ulp",
        "// below the correctly rounded root, keyed by (exponent parity << 23 | mantissa) of",
        "// the input (subnormals scaled by an even power of two first). Sorted keys, stored",
        f"// as gaps from the previous key (the first from 0). {keys.size} keys, sha256 {digest}",
        "#pragma once",
        "#include <stdint.h>",
        "",
        f"#define QS_SQRT_DOWN_N {keys.size}",
        f"static const uint16_t QS_SQRT_DOWN_GAPS[{keys.size}] = {{",
    ]
    for i in range(0, keys.size, 20):
        lines.append("    " + ", ".join(str(int(v)) for v in deltas[i:i + 20]) + ",")
    lines.append("};")
    OUT.write_text("\n".join(lines) + "\n")
    print(f"{OUT}: {keys.size} keys ({keys.size / (1 << 24) * 100:.3f}% of keys)")


if __name__ == "__main__":
    main()
