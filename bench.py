#!/usr/bin/env python3
"""Benchmark: input GB/s (bf16) of the GPU block quantizers on one MI355X.

Headline workload: Q4_K with an imatrix on the two ffn-shaped bf16 tensors
9728x2560 and 2560x9728 (weights N(0, 0.02) with log-normal per-row std
jitter, sigma 0.3; per-column log-normal imatrix). One step = one quantization
pass over both tensors, inputs already resident in HBM; the buffers rotate over
>= 1 GiB of distinct copies so the 256 MB MALL cannot serve them.

The JSON line also carries, per quant type (same shapes, with and without
imatrix), the kernel GB/s, its HBM-roofline fraction and the identical-block
percentage against the CPU oracle on a row sample; plus the CPU baseline (the
oracle, a C restatement of the reference's eager CPU path, timed on this host's
cores on the full headline workload).

usage: python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--types all|none|q4_k,...]
"""

from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
# output bytes per 256 input values (per 32 for Q4_0 -> scaled to 256)
OUT_BYTES_PER_256 = {"q4_0": 144, "q2_k": 84, "q3_k": 110, "q4_k": 144, "q5_k": 176,
                     "q6_k": 210, "iq4_xs": 136, "iq2_xxs": 66, "iq2_xs": 74, "iq2_s": 82,
                     "iq3_xxs": 98, "iq3_s": 110}
TYPE_IDS = {"q4_0": 2, "q2_k": 10, "q3_k": 11, "q4_k": 12, "q5_k": 13, "q6_k": 14, "iq4_xs": 23,
            "iq2_xxs": 16, "iq2_xs": 17, "iq2_s": 22, "iq3_xxs": 18, "iq3_s": 21}
NEEDS_IMATRIX = {"iq2_xxs", "iq2_xs", "iq2_s", "iq3_xxs"}
SHAPES = [(9728, 2560), (2560, 9728)]   # (rows, k)
ROTATE_BYTES = 1 << 30


def make_inputs(torch, dev, seed: int = 0):
    """bf16 tensors of the headline config on the device, plus per-column imatrix."""
    import numpy as np
    rng = np.random.default_rng(seed)
    xs, qws, host = [], [], []
    for rows, k in SHAPES:
        a = rng.standard_normal((rows, k), dtype=np.float32) * np.float32(0.02)
        a *= np.exp(np.float32(0.3) * rng.standard_normal((rows, 1), dtype=np.float32))
        t = torch.from_numpy(a).to(torch.bfloat16)
        host.append(t)
        xs.append(t.to(dev))
        qws.append(torch.from_numpy(rng.lognormal(0.0, 1.0, k).astype(np.float32)).to(dev))
    return xs, qws, host


def profiled_traffic() -> int | None:
    """HBM bytes per launch of the headline kernel, from the rocprofv3 FETCH_SIZE /
    WRITE_SIZE runs summarised in profiles/ (scaled by a copy of known size)."""
    f = ROOT / "profiles" / "counters_q4_k_imat_9728x2560.md"
    if f.exists():
        for ln in f.read_text().splitlines():
            if ln.startswith("traffic_bytes_per_launch:"):
                return int(ln.split(":")[1])
    return None


def algorithmic_bytes(qtype: str, n_elems: int, k: int) -> int:
    return 2 * n_elems + n_elems * OUT_BYTES_PER_256[qtype] // 256 + 4 * k


def time_type(torch, qs, qtype, imat, xs_rot, qws, outs, steps, warmup):
    """Returns (ms per step, per-shape average kernel ms) for one type."""
    tid = TYPE_IDS[qtype]
    nrot = len(xs_rot)
    stream = torch.cuda.current_stream()

    def step(i, evs=None):
        xs = xs_rot[i % nrot]
        for j, x in enumerate(xs):
            if evs is not None:
                evs[j][0].record(stream)
            qs.quantize(tid, x, qws[j] if imat else None, out=outs[j])
            if evs is not None:
                evs[j][1].record(stream)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / steps
    # per-launch kernel durations from HIP events on the launch stream
    kms = [0.0] * len(SHAPES)
    for i in range(steps):
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in SHAPES]
        step(i, evs)
        torch.cuda.synchronize()
        for j, (a, b) in enumerate(evs):
            kms[j] += a.elapsed_time(b) / steps
    return ms_step, kms


def identical_pct(torch, qs, oracle, qtype, imat, host, qws, rows=256):
    import numpy as np
    same = total = 0
    for j, (r, k) in enumerate(SHAPES):
        xb = host[j][:rows]
        qw = qws[j].cpu().numpy() if imat else None
        got = qs.quantize(TYPE_IDS[qtype], xb.to(qws[j].device), qws[j] if imat else None)
        got = got.cpu().numpy()
        ref = oracle.quantize(qtype, xb.float().numpy(), qw,
                              n_threads=len(os.sched_getaffinity(0)))
        bb = OUT_BYTES_PER_256[qtype] if qtype != "q4_0" else 18
        a, b = got.reshape(-1, bb), ref.reshape(-1, bb)
        same += int((a == b).all(1).sum())
        total += a.shape[0]
    return 100.0 * same / total


def cpu_baseline(oracle, host, qws):
    """The oracle on the full headline workload (Q4_K + imatrix), all host cores."""
    cores = len(os.sched_getaffinity(0))
    n = 0
    t0 = time.perf_counter()
    for j in range(len(SHAPES)):
        x = host[j].float().numpy()
        oracle.quantize("q4_k", x, qws[j].cpu().numpy(), n_threads=cores)
        n += x.size
    dt = time.perf_counter() - t0
    return {"value": round(2 * n / dt / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"full workload: Q4_K+imatrix on bf16 {SHAPES[0][0]}x{SHAPES[0][1]} and "
                      f"{SHAPES[1][0]}x{SHAPES[1][1]} ({n} values), {dt:.2f} s, one pass"}


def copy_peak(torch, dev, steps: int, warmup: int) -> int:
    """1 GiB device-to-device copy: measured HBM copy rate (read + write bytes)."""
    nbytes = 1 << 30
    a = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a)
    for _ in range(warmup):
        b.copy_(a)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        b.copy_(a)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes,
                      "ms_per_copy": round(dt * 1e3, 4),
                      "copy_GBps_read_plus_write": round(2 * nbytes / dt / 1e9, 1)}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--types", default="all", help="per-type table: all, none or a comma list")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--copy-only", action="store_true",
                    help="time a plain 1 GiB device copy instead (HBM copy peak, and the "
                         "reference size for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE counts)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this quantizer runs on one GPU; --gpus must be 1 "
              "(the path shards by tensor with no exchange, see the design notes)", file=sys.stderr)
        return 2

    import torch
    qs = importlib.import_module("quant-studio_amd")
    import oracle

    dev = torch.device("cuda:0")
    if args.copy_only:
        return copy_peak(torch, dev, args.steps, args.warmup)
    xs, qws, host = make_inputs(torch, dev)
    per_step_bytes = sum(2 * r * k for r, k in SHAPES)
    nrot = max(1, -(-ROTATE_BYTES // per_step_bytes))
    xs_rot = [xs] + [[x.clone() for x in xs] for _ in range(nrot - 1)]
    n_elems = sum(r * k for r, k in SHAPES)

    def outs_for(qtype):
        return [torch.empty((r, k // 256 * OUT_BYTES_PER_256[qtype]), dtype=torch.uint8, device=dev)
                for r, k in SHAPES]

    # headline: Q4_K + imatrix
    ms_step, kms = time_type(torch, qs, "q4_k", True, xs_rot, qws, outs_for("q4_k"),
                             args.steps, args.warmup)
    value = 2 * n_elems / (ms_step * 1e-3) / 1e9
    # dominant kernel: the 9728x2560 launch
    r0, k0 = SHAPES[0]
    alg = algorithmic_bytes("q4_k", r0 * k0, k0)
    achieved = alg / (kms[0] * 1e-3) / 1e9

    per_type = {}
    sel = [] if args.types == "none" else (list(TYPE_IDS) if args.types == "all"
                                           else args.types.split(","))
    for qtype in sel:
        modes = (False,) if qtype == "q4_0" else (True,) if qtype in NEEDS_IMATRIX else (False, True)
        for imat in modes:
            st, km = time_type(torch, qs, qtype, imat, xs_rot, qws, outs_for(qtype),
                               max(3, args.steps // 4), 1)
            a = sum(algorithmic_bytes(qtype, r * k, k) for r, k in SHAPES) / (sum(km) * 1e-3) / 1e9
            per_type[f"{qtype}{'+imat' if imat else ''}"] = {
                "input_GBps": round(2 * n_elems / (st * 1e-3) / 1e9, 2),
                "ms_per_step": round(st, 4),
                "kernel_ms": [round(v, 4) for v in km],
                "hbm_frac": round(a / HBM_PEAK_GBS, 4),
                "identical_pct_vs_oracle": round(identical_pct(torch, qs, oracle, qtype, imat,
                                                               host, qws), 3),
            }

    line = {
        "metric": "input GB/s (bf16) per quant type at 1 GPU + % identical blocks vs reference",
        "value": round(value, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded bf16 tensors resident in HBM, rotated over >=1 GiB)",
        "config": {"workload": "Q4_K + imatrix on bf16 ffn tensors 9728x2560 and 2560x9728",
                   "types": "q4_k", "imatrix": True, "n_values": n_elems,
                   "parallelism": "1 GPU (no exchange)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 5),
                     "traffic": profiled_traffic(),
                     "kernel": "k_q45_k<bf16, imatrix, 15>", "kernel_ms": round(kms[0], 4),
                     "algorithmic_bytes": alg},
        "per_type": per_type,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(oracle, host, qws)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
