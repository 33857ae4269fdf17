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
# output bytes per 256 input values (32-value formats: 8 blocks)
OUT_BYTES_PER_256 = {"q4_0": 144, "q2_k": 84, "q3_k": 110, "q4_k": 144, "q5_k": 176,
                     "q6_k": 210, "iq4_xs": 136, "iq2_xxs": 66, "iq2_xs": 74, "iq2_s": 82,
                     "iq3_xxs": 98, "iq3_s": 110, "q4_1": 160, "q5_0": 176, "q5_1": 192,
                     "q8_0": 272, "iq4_nl": 144}
TYPE_IDS = {"q4_0": 2, "q2_k": 10, "q3_k": 11, "q4_k": 12, "q5_k": 13, "q6_k": 14, "iq4_xs": 23,
            "iq2_xxs": 16, "iq2_xs": 17, "iq2_s": 22, "iq3_xxs": 18, "iq3_s": 21,
            "q4_1": 3, "q5_0": 6, "q5_1": 7, "q8_0": 8, "iq4_nl": 20}
NEEDS_IMATRIX = {"iq2_xxs", "iq2_xs", "iq2_s", "iq3_xxs"}
IGNORE_IMATRIX = {"q4_0", "q4_1", "q5_0", "q5_1", "q8_0"}
BLOCK_BYTES = {t: (b // 8 if t in IGNORE_IMATRIX | {"iq4_nl"} else b) for t, b in OUT_BYTES_PER_256.items()}
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


def profiled(key: str) -> int | None:
    """A per-launch figure of the headline kernel from the rocprofv3 counter runs
    summarised in profiles/: HBM bytes (FETCH_SIZE + WRITE_SIZE, scaled by a copy
    of known size) or VALU wave instructions (SQ_INSTS_VALU)."""
    f = ROOT / "profiles" / "counters_q4_k_imat_9728x2560.md"
    if f.exists():
        for ln in f.read_text().splitlines():
            if ln.startswith(key + ":"):
                return int(ln.split(":")[1])
    return None


def profiled_valu_per_type() -> dict:
    """SQ_INSTS_VALU per launch of every per-type kernel (rocprofv3 counter run
    summarised in profiles/), keyed like per_type."""
    f = ROOT / "profiles" / "valu_insts_per_type_ffn_9728x2560_2560x9728.md"
    out = {}
    if f.exists():
        for ln in f.read_text().splitlines():
            if ln.startswith("valu_insts[") and "]:" in ln:
                key, val = ln[len("valu_insts["):].split("]:")
                out[key] = float(val)
    return out


def valu_peak(torch, dev, launches: int = 5) -> float:
    """Measured VALU issue rate (wave instructions per second) of a kernel that
    issues only independent f32 multiplies and adds (libqs_calib.so)."""
    import ctypes
    lib = ctypes.CDLL(str(ROOT / "quant-studio_amd" / "_build" / "libqs_calib.so"))
    lib.qs_calib_valu.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.qs_calib_valu_insts.restype = ctypes.c_double
    lib.qs_calib_valu_insts.argtypes = [ctypes.c_int, ctypes.c_int]
    grid, iters = 8192, 4096       # ~7 ms per launch
    out = torch.empty(1, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream()
    run = lambda: lib.qs_calib_valu(grid, iters, ctypes.c_void_p(out.data_ptr()),
                                    ctypes.c_void_p(stream.cuda_stream))
    assert run() == 0
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(launches):
        run()
    b.record(stream)
    torch.cuda.synchronize()
    sec = a.elapsed_time(b) * 1e-3 / launches
    return lib.qs_calib_valu_insts(grid, iters) / sec


def algorithmic_bytes(qtype: str, n_elems: int, k: int) -> int:
    return 2 * n_elems + n_elems * OUT_BYTES_PER_256[qtype] // 256 + 4 * k


def time_type(torch, qs, qtype, imat, xs_rot, qws, outs, steps, warmup):
    """Returns (ms per step, per-shape average kernel ms) for one type."""
    tid = TYPE_IDS[qtype]
    nrot = len(xs_rot)
    stream = torch.cuda.current_stream()

    def step(i):
        xs = xs_rot[i % nrot]
        for j, x in enumerate(xs):
            qs.quantize(tid, x, qws[j] if imat else None, out=outs[j])

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / steps
    # per-launch kernel durations from HIP events on the launch stream: each
    # shape's launches back to back between one pair of events, so the host's
    # launch overhead (~8 us per call) overlaps the queued kernels instead of
    # being counted in short ones
    kms = []
    for j, _ in enumerate(SHAPES):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(steps):
            qs.quantize(tid, xs_rot[i % nrot][j], qws[j] if imat else None, out=outs[j])
        b.record(stream)
        torch.cuda.synchronize()
        kms.append(a.elapsed_time(b) / steps)
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
        bb = BLOCK_BYTES[qtype]
        a, b = got.reshape(-1, bb), ref.reshape(-1, bb)
        same += int((a == b).all(1).sum())
        total += a.shape[0]
    return 100.0 * same / total


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or "unknown"."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(oracle, host, qws):
    """The oracle on the full headline workload (Q4_K + imatrix), all host
    cores; plus one thread on the first eighth of each tensor's rows."""
    cores = len(os.sched_getaffinity(0))

    def run(rows_frac, threads):
        n = 0
        t0 = time.perf_counter()
        for j in range(len(SHAPES)):
            x = host[j][: max(1, SHAPES[j][0] // rows_frac)].float().numpy()
            oracle.quantize("q4_k", x, qws[j].cpu().numpy(), n_threads=threads)
            n += x.size
        return n, time.perf_counter() - t0

    n, dt = run(1, cores)
    n1, dt1 = run(8, 1)
    return {"value": round(2 * n / dt / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "value_1_thread": round(2 * n1 / dt1 / 1e9, 5), "cpu": cpu_model(),
            "sample": f"full workload: Q4_K+imatrix on bf16 {SHAPES[0][0]}x{SHAPES[0][1]} and "
                      f"{SHAPES[1][0]}x{SHAPES[1][1]} ({n} values), {dt:.2f} s, one pass; "
                      f"1 thread: the first 1/8 of each tensor's rows ({n1} values), {dt1:.2f} s"}


def q4_0_large(torch, qs, dev, steps: int) -> dict:
    """Q4_0 on a token_embd-shaped bf16 tensor (151936 x 2560, 778 MB), two
    rotating copies: the HBM-bound case at a size where launch ramp-up is small."""
    rows, k = 151936, 2560
    g = torch.Generator(device=dev).manual_seed(1)
    xs = [(torch.randn(rows, k, device=dev, generator=g) * 0.01).to(torch.bfloat16) for _ in range(2)]
    out = torch.empty((rows, k // 32 * 18), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    # ~6 ms of warm-up: the first launches after the other kernels run below
    # the GPU's sustained clocks; then the median of three timed groups
    for i in range(30):
        qs.quantize(2, xs[i % 2], None, out=out)
    groups = []
    for _ in range(3):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(steps):
            qs.quantize(2, xs[i % 2], None, out=out)
        b.record(stream)
        torch.cuda.synchronize()
        groups.append(a.elapsed_time(b) / steps)
    ms = sorted(groups)[1]
    alg = algorithmic_bytes("q4_0", rows * k, k) - 4 * k
    return {"input_GBps": round(2 * rows * k / (ms * 1e-3) / 1e9, 1), "kernel_ms": round(ms, 4),
            "hbm_GBps": round(alg / (ms * 1e-3) / 1e9, 1), "hbm_frac": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


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


# ---------------------------------------------------------------------------
# end-to-end: the CLI on a synthetic 4B-class bf16 GGUF
# ---------------------------------------------------------------------------

def synth_model(torch, dev, path: Path, im_path: Path, seed: int = 0) -> int:
    """Qwen3-like 4B-class bf16 model: 36 layers, hidden 2560, ffn 9728, 32 q /
    8 kv heads of dim 128, vocab 151936, tied embeddings; weights N(0, 0.02),
    embedding N(0, 0.01). Imatrix per tensor: per-column log-normal(0, 1).
    Values are drawn on the GPU; returns the number of weight values."""
    import numpy as np
    qs_io = importlib.import_module("quant-studio_amd.gguf_io")
    GT = importlib.import_module("quant-studio_amd.gguf_types").GGMLQuantizationType
    KV, VT = qs_io.KV, qs_io.VT
    L, H, F, V = 36, 2560, 9728, 151936
    tensors = [("token_embd.weight", (H, V), 0.01)]
    for i in range(L):
        p = f"blk.{i}."
        tensors += [(p + "attn_norm.weight", (H,), None), (p + "attn_q.weight", (H, 4096), 0.02),
                    (p + "attn_k.weight", (H, 1024), 0.02), (p + "attn_v.weight", (H, 1024), 0.02),
                    (p + "attn_q_norm.weight", (128,), None), (p + "attn_k_norm.weight", (128,), None),
                    (p + "attn_output.weight", (4096, H), 0.02), (p + "ffn_norm.weight", (H,), None),
                    (p + "ffn_gate.weight", (H, F), 0.02), (p + "ffn_up.weight", (H, F), 0.02),
                    (p + "ffn_down.weight", (F, H), 0.02)]
    tensors.append(("output_norm.weight", (H,), None))
    kvs = [KV("qwen3.block_count", VT.UINT32, L), KV("qwen3.context_length", VT.UINT32, 40960),
           KV("qwen3.embedding_length", VT.UINT32, H), KV("qwen3.feed_forward_length", VT.UINT32, F),
           KV("qwen3.attention.head_count", VT.UINT32, 32),
           KV("qwen3.attention.head_count_kv", VT.UINT32, 8),
           KV("qwen3.attention.key_length", VT.UINT32, 128),
           KV("general.file_type", VT.UINT32, 32), KV("general.name", VT.STRING, "synthetic-4b")]
    w = qs_io.GGUFWriter(path, "qwen3")
    for kv in kvs:
        w.add_kv(kv)
    for name, ne, std in tensors:
        n = int(np.prod(ne))
        w.add_tensor_info(name, ne, GT.BF16 if std else GT.F32, n * (2 if std else 4))
    f = w.write_header()
    g = torch.Generator(device=dev).manual_seed(seed)
    rng = np.random.default_rng(seed)
    n_weights = 0
    im_tensors = []
    for name, ne, std in tensors:
        w.pad()
        n = int(np.prod(ne))
        if std is None:
            f.write(np.ones(n, np.float32).tobytes())
            continue
        t = (torch.randn(n, device=dev, generator=g) * std).to(torch.bfloat16)
        f.write(t.view(torch.int16).cpu().numpy().tobytes())
        n_weights += n
        v = rng.lognormal(0.0, 1.0, ne[0]).astype(np.float32)
        im_tensors += [(name + ".in_sum2", (ne[0],), GT.F32, v * np.float32(100.0)),
                       (name + ".counts", (1,), GT.F32, np.array([100.0], np.float32))]
    w.pad()
    w.close()
    qs_io.write_gguf(im_path, "imatrix", [KV("general.type", VT.STRING, "imatrix")], im_tensors)
    return n_weights


def run_e2e(torch, dev, schemes: list[str]) -> int:
    import re
    import subprocess
    import tempfile
    base = Path("/dev/shm") if Path("/dev/shm").is_dir() else Path(tempfile.gettempdir())
    with tempfile.TemporaryDirectory(dir=base) as d:
        d = Path(d)
        src, im = d / "model-bf16.gguf", d / "imatrix.gguf"
        t0 = time.perf_counter()
        n = synth_model(torch, dev, src, im)
        gen_s = time.perf_counter() - t0
        results = {}
        for sch in schemes:
            name, *extra = sch.split()
            out = d / f"out-{name}.gguf"
            cmd = [sys.executable, str(ROOT / "quant-studio.py"), str(src), str(out), name,
                   "--imatrix", str(im), *extra]
            t0 = time.perf_counter()
            r = subprocess.run(cmd, capture_output=True, text=True)
            wall = time.perf_counter() - t0
            if r.returncode != 0:
                print(r.stderr[-2000:], file=sys.stderr)
                return 1
            m = re.search(r"done in ([0-9.]+)s", r.stdout)
            results[sch] = {"pipeline_s": float(m.group(1)) if m else None,
                            "process_wall_s": round(wall, 2),
                            "input_GBps_pipeline": round(src.stat().st_size / 1e9 / float(m.group(1)), 2)
                            if m and float(m.group(1)) > 0 else None,
                            "out_bytes": out.stat().st_size}
            out.unlink()
            print(f"e2e {sch}: {results[sch]}", file=sys.stderr, flush=True)
        print(json.dumps({"e2e": "synthetic 4B-class bf16 GGUF (36 layers, 2560/9728, vocab 151936), "
                                 "file in page cache", "file_bytes": src.stat().st_size,
                          "weights": n, "generate_s": round(gen_s, 1), "runs": results}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--types", default="all", help="per-type table: all, none or a comma list")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--e2e", default=None,
                    help="run the CLI end to end on a synthetic 4B-class model for these "
                         "';'-separated schemes (e.g. 'IQ2_XXS;Q4_K_M') and print its own JSON line")
    ap.add_argument("--valu-peak", action="store_true",
                    help="time the VALU issue-rate kernel only (the reference for SQ_INSTS_VALU)")
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
    if args.valu_peak:
        print(json.dumps({"valu_wave_instr_per_s": round(valu_peak(torch, dev, args.steps))}), flush=True)
        return 0
    if args.e2e:
        return run_e2e(torch, dev, [x.strip() for x in args.e2e.split(";") if x.strip()])
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
    valu_counts = profiled_valu_per_type()
    peak_valu = valu_peak(torch, dev)
    sel = [] if args.types == "none" else (list(TYPE_IDS) if args.types == "all"
                                           else args.types.split(","))
    for qtype in sel:
        modes = (False,) if qtype in IGNORE_IMATRIX else (True,) if qtype in NEEDS_IMATRIX else (False, True)
        for imat in modes:
            st, km = time_type(torch, qs, qtype, imat, xs_rot, qws, outs_for(qtype),
                               max(3, args.steps // 4), 1)
            a = sum(algorithmic_bytes(qtype, r * k, k) for r, k in SHAPES) / (sum(km) * 1e-3) / 1e9
            key = f"{qtype}{'+imat' if imat else ''}"
            insts = valu_counts.get(key)
            per_type[key] = {
                "input_GBps": round(2 * n_elems / (st * 1e-3) / 1e9, 2),
                "ms_per_step": round(st, 4),
                "kernel_ms": [round(v, 4) for v in km],
                "hbm_frac": round(a / HBM_PEAK_GBS, 4),
                # VALU issue rate (SQ_INSTS_VALU per launch over the live launch
                # time) against the calibration kernel's rate
                "valu_frac": None if insts is None else
                round(insts / (sum(km) / len(km) * 1e-3) / peak_valu, 3),
                "identical_pct_vs_oracle": round(identical_pct(torch, qs, oracle, qtype, imat,
                                                               host, qws), 3),
            }

    if "q4_0" in sel:
        per_type["q4_0 token_embd 151936x2560"] = q4_0_large(torch, qs, dev, 20)
    insts = profiled("valu_insts_per_launch")

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
                     "traffic": profiled("traffic_bytes_per_launch"),
                     "kernel": "k_q45_k<bf16, imatrix, 15>", "kernel_ms": round(kms[0], 4),
                     "algorithmic_bytes": alg,
                     # the kernel is VALU-bound: its SQ_INSTS_VALU per launch over its
                     # live duration, against the measured issue rate of a pure
                     # mul/add kernel
                     "valu": None if insts is None else {
                         "insts_per_launch": insts, "unit": "G wave-instr/s",
                         "achieved": round(insts / (kms[0] * 1e-3) / 1e9, 1),
                         "peak": round(peak_valu / 1e9, 1),
                         "frac": round(insts / (kms[0] * 1e-3) / peak_valu, 4)}},
        "per_type": per_type,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(oracle, host, qws)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
