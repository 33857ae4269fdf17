#!/usr/bin/env python3
"""Benchmark: input GB/s (bf16) of the GPU block quantizers on one MI355X.

Headline workload: Q4_K with an imatrix on the two ffn-shaped bf16 tensors
9728x2560 and 2560x9728 (weights N(0, 0.02) with log-normal per-row std
jitter, sigma 0.3; per-column log-normal imatrix). One step = one quantization
pass over both tensors (two launches), inputs already resident in HBM; the
buffers rotate over >= 1 GiB of distinct copies so the 256 MB MALL cannot
serve them. The core clock follows VALU load, so the VALU-calibration kernel
(~0.2 s of full-chip VALU work, measured for the line anyway) runs right
before the headline's own warm-up and the timed launches queue behind VALU
work. The timed steps run back to back between two HIP events on the launch
stream; both launches of a step run the same kernel, so its average launch is
the step time over two.

The JSON line also carries:
  - per_type: every HIP type with and without imatrix on the same shapes:
    kernel GB/s, HBM-roofline fraction and VALU fraction; the 32-value
    formats also against a copy kernel (at 1 GiB, and moving the same bytes
    per launch: the ceiling of a launch that size);
  - configs: Q4_0 on one 4096x4096 bf16 tensor with 0.1% outliers (seed 0),
    and IQ2_XXS + imatrix on 36 heavy-tailed (Student-t, df 5) 2560x9728
    ffn_down tensors, each timed as its own workload;
  - cpu_baseline: the oracle (a C restatement of the reference's eager CPU
    path) on this host's cores: the full headline workload timed, and per
    type the full tensors, whose bytes also give each type's identical-block
    percentage against the GPU, with the weighted-MSE tie rule applied to
    every block that differs.

usage: python bench.py [--gpus 1] [--steps 100] [--warmup 300] [--types all|none|q4_k,...]
       python bench.py --e2e 'IQ2_XXS;Q4_K_M'   the command line end to end on a
                                               synthetic 4B-class model (warm and cold)
       python bench.py --e2e all               the same for the reference's published runs
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
NEEDS_IMATRIX = {"iq2_xxs", "iq2_xs", "iq2_s"}   # IQ3_XXS also runs without one (timed both ways)
IGNORE_IMATRIX = {"q4_0", "q4_1", "q5_0", "q5_1", "q8_0"}
B32_TYPES = IGNORE_IMATRIX          # the 32-value formats: HBM-bound, compared with a copy
BLOCK_VALUES = {t: (32 if t in IGNORE_IMATRIX | {"iq4_nl"} else 256) for t in OUT_BYTES_PER_256}
BLOCK_BYTES = {t: OUT_BYTES_PER_256[t] * BLOCK_VALUES[t] // 256 for t in OUT_BYTES_PER_256}
SHAPES = [(9728, 2560), (2560, 9728)]   # (rows, k)
ROTATE_BYTES = 1 << 30


def modes_of(qtype: str) -> tuple:
    return (False,) if qtype in IGNORE_IMATRIX else (True,) if qtype in NEEDS_IMATRIX else (False, True)


def bf16_from(torch, a):
    """float32 numpy array -> bf16 torch tensor (round to nearest even)."""
    return torch.from_numpy(a.astype("float32", copy=False)).to(torch.bfloat16)


def make_inputs(torch, dev, seed: int = 0):
    """bf16 tensors of the headline config on the device, plus per-column imatrix."""
    import numpy as np
    rng = np.random.default_rng(seed)
    xs, qws, host = [], [], []
    for rows, k in SHAPES:
        a = rng.standard_normal((rows, k), dtype=np.float32) * np.float32(0.02)
        a *= np.exp(np.float32(0.3) * rng.standard_normal((rows, 1), dtype=np.float32))
        t = bf16_from(torch, a)
        host.append(t)
        xs.append(t.to(dev))
        qws.append(torch.from_numpy(rng.lognormal(0.0, 1.0, k).astype(np.float32)).to(dev))
    return xs, qws, host


def profile_figure(name: str, key: str) -> float | None:
    """A figure recorded by a rocprofv3 summary in profiles/ (lines `key: value`)."""
    f = ROOT / "profiles" / name
    if f.exists():
        for ln in f.read_text().splitlines():
            if ln.startswith(key + ":"):
                return float(ln.split(":", 1)[1])
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
    global VALU_RATE
    VALU_RATE = lib.qs_calib_valu_insts(grid, iters) / sec
    return VALU_RATE


def _calib_lib():
    import ctypes
    lib = ctypes.CDLL(str(ROOT / "quant-studio_amd" / "_build" / "libqs_calib.so"))
    lib.qs_calib_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_longlong, ctypes.c_void_p]
    return lib


def copy_kernel_peak(torch, dev, nbytes: int = 1 << 30, launches: int = 10) -> float:
    """Measured copy rate (read + written bytes per second) of a streaming
    16-byte copy kernel shaped like the 32-value quantizer (libqs_calib.so),
    1 GiB each way, launches back to back."""
    import ctypes
    lib = _calib_lib()
    a = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a)
    stream = torch.cuda.current_stream()
    run = lambda: lib.qs_calib_copy(ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(b.data_ptr()),
                                    nbytes, ctypes.c_void_p(stream.cuda_stream))
    assert run() == 0
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(launches):
        run()
    e1.record(stream)
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) * 1e-3 / launches
    del a, b
    return 2 * nbytes / sec


def copy_kernel_rate(torch, dev, traffic: int, steps: int = 24) -> float:
    """Read + written bytes per second of the same copy kernel when one launch
    moves `traffic` bytes (half read, half written): the ceiling of a launch of
    that size, ramp-up and drain included. Buffer pairs rotate over >= 1 GiB so
    the MALL holds none of them; launches run back to back (time_steps)."""
    import ctypes
    lib = _calib_lib()
    n = max(16, traffic // 2 // 16 * 16)
    pairs = max(2, -(-(1 << 30) // (2 * n)))
    bufs = [(torch.empty(n, dtype=torch.uint8, device=dev).fill_(1),
             torch.empty(n, dtype=torch.uint8, device=dev)) for _ in range(pairs)]
    stream = torch.cuda.current_stream()

    def launch(i):
        a, b = bufs[i % pairs]
        rc = lib.qs_calib_copy(ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(b.data_ptr()), n,
                               ctypes.c_void_p(stream.cuda_stream))
        if rc:
            raise RuntimeError(f"qs_calib_copy failed ({rc})")
    # median of five short regions, as the 32-value rows it is compared with
    _, ms = sorted(time_steps(torch, [launch], steps, 5) for _ in range(5))[2]
    del bufs
    torch.cuda.empty_cache()
    return 2 * n / (ms * 1e-3)


def algorithmic_bytes(qtype: str, n_elems: int, k: int) -> int:
    """bf16 in + packed blocks out + the imatrix (4k bytes)."""
    return 2 * n_elems + n_elems * OUT_BYTES_PER_256[qtype] // 256 + 4 * k


# VALU wave instructions per second of k_valu_issue on this device (set by
# valu_peak(); before that a typical MI355X figure sizes the stream hold)
VALU_RATE = 1.1e12


def busy_hold(torch, seconds: float) -> None:
    """Hold the current stream for about `seconds` with the VALU issue kernel
    on every CU (libqs_calib.so). The core clock follows VALU load: after an
    idle stretch, a one-wave spin or a memory-bound kernel, the first ~60
    headline launches (~25 ms) ran up to 14% slower, while straight after VALU
    work they ran at their steady rate from the first launch. So the timed
    launches queue behind VALU work, not behind an idle spin."""
    import ctypes
    lib = ctypes.CDLL(str(ROOT / "quant-studio_amd" / "_build" / "libqs_calib.so"))
    lib.qs_calib_valu.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    grid = 8192
    iters = max(1, int(seconds * VALU_RATE / (grid * 4 * 2 * 16)))
    out = torch.empty(1, dtype=torch.float32, device=torch.device("cuda", torch.cuda.current_device()))
    if lib.qs_calib_valu(grid, iters, ctypes.c_void_p(out.data_ptr()),
                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) != 0:
        raise RuntimeError("qs_calib_valu failed")


def time_steps(torch, launches, steps: int, warmup: int):
    """Run `warmup` untimed steps, then time exactly `steps` steps, a step being
    the callables in `launches` (each queues one kernel; called with the step
    index). Returns (ms per step, mean ms per launch) from two events on the
    launch stream, one before the first timed launch and one after the last;
    the launches run back to back between them. No event sits between launches:
    each event marker costs the command processor 2-5 us, a third of a
    12-us kernel. The stream is held by VALU work (busy_hold) while the timed
    launches are queued, so kernels shorter than the host's launch cost still
    run back to back and the clock does not drop before them. The hold is not
    timed."""
    stream = torch.cuda.current_stream()
    t0 = time.perf_counter()
    for i in range(warmup):
        for f in launches:
            f(i)
    # host time to queue one launch, from the warm-up (at least 50 us assumed)
    per_launch_s = max(50e-6, (time.perf_counter() - t0) / max(1, warmup * len(launches)))
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    hold_s = min(2.0, 2.0 * per_launch_s * steps * len(launches) + 2e-3)
    busy_hold(torch, hold_s)
    e0.record(stream)
    for i in range(steps):
        for f in launches:
            f(i)
    e1.record(stream)
    torch.cuda.synchronize()
    step_ms = e0.elapsed_time(e1) / steps
    return step_ms, step_ms / len(launches)


def shape_launches(qs, qtype, imat, xs_rot, qws, outs):
    tid = TYPE_IDS[qtype]
    return [(lambda i, j=j: qs.quantize(tid, xs_rot[i % len(xs_rot)][j], qws[j] if imat else None,
                                        out=outs[j]))
            for j in range(len(SHAPES))]


def gpu_bytes(torch, qs, qtype, imat, xs, qws):
    """The GPU's bytes for the first input copy (both shapes), on the host."""
    out = [qs.quantize(TYPE_IDS[qtype], x, qws[j] if imat else None) for j, x in enumerate(xs)]
    torch.cuda.synchronize()
    return [o.cpu().numpy() for o in out]


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


def compare_blocks(qtype, got, ref, x_f32, qw):
    """Identical blocks of two packed outputs (one tensor), and for every
    block that differs whether the GPU's imatrix-weighted MSE is <= the
    oracle's (the tie rule): returns (blocks, identical, differing_with_le_mse)."""
    import numpy as np
    bb = BLOCK_BYTES[qtype]
    a, b = got.reshape(-1, bb), ref.reshape(-1, bb)
    same = (a == b).all(1)
    le = 0
    if not same.all():
        if str(ROOT / "tests") not in sys.path:
            sys.path.insert(0, str(ROOT / "tests"))
        import dequant
        rows = np.nonzero((~same).reshape(x_f32.shape[0], -1).any(1))[0]
        ea = dequant.block_weighted_mse(qtype, got[rows], x_f32[rows], qw)
        eb = dequant.block_weighted_mse(qtype, ref[rows], x_f32[rows], qw)
        d = ~same.reshape(x_f32.shape[0], -1)[rows].reshape(-1)
        le = int((ea[d] <= eb[d]).sum())
    return int(same.size), int(same.sum()), le


def cpu_baseline(oracle, host, qws, gpu_out: dict, seconds_per_type: float):
    """The CPU leg: the oracle on this host's cores.
      - value: the full headline workload (Q4_K + imatrix, both tensors), one
        pass, all cores; plus one thread on the first eighth of each tensor;
      - per_type: each type on the full tensors (or, past seconds_per_type of
        projected CPU time, on the leading rows that fit), its CPU GB/s, and
        its bytes compared with the GPU's: identical blocks and the tie rule."""
    import numpy as np
    cores = len(os.sched_getaffinity(0))
    xf = [h.float().numpy() for h in host]
    qwn = [q.cpu().numpy() for q in qws]

    def run(qtype, imat, rows, threads):
        outs, n = [], 0
        t0 = time.perf_counter()
        for j in range(len(SHAPES)):
            x = xf[j][:rows[j]]
            if x.shape[0] == 0:
                continue
            outs.append(oracle.quantize(qtype, x, qwn[j] if imat else None, n_threads=threads))
            n += x.size
        return outs, n, time.perf_counter() - t0

    full = [r for r, _ in SHAPES]
    ref, n, dt = run("q4_k", True, full, cores)
    _, n1, dt1 = run("q4_k", True, [r // 8 for r in full], 1)
    per_type = {}
    for key, outs in gpu_out.items():
        qtype, imat = key.split("+")[0], key.endswith("+imat")
        if key == "q4_k+imat":
            refs, m, t = ref, n, dt
        else:
            # projected time from a 64-row probe of the first tensor
            _, mp, tp = run(qtype, imat, [64, 0], cores)
            frac = min(1.0, seconds_per_type / max(1e-9, tp / mp * n))
            rows = [max(1, int(r * frac)) for r in full]
            refs, m, t = run(qtype, imat, rows, cores)
        blocks = same = le = 0
        for j in range(len(SHAPES)):
            r = refs[j].shape[0]
            b, s, l = compare_blocks(qtype, outs[j][:r], refs[j], xf[j][:r], qwn[j] if imat else None)
            blocks, same, le = blocks + b, same + s, le + l
        print(f"bench: cpu leg {key}: {m} values in {t:.1f} s, {blocks - same} of {blocks} blocks "
              f"differ", file=sys.stderr, flush=True)
        per_type[key] = {"cpu_GBps": round(2 * m / t / 1e9, 4), "values_checked": int(m),
                         "full_tensors": m == n,
                         "identical_pct": round(100.0 * same / blocks, 4),
                         "differing_blocks": blocks - same,
                         "differing_with_le_weighted_mse": le}
    return {"value": round(2 * n / dt / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "value_1_thread": round(2 * n1 / dt1 / 1e9, 5), "cpu": cpu_model(),
            "sample": f"full workload: Q4_K+imatrix on bf16 {SHAPES[0][0]}x{SHAPES[0][1]} and "
                      f"{SHAPES[1][0]}x{SHAPES[1][1]} ({n} values), {dt:.2f} s, one pass; "
                      f"1 thread: the first 1/8 of each tensor's rows ({n1} values), {dt1:.2f} s",
            "per_type": per_type}


def q4_0_outlier_tensor(torch, qs, dev, steps: int) -> dict:
    """Q4_0 on one 4096x4096 bf16 tensor, N(0, 0.02) with 0.1% of the values
    (16,777, chosen with seed 0) scaled x20, no imatrix; 32 distinct copies
    (1 GiB) rotate so the MALL cannot hold them."""
    import numpy as np
    rng = np.random.default_rng(0)
    a = rng.normal(0.0, 0.02, (4096, 4096))
    idx = rng.choice(a.size, 16777, replace=False)
    a.reshape(-1)[idx] *= 20.0
    x0 = bf16_from(torch, a).to(dev)
    xs = [x0] + [x0.clone() for _ in range(31)]
    out = torch.empty((4096, 4096 // 32 * 18), dtype=torch.uint8, device=dev)
    wall, ms = time_steps(torch, [lambda i: qs.quantize(2, xs[i % 32], None, out=out)],
                          max(steps, 64), 64)
    alg = algorithmic_bytes("q4_0", 4096 * 4096, 4096) - 4 * 4096
    return {"workload": "Q4_0 on bf16 4096x4096, N(0,0.02) + 0.1% outliers x20, seed 0",
            "input_GBps": round(2 * 4096 * 4096 / (ms * 1e-3) / 1e9, 1),
            "kernel_ms": round(ms, 5), "ms_per_step": round(wall, 5),
            "hbm_frac": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def iq2_xxs_ffn_down_tensors(torch, qs, dev, steps: int) -> dict:
    """IQ2_XXS + imatrix on 36 ffn_down tensors of 2560x9728 bf16: Student-t
    (df 5) weights scaled to std 0.02, a log-normal imatrix per tensor. One
    step = the 36 tensors."""
    g = torch.Generator(device=dev).manual_seed(4)
    rows, k, n = 2560, 9728, 36
    scale = 0.02 / (5.0 / 3.0) ** 0.5
    xs, qws = [], []
    for _ in range(n):
        # Student-t(5) = N(0,1) / sqrt(chi2(5) / 5)
        z = torch.randn(rows, k, device=dev, generator=g)
        c = torch.randn(5, rows, k, device=dev, generator=g).pow_(2).sum(0).div_(5.0).sqrt_()
        xs.append((z / c * scale).to(torch.bfloat16))
        qws.append(torch.randn(k, device=dev, generator=g).exp_())
        del z, c
    out = torch.empty((rows, k // 256 * 66), dtype=torch.uint8, device=dev)
    launches = [(lambda i, j=j: qs.quantize(16, xs[j], qws[j], out=out)) for j in range(n)]
    wall, kms = time_steps(torch, launches, max(1, steps // 50), 1)
    return {"workload": "IQ2_XXS + imatrix on 36 ffn_down tensors 2560x9728 bf16, Student-t df 5 "
                        "scaled to std 0.02, log-normal imatrix",
            "input_GBps": round(2 * rows * k * n / (wall * 1e-3) / 1e9, 2),
            "ms_per_step": round(wall, 3), "kernel_ms_mean": round(kms, 4),
            "kernel_GBps": round(2 * rows * k / (kms * 1e-3) / 1e9, 2),
            "hbm_frac": round(algorithmic_bytes("iq2_xxs", rows * k, k) / (kms * 1e-3) / 1e9
                              / HBM_PEAK_GBS, 5)}


def q4_0_large(torch, qs, dev, steps: int) -> dict:
    """Q4_0 on a token_embd-shaped bf16 tensor (151936 x 2560, 778 MB), two
    rotating copies: the HBM-bound case at a size where launch ramp-up is small."""
    rows, k = 151936, 2560
    g = torch.Generator(device=dev).manual_seed(1)
    xs = [(torch.randn(rows, k, device=dev, generator=g) * 0.01).to(torch.bfloat16) for _ in range(2)]
    out = torch.empty((rows, k // 32 * 18), dtype=torch.uint8, device=dev)
    wall, ms = time_steps(torch, [lambda i: qs.quantize(2, xs[i % 2], None, out=out)], steps, 30)
    alg = algorithmic_bytes("q4_0", rows * k, k) - 4 * k
    return {"input_GBps": round(2 * rows * k / (ms * 1e-3) / 1e9, 1), "kernel_ms": round(ms, 4),
            "hbm_GBps": round(alg / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def copy_peak(torch, dev, steps: int, warmup: int) -> int:
    """1 GiB device-to-device copy (torch's copy kernel: the reference size for
    scaling the FETCH_SIZE / WRITE_SIZE counters), then the streaming copy
    kernel's rate per launch size: the launches of the Q4_0 workloads (4096x4096,
    one 9728x2560 ffn tensor, the 151936x2560 token_embd) and 1 GiB each way."""
    nbytes = 1 << 30
    a = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a)
    wall, ms = time_steps(torch, [lambda i: b.copy_(a)], steps, warmup)
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes,
                      "ms_per_copy": round(ms, 4),
                      "copy_GBps_read_plus_write": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}),
          flush=True)
    del a, b
    torch.cuda.empty_cache()
    for name, traffic in [("q4_0 4096x4096", algorithmic_bytes("q4_0", 4096 * 4096, 4096) - 4 * 4096),
                          ("q4_0 9728x2560", algorithmic_bytes("q4_0", 9728 * 2560, 2560) - 4 * 2560),
                          ("q4_0 151936x2560", algorithmic_bytes("q4_0", 151936 * 2560, 2560) - 4 * 2560),
                          ("1 GiB each way", 2 << 30)]:
        r = copy_kernel_rate(torch, dev, traffic)
        print(json.dumps({"stream_copy_bytes_per_launch": traffic, "as_the_launch_of": name,
                          "us_per_launch": round(traffic / r * 1e6, 2),
                          "GBps_read_plus_write": round(r / 1e9, 1),
                          "frac_of_8TBps": round(r / 1e9 / HBM_PEAK_GBS, 4)}), flush=True)
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


def fs_type(path: Path) -> str:
    """Filesystem type of the mount holding `path` (/proc/mounts)."""
    best, kind = "", "unknown"
    p = str(path.resolve())
    try:
        for ln in open("/proc/mounts"):
            parts = ln.split()
            if len(parts) > 2 and (p == parts[1] or p.startswith(parts[1].rstrip("/") + "/")) \
                    and len(parts[1]) >= len(best):
                best, kind = parts[1], parts[2]
    except OSError:
        pass
    return kind


def drop_page_cache(path: Path) -> None:
    """Evict a file's clean pages (fsync, then POSIX_FADV_DONTNEED)."""
    fd = os.open(path, os.O_RDONLY)
    try:
        os.fsync(fd)
        os.posix_fadvise(fd, 0, 0, os.POSIX_FADV_DONTNEED)
    finally:
        os.close(fd)


# The reference's published end-to-end runs on a 4B bf16 model (README.md:28-49:
# every scheme with one imatrix, Q4_0 without; README.md:62-64: three --pure
# runs). A "--no-imatrix" token (bench.py's, not the command line's) runs
# the scheme without the imatrix.
E2E_PUBLISHED = ["IQ2_XXS", "IQ2_XS", "IQ2_S", "IQ2_M", "Q2_K_S", "Q2_K", "IQ3_XXS", "IQ3_XS",
                 "IQ3_S", "IQ3_M", "Q3_K_S", "Q3_K_M", "Q3_K_L", "IQ4_XS", "Q4_0 --no-imatrix",
                 "Q4_K_S", "Q4_K_M", "Q5_K_S", "Q5_K_M", "Q6_K",
                 "Q4_0 --pure --no-imatrix", "Q4_K --pure", "IQ2_XXS --pure"]
# the default run's end-to-end leg: the full-model IQ2_XXS run, the Q4_K_M mix
# with --mem 4G, and the IQ3_XXS and IQ2_S schemes with a Q4_0 token embedding
E2E_DEFAULT = ["IQ2_XXS", "Q4_K_M --mem 4G", "IQ3_XXS --token-embedding-type q4_0",
               "IQ2_S --token-embedding-type q4_0"]


def e2e_runs(torch, dev, schemes: list[str], where: str | None) -> dict:
    """The command line on the synthetic model, per scheme: one run with the
    input in the page cache (warm) and one after evicting the input and the
    imatrix from it (cold; only meaningful on a disk-backed filesystem).
    Returns the record (raises on a failed run)."""
    import re
    import subprocess
    import tempfile
    cands = [Path(where)] if where else [Path(os.environ.get("TMPDIR", "/tmp")), Path("/tmp"),
                                         Path("/var/tmp"), ROOT]
    base = next((c for c in cands if c.is_dir() and fs_type(c) not in ("tmpfs", "ramfs")), cands[0])
    with tempfile.TemporaryDirectory(dir=base, prefix="qs_e2e_") as d:
        d = Path(d)
        src, im = d / "model-bf16.gguf", d / "imatrix.gguf"
        t0 = time.perf_counter()
        n = synth_model(torch, dev, src, im)
        gen_s = time.perf_counter() - t0
        print(f"e2e: model written to {d} ({fs_type(d)}) in {gen_s:.1f} s", file=sys.stderr, flush=True)
        results = {}
        for sch in schemes:
            name, *extra = sch.split()
            use_im = "--no-imatrix" not in extra
            extra = [a for a in extra if a != "--no-imatrix"]
            for cache in ("warm", "cold"):
                out = d / f"out-{name}.gguf"
                if cache == "cold":
                    drop_page_cache(src)
                    drop_page_cache(im)
                cmd = [sys.executable, str(ROOT / "quant-studio.py"), str(src), str(out), name,
                       *(["--imatrix", str(im)] if use_im else []), *extra]
                t0 = time.perf_counter()
                r = subprocess.run(cmd, capture_output=True, text=True)
                wall = time.perf_counter() - t0
                if r.returncode != 0:
                    raise RuntimeError(f"e2e {sch}: the command line failed:\n{r.stderr[-2000:]}")
                m = re.search(r"done in ([0-9.]+)s", r.stdout)
                pipe_s = float(m.group(1)) if m else None
                results[f"{sch} {cache}"] = {
                    "pipeline_s": pipe_s, "process_wall_s": round(wall, 2),
                    "input_GBps_pipeline": round(src.stat().st_size / 1e9 / pipe_s, 2)
                    if pipe_s else None,
                    "out_bytes": out.stat().st_size}
                out.unlink()
                print(f"e2e {sch} {cache}: {results[f'{sch} {cache}']}", file=sys.stderr, flush=True)
        return {"e2e": "synthetic 4B-class bf16 GGUF (36 layers, 2560/9728, vocab 151936)",
                "filesystem": fs_type(d), "file_bytes": src.stat().st_size,
                "weights": n, "generate_s": round(gen_s, 1),
                "cold": "input and imatrix evicted from the page cache before the run "
                        "(fsync + POSIX_FADV_DONTNEED)",
                "runs": results}


def run_e2e(torch, dev, schemes: list[str], where: str | None) -> int:
    print(json.dumps(e2e_runs(torch, dev, schemes, where)), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--types", default="all", help="per-type table: all, none or a comma list")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-configs", action="store_true", help="skip the Q4_0 4096x4096 and "
                    "IQ2_XXS Student-t workloads")
    ap.add_argument("--configs", default="q4_0,iq2_xxs",
                    help="which of those workloads to run: a comma list of q4_0 (4096x4096 with "
                         "outliers) and iq2_xxs (36 Student-t ffn_down tensors)")
    ap.add_argument("--cpu-seconds", type=float, default=45.0,
                    help="CPU time per type for the identical-block check (full tensors when "
                         "the oracle fits in it)")
    ap.add_argument("--sqrt", default="torch-cpu", choices=["torch-cpu", "ieee", "torch-cpu-amd"],
                    help="square-root rounding of the weights (the oracle follows it)")
    ap.add_argument("--e2e", default=None,
                    help="run the CLI end to end on a synthetic 4B-class model for these "
                         "';'-separated schemes (e.g. 'IQ2_XXS;Q4_K_M'), or 'all' for the "
                         "reference's published runs, and print its own JSON line")
    ap.add_argument("--no-e2e", action="store_true",
                    help="skip the default end-to-end leg (the command line on the synthetic "
                         "4B-class model: IQ2_XXS, Q4_K_M --mem 4G, IQ3_XXS and IQ2_S with a "
                         "Q4_0 token embedding; warm and cold)")
    ap.add_argument("--e2e-dir", default=None, help="directory for the e2e model (default: the "
                    "first disk-backed of $TMPDIR, /tmp, /var/tmp, the repository)")
    ap.add_argument("--valu-peak", action="store_true",
                    help="time the VALU issue-rate kernel only (the reference for SQ_INSTS_VALU)")
    ap.add_argument("--copy-only", action="store_true",
                    help="time a plain 1 GiB device copy instead (HBM copy peak, and the "
                         "reference size for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE counts)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this quantizer runs on one GPU; --gpus must be 1 (the path shards by "
              "tensor with no exchange between GPUs, so a single GPU's rate is what it measures)",
              file=sys.stderr)
        return 2

    import torch
    qs = importlib.import_module("quant-studio_amd")

    dev = torch.device("cuda:0")
    if args.copy_only:
        return copy_peak(torch, dev, args.steps, args.warmup)
    if args.valu_peak:
        print(json.dumps({"valu_wave_instr_per_s": round(valu_peak(torch, dev, args.steps))}), flush=True)
        return 0
    if args.e2e:
        schemes = E2E_PUBLISHED if args.e2e == "all" else \
            [x.strip() for x in args.e2e.split(";") if x.strip()]
        return run_e2e(torch, dev, schemes, args.e2e_dir)
    qs.set_sqrt_rounding(args.sqrt)
    qs.init(0)
    xs, qws, host = make_inputs(torch, dev)
    per_step_bytes = sum(2 * r * k for r, k in SHAPES)
    nrot = max(1, -(-ROTATE_BYTES // per_step_bytes))
    xs_rot = [xs] + [[x.clone() for x in xs] for _ in range(nrot - 1)]
    n_elems = sum(r * k for r, k in SHAPES)

    def outs_for(qtype):
        return [torch.empty((r, k // 256 * OUT_BYTES_PER_256[qtype]), dtype=torch.uint8, device=dev)
                for r, k in SHAPES]

    # The calibration kernels run first, the VALU one last: their measurements
    # belong to the line anyway, and the core clock follows VALU load (after
    # idle time or memory-bound kernels the first ~60 headline launches ran up
    # to 14% slower; straight after VALU work, at their steady rate), so ~0.2 s
    # of VALU work right before the headline's own warm-up settles the clock
    # whatever --warmup is.
    copy_peak_gbs = copy_kernel_peak(torch, dev) / 1e9
    peak_valu = valu_peak(torch, dev, launches=30)

    # headline: Q4_K + imatrix; both launches of a step run the same kernel
    # (k_q45_k, 97,280 superblocks each), so the kernel's average launch is
    # the step time over the two launches
    ms_step, kms = time_steps(torch, shape_launches(qs, "q4_k", True, xs_rot, qws, outs_for("q4_k")),
                              args.steps, args.warmup)
    value = 2 * n_elems / (ms_step * 1e-3) / 1e9
    print(f"bench: headline {ms_step:.4f} ms per step, {kms:.4f} ms per launch",
          file=sys.stderr, flush=True)
    # algorithmic bytes of the average launch (the two shapes differ only in
    # the imatrix's 4k bytes)
    alg = sum(algorithmic_bytes("q4_k", r * k, k) for r, k in SHAPES) // len(SHAPES)
    achieved = alg / (kms * 1e-3) / 1e9
    insts = profile_figure("counters_q4_k_imat_9728x2560.md", "valu_insts_per_launch")
    traffic = profile_figure("counters_q4_k_imat_9728x2560.md", "traffic_bytes_per_launch")

    per_type, gpu_out = {}, {}
    valu_counts = profiled_valu_per_type()
    copy_rates = {}

    def same_size_copy(traffic: int) -> float:
        """GB/s of the copy kernel at this traffic per launch (measured once per size)."""
        if traffic not in copy_rates:
            copy_rates[traffic] = copy_kernel_rate(torch, dev, traffic) / 1e9
        return copy_rates[traffic]
    sel = [] if args.types == "none" else (list(TYPE_IDS) if args.types == "all"
                                           else args.types.split(","))
    for qtype in sel:
        for imat in modes_of(qtype):
            key = f"{qtype}{'+imat' if imat else ''}"
            # the 32-value launches take ~13 us, so one late launch moves a
            # 10-step region by several percent: median of five regions
            runs = [time_steps(torch, shape_launches(qs, qtype, imat, xs_rot, qws, outs_for(qtype)),
                               max(10, args.steps // 4), 20)
                    for _ in range(5 if qtype in B32_TYPES else 1)]
            st, km = sorted(runs)[len(runs) // 2]
            a = sum(algorithmic_bytes(qtype, r * k, k) for r, k in SHAPES) / (st * 1e-3) / 1e9
            n_insts = valu_counts.get(key)
            print(f"bench: {key}: {km:.4f} ms per launch", file=sys.stderr, flush=True)
            per_type[key] = {
                "input_GBps": round(2 * n_elems / (st * 1e-3) / 1e9, 2),
                "ms_per_step": round(st, 4),
                "kernel_ms": round(km, 4),
                "hbm_frac": round(a / HBM_PEAK_GBS, 4),
                "copy_frac": round(a / copy_peak_gbs, 4),
                # against the copy kernel moving this launch's bytes (the
                # ceiling of a launch this size, ramp-up and drain included)
                "copy_frac_same_size": round(a / same_size_copy(
                    algorithmic_bytes(qtype, SHAPES[0][0] * SHAPES[0][1], SHAPES[0][1])), 4)
                if qtype in B32_TYPES else None,
                # VALU issue rate (SQ_INSTS_VALU per launch over the live launch
                # time) against the calibration kernel's rate
                "valu_frac": None if n_insts is None else
                round(n_insts / (km * 1e-3) / peak_valu, 3),
            }
            if not args.no_cpu:
                gpu_out[key] = gpu_bytes(torch, qs, qtype, imat, xs, qws)
    if not args.no_cpu and "q4_k+imat" not in gpu_out:
        gpu_out["q4_k+imat"] = gpu_bytes(torch, qs, "q4_k", True, xs, qws)

    configs = {}
    which = set() if args.no_configs else {c.strip() for c in args.configs.split(",") if c.strip()}
    if which - {"q4_0", "iq2_xxs"}:
        raise SystemExit(f"bench.py: unknown --configs {sorted(which - {'q4_0', 'iq2_xxs'})}")
    if which:
        del xs_rot
        if "q4_0" in which:
            configs["q4_0_4096x4096_outliers"] = q4_0_outlier_tensor(torch, qs, dev, args.steps)
        if "iq2_xxs" in which:
            configs["iq2_xxs_imat_36x2560x9728_student_t"] = iq2_xxs_ffn_down_tensors(torch, qs, dev,
                                                                                       args.steps)
        torch.cuda.empty_cache()
    if "q4_0" in sel:
        per_type["q4_0 token_embd 151936x2560"] = q4_0_large(torch, qs, dev, 20)
    for row, alg_b in [(per_type.get("q4_0 token_embd 151936x2560"),
                        algorithmic_bytes("q4_0", 151936 * 2560, 2560) - 4 * 2560),
                       (configs.get("q4_0_4096x4096_outliers"),
                        algorithmic_bytes("q4_0", 4096 * 4096, 4096) - 4 * 4096)]:
        if row:
            row["copy_frac"] = round(row["hbm_frac"] * HBM_PEAK_GBS / copy_peak_gbs, 4)
            row["copy_frac_same_size"] = round(row["hbm_frac"] * HBM_PEAK_GBS / same_size_copy(alg_b), 4)

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
                   "sqrt_rounding": args.sqrt, "parallelism": "1 GPU (no exchange)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 5),
                     "traffic": None if traffic is None else int(traffic),
                     "kernel": "k_q45_k<bf16, imatrix, 15>", "kernel_ms": round(kms, 4),
                     "algorithmic_bytes": alg,
                     # the binding roof: this kernel is VALU-bound, so its
                     # SQ_INSTS_VALU per launch over the same live duration is
                     # set against the measured issue rate of a pure mul/add kernel
                     "binding": "valu",
                     "valu": None if insts is None else {
                         "insts_per_launch": int(insts), "unit": "G wave-instr/s",
                         "achieved": round(insts / (kms * 1e-3) / 1e9, 1),
                         "peak": round(peak_valu / 1e9, 1),
                         "frac": round(insts / (kms * 1e-3) / peak_valu, 4)}},
        "copy_peak": {"GBps": round(copy_peak_gbs, 1), "unit": "GB/s read + written",
                      "kernel": "k_copy_stream (libqs_calib.so), 1 GiB, 16-byte non-temporal "
                                "loads and stores, 10 launches back to back"},
        "valu_peak": {"G_wave_instr_per_s": round(peak_valu / 1e9, 1),
                      "kernel": "k_valu_issue (libqs_calib.so), 30 launches of ~7 ms, "
                                "before the headline"},
        "per_type": per_type,
        "configs": configs,
    }
    if not args.no_cpu:
        import oracle
        if args.sqrt == "ieee":
            oracle.use_ieee_sqrt(True)
        elif args.sqrt == "torch-cpu-amd":
            sys.path.insert(0, str(ROOT / "tests"))
            import sqrt_hosts
            oracle.use_amd_host_sqrt(sqrt_hosts.amd_ulps())
        cb = cpu_baseline(oracle, host, qws, gpu_out, args.cpu_seconds)
        line["cpu_baseline"] = cb
        head = cb["per_type"].get("q4_k+imat")
        line["identical_pct_vs_oracle"] = None if head is None else head["identical_pct"]
    if not args.no_e2e:
        # the command line end to end on the synthetic 4B-class model
        # (E2E_DEFAULT), warm and cold page cache; supplementary to the
        # headline, so a failure is reported in the line
        try:
            line["e2e"] = e2e_runs(torch, dev, E2E_DEFAULT, args.e2e_dir)
        except Exception as e:
            print(f"bench: e2e leg failed: {e}", file=sys.stderr, flush=True)
            line["e2e"] = {"error": str(e)[-500:]}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
