"""CPU oracle for the GGUF block quantizers -- TEST INFRASTRUCTURE ONLY.

A plain-C restatement of the reference's eager CPU path (kernels/*.py under
torch on CPU), loaded with ctypes. Only tests/, __graft_entry__.smoke() and the
CPU-baseline leg of bench.py use it, always as the expected result to compare
against or as the timed CPU baseline; the product library never calls it.

Parity pinning: every type is checked against golden vectors written by the
reference itself (tests/golden/gen_golden.py); the reduction-order helpers and
the fp16 conversion are also checked against torch and numpy directly.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libqs_oracle.so"

TYPE_IDS = {"q4_0": 2, "q2_k": 10, "q3_k": 11, "q4_k": 12, "q5_k": 13, "q6_k": 14,
            "iq2_xxs": 16, "iq2_xs": 17, "iq3_xxs": 18, "iq3_s": 21, "iq2_s": 22,
            "iq4_xs": 23,
            # ggml formats without a reference module (parity unpinned against
            # the reference; pinned by known answers and dequantisation bounds)
            "q4_1": 3, "q5_0": 6, "q5_1": 7, "q8_0": 8, "iq4_nl": 20}

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.qso_row_bytes.restype = ctypes.c_int64
        L.qso_row_bytes.argtypes = [ctypes.c_int, ctypes.c_int64]
        L.qso_quantize.restype = ctypes.c_int
        L.qso_quantize.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                   ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        L.qso_sum_cascade8.restype = ctypes.c_float
        L.qso_sum_cascade8.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.qso_sum_tree.restype = ctypes.c_float
        L.qso_sum_tree.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.qso_f32_to_f16.restype = ctypes.c_uint16
        L.qso_f32_to_f16.argtypes = [ctypes.c_float]
        L.qso_set_sqrt_hook.restype = None
        L.qso_set_sqrt_hook.argtypes = [ctypes.c_void_p]
        L.qso_set_sqrt_ieee.restype = None
        L.qso_set_sqrt_ieee.argtypes = [ctypes.c_int]
        L.qso_set_sqrt_table.restype = None
        L.qso_set_sqrt_table.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.qso_sqrt.restype = ctypes.c_float
        L.qso_sqrt.argtypes = [ctypes.c_float]
        L.qso_sqrt_ref.restype = ctypes.c_float
        L.qso_sqrt_ref.argtypes = [ctypes.c_float]
        L.qso_set_mutation.restype = None
        L.qso_set_mutation.argtypes = [ctypes.c_int]
        _lib = L
    return _lib


def row_bytes(qtype: str, k: int) -> int:
    return int(lib().qso_row_bytes(TYPE_IDS[qtype], k))


def quantize(qtype: str, x: np.ndarray, qw: np.ndarray | None = None,
             n_threads: int | None = None) -> np.ndarray:
    """x: (n, k) float32 (or bf16 bits as uint16); qw: (k,) float32 or None.
    Returns (n, row_bytes) uint8."""
    if x.dtype == np.uint16:
        x = (x.astype(np.uint32) << 16).view(np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, k = x.shape
    rb = row_bytes(qtype, k)
    if rb < 0:
        raise ValueError(f"{qtype}: unsupported row length {k}")
    out = np.empty((n, rb), dtype=np.uint8)
    q = None
    if qw is not None:
        q = np.ascontiguousarray(qw, dtype=np.float32)
        if q.shape != (k,):
            raise ValueError("imatrix must have k entries")
    nt = n_threads or len(os.sched_getaffinity(0))
    rc = lib().qso_quantize(TYPE_IDS[qtype], x.ctypes.data, n, k,
                            None if q is None else q.ctypes.data, out.ctypes.data, nt)
    if rc != 0:
        raise RuntimeError(f"oracle: quantize {qtype} failed ({rc})")
    return out


SQRT_FN = ctypes.CFUNCTYPE(ctypes.c_float, ctypes.c_float)
_hook_ref = None


def sqrt_ref(v: float) -> np.float32:
    """The oracle's square root: IEEE sqrtf minus one ulp on the tabulated set
    where the reference's torch.sqrt (CPU) rounds down."""
    return np.float32(lib().qso_sqrt_ref(float(v)))


def use_ieee_sqrt(enable: bool) -> None:
    """Make the oracle use plain IEEE sqrtf for its weights (tests only)."""
    lib().qso_set_sqrt_ieee(1 if enable else 0)


_sqrt_table = None


def use_sqrt_table(ulps, subnormal_ieee: bool = False) -> None:
    """Make the oracle round its square roots by a per-key table: `ulps` holds
    2^24 int8 offsets from the IEEE root (torch.sqrt measured on another host),
    keyed like qso_sqrt_ref; with subnormal_ieee, subnormal inputs keep the IEEE
    root; None switches the table off (tests only)."""
    global _sqrt_table
    if ulps is None:
        lib().qso_set_sqrt_table(None, 0)
        _sqrt_table = None
        return
    t = np.ascontiguousarray(ulps, dtype=np.int8)
    if t.size != 1 << 24:
        raise ValueError("the square-root table holds one offset per 2^24 keys")
    lib().qso_set_sqrt_table(t.ctypes.data, 1 if subnormal_ieee else 0)
    _sqrt_table = t


def use_amd_host_sqrt(ulps) -> None:
    """The AMD EPYC host's torch.sqrt: the table `ulps` on normal inputs, the
    IEEE root on subnormal ones (tests only; None switches it off)."""
    use_sqrt_table(ulps, subnormal_ieee=True)


def use_torch_sqrt(enable: bool) -> None:
    """Make the oracle call torch's CPU sqrt live (the routine the reference's
    eager path calls) instead of its tabulated reproduction. Single-threaded
    use only (the callback takes the GIL)."""
    global _hook_ref
    if enable:
        import torch

        def f(v):
            return torch.sqrt(torch.tensor(v, dtype=torch.float32)).item()
        _hook_ref = SQRT_FN(f)
        lib().qso_set_sqrt_hook(ctypes.cast(_hook_ref, ctypes.c_void_p))
    else:
        lib().qso_set_sqrt_hook(None)
        _hook_ref = None


def sum_cascade8(v: np.ndarray) -> np.float32:
    v = np.ascontiguousarray(v, dtype=np.float32)
    return np.float32(lib().qso_sum_cascade8(v.ctypes.data, v.size))


def sum_tree(v: np.ndarray) -> np.float32:
    v = np.ascontiguousarray(v, dtype=np.float32)
    return np.float32(lib().qso_sum_tree(v.ctypes.data, v.size))


def f32_to_f16_bits(f: float) -> int:
    return int(lib().qso_f32_to_f16(float(f)))
