"""CPU tests of the C-ABI library: it loads, exports every function the public
header declares, reports the reference's type table, and rejects bad
arguments before any device work (no GPU needed)."""

from __future__ import annotations

import ctypes
import re
import subprocess
import sys
from pathlib import Path

import pytest

from golden_data import TYPES

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "quant_studio.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(qs_\w+)\s*\(", text, flags=re.M)


def test_header_declares_the_api():
    names = set(declared_functions())
    assert {"qs_abi_version", "qs_row_bytes", "qs_quantize", "qs_last_error",
            "qs_type_supported", "qs_type_needs_imatrix", "qs_type_uses_imatrix",
            "qs_device_count", "qs_pipeline_create", "qs_pipeline_quantize", "qs_pipeline_write",
            "qs_pipeline_finish", "qs_pipeline_destroy", "qs_init", "qs_set_sqrt_rounding",
            "qs_get_sqrt_rounding"} <= names


def test_library_exports_every_declared_symbol(qs):
    L = qs.library()
    for name in declared_functions():
        assert hasattr(L, name), f"libqs_hip.so does not export {name}"
    assert L.qs_abi_version() == qs.ABI_VERSION == 3


@pytest.mark.parametrize("qtype", sorted(TYPES))
def test_row_bytes_match_reference_block_sizes(qs, qtype):
    tid, blk, nbytes = TYPES[qtype]
    L = qs.library()
    assert L.qs_row_bytes(tid, 4 * blk) == 4 * nbytes
    assert L.qs_row_bytes(tid, blk + 1) == -22
    assert L.qs_row_bytes(tid, 0) == -22


def test_type_flags_match_reference_specs(qs):
    L = qs.library()
    for name, spec in qs.ALL_SPECS.items():
        t = int(spec.ggml_type)
        assert L.qs_type_needs_imatrix(t) == int(spec.needs_imatrix), name
        assert L.qs_type_uses_imatrix(t) == int(spec.uses_imatrix), name
    assert L.qs_type_needs_imatrix(99) == -95


def test_registry_lists_only_types_with_kernels(qs):
    L = qs.library()
    for name, spec in qs.ALL_SPECS.items():
        assert (name in qs.QUANT_TYPES) == bool(L.qs_type_supported(int(spec.ggml_type)))
    for name in ("q4_0", "q2_k", "q3_k", "q4_k", "q5_k", "q6_k", "iq4_xs"):
        assert name in qs.QUANT_TYPES


def _call(L, t, src_type=30, src=16, n=4, k=256, stride=512, qw=None, dst=64, dst_bytes=10 ** 6):
    return L.qs_quantize(t, src_type, ctypes.c_void_p(src), n, k, stride,
                         None if qw is None else ctypes.c_void_p(qw), ctypes.c_void_p(dst),
                         dst_bytes, None)


def test_quantize_rejects_bad_arguments_before_launch(qs):
    L = qs.library()
    assert _call(L, 99) == -95                       # unknown type
    assert _call(L, 12, k=100) == -22                # k not a multiple of 256
    assert _call(L, 12, src_type=5) == -22           # unsupported source dtype
    assert _call(L, 12, n=-1) == -22
    assert _call(L, 12, src=0) == -22                # null source
    assert _call(L, 12, src=8) == -22                # misaligned source
    assert _call(L, 12, stride=500) == -22           # stride below k*2 / not 16-aligned
    assert _call(L, 12, dst_bytes=10) == -22         # dst too small
    assert b"dst holds 10 bytes" in L.qs_last_error()
    assert _call(L, 12, n=0) == 0                    # empty input: no work, no launch
    # sizes whose products would wrap int64 are refused before any arithmetic
    assert _call(L, 12, n=1 << 40, k=1 << 20) == -22
    assert b"exceed the 2^34" in L.qs_last_error()
    assert _call(L, 12, n=1 << 20, k=1 << 14, stride=1 << 50) == -22
    assert b"2^62-byte span" in L.qs_last_error()
    assert _call(L, 12, n=(1 << 34) // 256 + 1, k=256, stride=512) == -22


def test_needs_imatrix_types_reject_missing_imatrix(qs):
    L = qs.library()
    for name, spec in qs.ALL_SPECS.items():
        if spec.needs_imatrix and L.qs_type_supported(int(spec.ggml_type)):
            assert _call(L, int(spec.ggml_type)) == -22
            assert b"requires an imatrix" in L.qs_last_error()


def test_cpu_quant_fn_needs_a_rocm_device(qs):
    """A quant_fn for a CPU device stages its tensors through the ROCm device;
    with none present it fails loudly (there is no CPU arithmetic to fall back
    on). The staged path itself is a GPU test."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a ROCm device is present: covered by the GPU tests")
    for qw in (None, torch.ones(256)):
        fn = qs.QUANT_TYPES["q4_k"].make_kernel(torch.device("cpu"), qw)
        with pytest.raises(qs.QuantSpecError, match="no ROCm device"):
            fn(torch.zeros(2, 256))


def test_pipeline_rejects_bad_arguments_without_device_work(qs):
    import ctypes
    L = qs.library()
    h = ctypes.c_void_p()
    assert L.qs_pipeline_create(0, 1, 4, ctypes.byref(h)) == -22          # too few slots
    assert "n_slots" in qs.last_error()
    assert L.qs_pipeline_create(0, 3, 0, ctypes.byref(h)) == -22          # no copy threads
    assert L.qs_pipeline_create(-1, 3, 4, ctypes.byref(h)) == -22         # no such device
    assert "not present" in qs.last_error() and not h.value
    assert L.qs_pipeline_create(0, 3, 4, None) == -22
    assert L.qs_pipeline_quantize(None, 12, 30, None, 1, 256, None, 1, 1, 0) == -22
    assert L.qs_pipeline_write(None, None, 0, 1, 0) == -22
    assert L.qs_pipeline_finish(None) == -22
    L.qs_pipeline_destroy(None)
    assert L.qs_device_count() >= 0


def test_one_hip_runtime_in_any_import_order():
    """Package first, torch second: the process must map a single HIP runtime
    (two runtimes make the library's device calls fail)."""
    code = ("import importlib, sys; sys.path.insert(0, sys.argv[1]); "
            "importlib.import_module('quant-studio_amd'); import torch; "
            "m = open('/proc/self/maps').read().splitlines(); "
            "print(len({l.split()[-1] for l in m if 'libamdhip64' in l}))")
    r = subprocess.run([sys.executable, "-c", code, str(ROOT)], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "1"


def test_sqrt_rounding_modes(qs):
    """The process-wide square-root mode: torch-cpu by default, ieee on
    request, anything else refused without changing the mode."""
    L = qs.library()
    assert qs.sqrt_rounding() == "torch-cpu"
    try:
        qs.set_sqrt_rounding("ieee")
        assert L.qs_get_sqrt_rounding() == 1 and qs.sqrt_rounding() == "ieee"
        assert L.qs_set_sqrt_rounding(7) == -22 and "square-root mode 7" in qs.last_error()
        assert qs.sqrt_rounding() == "ieee"
        with pytest.raises(ValueError):
            qs.set_sqrt_rounding("fast")
    finally:
        qs.set_sqrt_rounding("torch-cpu")
    assert L.qs_get_sqrt_rounding() == 0


def test_init_refuses_absent_devices(qs):
    L = qs.library()
    assert L.qs_init(-1) == -22
    assert L.qs_init(1 << 20) == -22 and "not present" in qs.last_error()
