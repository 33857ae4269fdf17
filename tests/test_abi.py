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
            "qs_device_count", "qs_pipeline_create", "qs_pipeline_quantize", "qs_pipeline_quantize_fd",
            "qs_pipeline_write",
            "qs_pipeline_finish", "qs_pipeline_destroy", "qs_init", "qs_set_sqrt_rounding",
            "qs_get_sqrt_rounding"} <= names


def test_library_exports_every_declared_symbol(qs):
    L = qs.library()
    for name in declared_functions():
        assert hasattr(L, name), f"libqs_hip.so does not export {name}"
    assert L.qs_abi_version() == qs.ABI_VERSION == 4


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


# the reference's per-type modules: module -> (function, its parameters)
# (kernels/q4_0.py:14, q2_k.py:25, q3_k.py:23, q4_k.py:25, q5_k.py:25,
# q6_k.py:22, iq4_xs.py:149, iq2.py:418, iq2_xs.py:20, iq2_s.py:21,
# iq3_xxs.py:31, iq3_s.py:31), each with a SPECS dict of its type
REFERENCE_MODULES = {
    "q4_0": ("quantize_q4_0", ["x"]), "q2_k": ("quantize_q2_k", ["x", "qw"]),
    "q3_k": ("quantize_q3_k", ["x", "qw"]), "q4_k": ("quantize_q4_k", ["x", "qw"]),
    "q5_k": ("quantize_q5_k", ["x", "qw"]), "q6_k": ("quantize_q6_k", ["x", "qw"]),
    "iq4_xs": ("quantize_iq4_xs", ["x", "qw"]), "iq2": ("quantize_iq2_xxs", ["x", "qw", "T"]),
    "iq2_xs": ("quantize_iq2_xs", ["x", "qw"]), "iq2_s": ("quantize_iq2_s", ["x", "qw"]),
    "iq3_xxs": ("quantize_iq3_xxs", ["x", "qw"]), "iq3_s": ("quantize_iq3_s", ["x", "qw"]),
}


def test_per_type_modules_mirror_the_reference(qs):
    """`kernels.<module>.quantize_<type>` callers (tools/dev_gpu_check.py:22-24)
    find the same module, function and parameter names, and each module's
    SPECS holds its registry entry; the five extra types follow the pattern."""
    import importlib
    import inspect
    extra = {t: (f"quantize_{t}", ["x", "qw"]) for t in ("q4_1", "q5_0", "q5_1", "q8_0", "iq4_nl")}
    for mod, (fn, params) in {**REFERENCE_MODULES, **extra}.items():
        m = importlib.import_module(f"quant-studio_amd.{mod}")
        f = getattr(m, fn)
        assert list(inspect.signature(f).parameters) == params, mod
        (name, spec), = m.SPECS.items()
        assert fn == f"quantize_{name}" and spec is qs.ALL_SPECS[name], mod


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


def test_iq2_types_reject_missing_imatrix(qs):
    """IQ2_XXS / IQ2_XS / IQ2_S refuse a NULL imatrix before any device work
    (their reference quantizers index qw unconditionally, iq2.py:418-431,
    iq2_xs.py:20-29, iq2_s.py:21-30). IQ3_XXS, whose QuantSpec also has
    needs_imatrix (a command-line policy), goes on without one as
    quantize_iq3_xxs(x, None) does (iq3_xxs.py:41-42): with no device here it
    fails later, at the table upload, not at the imatrix check."""
    L = qs.library()
    required = {"iq2_xxs", "iq2_xs", "iq2_s"}
    assert {n for n, sp in qs.ALL_SPECS.items() if sp.needs_imatrix} == required | {"iq3_xxs"}
    for name in required:
        assert _call(L, int(qs.ALL_SPECS[name].ggml_type)) == -22, name
        assert b"requires an imatrix" in L.qs_last_error(), name
    if L.qs_device_count() == 0:        # with a device the call would launch on the dummy pointers
        assert _call(L, int(qs.ALL_SPECS["iq3_xxs"].ggml_type)) != 0
        assert b"requires an imatrix" not in L.qs_last_error()


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
    assert L.qs_pipeline_quantize_fd(None, 12, 30, 0, 0, 1, 256, None, 1, 1, 0) == -22
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
