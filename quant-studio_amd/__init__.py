"""MI355X-native GGUF block quantizers behind the reference's plugin API.

Mirrors the reference's kernel registry (kernels/__init__.py:18-27,
kernels/common.py:20-37): `QUANT_TYPES` maps a lowercase type name to a
`QuantSpec`, whose `make_kernel(device, qw)` returns `quant_fn(x) -> uint8`.
Here every quant_fn is one call into the gfx950 HIP library (libqs_hip.so,
C ABI in include/quant_studio.h) on torch's current stream. A quant_fn made
for a CPU device (the reference's CPU path, quant-studio.py:216-232) takes
CPU tensors and returns a CPU tensor, computing on the current ROCm device
(the bytes are the reference CPU path's either way). There is no CPU
arithmetic: the library must be built (build.py) and a ROCm device present,
and every failure raises. torch is imported on first use of the tensor API
only; the command line runs on the library's own pipeline without it.

Import with `importlib.import_module("quant-studio_amd")` (the directory name
is not an identifier).
"""

from __future__ import annotations

import ctypes
import sys
import threading
from pathlib import Path

from .gguf_types import GGMLQuantizationType, LlamaFileType

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "_build" / "libqs_hip.so"
ABI_VERSION = 4

_lib: ctypes.CDLL | None = None


def __getattr__(name: str):
    # torch-valued constants, created when first asked for
    if name in ("TORCH_DTYPES", "F32_TINY"):
        import torch
        # source dtypes the quantizers read directly (kernels/common.py:20-24)
        globals()["TORCH_DTYPES"] = {
            GGMLQuantizationType.F32: torch.float32,
            GGMLQuantizationType.F16: torch.float16,
            GGMLQuantizationType.BF16: torch.bfloat16,
        }
        globals()["F32_TINY"] = torch.finfo(torch.float32).tiny
        return globals()[name]
    raise AttributeError(name)


def _src_id(dtype) -> int | None:
    import torch
    return {torch.float32: 0, torch.float16: 1, torch.bfloat16: 30}.get(dtype)


class QuantSpecError(RuntimeError):
    """A quantizer call was rejected or failed in the HIP library."""


def _bind_torch_hip_runtime() -> None:
    """torch's ROCm wheel carries its own HIP runtime (torch/lib/libamdhip64.so,
    soname libamdhip64.so.7), which torch's libraries load by file name. If this
    library were loaded first it would bind the system copy, and a later
    `import torch` would map a second HIP and HSA runtime into the process,
    after which this library's device calls fail. So when torch is installed,
    its runtime is loaded first (without importing torch) and this library binds
    to it; in any import order the process then has one HIP runtime."""
    import importlib.util
    spec = importlib.util.find_spec("torch")
    for loc in (spec.submodule_search_locations or []) if spec else []:
        rt = Path(loc) / "lib" / "libamdhip64.so"
        if rt.exists():
            ctypes.CDLL(str(rt), mode=ctypes.RTLD_GLOBAL)
            return


_lib_lock = threading.Lock()


def library() -> ctypes.CDLL:
    """Load libqs_hip.so (built in-tree by build.py); raises if it is missing.
    Thread-safe: the command line may load it from a pipeline-creating thread
    while the main thread gets to it too."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        return _load_library()


def _load_library() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is missing: build it with "
                              "quant-studio_amd/build.py (or __graft_entry__.build())")
        _bind_torch_hip_runtime()
        L = ctypes.CDLL(str(LIB_PATH))
        L.qs_abi_version.restype = ctypes.c_int
        L.qs_type_supported.restype = ctypes.c_int
        L.qs_type_supported.argtypes = [ctypes.c_int]
        L.qs_type_needs_imatrix.restype = ctypes.c_int
        L.qs_type_needs_imatrix.argtypes = [ctypes.c_int]
        L.qs_type_uses_imatrix.restype = ctypes.c_int
        L.qs_type_uses_imatrix.argtypes = [ctypes.c_int]
        L.qs_row_bytes.restype = ctypes.c_int64
        L.qs_row_bytes.argtypes = [ctypes.c_int, ctypes.c_int64]
        L.qs_quantize.restype = ctypes.c_int
        L.qs_quantize.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                  ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                  ctypes.c_int64, ctypes.c_void_p]
        L.qs_init.restype = ctypes.c_int
        L.qs_init.argtypes = [ctypes.c_int]
        L.qs_set_sqrt_rounding.restype = ctypes.c_int
        L.qs_set_sqrt_rounding.argtypes = [ctypes.c_int]
        L.qs_get_sqrt_rounding.restype = ctypes.c_int
        L.qs_last_error.restype = ctypes.c_char_p
        L.qs_device_count.restype = ctypes.c_int
        L.qs_pipeline_create.restype = ctypes.c_int
        L.qs_pipeline_create.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.POINTER(ctypes.c_void_p)]
        L.qs_pipeline_quantize.restype = ctypes.c_int
        L.qs_pipeline_quantize.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                           ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                           ctypes.c_int64, ctypes.c_int, ctypes.c_int64]
        L.qs_pipeline_quantize_fd.restype = ctypes.c_int
        L.qs_pipeline_quantize_fd.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                              ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                              ctypes.c_int64, ctypes.c_int, ctypes.c_int64]
        L.qs_pipeline_write.restype = ctypes.c_int
        L.qs_pipeline_write.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                        ctypes.c_int64]
        L.qs_pipeline_finish.restype = ctypes.c_int
        L.qs_pipeline_finish.argtypes = [ctypes.c_void_p]
        L.qs_pipeline_destroy.restype = None
        L.qs_pipeline_destroy.argtypes = [ctypes.c_void_p]
        if L.qs_abi_version() != ABI_VERSION:
            raise ImportError(f"{LIB_PATH}: ABI version {L.qs_abi_version()} != {ABI_VERSION}")
        _lib = L
    return _lib


def last_error() -> str:
    return library().qs_last_error().decode()


def row_bytes(ggml_type: int, k: int) -> int:
    rb = library().qs_row_bytes(int(ggml_type), int(k))
    if rb < 0:
        raise ValueError(last_error())
    return rb


MAX_VALUES_PER_CALL = 1 << 34      # qs_quantize's per-call limit (include/quant_studio.h)

# square-root rounding of the weights (QS_SQRT_* in include/quant_studio.h):
# torch.sqrt on an Intel host's CPU (the default), the IEEE root, torch.sqrt on
# an AMD EPYC host's CPU
SQRT_ROUNDING = {"torch-cpu": 0, "ieee": 1, "torch-cpu-amd": 2}


def init(device: int = 0) -> None:
    """Upload the library's constant tables to ROCm device `device` now
    (qs_init), so no later quant_fn call on it allocates or blocks."""
    if library().qs_init(int(device)) != 0:
        raise QuantSpecError(last_error())


def set_sqrt_rounding(mode: str) -> None:
    """Square-root rounding of the weights, process-wide: "torch-cpu" (the
    default: torch.sqrt on an Intel host's CPU, where the golden vectors were
    written), "ieee" (the correctly rounded root: torch.sqrt on a GPU tensor,
    C sqrtf) or "torch-cpu-amd" (torch.sqrt on an AMD EPYC host's CPU)."""
    if mode not in SQRT_ROUNDING:
        raise ValueError(f"square-root rounding {mode!r}: one of {', '.join(SQRT_ROUNDING)}")
    if library().qs_set_sqrt_rounding(SQRT_ROUNDING[mode]) != 0:
        raise QuantSpecError(last_error())


def sqrt_rounding() -> str:
    code = library().qs_get_sqrt_rounding()
    return next(name for name, c in SQRT_ROUNDING.items() if c == code)


def _rocm_device():
    import torch
    if not torch.cuda.is_available():
        raise QuantSpecError("quant_fn: no ROCm device; this build computes every type on the GPU "
                             "(a CPU tensor is staged through the current ROCm device)")
    return torch.device("cuda", torch.cuda.current_device())


def _quantize_host(ggml_type: int, x, qw, out):
    """A CPU (or other non-ROCm) x: copy it and qw to the current ROCm device,
    quantize there and return the bytes on x's device (synchronous)."""
    dev = _rocm_device()
    q = None if qw is None else qw.to(dev)
    got = quantize(ggml_type, x.to(dev), q)
    if out is None:
        return got.to(x.device)
    out.view(got.shape).copy_(got)
    return out


def quantize(ggml_type: int, x, qw, out=None):
    """Quantize the rows of x (n, k); returns uint8 (n, row_bytes) on x's device.

    x: float32 / float16 / bfloat16, any strides (layouts the C call does not
    take -- a column stride other than 1, rows not 16-byte aligned, a row
    stride that is not a multiple of 16 bytes or shorter than a row -- are
    copied to a contiguous tensor first).
    qw: (k,) float32 imatrix column weights on x's device, or None.
    On a ROCm device the launch goes on torch's current stream and nothing is
    synchronised; a tensor on any other device is staged through the current
    ROCm device and the call returns when the bytes are back."""
    import torch
    if x.dim() != 2:
        raise ValueError(f"quant_fn: x must be 2-D (n, k), got shape {tuple(x.shape)}")
    src_id = _src_id(x.dtype)
    if src_id is None:
        raise ValueError(f"quant_fn: unsupported dtype {x.dtype}")
    if x.device.type != "cuda":
        return _quantize_host(ggml_type, x, qw, out)
    n, k = x.shape
    esz = x.element_size()
    if n > 0 and ((k > 1 and x.stride(1) != 1) or x.data_ptr() % 16 or
                  (n > 1 and (x.stride(0) < k or (x.stride(0) * esz) % 16))):
        # an explicit copy: x.contiguous() returns x itself for a contiguous
        # view that starts off a 16-byte boundary; a fresh allocation does not
        x = torch.empty((n, k), dtype=x.dtype, device=x.device).copy_(x)
    rb = row_bytes(ggml_type, k)
    if out is None:
        out = torch.empty((n, rb), dtype=torch.uint8, device=x.device)
    elif out.dtype != torch.uint8 or not out.is_contiguous() or out.numel() < n * rb:
        raise ValueError("quant_fn: out must be contiguous uint8 with n*row_bytes elements")
    qptr = None
    if qw is not None:
        if qw.device != x.device or qw.dtype != torch.float32 or qw.numel() < k:
            raise ValueError("quant_fn: qw must be float32 with k values on x's device")
        qw = qw.contiguous()
        qptr = qw.data_ptr()
    stride_bytes = (x.stride(0) if n > 1 else k) * x.element_size()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    # one C call takes at most MAX_VALUES_PER_CALL values: larger inputs go in
    # row ranges (the bytes do not depend on the split)
    rows = max(1, MAX_VALUES_PER_CALL // max(k, 1))
    for r0 in range(0, max(n, 1), rows):
        m = max(0, min(rows, n - r0))
        rc = library().qs_quantize(int(ggml_type), src_id, x.data_ptr() + r0 * stride_bytes, m, k,
                                   stride_bytes, qptr, out.data_ptr() + r0 * rb,
                                   out.numel() - r0 * rb, stream)
        if rc != 0:
            raise QuantSpecError(last_error())
    return out.view(n, rb) if out.dim() != 2 else out


class QuantSpec:
    """Same fields and meaning as the reference's QuantSpec (kernels/common.py:27-37)."""

    def __init__(self, ggml_type: GGMLQuantizationType, ftype: LlamaFileType,
                 bytes_per_elem: int, needs_imatrix: bool, make_kernel,
                 uses_imatrix: bool | None = None):
        self.ggml_type = ggml_type
        self.ftype = ftype
        self.bytes_per_elem = bytes_per_elem  # rough full-pipeline working set per element
        self.needs_imatrix = needs_imatrix
        self.make_kernel = make_kernel        # (device, qw_tensor|None) -> fn(x)->uint8
        self.uses_imatrix = needs_imatrix if uses_imatrix is None else uses_imatrix


def _kernel_factory(ggml_type: GGMLQuantizationType, uses_imatrix: bool):
    def make_kernel(device, qw):
        import torch
        q = qw if uses_imatrix else None    # Q4_0 ignores an imatrix (q4_0.py:36-37), as do
                                            # the other 32-value integer formats
        if q is not None:
            q = q.to(device=device, dtype=torch.float32).contiguous()
        if torch.device(device).type == "cuda" or q is None:
            return lambda x: quantize(ggml_type, x, q)
        # a CPU (or MPS) kernel: its imatrix goes to the ROCm device once, on
        # first use, instead of once per call
        staged = {}

        def quant_fn(x):
            if x.device.type == "cuda":
                return quantize(ggml_type, x, q.to(x.device))
            if "q" not in staged:
                staged["q"] = q.to(_rocm_device())
            got = quantize(ggml_type, x.to(staged["q"].device), staged["q"])
            return got.to(x.device)
        return quant_fn
    return make_kernel


# (name, ggml type, file type, bytes_per_elem, needs_imatrix, uses_imatrix): the
# SPECS entries of the reference modules (q4_0.py:40-43, q2_k.py:88-91,
# q3_k.py:85-88, q4_k.py:86-89, q5_k.py:89-92, q6_k.py:72-75, iq4_xs.py:195-198,
# iq2.py:506-509, iq2_xs.py:77-80, iq2_s.py:70-73, iq3_xxs.py:143-146,
# iq3_s.py:148-151)
_T, _F = GGMLQuantizationType, LlamaFileType
_SPECS = [
    ("q4_0", _T.Q4_0, _F.MOSTLY_Q4_0, 16, False, False),
    ("q2_k", _T.Q2_K, _F.MOSTLY_Q2_K, 24, False, True),
    ("q3_k", _T.Q3_K, _F.MOSTLY_Q3_K_M, 24, False, True),
    ("q4_k", _T.Q4_K, _F.MOSTLY_Q4_K_M, 24, False, True),
    ("q5_k", _T.Q5_K, _F.MOSTLY_Q5_K_M, 24, False, True),
    ("q6_k", _T.Q6_K, _F.MOSTLY_Q6_K, 24, False, True),
    ("iq4_xs", _T.IQ4_XS, _F.MOSTLY_IQ4_XS, 24, False, True),
    ("iq2_xxs", _T.IQ2_XXS, _F.MOSTLY_IQ2_XXS, 64, True, True),
    ("iq2_xs", _T.IQ2_XS, _F.MOSTLY_IQ2_XS, 64, True, True),
    ("iq2_s", _T.IQ2_S, _F.MOSTLY_IQ2_S, 64, True, True),
    ("iq3_xxs", _T.IQ3_XXS, _F.MOSTLY_IQ3_XXS, 64, True, True),
    ("iq3_s", _T.IQ3_S, _F.MOSTLY_IQ3_S, 64, False, True),
    # ggml formats the reference has no module for (quant-studio.py:396-399
    # stops on them); working-set sizes as for the reference's Q4_0 and IQ4_XS
    ("q4_1", _T.Q4_1, _F.MOSTLY_Q4_1, 16, False, False),
    ("q5_0", _T.Q5_0, _F.MOSTLY_Q5_0, 16, False, False),
    ("q5_1", _T.Q5_1, _F.MOSTLY_Q5_1, 16, False, False),
    ("q8_0", _T.Q8_0, _F.MOSTLY_Q8_0, 16, False, False),
    ("iq4_nl", _T.IQ4_NL, _F.MOSTLY_IQ4_NL, 24, False, True),
]
ALL_SPECS: dict[str, QuantSpec] = {
    name: QuantSpec(t, f, bpe, needs, _kernel_factory(t, uses), uses)
    for name, t, f, bpe, needs, uses in _SPECS
}


def _registry() -> dict[str, QuantSpec]:
    """Types with a HIP quantizer in the loaded library (registry semantics of
    kernels/__init__.py:18-27: a type without a kernel is simply absent)."""
    try:
        L = library()
    except ImportError as e:  # like a kernel module that fails to import: warn, register nothing
        print(f"warning: quant-studio_amd: {e}", file=sys.stderr)
        return {}
    return {n: s for n, s in ALL_SPECS.items() if L.qs_type_supported(int(s.ggml_type))}


QUANT_TYPES: dict[str, QuantSpec] = _registry()

__all__ = ["QUANT_TYPES", "ALL_SPECS", "QuantSpec", "QuantSpecError", "TORCH_DTYPES",
           "GGMLQuantizationType", "LlamaFileType", "library", "quantize", "row_bytes", "init",
           "set_sqrt_rounding", "sqrt_rounding"]
