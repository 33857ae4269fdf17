"""Host pipeline of the command line, driven from Python over the C ABI.

The staging itself is native (qs_pipeline_* in libqs_hip.so): a ring of
pinned slots, a thread pool for the mapping -> pinned copies, H2D/D2H on a
copy stream, kernels on a compute stream, and a writer thread that pwrite()s
each chunk at its own file offset once its D2H event has fired. It replaces
the reference's CudaPipeline, OutputWriter and copy_tensor
(quant-studio.py:103-131, :148-213, :235-241). Python keeps what the
reference keeps in Python: the GGUF header, tensor order and offsets, the type
plan, and the chunk size derived from --mem (quant-studio.py:457).

No torch: the command line starts without importing it.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

from . import library, last_error
from .gguf_io import TensorInfo
from .gguf_types import GGMLQuantizationType as GT

# source ids of the C ABI (QS_SRC_*)
SRC_IDS = {GT.F32: 0, GT.F16: 1, GT.BF16: 30}


class PipelineError(RuntimeError):
    pass


def device_count() -> int:
    return int(library().qs_device_count())


class NativePipeline:
    def __init__(self, device: int, fd: int, slots: int = 3, copy_threads: int | None = None):
        self.L = library()
        self.fd = fd
        n = copy_threads or min(16, len(os.sched_getaffinity(0)))
        h = ctypes.c_void_p()
        self._check(self.L.qs_pipeline_create(int(device), int(slots), int(n), ctypes.byref(h)))
        self.h = h
        self._keep: list = []          # host buffers that must outlive finish()

    @staticmethod
    def _check(rc: int) -> None:
        if rc != 0:
            raise PipelineError(last_error())

    def quantize_tensor(self, t: TensorInfo, ggml_type: int, qw: np.ndarray | None,
                        rows_per_chunk: int, offset: int, row_bytes: int) -> int:
        """Queue tensor t (rows from the input mapping) for quantization to
        ggml_type, written at `offset` of the output file; returns its bytes."""
        rows = t.rows()
        n_rows = rows.shape[0]
        k = t.ne[0]
        qptr = None
        if qw is not None:
            qw = np.ascontiguousarray(qw[:k], dtype=np.float32)
            self._keep.append(qw)
            qptr = qw.ctypes.data
        self._check(self.L.qs_pipeline_quantize(self.h, int(ggml_type), SRC_IDS[t.ggml_type],
                                                rows.ctypes.data, n_rows, k, qptr, int(rows_per_chunk),
                                                self.fd, int(offset)))
        return n_rows * row_bytes

    def write(self, data: np.ndarray, offset: int) -> int:
        """Queue host bytes (a passthrough tensor's mapping) for writing at offset."""
        data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        self._keep.append(data)
        self._check(self.L.qs_pipeline_write(self.h, data.ctypes.data, data.size, self.fd, int(offset)))
        return int(data.size)

    def finish(self) -> None:
        self._check(self.L.qs_pipeline_finish(self.h))
        self._keep.clear()

    def close(self) -> None:
        if self.h:
            self.L.qs_pipeline_destroy(self.h)
            self.h = None
            self._keep.clear()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
