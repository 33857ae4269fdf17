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


class Readahead:
    """Asks the kernel to read the input tensors into the page cache ahead of
    the pipeline's copies (madvise MADV_WILLNEED, in plan order, from a
    thread of its own, a window at a time), at most `budget` bytes past the
    tensor being queued.
    The copies fault the mapping in a few MB at a time and the pipeline waits
    for a free slot between chunks, so with a cold page cache the disk idles
    between reads; with the requests queued ahead it streams. Best effort:
    a failing madvise is ignored (the copies fault the pages in anyway)."""

    MADV_WILLNEED = 3

    def __init__(self, tensors: list[TensorInfo], budget: int = 1 << 30, madvise=None):
        import threading
        if madvise is None:
            libc = ctypes.CDLL(None, use_errno=True)
            libc.madvise.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
            libc.madvise.restype = ctypes.c_int
            madvise = libc.madvise        # ctypes releases the GIL during the call
        self._madvise = madvise
        self._page = os.sysconf("SC_PAGE_SIZE")
        self._ranges = [(t.data.ctypes.data, t.nbytes) for t in tensors if t.nbytes > 0]
        self._budget = budget
        self._queued = 0             # bytes of input the pipeline has been handed so far
        self._cv = threading.Condition()
        self._stop = False
        self._thread = threading.Thread(target=self._run, name="qs-readahead", daemon=True)
        self._thread.start()

    def advance(self, nbytes: int) -> None:
        """The pipeline is about to take nbytes more of the input."""
        with self._cv:
            self._queued += nbytes
            self._cv.notify()

    def close(self) -> None:
        with self._cv:
            self._stop = True
            self._cv.notify()
        self._thread.join()

    WINDOW = 2 << 20         # one request per 2 MiB: the kernel reads at most its
                             # readahead limit (a few MiB) per madvise call

    def _run(self) -> None:
        done = 0                 # input bytes advised so far, in plan order
        for addr, n in self._ranges:
            a = addr - addr % self._page
            end = addr + n
            while a < end:
                with self._cv:
                    while not self._stop and done - self._queued > self._budget:
                        self._cv.wait()
                    if self._stop:
                        return
                w = min(self.WINDOW, end - a)
                self._madvise(a, w, self.MADV_WILLNEED)
                done += w
                a += w


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
