"""Host pipeline of the command line, driven from Python over the C ABI.

The staging itself is native (qs_pipeline_* in libqs_hip.so): a ring of
pinned slots, a thread pool that reads each chunk's rows from the input file
(pread) into its slot one chunk ahead of the launches, uploads on a copy
stream, kernels on two compute streams writing each chunk's output into a
pinned host slot, and a writer thread that pwrite()s each chunk at its own
file offset once its kernel has finished. It replaces
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
from .pipeline_start import PipelineStart  # noqa: F401  (created before numpy is imported)

# source ids of the C ABI (QS_SRC_*)
SRC_IDS = {GT.F32: 0, GT.F16: 1, GT.BF16: 30}


class PipelineError(RuntimeError):
    pass


class Readahead:
    """Asks the kernel to read the input tensors into the page cache ahead of
    the pipeline's copies (madvise MADV_WILLNEED, in plan order, from a
    thread of its own, a window at a time), at most `budget` bytes past the
    tensor being queued.
    The pipeline reads a chunk at a time and waits for a free slot between
    chunks, so with a cold page cache the disk would idle between reads; with
    the requests queued ahead it streams. The advice goes through the file's
    mapping but maps nothing into the process (no page-table entries are
    made). Best effort: a failing madvise is ignored (the reads fetch the
    pages anyway)."""

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


# Input bytes per staged chunk. --mem bounds a chunk (the reference's budget
# per row chunk, quant-studio.py:457); the pipeline stages at most this much
# per chunk within it. The output does not depend on the chunking, and with
# chunks of this size the read, upload, kernel and write of
# consecutive chunks overlap inside every tensor instead of across whole
# tensors, and the pinned slots stay small. Measured on the synthetic
# 4B-class model, warm (process wall, one MI355X, when this size was chosen):
# IQ2_XXS 0.77 s with whole tensors per chunk (--mem 4G) -> 0.61 s at 16 MiB
# (8 MiB 0.62, 32 MiB 0.62, 64 MiB 0.67, 128 MiB 0.73); Q4_K_M 0.74 -> 0.49
# s; IQ3_XXS 0.74 -> 0.60 s (at 32 MiB); IQ2_S 0.89 -> 0.76 s (at 32 MiB).
STAGE_BYTES = 16 << 20


def default_copy_threads() -> int:
    return min(16, len(os.sched_getaffinity(0)))


class NativePipeline:
    def __init__(self, device: int, fd: int, slots: int = 3, copy_threads: int | None = None,
                 handle: ctypes.c_void_p | None = None):
        """A pipeline on `device` writing to fd, or the one `handle` holds
        (made by PipelineStart)."""
        self.L = library()
        self.fd = fd
        if handle is None:
            handle = ctypes.c_void_p()
            self._check(self.L.qs_pipeline_create(int(device), int(slots),
                                                  int(copy_threads or default_copy_threads()),
                                                  ctypes.byref(handle)))
        self.h = handle
        self._keep: list = []          # host buffers that must outlive finish()

    @staticmethod
    def _check(rc: int) -> None:
        if rc != 0:
            raise PipelineError(last_error())

    def quantize_tensor(self, t: TensorInfo, ggml_type: int, qw: np.ndarray | None,
                        rows_per_chunk: int, offset: int, row_bytes: int, src_fd: int = -1) -> int:
        """Queue tensor t for quantization to ggml_type, written at `offset` of
        the output file, staged in chunks of at most rows_per_chunk rows and
        STAGE_BYTES input bytes; returns its bytes. With src_fd (the input
        file's descriptor, t read from it) the rows are read with pread at
        t.file_offset, else copied from t's mapping. The last chunk's rows may
        still be being read when this returns: the descriptor and the rows
        stay in use until finish()."""
        rows = t.rows()
        n_rows = rows.shape[0]
        k = t.ne[0]
        rows_per_chunk = max(1, min(int(rows_per_chunk), STAGE_BYTES // max(1, rows.shape[1])))
        qptr = None
        if qw is not None:
            qw = np.ascontiguousarray(qw[:k], dtype=np.float32)
            self._keep.append(qw)
            qptr = qw.ctypes.data
        if src_fd >= 0 and t.file_offset >= 0:
            self._check(self.L.qs_pipeline_quantize_fd(self.h, int(ggml_type), SRC_IDS[t.ggml_type],
                                                       int(src_fd), int(t.file_offset), n_rows, k, qptr,
                                                       int(rows_per_chunk), self.fd, int(offset)))
        else:
            self._keep.append(rows)
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
