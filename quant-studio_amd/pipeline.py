"""Host pipeline: mapped GGUF rows -> pinned staging -> HBM -> HIP quantizer ->
pinned -> output file.

Replaces the reference's CudaPipeline / OutputWriter / copy_tensor
(quant-studio.py:103-131, :148-213, :235-241) with:
  - a ring of pinned slots (default 3) so the host copy of chunk i+2, the H2D
    of chunk i+1 and the kernel of chunk i overlap;
  - the mmap -> pinned copy split over a thread pool (one thread would cap the
    pipeline well below PCIe rate);
  - H2D and D2H on a dedicated copy stream, kernels on the compute stream,
    ordered by events; no host synchronisation inside a chunk;
  - bf16/f16/f32 rows handed to the kernel as stored (no f32 upcast pass);
  - a single writer thread that keeps file order and waits on each chunk's
    D2H event before writing it.
The output bytes do not depend on the chunking.
"""

from __future__ import annotations

import os
from collections import deque
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

from .gguf_io import GGUFWriter, TensorInfo
from .gguf_types import GGMLQuantizationType as GT

_TORCH_SRC = {GT.F32: torch.float32, GT.F16: torch.float16, GT.BF16: torch.bfloat16}


class OrderedWriter:
    """All file writes on one thread, in submission order; errors surface on the
    next submit or at flush."""

    def __init__(self, writer: GGUFWriter):
        self.w = writer
        self.pool = ThreadPoolExecutor(max_workers=1)
        self.futs: deque = deque()

    def submit(self, fn):
        while self.futs and self.futs[0].done():
            self.futs.popleft().result()
        f = self.pool.submit(fn)
        self.futs.append(f)
        return f

    def pad(self):
        return self.submit(self.w.pad)

    def write(self, buf):
        return self.submit(lambda: self.w.fout.write(buf))

    def flush(self):
        while self.futs:
            self.futs.popleft().result()

    def close(self):
        self.flush()
        self.pool.shutdown()


class _Slot:
    def __init__(self):
        self.in_pin = self.out_pin = None
        self.x_dev = self.out_dev = None
        self.h2d = self.kern = self.d2h = None
        self.write_fut = None


def _grow_pinned(buf, nbytes):
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 1), dtype=torch.uint8, pin_memory=True)
    return buf


def _grow_dev(buf, nbytes, dev):
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    return buf


class HipPipeline:
    def __init__(self, device: torch.device, out: OrderedWriter, slots: int = 3,
                 copy_threads: int | None = None):
        self.dev = device
        self.out = out
        self.slots = [_Slot() for _ in range(slots)]
        self.next = 0
        self.copy_stream = torch.cuda.Stream(device)          # default priority
        self.compute = torch.cuda.current_stream(device)
        n = copy_threads or min(16, len(os.sched_getaffinity(0)))
        self.copy_pool = ThreadPoolExecutor(max_workers=n)
        self.n_copy = n

    def _host_copy(self, dst: np.ndarray, src: np.ndarray) -> None:
        """mmap rows -> pinned, split across the copy threads (numpy releases
        the GIL for these copies; page faults are taken in parallel)."""
        n = src.shape[0]
        parts = min(self.n_copy, max(1, src.nbytes >> 22))
        if parts <= 1:
            np.copyto(dst, src)
            return
        bounds = np.linspace(0, n, parts + 1, dtype=np.int64)
        futs = [self.copy_pool.submit(np.copyto, dst[a:b], src[a:b])
                for a, b in zip(bounds[:-1], bounds[1:]) if b > a]
        for f in futs:
            f.result()

    def quantize_tensor(self, t: TensorInfo, ggml_type: int, qw: torch.Tensor | None,
                        rows_per_chunk: int, quantize) -> int:
        rows = t.rows()
        n_rows, in_row_bytes = rows.shape
        k = t.ne[0]
        src_dtype = _TORCH_SRC[t.ggml_type]
        out_row_bytes = None
        written = 0
        for i0 in range(0, n_rows, rows_per_chunk):
            n = min(rows_per_chunk, n_rows - i0)
            s = self.slots[self.next]
            self.next = (self.next + 1) % len(self.slots)
            # this slot's pinned input was last read by its H2D; its pinned
            # output by the writer thread
            if s.h2d is not None:
                s.h2d.synchronize()
            if s.write_fut is not None:
                s.write_fut.result()
            nin = n * in_row_bytes
            s.in_pin = _grow_pinned(s.in_pin, nin)
            self._host_copy(s.in_pin[:nin].numpy().reshape(n, in_row_bytes), rows[i0:i0 + n])
            with torch.cuda.stream(self.copy_stream):
                if s.kern is not None:                # the kernel that read x_dev is done
                    self.copy_stream.wait_event(s.kern)
                s.x_dev = _grow_dev(s.x_dev, nin, self.dev)
                s.x_dev[:nin].copy_(s.in_pin[:nin], non_blocking=True)
                s.h2d = torch.cuda.Event()
                s.h2d.record(self.copy_stream)
            self.compute.wait_event(s.h2d)
            if s.d2h is not None:                     # out_dev's previous D2H is done
                self.compute.wait_event(s.d2h)
            x = s.x_dev[:nin].view(src_dtype).view(n, k)
            if out_row_bytes is None:
                from . import row_bytes
                out_row_bytes = row_bytes(ggml_type, k)
            nout = n * out_row_bytes
            s.out_dev = _grow_dev(s.out_dev, nout, self.dev)
            quantize(ggml_type, x, qw, out=s.out_dev[:nout])
            s.kern = torch.cuda.Event()
            s.kern.record(self.compute)
            with torch.cuda.stream(self.copy_stream):
                self.copy_stream.wait_event(s.kern)
                s.out_pin = _grow_pinned(s.out_pin, nout)
                s.out_pin[:nout].copy_(s.out_dev[:nout], non_blocking=True)
                s.d2h = torch.cuda.Event()
                s.d2h.record(self.copy_stream)
            buf, ev = s.out_pin[:nout].numpy(), s.d2h

            def _write(ev=ev, buf=buf):
                ev.synchronize()
                self.out.w.fout.write(buf.data)
            s.write_fut = self.out.submit(_write)
            written += nout
        return written

    def close(self) -> None:
        self.copy_pool.shutdown()


def copy_tensor(t: TensorInfo, mem_bytes: int, out: OrderedWriter) -> int:
    """Pass a tensor through untouched (the writer thread reads the mapping)."""
    flat = t.data
    step = max(1 << 20, mem_bytes)
    for off in range(0, flat.shape[0], step):
        out.submit(lambda a=flat[off:off + step]: out.w.fout.write(a.data))
    return int(flat.shape[0])
