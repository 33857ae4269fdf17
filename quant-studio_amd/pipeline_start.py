"""The native pipeline's creation on a thread of its own, started as early as
the command line can: its first stream creation sets up the device's queues
(~0.08 s on the MI355X), which then overlaps the imports, argument parsing,
imatrix loading and planning. Imports neither numpy nor torch, so the entry
script can start it before the command line's own imports.

Which device is used, and every error, is still decided by the command line
in the reference's order (its pipeline is created after the plan,
quant-studio.py:445-449): a start for another device, or one whose creation
failed, is closed and not used."""

from __future__ import annotations

import ctypes
import os
import threading


def _default_copy_threads() -> int:
    return min(16, len(os.sched_getaffinity(0)))


class PipelineStart:
    """qs_pipeline_create on a thread of its own. The thread loads the library
    and makes the C calls, which release the GIL, so the device's
    initialisation runs while the calling thread goes on with Python work.
    take() joins it and returns the NativePipeline, or None if the device is
    absent or the creation failed (the caller then creates one itself and sees
    the error on its own thread)."""

    def __init__(self, device: int, slots: int = 3, copy_threads: int | None = None):
        self.device = int(device)
        self._L = None
        self._h = ctypes.c_void_p()
        self._rc: int | None = None
        threads = int(copy_threads or _default_copy_threads())

        def run() -> None:
            from . import library
            try:
                L = library()
                if not 0 <= self.device < L.qs_device_count():
                    return
                self._L = L
                self._rc = L.qs_pipeline_create(self.device, int(slots), threads, ctypes.byref(self._h))
            except Exception:           # a missing library: reported by the caller's own attempt
                self._rc = None

        self._thread = threading.Thread(target=run, name="qs-pipeline-create", daemon=True)
        self._thread.start()

    def take(self, fd: int):
        self._thread.join()
        if self._rc != 0 or not self._h.value:
            return None
        from .pipeline import NativePipeline
        h, self._h = self._h, ctypes.c_void_p()
        return NativePipeline(self.device, fd, handle=h)

    def close(self) -> None:
        """Release a pipeline that was not taken."""
        self._thread.join()
        if self._rc == 0 and self._h.value:
            self._L.qs_pipeline_destroy(self._h)
            self._h = ctypes.c_void_p()


def requested_device(argv: list[str]) -> int | None:
    """The ROCm device a command line will use, read from argv without the
    full parser (--device cuda:N or --device=cuda:N; every other device
    choice, cpu and mps included, computes on device 0), or None for a run
    that will not use a device (--dry-run, help, no arguments)."""
    if not argv or any(a in ("--dry-run", "-h", "--help") for a in argv):
        return None
    dev = "auto"
    for i, a in enumerate(argv):
        if a == "--device" and i + 1 < len(argv):
            dev = argv[i + 1]
        elif a.startswith("--device="):
            dev = a.split("=", 1)[1]
    if ":" in dev:
        try:
            return int(dev.split(":", 1)[1])
        except ValueError:
            return None
    return 0


def early_start(argv: list[str]) -> PipelineStart | None:
    """A PipelineStart for the device argv asks for, or None."""
    dev = requested_device(argv)
    return None if dev is None or dev < 0 else PipelineStart(dev)
