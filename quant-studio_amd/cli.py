"""quant-studio command line: GGUF -> GGUF quantization on one MI355X.

The command-line contract is the reference driver's (quant-studio.py:267-476):
the same argv (`in.gguf [out.gguf] <scheme> [nthreads] [options]`), defaults,
scheme table, per-tensor plan (scheme.py here), checks, error messages, exit
codes and output layout. The code is organised differently: the options are
a table (OPTIONS / REJECTED below), a parse produces a `Request`, and the run
is three phases -- plan every tensor, then either print the plan (--dry-run)
or stream the tensors through the native pipeline (pipeline.py).

Devices: quantization runs on a ROCm device. `--device cpu` and `--device mps`
(the reference's CPU / Apple paths, quant-studio.py:51-58, :216-232) are
accepted and also compute on the ROCm device: the blocks are the bytes of the
reference's CPU path either way. `--sqrt-rounding` (an addition) selects whose
torch.sqrt rounding the weights follow (the library's QS_SQRT_* modes).
"""

from __future__ import annotations

import argparse
import os
import sys
import time
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from . import scheme
from .gguf_io import VT, GGUFReader, GGUFWriter, KV, load_imatrix, tensor_nbytes
from .gguf_types import GGMLQuantizationType as GT

QUANTIZATION_VERSION = 2
_SOURCE_TYPES = (GT.F32, GT.F16, GT.BF16)

# ---------------------------------------------------------------------------
# the option table
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class Option:
    flag: str
    kind: str                 # "value", "switch" (store_true), "list" (append), "path"
    default: object = None
    metavar: str | None = None
    help: str | None = None   # None: accepted but not listed


OPTIONS = (
    Option("--mem", "value", "4G", None, "host/device budget per row chunk (e.g. 4G, 512M)"),
    Option("--device", "value", "auto", None,
           "auto / cuda / hip / cuda:N; cpu and mps are accepted and computed on the ROCm device"),
    Option("--imatrix", "path", None, None, "importance matrix (GGUF)"),
    Option("--pure", "switch", False, None,
           "one type for every eligible tensor: no k-quant mixture"),
    Option("--leave-output-tensor", "switch", False, None, "keep output.weight as it is"),
    Option("--output-tensor-type", "value", None, "ggml_type", "type for output.weight"),
    Option("--token-embedding-type", "value", None, "ggml_type", "type for the token embeddings"),
    Option("--tensor-type", "list", [], "name=ggml_type",
           "type for tensors whose name matches the regex (may repeat)"),
    Option("--tensor-type-file", "path", None, "file",
           "name=ggml_type entries, whitespace-separated"),
    Option("--dry-run", "switch", False, None, "print the per-tensor plan and sizes, write nothing"),
    Option("--sqrt-rounding", "value", "torch-cpu", None,
           "whose torch.sqrt the weights follow: torch-cpu (the reference's eager CPU "
           "path on an Intel host, default, for every --device), torch-cpu-amd (the "
           "same on an AMD EPYC host) or ieee (correctly rounded, as the reference's "
           "GPU path computes it); --device auto/cuda does not select ieee"),
)

# llama-quantize options the reference recognises and refuses (quant-studio.py:305-312)
REJECTED = (
    Option("--allow-requantize", "switch", False),
    Option("--include-weights", "value"),
    Option("--exclude-weights", "value"),
    Option("--prune-layers", "value"),
    Option("--keep-split", "switch", False),
    Option("--override-kv", "list", []),
)

_DEVICES = ("auto", "cuda", "hip", "cpu", "mps")


def _dest(opt: Option) -> str:
    return opt.flag.lstrip("-").replace("-", "_")


def _add(group, opt: Option) -> None:
    kw: dict = {"help": opt.help if opt.help is not None else argparse.SUPPRESS}
    if opt.kind == "switch":
        kw["action"] = "store_true"
    elif opt.kind == "list":
        kw.update(action="append", default=list(opt.default or []))
    else:
        kw["default"] = opt.default
        if opt.kind == "path":
            kw["type"] = Path
    if opt.metavar is not None:
        kw["metavar"] = opt.metavar
    group.add_argument(opt.flag, **kw)


def build_parser() -> argparse.ArgumentParser:
    ap = argparse.ArgumentParser(
        prog="quant-studio.py",
        usage="%(prog)s input.gguf [output.gguf] type [options]",
        description="Quantize a GGUF model on an AMD Instinct MI355X; argv of llama-quantize.",
        formatter_class=argparse.RawDescriptionHelpFormatter,
        epilog=scheme.format_scheme_table())
    ap.add_argument("input", type=Path, help="F32 / F16 / BF16 source model")
    ap.add_argument("words", nargs="*", metavar="[output.gguf] type",
                    help="output path (default ggml-model-<TYPE>.gguf beside the input) and "
                         "scheme from the table below")
    for opt in OPTIONS:
        _add(ap, opt)
    refused = ap.add_argument_group("llama-quantize options that are refused")
    for opt in REJECTED:
        _add(refused, opt)
    return ap


# ---------------------------------------------------------------------------
# parsing into a request
# ---------------------------------------------------------------------------


@dataclass
class Request:
    src: Path
    dst: Path
    option: scheme.SchemeOption
    mem_bytes: int
    mem_text: str
    device: str
    imatrix: Path | None
    pure: bool
    keep_output: bool
    output_type: GT | None
    embedding_type: GT | None
    overrides: list = field(default_factory=list)
    dry_run: bool = False
    sqrt_rounding: str = "torch-cpu"


def parse_mem(text: str) -> int:
    """--mem: a byte count, or a number with a binary K / M / G suffix."""
    t = text.strip().upper()
    scale = {"K": 1 << 10, "M": 1 << 20, "G": 1 << 30}.get(t[-1:])
    return int(float(t[:-1]) * scale) if scale else int(t)


def parse_ggml_type(name: str) -> GT:
    found = GT.__members__.get(name.upper())
    if found is None:
        sys.exit(f"error: unknown ggml type: {name}")
    return found


def fmt_size(n: float) -> str:
    """Size for the progress lines: bytes below 1 KiB, else KiB / MiB / GiB."""
    if n < 1024:
        return f"{int(n):8d} B  "
    for unit, scale in (("KiB", 1 << 10), ("MiB", 1 << 20), ("GiB", 1 << 30)):
        if n < scale * 1024 or unit == "GiB":
            return f"{n / scale:8.1f} {unit}"
    raise AssertionError("unreachable")


def split_positionals(ap: argparse.ArgumentParser, words: list[str]):
    """The words after the input, in llama-quantize's two forms:
         output type [nthreads]       and       type [nthreads]
    The output is taken as omitted when the first word names a scheme and the
    next is absent or a thread count (quant-studio.py:314-319). Returns
    (output or None, type or None, nthreads or None)."""
    if len(words) > 3:
        ap.error("unrecognized arguments: " + " ".join(words[3:]))
    first, second, third = (list(words) + [None, None, None])[:3]
    output_omitted = (first is not None and scheme.parse_scheme(first) is not None
                      and (second is None or second.isdigit()))
    if output_omitted:
        return None, first, second
    return first, second, third


def parse_request(argv: list[str] | None = None) -> Request:
    ap = build_parser()
    ns = ap.parse_args(argv)
    for opt in REJECTED:
        if getattr(ns, _dest(opt)):
            sys.exit(f"error: {opt.flag} is not supported by quant-studio")
    output, qtype, nthreads = split_positionals(ap, ns.words)
    if qtype is None:
        ap.error("missing quantization type")
    if nthreads is not None:
        sys.exit("error: the nthreads argument is not supported by quant-studio (GPU pipeline)")

    option = scheme.parse_scheme(qtype)
    if option is None:
        sys.exit(f"error: unknown quantization scheme {qtype!r}\n\n" + scheme.format_scheme_table())
    if not option.supported:
        sys.exit(f"error: scheme {option.name} is not supported by quant-studio\n\n"
                 + scheme.format_scheme_table())

    entries = list(ns.tensor_type)
    if ns.tensor_type_file is not None:
        entries += ns.tensor_type_file.read_text().split()
    overrides = []
    for entry in entries:
        pattern, sep, tname = entry.partition("=")
        if not tname:
            sys.exit(f"error: invalid --tensor-type {entry!r}, expected name=ggml_type")
        overrides.append((pattern, parse_ggml_type(tname)))

    device = ns.device
    if device not in _DEVICES and not (device.startswith(("cuda:", "hip:"))
                                       and device.split(":", 1)[1].isdigit()):
        sys.exit(f"error: device {device!r}: use auto, cuda, hip, cuda:N, cpu or mps")
    if ns.sqrt_rounding not in ("torch-cpu", "torch-cpu-amd", "ieee"):
        sys.exit(f"error: --sqrt-rounding {ns.sqrt_rounding!r}: use torch-cpu, torch-cpu-amd or ieee")

    return Request(
        src=ns.input,
        dst=Path(output) if output else ns.input.parent / f"ggml-model-{option.name}.gguf",
        option=option, mem_bytes=parse_mem(ns.mem), mem_text=ns.mem, device=device,
        imatrix=ns.imatrix, pure=ns.pure, keep_output=ns.leave_output_tensor,
        output_type=parse_ggml_type(ns.output_tensor_type) if ns.output_tensor_type else None,
        embedding_type=parse_ggml_type(ns.token_embedding_type) if ns.token_embedding_type else None,
        overrides=overrides, dry_run=ns.dry_run, sqrt_rounding=ns.sqrt_rounding)


# ---------------------------------------------------------------------------
# the plan
# ---------------------------------------------------------------------------


@dataclass
class Step:
    tensor: object               # gguf_io.TensorInfo
    dst: GT | None = None        # None: written as it is
    spec: object = None          # QuantSpec of dst

    def out_nbytes(self) -> int:
        t = self.tensor
        if self.dst is None:
            return t.nbytes
        return t.n_elements // t.ne[0] * tensor_nbytes(self.dst, (t.ne[0],))


def plan_tensors(req: Request, reader: GGUFReader, imatrix: dict) -> list[Step]:
    """One step per tensor in the loader's order (the counters of the policy
    depend on it), with the type the policy picks; exits on types without a
    kernel and on tensors that need imatrix data (quant-studio.py:362-419)."""
    from . import QUANT_TYPES
    tensors = sorted(reader.tensors, key=lambda t: scheme.weight_name_key(t.name))
    kv = reader.values()
    model = scheme.ModelInfo.from_kv(kv)
    state = scheme.init_state(model, [t.name for t in tensors], bool(imatrix), req.overrides)
    spec_of = {s.ggml_type: s for s in QUANT_TYPES.values()}
    steps, missing, needs_data = [], {}, []
    for t in tensors:
        dst = t.ggml_type
        if t.ggml_type in _SOURCE_TYPES:
            try:
                dst = scheme.tensor_get_type(
                    state, model, t.name, t.ne, t.ggml_type, req.option.ftype, pure=req.pure,
                    quantize_output_tensor=not req.keep_output,
                    token_embedding_type=req.embedding_type, output_tensor_type=req.output_type)
            except ValueError as e:
                print(f"warning: {t.name}: {e}; keeping {t.ggml_type.name}", file=sys.stderr)
        if dst == t.ggml_type:
            steps.append(Step(t))
            continue
        spec = spec_of.get(dst)
        if spec is None:
            missing.setdefault(dst.name, []).append(t.name)
            steps.append(Step(t))
            continue
        wants_data = spec.needs_imatrix or scheme.tensor_requires_imatrix(t.name, dst, req.option.ftype)
        if wants_data and t.name not in imatrix:
            needs_data.append(t.name)
        steps.append(Step(t, dst, spec))

    if missing:
        detail = "; ".join(f"{ty} for {len(names)} tensors (e.g. {names[0]})"
                           for ty, names in sorted(missing.items()))
        sys.exit(f"error: this scheme needs kernel types quant-studio does not have yet: {detail}")
    if needs_data:
        names = sorted(set(needs_data))
        hint = "" if req.imatrix else " (pass --imatrix)"
        if "token_embd.weight" in names:
            hint += " (token_embd can be overridden with --token-embedding-type)"
        sys.exit(f"error: {len(names)} tensors require importance matrix data{hint}: "
                 + ", ".join(names[:4]) + ("..." if len(names) > 4 else ""))
    return steps


def print_plan(steps: list[Step]) -> None:
    total_in = total_out = 0
    for st in steps:
        nb = st.out_nbytes()
        total_in += st.tensor.nbytes
        total_out += nb
        kind = st.tensor.ggml_type.name
        print(f"{st.tensor.name:48s} {kind:>8s} -> {st.dst.name if st.dst else kind:<8s} {fmt_size(nb)}")
    print(f"dry run: {fmt_size(total_in)} -> {fmt_size(total_out)} tensor data "
          f"({total_out / max(total_in, 1) * 100:.1f}%)")


# ---------------------------------------------------------------------------
# writing the output
# ---------------------------------------------------------------------------


def copied_kvs(reader: GGUFReader, ftype: int) -> list[KV]:
    """The input's KVs in order, without general.architecture (the writer puts
    it first) and the GGUF.* entries, then general.file_type and
    general.quantization_version (quant-studio.py:249-264)."""
    tail = [KV("general.file_type", VT.UINT32, int(ftype)),
            KV("general.quantization_version", VT.UINT32, QUANTIZATION_VERSION)]
    replaced = {kv.name for kv in tail} | {"general.architecture"}
    keep = [kv for name, kv in reader.kv.items() if name not in replaced and not name.startswith("GGUF.")]
    return keep + tail


def device_index(req: Request, ndev: int) -> int:
    if ndev == 0:
        sys.exit("error: no ROCm device available (this build has no CPU quantization path)")
    index = int(req.device.split(":", 1)[1]) if ":" in req.device else 0
    if index >= ndev:
        sys.exit(f"error: device {req.device!r} not present ({ndev} ROCm devices)")
    return index


def preallocate(fd: int, size: int) -> bool:
    """Allocate the output file's blocks up front with the fallocate(2) system
    call: writes into the page cache then skip ext4's per-page delayed
    allocation (about twice the pwrite rate there). Where the filesystem
    cannot (EOPNOTSUPP) nothing happens and the writes allocate as usual; glibc's
    posix_fallocate would instead write a byte into every block."""
    import ctypes
    try:
        libc = ctypes.CDLL(None, use_errno=True)
        fn = libc.fallocate
    except (OSError, AttributeError):
        return False
    fn.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64]
    fn.restype = ctypes.c_int
    return size > 0 and fn(fd, 0, 0, size) == 0


def start_device(req: Request, early=None):
    """The native pipeline's creation on a thread of its own (a
    PipelineStart), so the device's initialisation overlaps loading the
    imatrix, parsing the input and planning the tensors: `early` (started by
    the entry script from argv) if it is for the requested device, else one
    started now; None for a dry run. Which device is used, and every error, is
    still decided by write_output in the reference's order (its pipeline is
    created after the plan, quant-studio.py:445-449)."""
    from .pipeline_start import PipelineStart
    try:
        dev = None if req.dry_run else (int(req.device.split(":", 1)[1]) if ":" in req.device else 0)
    except ValueError:
        dev = None
    if early is not None and early.device == dev:
        return early
    if early is not None:
        early.close()
    return None if dev is None or dev < 0 else PipelineStart(dev)


def write_output(req: Request, reader: GGUFReader, steps: list[Step], imatrix: dict,
                 start=None) -> None:
    """Streams the planned tensors through the native pipeline into req.dst;
    `start` is start_device()'s pipeline in the making, if any."""
    from . import library, row_bytes, SQRT_ROUNDING
    from .pipeline import NativePipeline, PipelineError, Readahead, device_count
    dev = device_index(req, device_count())
    if req.device in ("cpu", "mps"):
        print(f"note: --device {req.device}: computed on ROCm device {dev} (the same bytes as the "
              f"reference's {req.device} path)")
    if library().qs_set_sqrt_rounding(SQRT_ROUNDING[req.sqrt_rounding]) != 0:
        sys.exit("error: cannot select the square-root rounding")
    for st in steps:            # imatrix lengths are checked before anything is written
        t = st.tensor
        if st.dst is not None and st.spec.uses_imatrix and t.name in imatrix \
                and imatrix[t.name].size < t.ne[0]:
            sys.exit(f"error: imatrix data for {t.name} has {imatrix[t.name].size} values, "
                     f"rows have {t.ne[0]}")

    writer = GGUFWriter(req.dst, reader.values()["general.architecture"])
    for kv in copied_kvs(reader, req.option.ftype):
        writer.add_kv(kv)
    for st in steps:
        writer.add_tensor_info(st.tensor.name, st.tensor.ne, st.dst or st.tensor.ggml_type,
                               st.out_nbytes())
    writer.write_header()
    base = writer.data_start()
    writer.fout.flush()
    fd = writer.fout.fileno()
    preallocate(fd, writer.total_size())

    total_in = total_out = 0
    t0 = time.time()
    ahead = Readahead([st.tensor for st in steps])
    try:
        early = start.take(fd) if start is not None and start.device == dev else None
        with early or NativePipeline(dev, fd) as pipe:
            for i, (st, info) in enumerate(zip(steps, writer.infos)):
                t, off = st.tensor, base + info[3]
                ahead.advance(t.nbytes)
                if st.dst is None:
                    nbytes = pipe.write(t.data, off)
                else:
                    qw = imatrix.get(t.name) if st.spec.uses_imatrix else None
                    rows = max(1, req.mem_bytes // (t.ne[0] * st.spec.bytes_per_elem))
                    nbytes = pipe.quantize_tensor(t, int(st.dst), qw, rows, off,
                                                  row_bytes(int(st.dst), t.ne[0]), reader.fileno())
                total_in += t.nbytes
                total_out += nbytes
                shape = "x".join(str(d) for d in t.ne)
                src, dst = t.ggml_type.name, (st.dst or t.ggml_type).name
                print(f"[{i + 1:4d}/{len(steps)}] {t.name:48s} {shape:>16s}  {src:>5s} -> "
                      f"{dst:<8s} {fmt_size(t.nbytes)} -> {fmt_size(nbytes)}")
            pipe.finish()
    except PipelineError as e:
        writer.close()
        sys.exit(f"error: {e}")
    finally:
        ahead.close()
    os.ftruncate(fd, writer.total_size())     # the trailing padding is zeros
    writer.close()
    print(f"done in {time.time() - t0:.1f}s: {fmt_size(total_in)} -> {fmt_size(total_out)} "
          f"({total_out / max(total_in, 1) * 100:.1f}%)")


def main(argv: list[str] | None = None, early=None) -> int:
    """The command line; `early` is a PipelineStart the entry script began
    from argv before importing this module (pipeline_start.early_start)."""
    start = early
    try:
        req = parse_request(argv)
        device_shown = "rocm" if req.device not in ("cpu", "mps") else f"{req.device} (on rocm)"
        print(f"quant-studio: {req.src} -> {req.dst} [{req.option.name}] device={device_shown} "
              f"mem={req.mem_text} sqrt-rounding={req.sqrt_rounding}")
        start = start_device(req, early)
        imatrix: dict[str, np.ndarray] = {}
        if req.imatrix is not None:
            imatrix = load_imatrix(req.imatrix)
            print(f"imatrix: {len(imatrix)} entries from {req.imatrix}")
        reader = GGUFReader(req.src)
        if "general.architecture" not in reader.values():
            sys.exit("error: input has no general.architecture key")
        steps = plan_tensors(req, reader, imatrix)
        if req.dry_run:
            print_plan(steps)
            return 0
        write_output(req, reader, steps, imatrix, start)
    finally:
        if start is not None:
            start.close()           # a pipeline that was not taken (an error stopped the run)
    return 0
