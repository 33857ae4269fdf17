"""quant-studio command line: GGUF -> GGUF quantization on one MI355X.

Same argv, plan, checks, messages and output layout as the reference's
driver (quant-studio.py:267-476): llama-quantize scheme names, the
llama-quant tensor-type policy (scheme.py here), --imatrix / --mem / --pure /
--leave-output-tensor / --output-tensor-type / --token-embedding-type /
--tensor-type / --tensor-type-file / --dry-run, the rejected llama-quantize
flags and the positional output/type/nthreads shuffle. Quantization runs only
on a ROCm device (`--device auto|cuda|hip`); there is no CPU path.
"""

from __future__ import annotations

import argparse
import os
import sys
import time
from pathlib import Path

import numpy as np

from . import scheme
from .gguf_io import VT, GGUFReader, GGUFWriter, KV, load_imatrix, tensor_nbytes
from .gguf_types import GGMLQuantizationType as GT

QUANTIZATION_VERSION = 2
_SOURCE_TYPES = (GT.F32, GT.F16, GT.BF16)


def parse_mem(s: str) -> int:
    s = s.strip().upper()
    units = {"K": 1 << 10, "M": 1 << 20, "G": 1 << 30}
    if s and s[-1] in units:
        return int(float(s[:-1]) * units[s[-1]])
    return int(s)


def parse_ggml_type(s: str) -> GT:
    try:
        return GT[s.upper()]
    except KeyError:
        sys.exit(f"error: unknown ggml type: {s}")


def fmt_size(n: float) -> str:
    for unit in ("B", "KiB", "MiB", "GiB"):
        if n < 1024 or unit == "GiB":
            return f"{n:8.1f} {unit}" if unit != "B" else f"{int(n):8d} B  "
        n /= 1024
    return f"{n} B"


def build_parser() -> argparse.ArgumentParser:
    ap = argparse.ArgumentParser(
        prog="quant-studio.py",
        description="GGUF quantizer on AMD Instinct MI355X, drop-in for llama-quantize",
        formatter_class=argparse.RawDescriptionHelpFormatter,
        epilog=scheme.format_scheme_table())
    ap.add_argument("input", type=Path, help="source GGUF (F32/F16/BF16)")
    ap.add_argument("output", nargs="?", default=None,
                    help="output GGUF (default: ggml-model-<TYPE>.gguf next to the input)")
    ap.add_argument("qtype", nargs="?", default=None, metavar="type",
                    help="quantization scheme, see the table below")
    ap.add_argument("nthreads", nargs="?", default=None, help=argparse.SUPPRESS)
    ap.add_argument("--mem", default="4G", help="memory budget per chunk, e.g. 4G / 512M")
    ap.add_argument("--device", default="auto", help="ROCm device: auto / cuda / hip (/ cuda:N)")
    ap.add_argument("--imatrix", type=Path, default=None, help="GGUF importance matrix")
    ap.add_argument("--pure", action="store_true",
                    help="disable k-quant mixtures and quantize all tensors to the same type")
    ap.add_argument("--leave-output-tensor", action="store_true",
                    help="leave output.weight un(re)quantized")
    ap.add_argument("--output-tensor-type", default=None, metavar="ggml_type",
                    help="use this ggml_type for the output.weight tensor")
    ap.add_argument("--token-embedding-type", default=None, metavar="ggml_type",
                    help="use this ggml_type for the token embeddings tensor")
    ap.add_argument("--tensor-type", action="append", default=[], metavar="name=ggml_type",
                    help="quantize tensors matching this name regex to this type; repeatable")
    ap.add_argument("--tensor-type-file", type=Path, default=None, metavar="file",
                    help="file with name=ggml_type entries, separated by spaces or newlines")
    ap.add_argument("--dry-run", action="store_true",
                    help="show the per-tensor plan and final size without quantizing")
    rej = ap.add_argument_group("rejected llama-quantize options")
    rej.add_argument("--allow-requantize", action="store_true", help=argparse.SUPPRESS)
    rej.add_argument("--include-weights", default=None, help=argparse.SUPPRESS)
    rej.add_argument("--exclude-weights", default=None, help=argparse.SUPPRESS)
    rej.add_argument("--prune-layers", default=None, help=argparse.SUPPRESS)
    rej.add_argument("--keep-split", action="store_true", help=argparse.SUPPRESS)
    rej.add_argument("--override-kv", action="append", default=[], help=argparse.SUPPRESS)
    return ap


def copied_kvs(reader: GGUFReader, ftype: int) -> list[KV]:
    """Input KVs in order minus general.architecture (written first by the
    writer), then general.file_type and general.quantization_version."""
    over = {"general.file_type": KV("general.file_type", VT.UINT32, int(ftype)),
            "general.quantization_version": KV("general.quantization_version", VT.UINT32,
                                               QUANTIZATION_VERSION)}
    kvs = [kv for name, kv in reader.kv.items()
           if name != "general.architecture" and not name.startswith("GGUF.") and name not in over]
    return kvs + list(over.values())


def main(argv: list[str] | None = None) -> int:
    ap = build_parser()
    args = ap.parse_args(argv)
    for flag, val in (("--allow-requantize", args.allow_requantize),
                      ("--include-weights", args.include_weights),
                      ("--exclude-weights", args.exclude_weights),
                      ("--prune-layers", args.prune_layers),
                      ("--keep-split", args.keep_split),
                      ("--override-kv", args.override_kv)):
        if val:
            sys.exit(f"error: {flag} is not supported by quant-studio")

    # llama-quantize positional style: the output name may be omitted
    if args.output is not None and scheme.parse_scheme(args.output) is not None and \
            (args.qtype is None or args.qtype.isdigit()):
        args.nthreads, args.qtype, args.output = args.qtype, args.output, None
    if args.qtype is None:
        ap.error("missing quantization type")
    if args.nthreads is not None:
        sys.exit("error: the nthreads argument is not supported by quant-studio (GPU pipeline)")

    opt = scheme.parse_scheme(args.qtype)
    if opt is None:
        sys.exit(f"error: unknown quantization scheme {args.qtype!r}\n\n" + scheme.format_scheme_table())
    if not opt.supported:
        sys.exit(f"error: scheme {opt.name} is not supported by quant-studio\n\n"
                 + scheme.format_scheme_table())
    out_path = Path(args.output) if args.output else args.input.parent / f"ggml-model-{opt.name}.gguf"

    entries = list(args.tensor_type)
    if args.tensor_type_file is not None:
        entries += args.tensor_type_file.read_text().split()
    overrides = []
    for ent in entries:
        pat, _, tname = ent.partition("=")
        if not tname:
            sys.exit(f"error: invalid --tensor-type {ent!r}, expected name=ggml_type")
        overrides.append((pat, parse_ggml_type(tname)))
    tet = parse_ggml_type(args.token_embedding_type) if args.token_embedding_type else None
    ott = parse_ggml_type(args.output_tensor_type) if args.output_tensor_type else None
    mem_bytes = parse_mem(args.mem)
    if args.device not in ("auto", "cuda", "hip") and not args.device.startswith(("cuda:", "hip:")):
        sys.exit(f"error: device {args.device!r}: this build quantizes on ROCm devices only")
    print(f"quant-studio: {args.input} -> {out_path} [{opt.name}] device=rocm mem={args.mem}")

    imatrix: dict[str, np.ndarray] = {}
    if args.imatrix is not None:
        imatrix = load_imatrix(args.imatrix)
        print(f"imatrix: {len(imatrix)} entries from {args.imatrix}")

    reader = GGUFReader(args.input)
    kv = reader.values()
    if "general.architecture" not in kv:
        sys.exit("error: input has no general.architecture key")
    arch = kv["general.architecture"]

    from . import QUANT_TYPES
    tensors = sorted(reader.tensors, key=lambda t: scheme.weight_name_key(t.name))
    model = scheme.ModelInfo.from_kv(kv)
    st = scheme.init_state(model, [t.name for t in tensors], bool(imatrix), overrides)
    spec_by_type = {s.ggml_type: s for s in QUANT_TYPES.values()}

    plans = []
    missing: dict[str, list[str]] = {}
    need_imat: list[str] = []
    for t in tensors:
        src = t.ggml_type
        dst = src
        if src in _SOURCE_TYPES:
            try:
                dst = scheme.tensor_get_type(
                    st, model, t.name, t.ne, src, opt.ftype, pure=args.pure,
                    quantize_output_tensor=not args.leave_output_tensor,
                    token_embedding_type=tet, output_tensor_type=ott)
            except ValueError as e:
                print(f"warning: {t.name}: {e}; keeping {src.name}", file=sys.stderr)
        if dst == src:
            plans.append((t, None, None))
            continue
        spec = spec_by_type.get(dst)
        if spec is None:
            missing.setdefault(dst.name, []).append(t.name)
            plans.append((t, None, None))
            continue
        if (scheme.tensor_requires_imatrix(t.name, dst, opt.ftype) or spec.needs_imatrix) \
                and t.name not in imatrix:
            need_imat.append(t.name)
        plans.append((t, dst, spec))

    if missing:
        detail = "; ".join(f"{ty} for {len(names)} tensors (e.g. {names[0]})"
                           for ty, names in sorted(missing.items()))
        sys.exit(f"error: this scheme needs kernel types quant-studio does not have yet: {detail}")
    if need_imat:
        uniq = sorted(set(need_imat))
        hint = "" if args.imatrix else " (pass --imatrix)"
        if "token_embd.weight" in uniq:
            hint += " (token_embd can be overridden with --token-embedding-type)"
        sys.exit(f"error: {len(uniq)} tensors require importance matrix data{hint}: "
                 + ", ".join(uniq[:4]) + ("..." if len(uniq) > 4 else ""))

    def out_nbytes(t, dst):
        return t.nbytes if dst is None else t.n_elements // t.ne[0] * tensor_nbytes(dst, (t.ne[0],))

    if args.dry_run:
        total_in = total_out = 0
        for t, dst, _ in plans:
            nb = out_nbytes(t, dst)
            total_in += t.nbytes
            total_out += nb
            print(f"{t.name:48s} {t.ggml_type.name:>8s} -> "
                  f"{dst.name if dst else t.ggml_type.name:<8s} {fmt_size(nb)}")
        print(f"dry run: {fmt_size(total_in)} -> {fmt_size(total_out)} tensor data "
              f"({total_out / max(total_in, 1) * 100:.1f}%)")
        return 0

    from . import row_bytes
    from .pipeline import NativePipeline, PipelineError, device_count
    ndev = device_count()
    if ndev == 0:
        sys.exit("error: no ROCm device available (this build has no CPU quantization path)")
    dev_index = 0 if args.device in ("auto", "cuda", "hip") else int(args.device.split(":")[1])
    if dev_index >= ndev:
        sys.exit(f"error: device {args.device!r} not present ({ndev} ROCm devices)")

    # imatrix rows are checked before anything is written
    for t, dst, spec in plans:
        if dst is not None and spec.uses_imatrix and t.name in imatrix and imatrix[t.name].size < t.ne[0]:
            sys.exit(f"error: imatrix data for {t.name} has {imatrix[t.name].size} values, "
                     f"rows have {t.ne[0]}")

    writer = GGUFWriter(out_path, arch)
    for k in copied_kvs(reader, opt.ftype):
        writer.add_kv(k)
    for t, dst, _ in plans:
        writer.add_tensor_info(t.name, t.ne, dst if dst is not None else t.ggml_type, out_nbytes(t, dst))
    writer.write_header()
    data_start = writer.data_start()
    writer.fout.flush()
    fd = writer.fout.fileno()

    total_in = total_out = 0
    t0 = time.time()
    try:
        with NativePipeline(dev_index, fd) as pipe:
            for i, ((t, dst, spec), info) in enumerate(zip(plans, writer.infos)):
                off = data_start + info[3]
                if dst is not None:
                    qw = imatrix.get(t.name) if spec.uses_imatrix else None
                    rows_per_chunk = max(1, mem_bytes // (t.ne[0] * spec.bytes_per_elem))
                    nbytes = pipe.quantize_tensor(t, int(dst), qw, rows_per_chunk, off,
                                                  row_bytes(int(dst), t.ne[0]))
                else:
                    nbytes = pipe.write(t.data, off)
                total_in += t.nbytes
                total_out += nbytes
                shape = "x".join(str(d) for d in t.ne)
                src = t.ggml_type.name
                print(f"[{i + 1:4d}/{len(plans)}] {t.name:48s} {shape:>16s}  {src:>5s} -> "
                      f"{dst.name if dst else src:<8s} {fmt_size(t.nbytes)} -> {fmt_size(nbytes)}")
            pipe.finish()
    except PipelineError as e:
        writer.close()
        sys.exit(f"error: {e}")
    # the padding after each tensor and at the end is zeros: set the final size
    os.ftruncate(fd, writer.total_size())
    writer.close()
    dt = time.time() - t0
    print(f"done in {dt:.1f}s: {fmt_size(total_in)} -> {fmt_size(total_out)} "
          f"({total_out / max(total_in, 1) * 100:.1f}%)")
    return 0
