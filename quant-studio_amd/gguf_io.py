"""GGUF v3 container I/O: an mmap reader, a streaming writer, the imatrix loader.

Written from the public GGUF format (little-endian): header (magic, version,
tensor count, KV count), key/values, tensor infos (name, dims, ggml type, data
offset), padding to `general.alignment` (32 by default), aligned tensor data.
It replaces the reference's use of gguf-py's GGUFReader / GGUFWriter
(quant-studio.py:249-264, :355-359, :421-441, :470-472) and its imatrix
loader (quant-studio.py:68-87), with the same output layout: the writer emits
general.architecture first, then the KVs in the order given, tensor infos
with offsets that are running sums of alignment-padded sizes, padding after
the infos and after every tensor's data.
"""

from __future__ import annotations

import mmap
import struct
from dataclasses import dataclass
from enum import IntEnum
from pathlib import Path
from typing import Any, BinaryIO

import numpy as np

from .gguf_types import GGMLQuantizationType as GT
from .gguf_types import QUANT_SIZES

GGUF_MAGIC = 0x46554747          # "GGUF" little-endian
GGUF_VERSION = 3
DEFAULT_ALIGNMENT = 32


class VT(IntEnum):
    """GGUF metadata value types."""
    UINT8 = 0
    INT8 = 1
    UINT16 = 2
    INT16 = 3
    UINT32 = 4
    INT32 = 5
    FLOAT32 = 6
    BOOL = 7
    STRING = 8
    ARRAY = 9
    UINT64 = 10
    INT64 = 11
    FLOAT64 = 12


_SCALAR = {VT.UINT8: "<B", VT.INT8: "<b", VT.UINT16: "<H", VT.INT16: "<h", VT.UINT32: "<I",
           VT.INT32: "<i", VT.FLOAT32: "<f", VT.BOOL: "<?", VT.UINT64: "<Q", VT.INT64: "<q",
           VT.FLOAT64: "<d"}
_NP = {GT.F32: np.float32, GT.F16: np.float16, GT.F64: np.float64, GT.I8: np.int8,
       GT.I16: np.int16, GT.I32: np.int32, GT.I64: np.int64}


def pad_to(n: int, align: int) -> int:
    return (n + align - 1) // align * align


def tensor_nbytes(ggml_type: int, ne: tuple[int, ...]) -> int:
    blk, size = QUANT_SIZES[GT(ggml_type)]
    n = int(np.prod(ne, dtype=np.int64)) if ne else 1
    if ne and ne[0] % blk:
        raise ValueError(f"row length {ne[0]} is not a multiple of the {GT(ggml_type).name} block {blk}")
    return n // blk * size


@dataclass
class KV:
    name: str
    vtype: VT
    value: Any
    sub_type: VT | None = None     # item type of an ARRAY


@dataclass
class TensorInfo:
    name: str
    ne: tuple[int, ...]            # ggml order: ne[0] is the row length
    ggml_type: GT
    offset: int                    # relative to the data section
    nbytes: int
    data: np.ndarray | None = None  # uint8 view into the mapped file
    file_offset: int = -1          # absolute offset of the data in the file (-1: not from a file)

    @property
    def n_elements(self) -> int:
        return int(np.prod(self.ne, dtype=np.int64))

    def rows(self) -> np.ndarray:
        """(n_rows, row_bytes) uint8 view, higher dims folded into rows."""
        row_bytes = tensor_nbytes(self.ggml_type, (self.ne[0],))
        return self.data.reshape(-1, row_bytes)

    def array(self) -> np.ndarray:
        """Typed view for unquantized tensors, numpy order (reversed ne)."""
        if self.ggml_type == GT.BF16:
            return self.data.view(np.uint16).reshape(tuple(reversed(self.ne)))
        return self.data.view(_NP[self.ggml_type]).reshape(tuple(reversed(self.ne)))


class GGUFReader:
    """Parses a GGUF file and maps its tensor data read-only."""

    def __init__(self, path: str | Path):
        self.path = Path(path)
        self._f = open(self.path, "rb")
        self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        buf = memoryview(self._mm)
        self._pos = 0
        magic, version = struct.unpack_from("<II", buf, 0)
        if magic != GGUF_MAGIC:
            raise ValueError(f"{path}: not a GGUF file (magic {magic:#x})")
        if version not in (2, 3):
            raise ValueError(f"{path}: unsupported GGUF version {version}")
        self.version = version
        n_tensors, n_kv = struct.unpack_from("<QQ", buf, 8)
        self._pos = 24
        self.kv: dict[str, KV] = {}
        for _ in range(n_kv):
            name = self._str(buf)
            vtype = VT(self._u32(buf))
            if vtype == VT.ARRAY:
                sub = VT(self._u32(buf))
                count = self._u64(buf)
                if sub == VT.ARRAY:
                    raise ValueError(f"{path}: nested arrays ({name}) are not supported")
                val = [self._value(buf, sub) for _ in range(count)]
                self.kv[name] = KV(name, vtype, val, sub)
            else:
                self.kv[name] = KV(name, vtype, self._value(buf, vtype))
        infos = []
        for _ in range(n_tensors):
            name = self._str(buf)
            nd = self._u32(buf)
            ne = tuple(self._u64(buf) for _ in range(nd))
            gtype = GT(self._u32(buf))
            off = self._u64(buf)
            infos.append((name, ne, gtype, off))
        align = DEFAULT_ALIGNMENT
        if "general.alignment" in self.kv:
            align = int(self.kv["general.alignment"].value)
        self.alignment = align
        self.data_offset = pad_to(self._pos, align)
        self.tensors: list[TensorInfo] = []
        base = np.frombuffer(self._mm, dtype=np.uint8)
        for name, ne, gtype, off in infos:
            nbytes = tensor_nbytes(gtype, ne)
            start = self.data_offset + off
            if start + nbytes > len(self._mm):
                raise ValueError(f"{path}: tensor {name} extends past the end of the file")
            self.tensors.append(TensorInfo(name, ne, gtype, off, nbytes, base[start:start + nbytes], start))

    def _u32(self, buf) -> int:
        v = struct.unpack_from("<I", buf, self._pos)[0]
        self._pos += 4
        return v

    def _u64(self, buf) -> int:
        v = struct.unpack_from("<Q", buf, self._pos)[0]
        self._pos += 8
        return v

    def _str(self, buf) -> str:
        n = self._u64(buf)
        s = bytes(buf[self._pos:self._pos + n]).decode("utf-8")
        self._pos += n
        return s

    def _value(self, buf, vtype: VT):
        if vtype == VT.STRING:
            return self._str(buf)
        fmt = _SCALAR[vtype]
        v = struct.unpack_from(fmt, buf, self._pos)[0]
        self._pos += struct.calcsize(fmt)
        return v

    def fileno(self) -> int:
        """Descriptor of the input file (the pipeline reads tensor rows with pread)."""
        return self._f.fileno()

    def get(self, name: str, default=None):
        kv = self.kv.get(name)
        return default if kv is None else kv.value

    def values(self) -> dict[str, Any]:
        return {k: v.value for k, v in self.kv.items()}

    def close(self) -> None:
        self.tensors = []
        try:
            self._mm.close()
        except BufferError:      # numpy views still alive; the map closes with them
            pass
        self._f.close()


def _pack_str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _pack_value(vtype: VT, v) -> bytes:
    if vtype == VT.STRING:
        return _pack_str(v)
    return struct.pack(_SCALAR[vtype], v)


def pack_kv(kv: KV) -> bytes:
    out = _pack_str(kv.name) + struct.pack("<I", int(kv.vtype))
    if kv.vtype == VT.ARRAY:
        out += struct.pack("<IQ", int(kv.sub_type), len(kv.value))
        out += b"".join(_pack_value(kv.sub_type, v) for v in kv.value)
    else:
        out += _pack_value(kv.vtype, kv.value)
    return out


class GGUFWriter:
    """Streams a GGUF file: header, KVs and tensor infos first, then the caller
    appends each tensor's data in info order, padding to the alignment."""

    def __init__(self, path: str | Path, arch: str, alignment: int = DEFAULT_ALIGNMENT):
        self.path = Path(path)
        self.alignment = alignment
        self.kvs: list[KV] = [KV("general.architecture", VT.STRING, arch)]
        self.infos: list[tuple[str, tuple[int, ...], GT, int]] = []
        self._offset = 0
        self.fout: BinaryIO | None = None

    def add_kv(self, kv: KV) -> None:
        self.kvs.append(kv)

    def add_tensor_info(self, name: str, ne: tuple[int, ...], ggml_type: GT, nbytes: int) -> None:
        self.infos.append((name, tuple(int(d) for d in ne), GT(ggml_type), self._offset))
        self._offset += pad_to(nbytes, self.alignment)

    def write_header(self) -> BinaryIO:
        self.fout = open(self.path, "wb")
        hdr = struct.pack("<IIQQ", GGUF_MAGIC, GGUF_VERSION, len(self.infos), len(self.kvs))
        hdr += b"".join(pack_kv(kv) for kv in self.kvs)
        for name, ne, gtype, off in self.infos:
            hdr += _pack_str(name) + struct.pack("<I", len(ne))
            hdr += b"".join(struct.pack("<Q", d) for d in ne)
            hdr += struct.pack("<IQ", int(gtype), off)
        self.fout.write(hdr)
        self.data_start_offset = pad_to(len(hdr), self.alignment)
        return self.fout

    def data_start(self) -> int:
        """File offset of the tensor data section (after write_header)."""
        return self.data_start_offset

    def total_size(self) -> int:
        """Size of the complete file: data section start + padded tensor data."""
        return self.data_start_offset + self._offset

    def pad(self) -> None:
        pos = self.fout.tell()
        n = pad_to(pos, self.alignment) - pos
        if n:
            self.fout.write(bytes(n))

    def close(self) -> None:
        if self.fout is not None:
            self.fout.close()
            self.fout = None


def write_gguf(path: str | Path, arch: str, kvs: list[KV],
               tensors: list[tuple[str, tuple[int, ...], GT, np.ndarray]]) -> None:
    """Write a complete GGUF file (used to build inputs and imatrix files)."""
    w = GGUFWriter(path, arch)
    for kv in kvs:
        w.add_kv(kv)
    for name, ne, gtype, data in tensors:
        w.add_tensor_info(name, ne, gtype, data.nbytes)
    w.write_header()
    for _name, _ne, _t, data in tensors:
        w.pad()
        w.fout.write(np.ascontiguousarray(data).view(np.uint8).tobytes())
    w.pad()
    w.close()


def load_imatrix(path: str | Path) -> dict[str, np.ndarray]:
    """Per-tensor imatrix weights from a GGUF imatrix file (the format of
    load_imatrix, quant-studio.py:68-87): for each tensor name with both a
    `<name>.in_sum2` and a `<name>.counts` record, the mean squared input
    activation per column, in_sum2 / counts in float32 -- one row of values per
    count (per expert for 3-D tensors), 0 where that count is not positive --
    flattened in row order."""
    records: dict[str, dict[str, np.ndarray]] = {}
    reader = GGUFReader(path)
    try:
        for t in reader.tensors:
            base, _, field = t.name.rpartition(".")
            if base and field in ("in_sum2", "counts"):
                records.setdefault(base, {})[field] = np.array(t.data.view(np.float32), copy=True)
    finally:
        reader.close()
    weights = {}
    for base, rec in records.items():
        if "in_sum2" not in rec or "counts" not in rec:
            continue
        counts = rec["counts"].reshape(-1, 1)
        per_count = rec["in_sum2"].reshape(counts.shape[0], -1)
        live = counts > 0
        mean = per_count / np.where(live, counts, np.float32(1))
        weights[base] = np.where(live, mean, np.float32(0)).astype(np.float32).reshape(-1)
    return weights
