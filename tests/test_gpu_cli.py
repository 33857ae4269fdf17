"""GPU end-to-end: the command line quantizes synthetic GGUF files on the
MI355X; every quantized tensor must equal the CPU oracle byte for byte, and
the file must keep the reference's container contract (tests/test_q4_0.py:
73-125): KVs preserved, file_type / quantization_version set, loader order,
shapes, untouched passthroughs, output independent of --mem chunking."""

from __future__ import annotations

import importlib
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle
from cli_models import GT, fallback_model, imatrix_for, io, small_model

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
IGNORE_IMATRIX = {"q4_0", "q4_1", "q5_0", "q5_1", "q8_0"}    # 32-value integer formats
sch = importlib.import_module("quant-studio_amd.scheme")


def run_cli(*args):
    print("cli:", *args, flush=True)
    r = subprocess.run([sys.executable, str(ROOT / "quant-studio.py"), *map(str, args)],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr + r.stdout
    return r


def check_output(src: Path, dst: Path, expect: dict, ftype: int, imatrix: dict | None = None):
    r_in, r_out = io.GGUFReader(src), io.GGUFReader(dst)
    kin, kout = r_in.values(), r_out.values()
    for k, v in kin.items():
        if k not in ("general.file_type",):
            assert kout[k] == v, k
    assert kout["general.file_type"] == ftype
    assert kout["general.quantization_version"] == 2
    assert [t.name for t in r_out.tensors] == sorted((t.name for t in r_in.tensors), key=sch.weight_name_key)
    tin = {t.name: t for t in r_in.tensors}
    for t in r_out.tensors:
        s = tin[t.name]
        assert t.ne == s.ne, t.name
        if t.ggml_type == s.ggml_type:
            assert np.array_equal(t.data, s.data), f"{t.name}: passthrough bytes changed"
            continue
        name = {v: k for k, v in oracle.TYPE_IDS.items()}[int(t.ggml_type)]
        x = expect[t.name].reshape(-1, t.ne[0])
        qw = None
        if imatrix is not None and t.name in imatrix and name not in IGNORE_IMATRIX:
            qw = imatrix[t.name][:t.ne[0]].astype(np.float32)
        ref = oracle.quantize(name, x, qw)
        assert np.array_equal(t.rows(), ref), f"{t.name} ({name}) differs from the oracle"
    r_in.close()
    r_out.close()


def test_q4_0_small_model_multi_chunk(tmp_path):
    src = tmp_path / "in.gguf"
    expect = small_model(src)
    a, b = tmp_path / "a.gguf", tmp_path / "b.gguf"
    run_cli(src, a, "q4_0", "--mem", "64K")
    run_cli(src, b, "q4_0")
    assert a.read_bytes() == b.read_bytes()
    check_output(src, a, expect, ftype=2)


@pytest.mark.parametrize("scheme,ftype,extra", [
    ("Q4_K_M", 15, []), ("Q6_K", 18, []), ("IQ4_XS", 30, []), ("Q2_K", 10, []),
    ("IQ2_XXS", 19, ["--token-embedding-type", "q4_0"]),
    ("IQ3_XXS", 23, []), ("IQ2_S", 28, []), ("IQ3_S", 26, []), ("Q3_K_L", 13, []),
    ("Q4_1", 3, []), ("Q5_0", 8, []), ("Q5_1", 9, []), ("Q8_0", 7, []), ("IQ4_NL", 25, []),
])
def test_schemes_with_imatrix(tmp_path, scheme, ftype, extra):
    src = tmp_path / "in.gguf"
    expect = small_model(src, odd=False)
    im = tmp_path / "im.gguf"
    ks = {n: v.shape[-1] for n, v in expect.items()}
    imatrix_for(im, ks, n_mat={"blk.0.ffn_gate_exps.weight": 4})
    imat = io.load_imatrix(im)
    out = tmp_path / "o.gguf"
    run_cli(src, out, scheme, "--imatrix", im, "--mem", "128K", *extra)
    check_output(src, out, expect, ftype=ftype, imatrix=imat)


@pytest.mark.parametrize("scheme,ftype", [("IQ2_XXS", 19), ("Q4_K_M", 15), ("IQ3_S", 26), ("Q2_K", 10)])
def test_imatrix_with_zero_columns_and_an_unrouted_expert(tmp_path, scheme, ftype):
    """An imatrix whose columns partly never fired (in_sum2 = 0; every other
    16-column group and ~30% more) and whose 3-D expert tensor has a zero
    count for expert 0, the only expert the reference reads (quant-studio.py:
    80-85, :455): that tensor's weights are all zero. Every quantized tensor
    equals the oracle fed the same loaded weights."""
    src = tmp_path / "in.gguf"
    expect = small_model(src, odd=False)
    im = tmp_path / "im.gguf"
    imatrix_for(im, {n: v.shape[-1] for n, v in expect.items()},
                n_mat={"blk.0.ffn_gate_exps.weight": 4}, zero_frac=0.3,
                dead_counts={"blk.0.ffn_gate_exps.weight": [0]})
    imat = io.load_imatrix(im)
    assert not imat["blk.0.ffn_gate_exps.weight"][:256].any()
    assert (imat["blk.0.ffn_gate_exps.weight"][256:] > 0).any()
    assert (imat["blk.0.attn_k.weight"] == 0).mean() > 0.5
    out = tmp_path / "o.gguf"
    run_cli(src, out, scheme, "--imatrix", im, "--mem", "128K")
    check_output(src, out, expect, ftype=ftype, imatrix=imat)


def test_device_cpu_writes_the_same_file(tmp_path):
    """--device cpu (the reference's CPU path) and the default device give the
    same file, byte for byte."""
    src = tmp_path / "in.gguf"
    expect = small_model(src, odd=False)
    im = tmp_path / "im.gguf"
    imatrix_for(im, {n: v.shape[-1] for n, v in expect.items()},
                n_mat={"blk.0.ffn_gate_exps.weight": 4})
    a, b = tmp_path / "a.gguf", tmp_path / "b.gguf"
    run_cli(src, a, "Q4_K_M", "--imatrix", im)
    r = run_cli(src, b, "Q4_K_M", "--imatrix", im, "--device", "cpu")
    assert "device=cpu (on rocm)" in r.stdout
    assert a.read_bytes() == b.read_bytes()


@pytest.mark.parametrize("mode", ["torch-cpu-amd", "ieee"])
def test_sqrt_rounding_option(tmp_path, mode):
    """--sqrt-rounding reaches the kernels: every quantized tensor equals the
    oracle in the same square-root mode."""
    import sqrt_hosts
    src = tmp_path / "in.gguf"
    expect = small_model(src, odd=False)
    im = tmp_path / "im.gguf"
    imatrix_for(im, {n: v.shape[-1] for n, v in expect.items()},
                n_mat={"blk.0.ffn_gate_exps.weight": 4})
    out = tmp_path / "o.gguf"
    run_cli(src, out, "IQ4_XS", "--imatrix", im, "--sqrt-rounding", mode)
    if mode == "ieee":
        oracle.use_ieee_sqrt(True)
    else:
        oracle.use_amd_host_sqrt(sqrt_hosts.amd_ulps())
    try:
        check_output(src, out, expect, ftype=30, imatrix=io.load_imatrix(im))
    finally:
        oracle.use_ieee_sqrt(False)
        oracle.use_sqrt_table(None)


def test_pipeline_chunks_match_single_call_and_report_write_errors(tmp_path):
    """The native pipeline directly: any chunking writes the same bytes as one
    qs_quantize call (checked against the oracle), and a failing write (here a
    read-only descriptor) surfaces as an error no later than finish()."""
    import os
    qs = importlib.import_module("quant-studio_amd")
    pl = importlib.import_module("quant-studio_amd.pipeline")
    rng = np.random.default_rng(7)
    x = (rng.normal(size=(37, 512)) * 0.02).astype(np.float32)
    qw = rng.lognormal(size=512).astype(np.float32)
    ref = oracle.quantize("q4_k", x, qw)
    info = io.TensorInfo("t", (512, 37), GT.F32, 0, x.nbytes, x.view(np.uint8).reshape(-1))
    for rows_per_chunk in (1, 5, 37, 100):
        path = tmp_path / f"o{rows_per_chunk}.bin"
        fd = os.open(path, os.O_RDWR | os.O_CREAT | os.O_TRUNC, 0o644)
        try:
            with pl.NativePipeline(0, fd) as p:
                p.write(np.frombuffer(b"HEAD", np.uint8), 0)
                p.quantize_tensor(info, int(GT.Q4_K), qw, rows_per_chunk, 64, qs.row_bytes(int(GT.Q4_K), 512))
                p.finish()
        finally:
            os.close(fd)
        b = path.read_bytes()
        assert b[:4] == b"HEAD" and b[4:64] == bytes(60)
        assert np.array_equal(np.frombuffer(b[64:], np.uint8).reshape(ref.shape), ref), rows_per_chunk
    ro = tmp_path / "ro.bin"
    ro.write_bytes(b"")
    fd = os.open(ro, os.O_RDONLY)
    try:
        with pl.NativePipeline(0, fd) as p:
            # reported by a later queue call once the writer has failed, else by finish()
            with pytest.raises(pl.PipelineError, match="write failed"):
                p.quantize_tensor(info, int(GT.Q4_K), qw, 8, 0, qs.row_bytes(int(GT.Q4_K), 512))
                p.finish()
    finally:
        os.close(fd)


def test_pipeline_reads_rows_from_the_file(tmp_path):
    """qs_pipeline_quantize_fd (rows read with pread at a file offset) writes
    the oracle's bytes for any chunking, bf16 and f32 rows at unaligned file
    offsets alike; a tensor that runs past the end of the file fails with
    QS_EIO naming the read (no later than qs_pipeline_finish), and an invalid
    descriptor or offset is refused."""
    import ctypes
    import os
    qs = importlib.import_module("quant-studio_amd")
    pl = importlib.import_module("quant-studio_amd.pipeline")
    rng = np.random.default_rng(9)
    x = (rng.normal(size=(29, 512)) * 0.02).astype(np.float32)
    qw = rng.lognormal(size=512).astype(np.float32)
    xb = (x.view(np.uint32) >> 16).astype(np.uint16)          # bf16 by truncation
    xbf = (xb.astype(np.uint32) << 16).view(np.float32)
    src = tmp_path / "rows.bin"
    lead = 37                                                    # an odd file offset
    src.write_bytes(bytes(lead) + x.tobytes() + xb.tobytes())
    cases = [(GT.F32, x, x, lead), (GT.BF16, xb, xbf, lead + x.nbytes)]
    sfd = os.open(src, os.O_RDONLY)
    try:
        for gt, raw, xf, off in cases:
            ref = oracle.quantize("q4_k", xf, qw)
            info = io.TensorInfo("t", (512, 29), gt, 0, raw.nbytes, raw.view(np.uint8).reshape(-1), off)
            for rows_per_chunk in (1, 6, 29):
                path = tmp_path / f"o{int(gt)}_{rows_per_chunk}.bin"
                fd = os.open(path, os.O_RDWR | os.O_CREAT | os.O_TRUNC, 0o644)
                try:
                    with pl.NativePipeline(0, fd) as p:
                        p.quantize_tensor(info, int(GT.Q4_K), qw, rows_per_chunk, 0,
                                          qs.row_bytes(int(GT.Q4_K), 512), sfd)
                        p.finish()
                finally:
                    os.close(fd)
                got = np.frombuffer(path.read_bytes(), np.uint8).reshape(ref.shape)
                assert np.array_equal(got, ref), (gt.name, rows_per_chunk)
        fd = os.open(tmp_path / "short.bin", os.O_RDWR | os.O_CREAT | os.O_TRUNC, 0o644)
        try:
            with pl.NativePipeline(0, fd) as p:
                # 4 more rows than the file holds after the bf16 block: the
                # read fails on the pool, reported by the call or by finish
                rc = p.L.qs_pipeline_quantize_fd(p.h, int(GT.Q4_K), 30, sfd, lead + x.nbytes, 33, 512,
                                                 None, 64, fd, 0)
                if rc == 0:
                    rc = p.L.qs_pipeline_finish(p.h)
                assert rc == -5 and "reading the input rows failed" in qs.last_error()
                assert p.L.qs_pipeline_quantize_fd(p.h, int(GT.Q4_K), 30, -1, 0, 1, 512, None, 1,
                                                   fd, 0) == -22
                assert p.L.qs_pipeline_quantize_fd(p.h, int(GT.Q4_K), 30, sfd, -1, 1, 512, None, 1,
                                                   fd, 0) == -22
        finally:
            os.close(fd)
    finally:
        os.close(sfd)


def test_pipeline_tensors_back_to_back(tmp_path):
    """Tensors of other widths, types and sources queued back to back: each
    queue call leaves its last chunk pending (its rows still being read) and
    the next call launches it, input slots are reused by rows of other widths
    and imatrices of other lengths, rows come from the file (bf16, pread) and
    from host memory (f32) in turn; every tensor's bytes are the oracle's."""
    import os
    qs = importlib.import_module("quant-studio_amd")
    pl = importlib.import_module("quant-studio_amd.pipeline")
    rng = np.random.default_rng(11)
    # (type, k, rows, rows per chunk)
    specs = [(GT.Q4_K, 512, 23, 5), (GT.IQ4_XS, 1024, 9, 4), (GT.Q6_K, 256, 40, 40), (GT.Q4_0, 2048, 7, 3),
             (GT.Q3_K, 768, 13, 1), (GT.Q4_K, 256, 64, 17), (GT.IQ3_XXS, 4096, 3, 2)]
    src = tmp_path / "rows.bin"
    blob, tensors, want = bytearray(b"\0" * 11), [], []
    for i, (gt, k, n, rpc) in enumerate(specs):
        x = (rng.normal(size=(n, k)) * 0.02).astype(np.float32)
        qw = rng.lognormal(size=k).astype(np.float32)
        if i % 2 == 0:      # bf16 rows in the file at an odd offset
            raw = (x.view(np.uint32) >> 16).astype(np.uint16)
            xf = (raw.astype(np.uint32) << 16).view(np.float32)
            info = io.TensorInfo(f"t{i}", (k, n), GT.BF16, 0, raw.nbytes, raw.view(np.uint8).reshape(-1), len(blob))
            blob += raw.tobytes()
        else:               # f32 rows from host memory
            xf = x
            info = io.TensorInfo(f"t{i}", (k, n), GT.F32, 0, x.nbytes, x.view(np.uint8).reshape(-1))
        name = gt.name.lower()
        want.append(oracle.quantize(name, xf, None if gt == GT.Q4_0 else qw))
        tensors.append((info, gt, qw, rpc))
    src.write_bytes(bytes(blob))
    out = tmp_path / "o.bin"
    sfd = os.open(src, os.O_RDONLY)
    fd = os.open(out, os.O_RDWR | os.O_CREAT | os.O_TRUNC, 0o644)
    try:
        with pl.NativePipeline(0, fd) as p:
            off = 0
            for info, gt, qw, rpc in tensors:
                print(f"queue {gt.name} {info.ne} rows/chunk {rpc}", flush=True)
                off += p.quantize_tensor(info, int(gt), qw, rpc, off, qs.row_bytes(int(gt), info.ne[0]),
                                         sfd if info.ggml_type == GT.BF16 else -1)
            p.finish()
    finally:
        os.close(fd)
        os.close(sfd)
    got, off = out.read_bytes(), 0
    for (info, gt, _, _), ref in zip(tensors, want):
        part = np.frombuffer(got[off:off + ref.nbytes], np.uint8).reshape(ref.shape)
        assert np.array_equal(part, ref), (gt.name, info.ne)
        off += ref.nbytes
    assert off == len(got)


def test_two_pipelines_on_two_threads(tmp_path):
    """Two pipelines driven at once from two threads (each its own input
    file, output file, copy threads, writer and streams; calls on one
    pipeline never overlap): both outputs are the oracle's bytes."""
    import os
    import threading
    qs = importlib.import_module("quant-studio_amd")
    pl = importlib.import_module("quant-studio_amd.pipeline")
    rng = np.random.default_rng(12)
    jobs = []
    for name, gts in (("a", [GT.Q4_K, GT.IQ2_XS, GT.Q6_K]), ("b", [GT.IQ3_S, GT.Q4_0, GT.IQ2_XXS])):
        k, n = 1024, 40
        src = tmp_path / f"{name}.bin"
        xs = [(rng.normal(size=(n, k)) * 0.02).astype(np.float32) for _ in gts]
        raws = [(x.view(np.uint32) >> 16).astype(np.uint16) for x in xs]
        src.write_bytes(b"".join(r.tobytes() for r in raws))
        qw = rng.lognormal(size=k).astype(np.float32)
        want = [oracle.quantize(gt.name.lower(), (r.astype(np.uint32) << 16).view(np.float32),
                                None if gt == GT.Q4_0 else qw) for gt, r in zip(gts, raws)]
        jobs.append((name, gts, raws, qw, want, src, tmp_path / f"{name}.out"))
    errors = []

    def run(name, gts, raws, qw, want, src, out):
        try:
            sfd = os.open(src, os.O_RDONLY)
            fd = os.open(out, os.O_RDWR | os.O_CREAT | os.O_TRUNC, 0o644)
            try:
                with pl.NativePipeline(0, fd) as p:
                    off = foff = 0
                    for gt, raw in zip(gts, raws):
                        info = io.TensorInfo(name, (raw.shape[1], raw.shape[0]), GT.BF16, 0, raw.nbytes,
                                             raw.view(np.uint8).reshape(-1), foff)
                        off += p.quantize_tensor(info, int(gt), qw, 7, off, qs.row_bytes(int(gt), raw.shape[1]),
                                                 sfd)
                        foff += raw.nbytes
                    p.finish()
            finally:
                os.close(fd)
                os.close(sfd)
        except Exception as e:          # reported on the main thread
            errors.append(f"{name}: {e}")

    threads = [threading.Thread(target=run, args=j) for j in jobs]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a pipeline thread did not finish"
    assert not errors, errors
    for name, gts, raws, qw, want, src, out in jobs:
        got, off = out.read_bytes(), 0
        for gt, ref in zip(gts, want):
            part = np.frombuffer(got[off:off + ref.nbytes], np.uint8).reshape(ref.shape)
            assert np.array_equal(part, ref), (name, gt.name)
            off += ref.nbytes
        assert off == len(got)


def test_pipeline_made_on_another_thread(tmp_path):
    """PipelineStart: a pipeline created on its own thread works when taken on
    this one (the oracle's bytes), can be taken only once, and one that is
    never taken is released by close()."""
    import os
    qs = importlib.import_module("quant-studio_amd")
    pl = importlib.import_module("quant-studio_amd.pipeline")
    rng = np.random.default_rng(10)
    x = (rng.normal(size=(9, 512)) * 0.02).astype(np.float32)
    info = io.TensorInfo("t", (512, 9), GT.F32, 0, x.nbytes, x.view(np.uint8).reshape(-1))
    ref = oracle.quantize("q6_k", x, None)
    path = tmp_path / "o.bin"
    fd = os.open(path, os.O_RDWR | os.O_CREAT | os.O_TRUNC, 0o644)
    try:
        start = pl.PipelineStart(0)
        p = start.take(fd)
        assert p is not None and start.take(fd) is None
        with p:
            p.quantize_tensor(info, int(GT.Q6_K), None, 4, 0, qs.row_bytes(int(GT.Q6_K), 512))
            p.finish()
        start.close()
    finally:
        os.close(fd)
    assert np.array_equal(np.frombuffer(path.read_bytes(), np.uint8).reshape(ref.shape), ref)
    unused = pl.PipelineStart(0)
    unused.close()
    unused.close()


@pytest.mark.parametrize("scheme,ftype", [("Q4_K_M", 15), ("Q5_K_S", 16), ("IQ4_XS", 30)])
def test_shape_fallback_types_end_to_end(tmp_path, scheme, ftype):
    """288-value rows fall back to Q5_0 / Q5_1 / Q8_0 / IQ4_NL (scheme.py:364-384)."""
    src = tmp_path / "in.gguf"
    expect = fallback_model(src)
    im = tmp_path / "im.gguf"
    imatrix_for(im, {n: 288 for n in expect})
    out = tmp_path / "o.gguf"
    run_cli(src, out, scheme, "--imatrix", im)
    types = {int(t.ggml_type) for t in io.GGUFReader(out).tensors}
    assert types & {int(GT.Q5_0), int(GT.Q5_1), int(GT.Q8_0), int(GT.IQ4_NL)}
    check_output(src, out, expect, ftype=ftype, imatrix=io.load_imatrix(im))


def test_pipeline_refuses_sizes_that_would_wrap(tmp_path):
    """A tensor of more than 2^34 values is refused before any chunk size is
    formed from n_rows * k (those products could wrap int64)."""
    import ctypes
    import os
    qs = importlib.import_module("quant-studio_amd")
    pl = importlib.import_module("quant-studio_amd.pipeline")
    fd = os.open(tmp_path / "o.bin", os.O_RDWR | os.O_CREAT | os.O_TRUNC, 0o644)
    try:
        with pl.NativePipeline(0, fd) as p:
            rc = p.L.qs_pipeline_quantize(p.h, 12, 30, ctypes.c_void_p(16), 1 << 40, 1 << 20, None,
                                          1, fd, 0)
            assert rc == -22 and "exceed the 2^34" in qs.last_error()
            p.finish()
    finally:
        os.close(fd)


def test_pipeline_imatrix_rule(tmp_path):
    """The pipeline takes a missing imatrix where qs_quantize does: IQ3_XXS
    runs without one (quantize_iq3_xxs(x, None), iq3_xxs.py:41-42) with the
    oracle's bytes, and IQ2_XXS is refused when queued (its quantizer has no
    path without one, iq2.py:418-431)."""
    import os
    qs = importlib.import_module("quant-studio_amd")
    pl = importlib.import_module("quant-studio_amd.pipeline")
    rng = np.random.default_rng(8)
    x = (rng.normal(size=(11, 512)) * 0.02).astype(np.float32)
    info = io.TensorInfo("t", (512, 11), GT.F32, 0, x.nbytes, x.view(np.uint8).reshape(-1))
    ref = oracle.quantize("iq3_xxs", x, None)
    path = tmp_path / "o.bin"
    fd = os.open(path, os.O_RDWR | os.O_CREAT | os.O_TRUNC, 0o644)
    try:
        with pl.NativePipeline(0, fd) as p:
            p.quantize_tensor(info, int(GT.IQ3_XXS), None, 4, 0, qs.row_bytes(int(GT.IQ3_XXS), 512))
            with pytest.raises(pl.PipelineError, match="requires an imatrix"):
                p.quantize_tensor(info, int(GT.IQ2_XXS), None, 4, ref.nbytes,
                                  qs.row_bytes(int(GT.IQ2_XXS), 512))
            p.finish()
    finally:
        os.close(fd)
    assert np.array_equal(np.frombuffer(path.read_bytes()[:ref.nbytes], np.uint8).reshape(ref.shape), ref)
