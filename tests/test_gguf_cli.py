"""CPU tests of the GGUF container I/O and the command line (plan, dry run,
error paths) -- the parts of the drop-in that need no GPU."""

from __future__ import annotations

import importlib
import struct
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from cli_models import GT, KV, VT, fallback_model, imatrix_for, io, small_model

ROOT = Path(__file__).resolve().parent.parent
CLI = [sys.executable, str(ROOT / "quant-studio.py")]


def run_cli(*args, check=True):
    r = subprocess.run([*CLI, *map(str, args)], capture_output=True, text=True, timeout=300)
    if check and r.returncode != 0:
        raise AssertionError(f"exit {r.returncode}: {r.stderr}")
    return r


def test_header_bytes_follow_the_format(tmp_path):
    p = tmp_path / "t.gguf"
    io.write_gguf(p, "llama", [KV("a.b", VT.UINT32, 7)],
                  [("w", (4, 2), GT.F32, np.arange(8, dtype=np.float32).reshape(2, 4))])
    b = p.read_bytes()
    assert b[:4] == b"GGUF" and struct.unpack_from("<IQQ", b, 4) == (3, 1, 2)
    off = 24
    key_len = struct.unpack_from("<Q", b, off)[0]
    assert b[off + 8:off + 8 + key_len] == b"general.architecture"     # written first
    r = io.GGUFReader(p)
    assert list(r.kv) == ["general.architecture", "a.b"]
    t = r.tensors[0]
    assert (t.name, t.ne, t.ggml_type, t.offset) == ("w", (4, 2), GT.F32, 0)
    assert r.data_offset % 32 == 0 and len(b) % 32 == 0
    assert np.array_equal(t.array(), np.arange(8, dtype=np.float32).reshape(2, 4))


def test_roundtrip_every_value_type(tmp_path):
    p = tmp_path / "m.gguf"
    small_model(p)
    r = io.GGUFReader(p)
    q = tmp_path / "copy.gguf"
    io.write_gguf(q, r.get("general.architecture"),
                  [kv for n, kv in r.kv.items() if n != "general.architecture"],
                  [(t.name, t.ne, t.ggml_type, t.data) for t in r.tensors])
    assert q.read_bytes() == p.read_bytes()
    assert r.get("tokenizer.ggml.tokens") == ["<s>", "</s>", "hello"]
    assert r.get("test.flag") is True and r.get("test.i64") == -(1 << 40)
    assert r.get("llama.attention.layer_norm_rms_epsilon") == np.float32(1e-5)


def test_imatrix_loader_divides_by_counts(tmp_path):
    p = tmp_path / "im.gguf"
    vals = imatrix_for(p, {"a.weight": 64, "b.weight": 32}, n_mat={"b.weight": 3})
    got = io.load_imatrix(p)
    assert set(got) == {"a.weight", "b.weight"}
    np.testing.assert_array_equal(got["a.weight"], vals["a.weight"])
    assert got["b.weight"].shape == (96,)


def test_imatrix_loader_per_expert_counts(tmp_path):
    """One row of in_sum2 per count (per expert), divided by its own count in
    float32; a zero count gives zeros; a name without both records is left out."""
    GT = io.GT if hasattr(io, "GT") else __import__("importlib").import_module(
        "quant-studio_amd.gguf_types").GGMLQuantizationType
    p = tmp_path / "im.gguf"
    s = np.arange(1, 13, dtype=np.float32) / np.float32(3.0)
    c = np.array([3.0, 0.0, 7.0], np.float32)
    io.write_gguf(p, "imatrix", [], [("e.weight.in_sum2", (12,), GT.F32, s),
                                     ("e.weight.counts", (3,), GT.F32, c),
                                     ("lonely.weight.in_sum2", (4,), GT.F32, s[:4])])
    got = io.load_imatrix(p)
    assert set(got) == {"e.weight"} and got["e.weight"].dtype == np.float32
    want = np.concatenate([s[:4] / np.float32(3.0), np.zeros(4, np.float32), s[8:] / np.float32(7.0)])
    assert np.array_equal(got["e.weight"], want)


def test_dry_run_plan(tmp_path):
    src = tmp_path / "in.gguf"
    small_model(src)
    r = run_cli(src, tmp_path / "o.gguf", "q4_0", "--dry-run")
    lines = {ln.split()[0]: ln.split() for ln in r.stdout.splitlines() if ln.startswith(("blk", "tok", "rope"))}
    assert lines["blk.0.attn_q.weight"][1:4] == ["F32", "->", "Q4_0"]
    assert lines["blk.0.attn_norm.weight"][3] == "F32"          # 1-D: passthrough
    assert lines["blk.0.odd.weight"][3] == "F32"                # 40 % 32: Q4_0 has no fallback
    assert "dry run:" in r.stdout
    assert "no tensor type fallback" in r.stderr


@pytest.mark.parametrize("argv,msg", [
    (["q4_0", "--allow-requantize"], "--allow-requantize is not supported"),
    (["q4_0", "--keep-split"], "--keep-split is not supported"),
    (["NOPE"], "unknown quantization scheme"),
    (["IQ1_S"], "not supported by quant-studio"),
    (["q4_0", "8"], "nthreads argument is not supported"),
    (["iq2_xxs"], "require importance matrix data"),
    (["q4_0", "--tensor-type", "attn"], "expected name=ggml_type"),
    (["q4_0", "--token-embedding-type", "q9_9"], "unknown ggml type"),
    (["q4_0", "--device", "tpu"], "use auto, cuda, hip, cuda:N, cpu or mps"),
    (["q4_0", "--device", "cuda:x"], "use auto, cuda, hip, cuda:N, cpu or mps"),
    (["q4_0", "--sqrt-rounding", "fast"], "--sqrt-rounding 'fast'"),
])
def test_cli_errors(tmp_path, argv, msg):
    src = tmp_path / "in.gguf"
    small_model(src, odd=False)
    args = [src] + ([tmp_path / "o.gguf"] if argv[0] != "q4_0" or "8" not in argv else []) + argv
    if argv == ["q4_0", "8"]:
        args = [src, "q4_0", "8"]
    r = run_cli(*args, "--dry-run", check=False)
    assert r.returncode != 0 and msg in (r.stderr + r.stdout)


@pytest.mark.parametrize("argv,msg", [
    ([], "missing quantization type"),
    (["out.gguf", "q4_0", "8", "extra"], "unrecognized arguments: extra"),
])
def test_cli_usage_errors_exit_2(tmp_path, argv, msg):
    """argparse-level errors: usage on stderr and exit status 2, as the
    reference's parser gives them."""
    src = tmp_path / "in.gguf"
    small_model(src, odd=False)
    r = run_cli(src, *argv, "--dry-run", check=False)
    assert r.returncode == 2 and msg in r.stderr and "usage:" in r.stderr


def test_cpu_and_mps_devices_are_accepted(tmp_path):
    """The reference's --device cpu / mps (quant-studio.py:51-58) run: this
    build computes on the ROCm device, which the header line says."""
    src = tmp_path / "in.gguf"
    small_model(src, odd=False)
    for dev in ("cpu", "mps"):
        r = run_cli(src, tmp_path / "o.gguf", "q4_0", "--device", dev, "--dry-run")
        assert f"device={dev} (on rocm)" in r.stdout and "dry run:" in r.stdout


def test_header_names_the_square_root_rounding(tmp_path):
    """The header line shows whose torch.sqrt rounding the weights follow, for
    the default and a chosen mode (--device does not change it)."""
    src = tmp_path / "in.gguf"
    small_model(src, odd=False)
    r = run_cli(src, tmp_path / "o.gguf", "q4_0", "--dry-run")
    assert "sqrt-rounding=torch-cpu" in r.stdout.splitlines()[0]
    r = run_cli(src, tmp_path / "o.gguf", "q4_0", "--device", "cuda", "--sqrt-rounding", "ieee", "--dry-run")
    assert "sqrt-rounding=ieee" in r.stdout.splitlines()[0]


def test_mem_and_size_helpers():
    cli = importlib.import_module("quant-studio_amd.cli")
    assert cli.parse_mem("4G") == 4 << 30 and cli.parse_mem(" 512m ") == 512 << 20
    assert cli.parse_mem("1.5K") == 1536 and cli.parse_mem("1000") == 1000
    with pytest.raises(ValueError):
        cli.parse_mem("1.5")
    assert cli.fmt_size(1023) == "    1023 B  "
    assert cli.fmt_size(1024) == "     1.0 KiB"
    assert cli.fmt_size(5 << 20) == "     5.0 MiB"
    assert cli.fmt_size((1 << 30) * 3 // 2) == "     1.5 GiB"
    assert cli.fmt_size(1 << 50) == f"{float(1 << 20):8.1f} GiB"


def test_default_output_name_and_positional_type(tmp_path):
    src = tmp_path / "in.gguf"
    small_model(src, odd=False)
    r = run_cli(src, "Q4_K_M", "--dry-run")
    assert f"-> {tmp_path / 'ggml-model-Q4_K_M.gguf'}" in r.stdout


def test_fallback_to_a_type_without_kernel_is_an_error(tmp_path):
    # IQ2_XXS on a 40-column tensor falls back to F16, which has no quantizer
    src = tmp_path / "in.gguf"
    small_model(src)
    r = run_cli(src, tmp_path / "o.gguf", "iq2_xxs", "--dry-run", check=False)
    assert r.returncode != 0 and "F16 for 1 tensors" in r.stderr


def ffn_down_model(path: Path, n_layer: int = 8) -> None:
    io.write_gguf(path, "llama", [KV("llama.block_count", VT.UINT32, n_layer)],
                  [(f"blk.{i}.ffn_down.weight", (256, 32), GT.F32,
                    np.zeros((32, 256), np.float32)) for i in range(n_layer)])


def test_missing_kernel_type_is_an_error(tmp_path):
    # an override to a type without a quantizer (IQ1_S)
    src = tmp_path / "in.gguf"
    ffn_down_model(src)
    r = run_cli(src, tmp_path / "o.gguf", "q4_0", "--tensor-type", "ffn_down=iq1_s", "--dry-run",
                check=False)
    assert r.returncode != 0 and "needs kernel types" in r.stderr and "IQ1_S" in r.stderr


def test_q4_0_with_imatrix_uses_q4_1_on_the_first_ffn_down_layers(tmp_path):
    # scheme.py:521-523: i_layer < n_layer / 8 with an imatrix -> Q4_1
    src = tmp_path / "in.gguf"
    ffn_down_model(src)
    im = tmp_path / "im.gguf"
    imatrix_for(im, {f"blk.{i}.ffn_down.weight": 256 for i in range(8)})
    r = run_cli(src, tmp_path / "o.gguf", "q4_0", "--imatrix", im, "--dry-run")
    lines = {ln.split()[0]: ln.split() for ln in r.stdout.splitlines() if ln.startswith("blk")}
    assert lines["blk.0.ffn_down.weight"][3] == "Q4_1"
    assert all(lines[f"blk.{i}.ffn_down.weight"][3] == "Q4_0" for i in range(1, 8))


@pytest.mark.parametrize("scheme,want", [
    ("Q4_K_M", {"attn_q": "Q5_0", "attn_v": "Q8_0", "ffn_down": "Q8_0"}),
    ("Q5_K_S", {"attn_q": "Q5_1"}),
    ("IQ4_XS", {"attn_q": "IQ4_NL"}),
])
def test_shape_fallback_types(tmp_path, scheme, want):
    # tensor_type_fallback (scheme.py:364-384): k % 256 != 0 -> a 32-value block type
    src = tmp_path / "in.gguf"
    fallback_model(src)
    r = run_cli(src, tmp_path / "o.gguf", scheme, "--dry-run")
    lines = {ln.split()[0]: ln.split() for ln in r.stdout.splitlines() if ln.startswith("blk")}
    for short, t in want.items():
        assert lines[f"blk.0.{short}.weight"][3] == t, (short, lines[f"blk.0.{short}.weight"])
    assert "falling back to" in r.stderr


def test_readahead_walks_the_plan_within_its_budget(tmp_path):
    """The input readahead advises the mapped tensors in plan order (page-aligned
    starts), stays within its byte budget of what the pipeline has taken, and
    stops cleanly when closed while waiting; the real madvise accepts its
    arguments on a mapped file (CPU only)."""
    import mmap
    import threading
    import time
    pipeline = importlib.import_module("quant-studio_amd.pipeline")
    path = tmp_path / "blob.bin"
    path.write_bytes(bytes(range(256)) * 4096)               # 1 MiB
    with open(path, "rb") as f:
        mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        base = np.frombuffer(mm, dtype=np.uint8)
        ts = [io.TensorInfo(f"t{i}", (1024,), GT.BF16, 0, 2048, base[i * 4096 + 7: i * 4096 + 7 + 2048])
              for i in range(200)]
        ra = pipeline.Readahead(ts[:4])                       # the libc madvise, on real pages
        for t in ts[:4]:
            ra.advance(t.nbytes)
        ra.close()
        advised, lock = [], threading.Lock()

        def record(a, n, adv):
            with lock:
                advised.append((a, n, adv))
            return 0

        page = pipeline.os.sysconf("SC_PAGE_SIZE")
        ra = pipeline.Readahead(ts, budget=16 * 1024, madvise=record)
        time.sleep(0.2)
        first = len(advised)
        assert 0 < first <= 16 * 1024 // 2048 + 1             # stopped at the budget
        for t in ts[:50]:
            ra.advance(t.nbytes)
        time.sleep(0.2)
        assert first < len(advised) <= 50 + 16 * 1024 // 2048 + 1
        ra.close()                                             # ends while waiting
        starts = [a for a, _, _ in advised]
        assert starts == sorted(starts)
        assert all(adv == pipeline.Readahead.MADV_WILLNEED for _, _, adv in advised)
        addr0 = ts[0].data.ctypes.data
        assert advised[0] == (addr0 - addr0 % page, 2048 + addr0 % page, 3)
        # a tensor longer than the window is advised window by window, in order
        big = [io.TensorInfo("big", (1 << 19,), GT.BF16, 0, 1 << 20, base[4096 + 5: 4096 + 5 + (1 << 20)])]
        win = []
        ra2 = type("R", (pipeline.Readahead,), {"WINDOW": 1 << 18})(
            big, madvise=lambda a, n, adv: win.append((a, n)) or 0)
        time.sleep(0.2)
        ra2.close()
        a0 = big[0].data.ctypes.data
        assert win[0][0] == a0 - a0 % page and all(n == 1 << 18 for _, n in win[:-1])
        assert sum(n for _, n in win) == (1 << 20) + a0 % page
        assert all(win[i + 1][0] == win[i][0] + win[i][1] for i in range(len(win) - 1))


def test_preallocate_keeps_written_bytes(tmp_path):
    """The output file's blocks are allocated up front (fallocate(2)); bytes
    already written stay, the size becomes the planned one, and a descriptor
    that cannot be extended reports False instead of raising."""
    import os
    cli = importlib.import_module("quant-studio_amd.cli")
    path = tmp_path / "o.bin"
    fd = os.open(path, os.O_RDWR | os.O_CREAT | os.O_TRUNC, 0o644)
    try:
        os.write(fd, b"GGUF-header")
        assert cli.preallocate(fd, 1 << 20)
        assert os.fstat(fd).st_size == 1 << 20
    finally:
        os.close(fd)
    assert path.read_bytes()[:11] == b"GGUF-header"
    fd = os.open(path, os.O_RDONLY)
    try:
        assert not cli.preallocate(fd, 2 << 20)
    finally:
        os.close(fd)


def test_requested_device_from_argv():
    """The entry script's early device start reads the device from argv the
    way the command line will use it (cuda:N -> N, everything else device 0)
    and starts nothing for runs that use no device."""
    ps = importlib.import_module("quant-studio_amd.pipeline_start")
    rd = ps.requested_device
    assert rd(["in.gguf", "out.gguf", "Q4_K_M"]) == 0
    assert rd(["in.gguf", "out.gguf", "Q4_K_M", "--device", "cuda:1"]) == 1
    assert rd(["in.gguf", "out.gguf", "Q4_K_M", "--device=cuda:2"]) == 2
    assert rd(["in.gguf", "out.gguf", "Q4_K_M", "--device", "cpu"]) == 0
    assert rd(["in.gguf", "out.gguf", "Q4_K_M", "--device", "cuda:x"]) is None
    assert rd(["in.gguf", "out.gguf", "Q4_K_M", "--dry-run"]) is None
    assert rd(["--help"]) is None and rd([]) is None


def test_early_start_without_a_device():
    """An early start for a device that is not there (no GPU here) ends on
    its own: take() hands back no pipeline, so the command line creates one
    itself and reports the missing device in the reference's words, and
    close() releases nothing."""
    ps = importlib.import_module("quant-studio_amd.pipeline_start")
    qs = importlib.import_module("quant-studio_amd")
    if qs.library().qs_device_count() > 0:
        pytest.skip("a ROCm device is visible")
    start = ps.early_start(["in.gguf", "out.gguf", "Q4_K_M"])
    assert start is not None and start.device == 0
    assert start.take(1) is None
    start.close()
    assert ps.early_start(["in.gguf", "out.gguf", "Q4_K_M", "--dry-run"]) is None
