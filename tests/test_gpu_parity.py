"""GPU parity: the HIP quantizers against the reference's golden vectors and the
CPU oracle, byte for byte. Runs on an MI355X (pytest -m gpu); every call goes
through the C ABI of libqs_hip.so."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import oracle
from golden_data import TYPES, block_identical, cases, nonfinite_case, zero_imatrix_cases

pytestmark = pytest.mark.gpu

HIP_TYPES = ["q4_0", "q2_k", "q3_k", "q4_k", "q5_k", "q6_k", "iq4_xs",
             "iq2_xxs", "iq2_xs", "iq2_s", "iq3_xxs", "iq3_s"]
NEEDS_IMATRIX = {"iq2_xxs", "iq2_xs", "iq2_s"}     # IQ3_XXS runs without one (iq3_xxs.py:41-42)
NTHREADS = min(16, len(os.sched_getaffinity(0)))


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return torch.device("cuda:0")


def to_device(x: np.ndarray, dev) -> torch.Tensor:
    if x.dtype == np.uint16:
        return torch.from_numpy(x.view(np.int16).copy()).view(torch.bfloat16).to(dev)
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dev)


def hip_quantize(qs, qtype, x, qw, dev) -> np.ndarray:
    tid = TYPES[qtype][0]
    xq = to_device(x, dev)
    q = None if qw is None else torch.from_numpy(qw).to(dev)
    out = qs.quantize(tid, xq, q)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def bf16_bits(a: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("qtype", HIP_TYPES)
def test_golden_vectors(qs, dev, qtype):
    """Golden inputs: identical to the reference's own bytes and to the oracle
    on every block (the kernels reproduce torch's CPU square root)."""
    for key, x, qw, expect in cases(qtype):
        print(f"{qtype} {key} shape={x.shape}", flush=True)
        got = hip_quantize(qs, qtype, x, qw, dev)
        same = block_identical(got, expect, qtype)
        assert same.all(), f"{qtype} {key}: {int((~same).sum())}/{same.size} blocks differ from the reference"
        ref = oracle.quantize(qtype, x, qw, n_threads=NTHREADS)
        assert np.array_equal(got, ref), f"{qtype} {key}: differs from the oracle"


ZERO_IMATRIX_TYPES = [t for t in HIP_TYPES if t != "q4_0"]


@pytest.mark.parametrize("qtype", ZERO_IMATRIX_TYPES)
def test_zero_imatrix_golden_vectors(qs, dev, qtype):
    """Imatrix vectors with zero entries (never-fired columns, zero 8/16/32/256
    -value groups, an all-zero vector; quant-studio.py:80-85 writes such zeros):
    identical to the reference's own bytes and to the oracle on every block."""
    for case, x, qw, expect in zero_imatrix_cases(qtype):
        print(f"{qtype} zero-imatrix {case} shape={x.shape}", flush=True)
        got = hip_quantize(qs, qtype, x, qw, dev)
        same = block_identical(got, expect, qtype)
        assert same.all(), f"{qtype} {case}: {int((~same).sum())}/{same.size} blocks differ from the reference"
        assert np.array_equal(got, oracle.quantize(qtype, x, qw, n_threads=NTHREADS)), case


@pytest.mark.parametrize("mode", ["ieee", "torch-cpu-amd"])
@pytest.mark.parametrize("qtype", ZERO_IMATRIX_TYPES)
def test_zero_imatrix_sqrt_modes(qs, dev, mode, qtype):
    """The same zero-imatrix inputs in the other square-root modes, against the
    oracle in that mode (sqrt(0) = +0 in every mode)."""
    import sqrt_hosts
    if mode == "ieee":
        oracle.use_ieee_sqrt(True)
    else:
        oracle.use_amd_host_sqrt(sqrt_hosts.amd_ulps())
    try:
        qs.set_sqrt_rounding(mode)
        for case, x, qw, _ in zero_imatrix_cases(qtype):
            print(f"{qtype} zero-imatrix {case} sqrt={mode}", flush=True)
            got = hip_quantize(qs, qtype, x, qw, dev)
            assert np.array_equal(got, oracle.quantize(qtype, x, qw, n_threads=NTHREADS)), case
    finally:
        qs.set_sqrt_rounding("torch-cpu")
        oracle.use_ieee_sqrt(False)
        oracle.use_sqrt_table(None)


EXTRA_TYPES = {"q4_1": 3, "q5_0": 6, "q5_1": 7, "q8_0": 8, "iq4_nl": 20}


# NaN bit patterns the hardware makes: an IQ4_XS / IQ3_S scale derived from a
# NaN the arithmetic created carries the sign of that default NaN (positive on
# the GPU, negative on x86), so their non-finite blocks are not compared
NAN_SIGN_TYPES = {"iq4_xs", "iq3_s"}


@pytest.mark.parametrize("qtype", HIP_TYPES + sorted(EXTRA_TYPES))
def test_nonfinite_inputs_match_the_oracle(qs, dev, qtype):
    """Rows holding NaN, +-Inf and +-1e38 values (f32 source), with and without
    imatrix: every kernel stays in bounds and returns the oracle's bytes on
    every block whose values are finite and below 1e18, and on every block for
    the types whose non-finite arithmetic the oracle shares (all but IQ4_XS and
    IQ3_S); Q4_0's bytes are then the reference's on every block
    (test_oracle.py pins the oracle's)."""
    from golden_data import clean_blocks
    x, qw, ref = nonfinite_case()
    tid = TYPES[qtype][0] if qtype in TYPES else EXTRA_TYPES[qtype]
    bs = 32 if qtype in ("q4_0", "iq4_nl") or qtype in EXTRA_TYPES else 256
    nb = TYPES[qtype][2] if qtype in TYPES else qs.row_bytes(tid, bs)
    clean = clean_blocks(x, bs)
    for imat in (False, True):
        if qtype in NEEDS_IMATRIX and not imat:
            continue
        q = qw if imat else None
        print(f"{qtype} imat={imat} non-finite rows", flush=True)
        got = qs.quantize(tid, to_device(x, dev), None if q is None else torch.from_numpy(q).to(dev))
        got = got.cpu().numpy()
        want = oracle.quantize(qtype, x, q, n_threads=NTHREADS)
        same = (got.reshape(-1, nb) == want.reshape(-1, nb)).all(1)
        assert same[clean].all(), f"{qtype} imat={imat}: finite blocks differ from the oracle"
        if qtype not in NAN_SIGN_TYPES:
            assert same.all(), f"{qtype} imat={imat}: non-finite blocks differ from the oracle"
        if qtype == "q4_0":
            assert np.array_equal(got, ref["q4_0.none"]), "q4_0: differs from the reference"


def ffn_like(rows: int, k: int, seed: int):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((rows, k)) * 0.02 * np.exp(0.3 * rng.standard_normal((rows, 1)))
    return bf16_bits(a), rng.lognormal(0.0, 1.0, k).astype(np.float32)


@pytest.mark.parametrize("qtype", HIP_TYPES)
@pytest.mark.parametrize("imat", [False, True])
def test_oracle_parity_random(qs, dev, qtype, imat):
    """Random ffn-like rows against the oracle; Q4_0 ignores an imatrix (the
    reference's Q4_0, q4_0.py:36-37), the IQ2 types refuse to run without one
    (their quantizers index qw unconditionally) and IQ3_XXS runs without one
    as quantize_iq3_xxs(x, None) does (iq3_xxs.py:41-42)."""
    x, qw = ffn_like(384, 2560, seed=sum(map(ord, qtype)) * 2 + int(imat))
    qw = qw if imat else None
    print(f"{qtype} imat={imat} 384x2560", flush=True)
    if qtype in NEEDS_IMATRIX and not imat:
        with pytest.raises(qs.QuantSpecError, match="requires an imatrix"):
            hip_quantize(qs, qtype, x, None, dev)
        return
    got = hip_quantize(qs, qtype, x, qw, dev)
    ref = oracle.quantize(qtype, x, None if qtype == "q4_0" else qw, n_threads=NTHREADS)
    same = block_identical(got, ref, qtype)
    assert same.all(), f"{int((~same).sum())}/{same.size} blocks differ"


@pytest.mark.parametrize("qtype", HIP_TYPES)
def test_tiny_magnitudes_match_the_oracle(qs, dev, qtype):
    """Rows scaled to ~1e-13 (their weighted error and distance terms,
    w*d*d ~ 1e-39, are f32 subnormals), rows around the groups' activity
    threshold (max |x| of 1e-15, GROUP_MAX_EPS) and rows of ordinary scale
    with an imatrix of ~1e-30 (every weighted term subnormal, the blocks'
    f16 scales representable) or of ~1e34 (sums and products that overflow),
    f32 source: the kernels keep subnormals and overflow as the reference's
    CPU arithmetic does, and the IQ searches' choice between full and reduced
    neighbour lists holds on terms that underflow to zero or overflow."""
    rng = np.random.default_rng(sum(map(ord, qtype)) + 17)
    k = 2560
    rows = []
    for scale in (1e-13, 3e-15, 1.2e-15, 8e-16):
        a = rng.standard_normal((24, k)) * scale
        rows.append(a)
    x = np.concatenate(rows).astype(np.float32)
    qw = rng.lognormal(0.0, 1.0, k).astype(np.float32)
    # values whose f16 block scales stay representable, with an imatrix of
    # ~1e-30: the weights are ~1e-34 and every weighted term subnormal
    x2 = (rng.standard_normal((32, k)) * 3e-4).astype(np.float32)
    qw2 = (rng.lognormal(0.0, 1.0, k) * 1e-30).astype(np.float32)
    # and an imatrix of ~1e34, whose weighted sums and products overflow to inf
    qw3 = (rng.lognormal(0.0, 1.0, k) * 1e34).astype(np.float32)
    for xs, q, what in ((x, qw, "tiny values"), (x, None, "tiny values"), (x2, qw2, "tiny imatrix"),
                        (x2, qw3, "huge imatrix")):
        if q is None and qtype in NEEDS_IMATRIX:
            continue
        print(f"{qtype} imat={q is not None} {what} {xs.shape}", flush=True)
        got = hip_quantize(qs, qtype, xs, q, dev)
        ref = oracle.quantize(qtype, xs, None if qtype == "q4_0" else q, n_threads=NTHREADS)
        same = block_identical(got, ref, qtype)
        assert same.all(), f"{qtype} imat={q is not None} {what}: {int((~same).sum())}/{same.size} blocks differ"


def nan_sign_cleared(b: np.ndarray, nb: int) -> np.ndarray:
    """Blocks with the sign bit of a NaN f16 block scale (bytes 0-1) cleared."""
    b = b.reshape(-1, nb).copy()
    d = b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8)
    nan = ((d & 0x7C00) == 0x7C00) & ((d & 0x03FF) != 0)
    b[nan, 1] &= 0x7F
    return b


@pytest.mark.parametrize("qtype", HIP_TYPES)
def test_special_weights_and_near_max_values(qs, dev, qtype):
    """Imatrix columns of +inf, NaN and -0 (whole superblocks, a 32-value
    group, a 4-value subgroup), and rows holding values near FLT_MAX next to
    zeros, f32 source. An IQ search whose distances are all +inf or NaN takes
    the list's first NaN, else its first entry, as torch's argmin does
    (iq2.py:366-371, iq3_common.py:228-235); -0 weights give -0 distances,
    which tie; values near FLT_MAX overflow x^2 and the superblock's sigma2,
    so their weights are +inf (or NaN at a zero importance). The GPU
    returns the oracle's bytes on every block (IQ4_XS and IQ3_S up to the sign
    of a NaN block scale, positive on the GPU and negative on x86)."""
    rng = np.random.default_rng(sum(map(ord, qtype)) + 29)
    k, nb = 2560, TYPES[qtype][2]
    x = (rng.standard_normal((64, k)) * 0.02).astype(np.float32)
    runs = []
    for what, val in (("+inf columns", np.inf), ("NaN columns", np.nan)):
        qw = rng.lognormal(0.0, 1.0, k).astype(np.float32)
        qw[rng.choice(k, 6, replace=False)] = val
        runs.append((what, x, qw))
    qw = rng.lognormal(0.0, 1.0, k).astype(np.float32)
    qw[256:512] = -0.0
    qw[1024:1056] = -0.0
    qw[2000:2004] = -0.0
    runs.append(("-0 columns", x, qw))
    xb = x.copy()
    xb[0:16, 5] = 3.0e38                 # one value near FLT_MAX, the rest of its group zero
    xb[0:16, 0:5] = 0.0
    xb[0:16, 6:32] = 0.0
    xb[16:32, 300] = -2.9e38
    xb[16:32, 288:300] = 0.0
    xb[32:48, 600] = 2.0e36              # beyond 2^120: full lists, no overflow
    xb[48:64, 1000:1004] = 0.0
    xb[48:64, 1004] = 3.3e38
    runs.append(("near-max values", xb, None))
    runs.append(("near-max values", xb, rng.lognormal(0.0, 1.0, k).astype(np.float32)))
    for what, xs, q in runs:
        if q is None and qtype in NEEDS_IMATRIX:
            continue
        print(f"{qtype} imat={q is not None} {what}", flush=True)
        got = hip_quantize(qs, qtype, xs, q, dev)
        ref = oracle.quantize(qtype, xs, None if qtype == "q4_0" else q, n_threads=NTHREADS)
        if qtype in NAN_SIGN_TYPES:
            got, ref = nan_sign_cleared(got, nb), nan_sign_cleared(ref, nb)
        same = (got.reshape(-1, nb) == ref.reshape(-1, nb)).all(1)
        assert same.all(), f"{qtype} imat={q is not None} {what}: {int((~same).sum())}/{same.size} blocks differ"


def test_q4_0_full_4096x4096(qs, dev):
    """Q4_0 on one bf16 4096x4096 tensor, N(0, 0.02) with 0.1%
    outliers x20, seed 0, byte-exact."""
    rng = np.random.default_rng(0)
    a = rng.normal(0.0, 0.02, (4096, 4096))
    idx = rng.choice(a.size, 16777, replace=False)
    a.reshape(-1)[idx] *= 20.0
    x = bf16_bits(a)
    got = hip_quantize(qs, "q4_0", x, None, dev)
    ref = oracle.quantize("q4_0", x, None, n_threads=NTHREADS)
    assert got.shape == (4096, 4096 // 32 * 18)
    assert np.array_equal(got, ref)


def test_q4_k_imatrix_full_ffn_shapes(qs, dev):
    """Q4_K with imatrix on the ffn shapes 9728x2560 and 2560x9728 bf16,
    per-row log-normal std jitter, log-normal per-column imatrix."""
    for rows, k, seed in ((9728, 2560, 1), (2560, 9728, 2)):
        print(f"q4_k imat {rows}x{k}", flush=True)
        x, qw = ffn_like(rows, k, seed)
        got = hip_quantize(qs, "q4_k", x, qw, dev)
        ref = oracle.quantize("q4_k", x, qw, n_threads=NTHREADS)
        same = block_identical(got, ref, "q4_k")
        assert same.all(), f"{rows}x{k}: {int((~same).sum())}/{same.size} blocks differ"


@pytest.mark.parametrize("qtype", ["q4_0", "q4_k", "q6_k", "q3_k", "iq2_xxs", "iq2_s", "iq3_s"])
def test_row_chunking_invariance(qs, dev, qtype):
    x, qw = ffn_like(300, 1024, seed=9)
    tid = TYPES[qtype][0]
    xd = to_device(x, dev)
    q = torch.from_numpy(qw).to(dev)
    whole = qs.quantize(tid, xd, q)
    parts = torch.cat([qs.quantize(tid, xd[a:b], q) for a, b in ((0, 7), (7, 150), (150, 300))])
    torch.cuda.synchronize()
    assert torch.equal(whole, parts)


@pytest.mark.parametrize("qtype", ["q4_0", "q5_k", "q2_k", "iq4_xs", "iq2_xs", "iq3_xxs"])
def test_f16_source(qs, dev, qtype):
    rng = np.random.default_rng(4)
    a = (rng.standard_normal((64, 512)) * 0.05).astype(np.float16)
    qw = rng.lognormal(0, 1, 512).astype(np.float32)
    tid = TYPES[qtype][0]
    got = qs.quantize(tid, torch.from_numpy(a).to(dev), torch.from_numpy(qw).to(dev)).cpu().numpy()
    ref = oracle.quantize(qtype, a.astype(np.float32), None if qtype == "q4_0" else qw)
    assert np.array_equal(got, ref)


def test_row_stride_and_unaligned_output(qs, dev):
    x, qw = ffn_like(40, 1024, seed=12)
    wide = torch.zeros((40, 1024 + 64), dtype=torch.bfloat16, device=dev)
    wide[:, :1024] = to_device(x, dev)
    view = wide[:, :1024]                       # row stride 1088 elements (2176 B)
    assert view.stride(0) == 1088
    for qtype in ("q4_0", "q6_k", "q4_k", "iq2_xxs", "iq2_s", "iq3_s"):
        tid = TYPES[qtype][0]
        rb = TYPES[qtype][2] * (1024 // TYPES[qtype][1])
        buf = torch.zeros(40 * rb + 3, dtype=torch.uint8, device=dev)
        out = buf[1:1 + 40 * rb]                # 1-byte offset: byte-store path
        qs.quantize(tid, view, torch.from_numpy(qw).to(dev), out=out)
        ref = oracle.quantize(qtype, x, None if qtype == "q4_0" else qw)
        b = buf.cpu().numpy()
        assert b[0] == 0 and b[-2:].tolist() == [0, 0]
        assert np.array_equal(b[1:1 + 40 * rb].reshape(40, rb), ref)


def test_empty_and_single_row(qs, dev):
    e = torch.zeros((0, 256), dtype=torch.bfloat16, device=dev)
    assert qs.quantize(12, e, None).shape == (0, 144)
    x, qw = ffn_like(1, 256, seed=3)
    got = hip_quantize(qs, "q4_k", x, qw, dev)
    assert np.array_equal(got, oracle.quantize("q4_k", x, qw))


def lattice_rows(rows: int, k: int, seed: int):
    """Rows whose values are small integer multiples of a power of two (a
    power of two per row, random signs, ~1 block in 8 of equal magnitudes)
    with a power-of-two imatrix holding ~10% zeros: the IQ searches' level
    terms then tie exactly, are exactly zero, and put values on the code's
    clamped top level with the grid's top level better -- the cases in which
    the searches choose between the full and the reduced neighbour lists."""
    rng = np.random.default_rng(seed)
    m = np.minimum(rng.geometric(0.25, (rows, k)) - 1, 15).astype(np.float64)
    m *= rng.choice([-1.0, 1.0], (rows, k))
    flat = rng.random((rows, k // 256)) < 0.125
    m = np.where(np.repeat(flat, 256, axis=1), np.sign(m) * 3 + (m == 0), m)
    a = m * 2.0 ** -rng.integers(5, 10, (rows, 1)).astype(np.float64)
    qw = (2.0 ** rng.integers(-2, 3, k)) * (rng.random(k) >= 0.1)
    return bf16_bits(a), qw.astype(np.float32)


@pytest.mark.parametrize("qtype", ["iq2_xxs", "iq2_xs", "iq2_s", "iq3_xxs", "iq3_s"])
def test_iq_searches_on_lattice_inputs(qs, dev, qtype):
    """Lattice rows (exact ties, zero terms, clamped top levels) against the
    oracle, with the imatrix and, where the type runs without one, without."""
    x, qw = lattice_rows(384, 2560, seed=sum(map(ord, qtype)))
    for q in (qw, None):
        if q is None and qtype in NEEDS_IMATRIX:
            continue
        print(f"{qtype} imat={q is not None} lattice 384x2560", flush=True)
        got = hip_quantize(qs, qtype, x, q, dev)
        ref = oracle.quantize(qtype, x, q, n_threads=NTHREADS)
        same = block_identical(got, ref, qtype)
        assert same.all(), f"{qtype} imat={q is not None}: {int((~same).sum())}/{same.size} blocks differ"


def test_iq2_xxs_full_ffn_down_tensor_heavy_tailed(qs, dev):
    """IQ2_XXS at full size: one 2560x9728 ffn_down tensor of
    Student-t (df 5) weights scaled to std 0.02 with a log-normal imatrix.
    Every row is quantized on the GPU; 64 rows spread over the tensor are
    compared with the oracle byte for byte, and the whole tensor's
    dequantized error stays at the format's level."""
    import dequant
    rng = np.random.default_rng(44)
    rows, k = 2560, 9728
    a = rng.standard_t(5, size=(rows, k)) * (0.02 / np.sqrt(5 / 3))
    x = bf16_bits(a)
    qw = rng.lognormal(0.0, 1.0, k).astype(np.float32)
    got = hip_quantize(qs, "iq2_xxs", x, qw, dev)
    sel = np.linspace(0, rows - 1, 64).astype(int)
    ref = oracle.quantize("iq2_xxs", x[sel], qw, n_threads=NTHREADS)
    same = block_identical(got[sel], ref, "iq2_xxs")
    assert same.all(), f"{int((~same).sum())}/{same.size} blocks differ"
    xf = (x.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    xh = dequant.dequantize("iq2_xxs", got, rows)
    rel = np.sqrt(((xf - xh) ** 2).mean() / (xf ** 2).mean())
    assert rel < 0.62, rel


def test_python_mirror_splits_calls_over_the_value_limit(dev, monkeypatch):
    """quant_fn inputs above the C call's value limit go in row ranges with the
    same bytes as one call (limit lowered here to 3 rows, 7 rows in all)."""
    import importlib
    qs = importlib.import_module("quant-studio_amd")
    rng = np.random.default_rng(21)
    x = (rng.normal(size=(7, 512)) * 0.02).astype(np.float32)
    qw = rng.lognormal(size=512).astype(np.float32)
    for qtype in ("q4_k", "iq2_xs"):
        whole = hip_quantize(qs, qtype, x, qw, dev)
        monkeypatch.setattr(qs, "MAX_VALUES_PER_CALL", 3 * 512)
        split = hip_quantize(qs, qtype, x, qw, dev)
        monkeypatch.undo()
        assert np.array_equal(whole, split), qtype
        assert np.array_equal(whole, oracle.quantize(qtype, x, qw, n_threads=NTHREADS)), qtype


# every type whose weights take a square root: the imatrix variants, Q4_K /
# Q5_K without one (av_x = sqrt(sum x^2 / 32), q4_k.py:34), and the IQ3 types
# without one, whose searches weigh by sqrt(w) with w = x*x (iq3_xxs.py:41-47,
# iq3_s.py:41-47)
SQRT_CASES = [(t, True) for t in HIP_TYPES + ["iq4_nl"] if t != "q4_0"] + \
    [("q4_k", False), ("q5_k", False), ("iq3_xxs", False), ("iq3_s", False)]


@pytest.mark.parametrize("mode", ["ieee", "torch-cpu-amd"])
@pytest.mark.parametrize("qtype,imat", SQRT_CASES)
def test_sqrt_rounding_modes(qs, dev, mode, qtype, imat):
    """The other square-root modes against the oracle in the same mode: the
    IEEE root, and torch.sqrt as an AMD EPYC host's MKL rounds it (the map the
    library embeds, decoded independently by the test)."""
    import sqrt_hosts
    x, qw = ffn_like(192, 2560, seed=77 + sum(map(ord, qtype)))
    qw = qw if imat else None
    print(f"{qtype} imat={imat} sqrt={mode}", flush=True)
    if mode == "ieee":
        oracle.use_ieee_sqrt(True)
    else:
        oracle.use_amd_host_sqrt(sqrt_hosts.amd_ulps())
    try:
        qs.set_sqrt_rounding(mode)
        tid = int(qs.ALL_SPECS[qtype].ggml_type)
        got = qs.quantize(tid, to_device(x, dev), None if qw is None else torch.from_numpy(qw).to(dev))
        got = got.cpu().numpy()
        ref = oracle.quantize(qtype, x, qw, n_threads=NTHREADS)
    finally:
        qs.set_sqrt_rounding("torch-cpu")
        oracle.use_ieee_sqrt(False)
        oracle.use_sqrt_table(None)
    assert np.array_equal(got, ref), f"{qtype} sqrt={mode}: differs from the oracle"
    # and the default mode is back: the golden-host bytes again
    if imat:
        back = qs.quantize(tid, to_device(x[:8], dev), torch.from_numpy(qw).to(dev)).cpu().numpy()
        assert np.array_equal(back, oracle.quantize(qtype, x[:8], qw, n_threads=NTHREADS))


@pytest.mark.parametrize("qtype", ["q4_0", "q4_k", "iq2_xs", "iq3_s"])
def test_cpu_device_quant_fn(qs, dev, qtype):
    """make_kernel(cpu, qw) returns a quant_fn that takes CPU tensors and
    returns a CPU uint8 tensor with the oracle's bytes (the reference's CPU
    path, quant-studio.py:216-232), computing on the ROCm device."""
    x, qw = ffn_like(33, 512, seed=5)
    spec = qs.QUANT_TYPES[qtype]
    fn = spec.make_kernel(torch.device("cpu"), torch.from_numpy(qw))
    xt = torch.from_numpy(x.view(np.int16).copy()).view(torch.bfloat16)
    got = fn(xt)
    assert got.device.type == "cpu" and got.dtype == torch.uint8
    ref = oracle.quantize(qtype, x, qw if spec.uses_imatrix else None, n_threads=NTHREADS)
    assert np.array_equal(got.numpy(), ref)
    # f32 CPU input, and the module-level call with a CPU tensor
    got32 = qs.quantize(int(spec.ggml_type), xt.float(), torch.from_numpy(qw) if spec.uses_imatrix else None)
    assert got32.device.type == "cpu" and np.array_equal(got32.numpy(), ref)


def test_layouts_the_c_call_refuses_are_copied(qs, dev):
    """Views the C call does not take (column offset not 16-byte aligned, row
    stride not a multiple of 16 bytes, a contiguous view starting off a
    16-byte boundary, an expanded row) are quantized from a contiguous copy:
    same bytes as the contiguous tensor."""
    x, qw = ffn_like(24, 512, seed=8)
    base = torch.zeros((24, 512 + 40), dtype=torch.bfloat16, device=dev)
    base[:, 1:513] = to_device(x, dev)
    odd = torch.zeros((24, 516), dtype=torch.bfloat16, device=dev)
    odd[:, :512] = to_device(x, dev)
    q = torch.from_numpy(qw).to(dev)
    flat = torch.zeros(24 * 512 + 8, dtype=torch.bfloat16, device=dev)
    flat[1:1 + 24 * 512] = to_device(x, dev).reshape(-1)
    shifted = flat[1:1 + 24 * 512].view(24, 512)
    assert shifted.is_contiguous() and shifted.data_ptr() % 16 == 2
    views = {"column offset 1 (2 bytes)": base[:, 1:513],
             "row stride 1032 bytes": odd[:, :512],
             "contiguous view 2 bytes past a 16-byte boundary": shifted}
    for qtype in ("q4_0", "q4_k", "iq3_xxs"):
        tid = TYPES[qtype][0]
        ref = oracle.quantize(qtype, x, None if qtype == "q4_0" else qw, n_threads=NTHREADS)
        for name, v in views.items():
            assert np.array_equal(qs.quantize(tid, v, q).cpu().numpy(), ref), (qtype, name)
        row = to_device(x[:1], dev).expand(5, 512)
        assert row.stride(0) == 0
        got = qs.quantize(tid, row, q).cpu().numpy()
        assert np.array_equal(got, np.repeat(ref[:1], 5, axis=0)), (qtype, "expanded")


def test_init_uploads_tables_up_front(qs, dev):
    """qs_init on the device succeeds (again, too), and quantization then
    behaves as before on every table it uploaded."""
    qs.init(0)
    qs.init(0)
    x, qw = ffn_like(16, 512, seed=6)
    for qtype in ("q4_k", "iq2_s", "iq3_s"):
        assert np.array_equal(hip_quantize(qs, qtype, x, qw, dev),
                              oracle.quantize(qtype, x, qw, n_threads=NTHREADS))


# (module, function, takes qw) for the reference's per-type modules and the
# five extra types
MODULE_FUNCTIONS = [("q4_0", "quantize_q4_0", False), ("q2_k", "quantize_q2_k", True),
                    ("q3_k", "quantize_q3_k", True), ("q4_k", "quantize_q4_k", True),
                    ("q5_k", "quantize_q5_k", True), ("q6_k", "quantize_q6_k", True),
                    ("iq4_xs", "quantize_iq4_xs", True), ("iq2", "quantize_iq2_xxs", True),
                    ("iq2_xs", "quantize_iq2_xs", True), ("iq2_s", "quantize_iq2_s", True),
                    ("iq3_xxs", "quantize_iq3_xxs", True), ("iq3_s", "quantize_iq3_s", True),
                    ("q4_1", "quantize_q4_1", True), ("q5_0", "quantize_q5_0", True),
                    ("q5_1", "quantize_q5_1", True), ("q8_0", "quantize_q8_0", True),
                    ("iq4_nl", "quantize_iq4_nl", True)]


@pytest.mark.parametrize("mod,fn,takes_qw", MODULE_FUNCTIONS)
def test_per_type_functions_cpu_and_gpu_agree(dev, mod, fn, takes_qw):
    """The reference's own device check (tools/dev_gpu_check.py:27-45) on the
    per-type functions: seed 7, shapes 512x256, 256x512, 37x1024, a zero row,
    constant rows of +-0.5 and a 1e-6 row with one 8.0; the function called on
    CPU tensors and on device tensors gives the same bytes, and both are the
    oracle's (the reference asks only >= 97% between its two paths). IQ3_XXS
    and the types that use an imatrix run with and without one where their
    function takes None."""
    import importlib
    m = importlib.import_module(f"quant-studio_amd.{mod}")
    f = getattr(m, fn)
    (qtype, spec), = m.SPECS.items()
    torch.manual_seed(7)
    for rows, k in ((512, 256), (256, 512), (37, 1024)):
        x = torch.randn(rows, k) * 0.05 * (0.2 + torch.rand(rows, 1) * 3.0)
        x[0] = 0.0
        x[1] = 0.5
        x[2] = -0.5
        x[3] = 1e-6
        x[3, 7] = 8.0
        qws = [torch.rand(k) * 4.0 + 0.05]
        if qtype not in NEEDS_IMATRIX:
            qws.append(None)
        for qw in qws:
            print(f"{mod}.{fn} {rows}x{k} imat={qw is not None}", flush=True)
            args = (x,) if not takes_qw else (x, qw)
            cpu = f(*args)
            gpu = f(x.to(dev), None if qw is None else qw.to(dev)) if takes_qw else f(x.to(dev))
            assert cpu.device.type == "cpu" and gpu.device == dev
            assert torch.equal(cpu, gpu.cpu()), (mod, rows, k)
            ref = oracle.quantize(qtype, x.numpy(), qw.numpy() if (qw is not None and spec.uses_imatrix)
                                  else None, n_threads=NTHREADS)
            assert np.array_equal(cpu.numpy(), ref), (mod, rows, k, qw is None)
