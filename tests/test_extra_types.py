"""Q4_1, Q5_0, Q5_1, Q8_0 and IQ4_NL: the ggml formats the reference has no
quantizer for (its command line stops on them, quant-studio.py:396-399).

There is no reference output to compare with, so the oracle is pinned by what
the formats and ggml's reference quantizers fix:
  - known answers: blocks lying exactly on a format's grid come back exactly,
    and the rounding rule of each format shows on chosen half-way values
    (Q8_0 rounds half away from zero, the others truncate after +0.5/+16.5);
  - dequantisation bounds on random data: every value within half a step of
    its reconstruction (plus the fp16 rounding of d and m);
  - special blocks: all-zero and constant blocks;
  - IQ4_NL's block search is the IQ4_XS one that the reference's golden
    vectors pin; here its levels must be the nearest LUT entries at 1/d.
The GPU tests (marked gpu) then require the HIP kernels to match the oracle
byte for byte, through the C ABI."""

from __future__ import annotations

import os

import numpy as np
import pytest

import dequant
import oracle

EXTRA = {"q4_1": (3, 20), "q5_0": (6, 22), "q5_1": (7, 24), "q8_0": (8, 34), "iq4_nl": (20, 18)}
NTHREADS = min(16, len(os.sched_getaffinity(0)))


def f16(v):
    return np.float64(np.float32(v).astype(np.float16))


def quant(qtype, x, qw=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    return oracle.quantize(qtype, x, qw, n_threads=NTHREADS)


def blocks(q, qtype):
    return q.reshape(-1, EXTRA[qtype][1])


def test_row_bytes():
    for qtype, (_, nb) in EXTRA.items():
        assert oracle.row_bytes(qtype, 64) == 2 * nb


# ---------------------------------------------------------------- known answers

def test_q8_0_grid_block_and_half_away_rounding():
    k = np.arange(-127, 128, 8, dtype=np.float32)            # 32 values, -127 .. 121
    x = np.concatenate([k[:31], [127.0]]).astype(np.float32) * np.float32(0.25)
    q = blocks(quant("q8_0", x[None]), "q8_0")[0]
    assert q[:2].view(np.float16)[0] == np.float16(0.25)
    assert np.array_equal(q[2:].view(np.int8), np.concatenate([k[:31], [127]]).astype(np.int8))
    # d = 127/127 = 1: 2.5 -> 3, -2.5 -> -3, 3.5 -> 4 (half away; half-even gives 2, -2, 4)
    y = np.zeros(32, np.float32)
    y[:4] = [127.0, 2.5, -2.5, 3.5]
    q = blocks(quant("q8_0", y[None]), "q8_0")[0]
    assert q[2:6].view(np.int8).tolist() == [127, 3, -3, 4]


@pytest.mark.parametrize("qtype,nmax", [("q4_1", 15), ("q5_1", 31)])
def test_q_1_grid_block(qtype, nmax):
    d, m = 0.125, -1.5
    L = np.arange(32) % (nmax + 1)
    L[:2] = [0, nmax]                                        # min and max present
    x = (m + d * L).astype(np.float32)
    q = quant(qtype, x[None])
    xh = dequant.dequantize(qtype, q, 1)[0]
    assert np.array_equal(xh, x.astype(np.float64))
    b = blocks(q, qtype)[0]
    assert b[:2].view(np.float16)[0] == np.float16(d) and b[2:4].view(np.float16)[0] == np.float16(m)


def test_q4_1_truncates_after_half():
    # min 0, max 15 -> d = 1: 2.49 -> 2, 2.5 -> 3 (trunc(2.5 + 0.5)), 2.51 -> 3
    x = np.zeros(32, np.float32)
    x[:4] = [15.0, 2.49, 2.5, 2.51]
    b = blocks(quant("q4_1", x[None]), "q4_1")[0]
    lo = b[4:20] & 15
    assert lo[:4].tolist() == [15, 2, 3, 3]


def test_q5_0_grid_block_and_rounding():
    s = 0.0625
    k = np.arange(-16, 16)
    x = (k * s).astype(np.float32)                           # max |x| at -16s -> d = s
    q = quant("q5_0", x[None])
    assert np.array_equal(dequant.dequantize("q5_0", q, 1)[0], x.astype(np.float64))
    b = blocks(q, "q5_0")[0]
    assert b[:2].view(np.float16)[0] == np.float16(s)
    # d = -16/-16 = 1: floor(2.5 + 16.5) = 19 -> 3, floor(-2.5 + 16.5) = 14 -> -2, 2.49 -> 2
    y = np.zeros(32, np.float32)
    y[:4] = [-16.0, 2.5, -2.5, 2.49]
    xh = dequant.dequantize("q5_0", quant("q5_0", y[None]), 1)[0]
    assert xh[:4].tolist() == [-16.0, 3.0, -2.0, 2.0]


def test_iq4_nl_grid_block():
    lut = dequant.IQ4NL
    d = 2.0 ** -9
    x = (np.concatenate([lut, lut[::-1]]) * d).astype(np.float32)
    q = quant("iq4_nl", x[None])
    b = blocks(q, "iq4_nl")[0]
    assert b[:2].view(np.float16)[0] == np.float16(d)
    assert np.array_equal(dequant.dequantize("iq4_nl", q, 1)[0], x.astype(np.float64))


# ---------------------------------------------------------------- special blocks

def test_zero_and_constant_blocks():
    z = np.zeros((1, 32), np.float32)
    for qtype in ("q4_1", "q5_1", "q8_0"):
        assert not quant(qtype, z).any(), qtype
    b = blocks(quant("q5_0", z), "q5_0")[0]                  # d = 0 / -16 = -0.0, L = 16
    assert b[:2].tolist() == [0x00, 0x80] and b[2:6].tolist() == [0xFF] * 4 and not b[6:].any()
    b = blocks(quant("iq4_nl", z), "iq4_nl")[0]              # d = 0; levels of 0 -> LUT entry 1
    assert not b[:2].any() and (b[2:] == 0x88).all()
    c = np.full((1, 32), 0.3, np.float32)
    for qtype in ("q4_1", "q5_1"):                          # d = 0, m = c
        xh = dequant.dequantize(qtype, quant(qtype, c), 1)[0]
        assert np.all(xh == f16(0.3)), qtype


# ---------------------------------------------------------------- bounds on random data

def _random(rows=64, k=512, seed=0):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((rows, k)) * 0.02 * np.exp(0.5 * rng.standard_normal((rows, 1)))
    a.reshape(-1)[rng.choice(a.size, a.size // 500, replace=False)] *= 20
    return a.astype(np.float32)


@pytest.mark.parametrize("qtype", ["q4_1", "q5_0", "q5_1", "q8_0"])
def test_every_value_within_half_a_step(qtype):
    """|x - xhat| <= d/2, plus the fp16 rounding of d (times the largest level)
    and of m; Q5_0's d = max / -16 (max: first value of largest |x|) clips
    values of the other sign near -max at level 31 (15 d), the format's
    asymmetry, which the bound allows for exactly those values."""
    x = _random(seed=EXTRA[qtype][0])
    q = quant(qtype, x)
    xh = dequant.dequantize(qtype, q, x.shape[0]).reshape(-1, 32)
    xb = x.astype(np.float64).reshape(-1, 32)
    b = blocks(q, qtype)
    d16 = np.abs(b[:, :2].copy().view(np.float16).astype(np.float64)[:, 0])
    clip = np.zeros_like(xb)
    if qtype in ("q4_1", "q5_1"):
        nmax = 15 if qtype == "q4_1" else 31
        d = (xb.max(1) - xb.min(1)) / nmax
        m = xb.min(1)
        slack = np.abs(m - f16(m.astype(np.float32))) + nmax * np.abs(d - d16)
    elif qtype == "q5_0":
        mx = np.take_along_axis(xb, np.abs(xb).argmax(1)[:, None], 1)[:, 0]
        ds = mx / -16
        d = np.abs(ds)
        slack = 16 * np.abs(d - d16)
        t = xb / np.where(ds == 0, 1, ds)[:, None] + 16.5
        clip = np.abs(xb - 15 * ds[:, None]) * (t >= 32)
    else:
        d = np.abs(xb).max(1) / 127
        slack = 127 * np.abs(d - d16)
    bound = 0.5 * d[:, None] * (1 + 1e-5) + slack[:, None] + clip + 1e-12
    assert (np.abs(xb - xh) <= bound).all()
    if qtype == "q5_0":
        assert 0 < (clip > 0).sum() < 0.01 * clip.size   # the clipping case occurs, rarely


def test_iq4_nl_levels_are_nearest_lut_entries_and_error_level():
    rng = np.random.default_rng(5)
    x = _random(seed=7)
    qw = rng.lognormal(0, 1, x.shape[1]).astype(np.float32)
    for w in (None, qw):
        q = quant("iq4_nl", x, w)
        b = blocks(q, "iq4_nl")
        d = b[:, :2].copy().view(np.float16).astype(np.float32)[:, 0]
        # levels: nearest LUT entry of x / d (at the f32 scale; the fp16 d only
        # differs in the last bits, so compare with a margin at the midpoints)
        L = np.concatenate([b[:, 2:] & 15, b[:, 2:] >> 4], 1).astype(np.int64)
        normal = np.abs(d) >= 2.0 ** -14                  # fp16 d with full precision
        assert normal.mean() > 0.9
        al = x.reshape(-1, 32)[normal] / d[normal, None]
        dist = np.abs(al[:, :, None] - dequant.IQ4NL[None, None, :])
        best = dist.min(-1)
        got = np.take_along_axis(dist, L[normal][:, :, None], -1)[:, :, 0]
        assert (got <= best + 1e-2 * (1 + np.abs(al))).all()
        xh = dequant.dequantize("iq4_nl", q, x.shape[0])
        rel = np.sqrt(((x - xh) ** 2).mean() / (x.astype(np.float64) ** 2).mean())
        assert rel < 0.12, rel


def test_iq4_nl_uses_the_imatrix():
    x = _random(seed=3)
    qw = np.random.default_rng(1).lognormal(0, 1, x.shape[1]).astype(np.float32)
    assert not np.array_equal(quant("iq4_nl", x), quant("iq4_nl", x, qw))


# ---------------------------------------------------------------- GPU parity

@pytest.fixture(scope="module")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return torch.device("cuda:0")


def _hip(qs, qtype, x, qw, dev, dtype="bf16"):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    t = {"bf16": t.to(torch.bfloat16), "f16": t.to(torch.float16), "f32": t}[dtype].to(dev)
    q = None if qw is None else torch.from_numpy(qw).to(dev)
    out = qs.quantize(EXTRA[qtype][0], t, q)
    torch.cuda.synchronize()
    ref_x = t.float().cpu().numpy()
    return out.cpu().numpy(), ref_x


@pytest.mark.gpu
@pytest.mark.parametrize("qtype", sorted(EXTRA))
@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_gpu_matches_oracle(qs, dev, qtype, dtype):
    x = _random(rows=257, k=1024, seed=EXTRA[qtype][0] + 11)
    x[0, :32] = 0.0                                        # zero block
    x[1, :32] = 0.3                                        # constant block
    x[2, :32] = -0.0
    x[3, :32] = np.float32(1e-30) * np.arange(32)          # tiny values
    qw = np.random.default_rng(2).lognormal(0, 1, 1024).astype(np.float32)
    for w in (None, qw):
        print(f"{qtype} {dtype} imat={w is not None} 257x1024", flush=True)
        got, xr = _hip(qs, qtype, x, w, dev, dtype)
        ref = quant(qtype, xr, w if qtype == "iq4_nl" else None)
        same = (blocks(got, qtype) == blocks(ref, qtype)).all(1)
        assert same.all(), f"{int((~same).sum())}/{same.size} blocks differ"


@pytest.mark.gpu
@pytest.mark.parametrize("qtype", sorted(EXTRA))
def test_gpu_row_stride_chunking_and_unaligned_output(qs, dev, qtype):
    import torch
    x = _random(rows=40, k=1024, seed=21)
    qw = np.random.default_rng(4).lognormal(0, 1, 1024).astype(np.float32)
    wide = torch.zeros((40, 1024 + 64), dtype=torch.bfloat16, device=dev)
    wide[:, :1024] = torch.from_numpy(x).to(torch.bfloat16).to(dev)
    view = wide[:, :1024]
    tid, nb = EXTRA[qtype]
    rb = nb * 32
    buf = torch.zeros(40 * rb + 3, dtype=torch.uint8, device=dev)
    out = buf[1:1 + 40 * rb]
    q = torch.from_numpy(qw).to(dev)
    qs.quantize(tid, view, q, out=out)
    parts = torch.cat([qs.quantize(tid, view[a:b], q) for a, b in ((0, 3), (3, 40))])
    torch.cuda.synchronize()
    xr = view.float().cpu().numpy()
    ref = quant(qtype, xr, qw if qtype == "iq4_nl" else None)
    b = buf.cpu().numpy()
    assert b[0] == 0 and b[-2:].tolist() == [0, 0]
    assert np.array_equal(b[1:1 + 40 * rb].reshape(40, rb), ref)
    assert np.array_equal(parts.cpu().numpy(), ref)


# ------------------------------------------- ulp-level pin: a second restatement

def _pin_inputs() -> np.ndarray:
    """131,072 blocks of 32: normal, uniform, heavy-tailed and bf16-rounded
    values at scales 1e-30 .. 1e4; exact half-way values of every format's
    rounding; zero, constant, one-signed, subnormal and tied-absmax blocks."""
    rng = np.random.default_rng(11)
    n = 1 << 17
    scale = np.exp(rng.uniform(np.log(1e-30), np.log(1e4), (n, 1)))
    kind = rng.integers(0, 4, (n, 1))
    v = np.where(kind == 0, rng.standard_normal((n, 32)),
                 np.where(kind == 1, rng.uniform(-1, 1, (n, 32)),
                          np.where(kind == 2, rng.standard_t(3, (n, 32)),
                                   rng.standard_normal((n, 32)) + 3.0)))
    x = (v * scale).astype(np.float32)
    bf = rng.random(n) < 0.5                                  # half of them bf16 values
    x[bf] = (x[bf].view(np.uint32) & np.uint32(0xffff0000)).view(np.float32)
    # half-way cases: d = 1 (Q8_0 absmax 127; Q4_1/Q5_1 range nmax), values at k + 1/2
    half = (rng.integers(-126, 126, (512, 32)) + 0.5).astype(np.float32)
    half[:, 0] = 127.0
    x[:512] = half
    r15 = (rng.integers(0, 15, (512, 32)) + 0.5).astype(np.float32)
    r15[:, 0], r15[:, 1] = 0.0, 15.0
    x[512:1024] = r15
    # Q5_0: d = -absmax/16 = 1 when the absmax is -16: x = k - 16.5 + ... lands on .5 after +16.5
    r16 = (rng.integers(-15, 15, (512, 32)) + 0.5).astype(np.float32)
    r16[:, 3] = -16.0
    x[1024:1536] = r16
    x[1536] = 0.0
    x[1537] = 0.37
    x[1538] = -0.0
    x[1539] = np.abs(x[1539])
    x[1540] = rng.integers(1, 1 << 23, 32).astype(np.uint32).view(np.float32)   # subnormals
    x[1541, :] = 1.0
    x[1541, 7] = -1.0                                         # tied |absmax|: first index wins
    return x


@pytest.mark.parametrize("qtype,imat", [("q4_1", False), ("q5_0", False), ("q5_1", False),
                                        ("q8_0", False), ("iq4_nl", False), ("iq4_nl", True)])
def test_oracle_matches_numpy_restatement_bit_for_bit(qtype, imat):
    """The oracle against an independent numpy restatement of the same
    formats, byte for byte on 131,072 blocks (the square root of IQ4_NL's
    weights taken as IEEE by both)."""
    import extra_types_np
    x = _pin_inputs().reshape(-1, 256)
    qw = np.random.default_rng(3).lognormal(0, 1, 256).astype(np.float32) if imat else None
    want = extra_types_np.quantize(qtype, x, qw)
    oracle.use_ieee_sqrt(True)
    try:
        got = quant(qtype, x, qw)
    finally:
        oracle.use_ieee_sqrt(False)
    diff = ~(blocks(got, qtype) == blocks(want, qtype)).all(1)
    assert not diff.any(), f"{int(diff.sum())} of {diff.size} blocks differ (first {np.nonzero(diff)[0][:5]})"


# planted division slips in the oracle and the types whose pin must catch them
DIVISION_SLIPS = {7: ("d = a * (1/n) instead of a / n", ["q4_1", "q5_1", "q8_0"]),
                  8: ("x / d instead of x * (1/d)", ["q4_1", "q5_0", "q5_1", "q8_0", "iq4_nl"])}


@pytest.mark.parametrize("mut", sorted(DIVISION_SLIPS))
def test_numpy_pin_catches_division_slips(mut):
    import extra_types_np
    what, types = DIVISION_SLIPS[mut]
    x = _pin_inputs().reshape(-1, 256)    # IQ4_NL's reprojection shows slip 8 in 1 block of them
    L = oracle.lib()
    L.qso_set_mutation(mut)
    try:
        for qtype in types:
            got = quant(qtype, x)
            want = extra_types_np.quantize(qtype, x)
            assert not np.array_equal(got, want), f"slip '{what}' not caught for {qtype}"
    finally:
        L.qso_set_mutation(0)
