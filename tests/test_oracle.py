"""CPU tests that pin the oracle before anything is checked against it.

- every supported type against the golden vectors the reference itself wrote
  (tests/golden/gen_golden.py imports the reference's kernels/*.py and runs
  its eager CPU quantizers);
- the reduction orders against torch's own CPU reductions (the runtime the
  reference's eager path runs on), the fp16 conversion against numpy;
- closed-form known answers for Q4_0, and planted mistakes in the oracle
  (wrong division form, sum order, rounding, accept test, a dropped
  candidate) that the golden vectors must each expose.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from golden_data import (ORACLE_TYPES, TYPES, block_identical, cases, clean_blocks, nonfinite_case,
                         zero_imatrix_cases)


@pytest.mark.parametrize("qtype", ORACLE_TYPES)
def test_oracle_matches_reference_golden(qtype):
    """The oracle (with its tabulated reproduction of torch's CPU square root)
    reproduces every golden block of every type."""
    for key, x, qw, expect in cases(qtype):
        got = oracle.quantize(qtype, x, qw, n_threads=4)
        same = block_identical(got, expect, qtype)
        assert same.all(), f"{qtype} {key}: {int((~same).sum())} of {same.size} blocks differ"


ZERO_IMATRIX_TYPES = [t for t in ORACLE_TYPES if t != "q4_0"]


@pytest.mark.parametrize("qtype", ZERO_IMATRIX_TYPES)
def test_oracle_matches_reference_zero_imatrix(qtype):
    """Imatrix vectors with zero entries (columns that never fired, whole 8-,
    16-, 32- and 256-value groups, an all-zero vector): the oracle reproduces
    every block the reference's eager quantizers wrote for them."""
    got_any = False
    for case, x, qw, expect in zero_imatrix_cases(qtype):
        assert (qw == 0).any() and (qw >= 0).all()
        got = oracle.quantize(qtype, x, qw, n_threads=4)
        same = block_identical(got, expect, qtype)
        assert same.all(), f"{qtype} {case}: {int((~same).sum())} of {same.size} blocks differ"
        got_any = True
    assert got_any


# planted mistakes that only zero weights expose, and the (type, case) pairs
# of the zero-imatrix vectors that must each expose them; the first set of
# golden vectors (strictly positive imatrix) misses 10-12 entirely and
# catches 9 only for the IQ3 types
ZERO_MUTANTS = {
    9: ("neighbour search keeps the last of equal distances",
        [("iq2_xxs", "zsub8"), ("iq2_xs", "zsub8"), ("iq2_s", "zsub8"), ("iq3_xxs", "zsub8"),
         ("iq3_s", "zall")]),
    10: ("make_qp accepts an equal error", [("q2_k", "zall"), ("q4_k", "zgroups"), ("q5_k", "zgroups")]),
    11: ("make_qx's first scale without its zero guard", [("q3_k", "zgroups"), ("q6_k", "zsub8")]),
    12: ("IQ2_XXS active without scale0*3 > 0", [("iq2_xxs", "zgroups"), ("iq2_xxs", "zsub8")]),
}


@pytest.mark.parametrize("mut", sorted(ZERO_MUTANTS))
def test_zero_imatrix_vectors_catch_planted_mistake(mut):
    what, pairs = ZERO_MUTANTS[mut]
    L = oracle.lib()
    L.qso_set_mutation(mut)
    try:
        for qtype, want in pairs:
            hit = [c for c in zero_imatrix_cases(qtype) if c[0] == want]
            assert hit, (qtype, want)
            case, x, qw, expect = hit[0]
            got = oracle.quantize(qtype, x, qw, n_threads=4)
            assert not block_identical(got, expect, qtype).all(), \
                f"planted mistake '{what}' not detected by {qtype} {case}"
    finally:
        L.qso_set_mutation(0)


def test_nonfinite_inputs_match_the_reference_on_every_finite_block():
    """Rows holding NaN, +-Inf and +-1e38 (whose squares overflow): the
    reference's quantizers raise on them for Q3_K, Q6_K and IQ2_XXS and
    otherwise follow torch's NaN propagation (argmax takes a NaN as the
    maximum), which the oracle and the kernels do not reproduce. Every block
    whose own values are finite and below 1e18 still matches the reference's
    bytes, and Q4_0's NaN and Inf blocks too (a NaN is the block's absmax, as
    torch's argmax takes it); the oracle returns bytes for every type."""
    x, qw, ref = nonfinite_case()
    assert {k.split(".")[0] for k in ref} == set(ORACLE_TYPES) - {"q3_k", "q6_k", "iq2_xxs"}
    n_clean = 0
    for key, expect in sorted(ref.items()):
        qtype, mode = key.split(".")
        clean = clean_blocks(x, TYPES[qtype][1])
        got = oracle.quantize(qtype, x, qw if mode == "imat" else None, n_threads=4)
        same = block_identical(got, expect, qtype)
        assert same[clean].all(), f"{key}: {int((clean & ~same).sum())} finite blocks differ"
        assert (~clean).any() and clean.any()
        if qtype == "q4_0":
            assert same.all(), f"q4_0: {int((~same).sum())} non-finite blocks differ"
        n_clean += int(clean.sum())
    for qtype in ("q3_k", "q6_k", "iq2_xxs"):
        assert oracle.quantize(qtype, x, qw, n_threads=4).shape[0] == x.shape[0]
    assert n_clean >= 300


# non-finite blocks (of 12 per case) whose bytes equal the reference's: the IQ
# searches whose distances are all +inf or NaN take torch's argmin, the first
# NaN else the first entry (a search returning "no index" matched 0 of IQ3_S's
# imatrix blocks); the rest differ where torch's NaN propagation elsewhere
# (max, round, clamp, integer casts of NaN) is not reproduced
NONFINITE_SAME = {"iq2_s.imat": 7, "iq2_xs.imat": 7, "iq3_s.imat": 7, "iq3_s.none": 1,
                  "iq3_xxs.imat": 7, "iq3_xxs.none": 7, "iq4_xs.imat": 0, "iq4_xs.none": 0,
                  "q2_k.imat": 2, "q2_k.none": 6, "q4_k.imat": 2, "q4_k.none": 6,
                  "q5_k.imat": 2, "q5_k.none": 6, "q4_0.none": 18}


def test_nonfinite_blocks_equal_to_the_reference():
    x, qw, ref = nonfinite_case()
    assert set(ref) == set(NONFINITE_SAME)
    for key, expect in sorted(ref.items()):
        qtype, mode = key.split(".")
        clean = clean_blocks(x, TYPES[qtype][1])
        got = oracle.quantize(qtype, x, qw if mode == "imat" else None, n_threads=4)
        same = block_identical(got, expect, qtype)
        assert int(same[~clean].sum()) >= NONFINITE_SAME[key], f"{key}: {int(same[~clean].sum())}"


@pytest.mark.parametrize("qtype", ["q4_k", "iq2_s", "iq3_xxs"])
def test_tabulated_sqrt_equals_live_torch_sqrt_in_the_oracle(qtype):
    """Calling torch.sqrt live from the oracle gives the same bytes as the table."""
    key, x, qw, expect = cases(qtype)[0]
    base = oracle.quantize(qtype, x, qw, n_threads=1)
    oracle.use_torch_sqrt(True)
    try:
        live = oracle.quantize(qtype, x, qw, n_threads=1)
    finally:
        oracle.use_torch_sqrt(False)
    assert np.array_equal(base, live)


def test_tabulated_sqrt_matches_torch_on_random_inputs():
    """qso_sqrt_ref == torch.sqrt (CPU) bit for bit: random positive normals and
    subnormals, powers of 4 apart, and the special values."""
    rng = np.random.default_rng(11)
    bits = np.concatenate([rng.integers(0x00800000, 0x7f800000, 200_000, dtype=np.uint32),
                           rng.integers(1, 0x00800000, 20_000, dtype=np.uint32)])
    x = bits.view(np.float32)
    x = np.concatenate([x, x[:1000] * np.float32(4.0), x[:1000] * np.float32(0.25),
                        np.array([0.0, -0.0, np.inf, -1.0, np.nan], np.float32)])
    want = torch.sqrt(torch.from_numpy(x)).numpy()
    got = np.array([oracle.sqrt_ref(v) for v in x], np.float32)
    assert np.array_equal(got.view(np.uint32)[:-2], want.view(np.uint32)[:-2])
    assert np.isnan(got[-2]) and np.isnan(got[-1])


@pytest.mark.parametrize("qtype", ["iq2_s"])
def test_ieee_sqrt_would_change_a_golden_block(qtype):
    """Why the table exists: with IEEE sqrtf instead of torch's rounding, one
    golden IQ2_S block (an exact tie in the sweep's accept test) differs."""
    oracle.use_ieee_sqrt(True)
    try:
        diff = 0
        for key, x, qw, expect in cases(qtype):
            diff += int((~block_identical(oracle.quantize(qtype, x, qw, n_threads=4), expect, qtype)).sum())
    finally:
        oracle.use_ieee_sqrt(False)
    assert diff >= 1


def test_torch_cpu_sqrt_is_not_correctly_rounded():
    """torch.sqrt on CPU returns one ulp below the correctly rounded root for
    some inputs (the set the table holds)."""
    v = np.array([0.019531157], np.float32)
    assert np.sqrt(v)[0] == np.float32(0.13975392)
    assert torch.sqrt(torch.from_numpy(v)).numpy()[0] == np.float32(0.13975391)
    assert oracle.sqrt_ref(v[0]) == np.float32(0.13975391)


@pytest.mark.parametrize("n", [8, 16, 32, 256])
def test_cascade8_is_torch_row_sum(n):
    rng = np.random.default_rng(n)
    rows = rng.standard_normal((2000, n)).astype(np.float32)
    rows[::7] *= rng.lognormal(0, 3, (rows[::7].shape[0], 1)).astype(np.float32)
    rows[::11] = np.abs(rows[::11]) ** 3
    ref = torch.from_numpy(rows).sum(-1).numpy()
    got = np.array([oracle.sum_cascade8(r) for r in rows], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("n", [16, 32])
def test_tree_sum_is_adjacent_pairs(n):
    rng = np.random.default_rng(5)
    for _ in range(500):
        v = rng.standard_normal(n).astype(np.float32) * np.float32(rng.lognormal(0, 2))
        t = v.copy()
        while t.size > 1:
            t = (t[0::2] + t[1::2]).astype(np.float32)
        assert oracle.sum_tree(v) == t[0]


def test_f16_round_to_nearest_even():
    rng = np.random.default_rng(3)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(1e-3),
        rng.standard_normal(4000).astype(np.float32) * np.float32(1e-6),   # f16 subnormal range
        rng.standard_normal(2000).astype(np.float32) * np.float32(3e4),
        # exact ties between two f16 neighbours (normal and subnormal)
        (np.arange(1, 1000, dtype=np.float32) * np.float32(2.0 ** -11) + np.float32(2.0 ** -12)),
        (np.arange(1, 1000, dtype=np.float32) * np.float32(2.0 ** -24) + np.float32(2.0 ** -25)),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e-8, -2.0 ** -25, 2.0 ** -24], np.float32),
    ])
    ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16_bits(v) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)


def test_python_float_over_tensor_is_reciprocal_multiply():
    """torch evaluates `c / t` (c a Python float) as t.reciprocal() * c, which the
    oracle's RDIV restates; on these inputs it differs from IEEE c / t."""
    rng = np.random.default_rng(11)
    t = (rng.standard_normal(20000) * 3).astype(np.float32)
    for c in (63.0, -32.0, -128.0, 4.0, 15.0, -4.1, 31.9):
        got = (c / torch.from_numpy(t)).numpy()
        recip = (np.float32(1.0) / t).astype(np.float32) * np.float32(c)
        ieee = (np.float32(c) / t).astype(np.float32)
        assert np.array_equal(got.view(np.uint32), recip.view(np.uint32))
        if np.log2(abs(c)) % 1:   # a power-of-two c scales exactly: both forms agree
            assert not np.array_equal(got.view(np.uint32), ieee.view(np.uint32))


def test_q4_0_known_answer():
    # block [-8..7]*s: max |x| is -8s (first), d = -8s/-8 = s, levels x/s + 8
    s = np.float32(0.125)
    x = (np.arange(-8, 8, dtype=np.float32) * s)
    x = np.concatenate([x, x])[None, :]
    out = oracle.quantize("q4_0", x)[0]
    assert out[:2].view(np.float16)[0] == np.float16(s)
    q = np.concatenate([np.arange(16), np.arange(16)])
    assert np.array_equal(out[2:], (q[:16] | (q[16:] << 4)).astype(np.uint8))


def test_q4_0_all_zero_block():
    out = oracle.quantize("q4_0", np.zeros((1, 32), np.float32))[0]
    # d = 0 / -8.0 = -0.0 (fp16 0x8000), id = 0, every level floor(0*0 + 8.5) = 8
    assert out[:2].tolist() == [0x00, 0x80] and (out[2:] == 0x88).all()


# planted mistakes in the oracle (qso_set_mutation) and a type whose golden
# vectors must expose each one
MUTANTS = {
    1: ("rdiv as IEEE division", ["q3_k", "q6_k", "iq4_xs"]),
    2: ("sequential sum for torch .sum(-1)", ["q4_k", "q2_k", "iq4_xs"]),
    3: ("sequential sum for tree_sum", ["q4_k", "q5_k", "q2_k"]),
    4: ("last make_qkx candidate dropped", ["q4_k", "q5_k", "q2_k"]),
    5: ("round half away from zero", ["q4_k", "q3_k", "q6_k"]),
    6: ("make_qx accept with >=", ["q6_k", "q3_k"]),
}


@pytest.mark.parametrize("mut", sorted(MUTANTS))
def test_golden_vectors_catch_planted_mistake(mut):
    what, types = MUTANTS[mut]
    L = oracle.lib()
    L.qso_set_mutation(mut)
    try:
        for qtype in types:
            caught = False
            for key, x, qw, expect in cases(qtype):
                got = oracle.quantize(qtype, x, qw, n_threads=4)
                if not block_identical(got, expect, qtype).all():
                    caught = True
                    break
            assert caught, f"planted mistake '{what}' not detected by {qtype} golden vectors"
    finally:
        L.qso_set_mutation(0)


def _sqrt_down_keys() -> np.ndarray:
    """The map's keys (parity << 23 | mantissa), from the generated header."""
    import re
    from pathlib import Path
    txt = (Path(__file__).resolve().parents[1] / "quant-studio_amd" / "csrc" / "qs_sqrt_table.h").read_text()
    gaps = np.array([int(v) for v in re.findall(r"\d+", txt[txt.index("{") + 1: txt.rindex("}")])], np.int64)
    return np.cumsum(gaps)


def _near_midpoint(v: np.ndarray) -> np.ndarray:
    """sqrt_near_midpoint of qs_device.h, op for op in float32: the remainder
    v - r^2 (exact, as the kernels' fma gives it) against -0.875 r ulp(r)."""
    r = np.sqrt(v)
    rem64 = v.astype(np.float64) - r.astype(np.float64) ** 2
    rem = rem64.astype(np.float32)
    ulp = (((r.view(np.uint32) & np.uint32(0x7f800000)) - np.uint32(23 << 23))).view(np.float32)
    lim = (np.float32(-0.875) * r) * ulp
    return (rem < lim) | (v.view(np.uint32) < np.uint32(0x17800000)), rem64, rem


def test_sqrt_map_is_read_for_every_listed_input():
    """The kernels read the square-root map only for inputs whose root lies
    within 1/16 ulp of the midpoint below the IEEE root: every one of the 2^24
    key classes in [1, 4) that the map lists passes that test, also scaled by
    powers of 4 down to the tiny-input cutoff and up to the largest floats, and
    about 6% of all inputs do."""
    keys = _sqrt_down_keys()
    m = np.arange(1 << 23, dtype=np.uint32)
    x = np.concatenate([(127 << 23) | m, (128 << 23) | m]).astype(np.uint32).view(np.float32)
    near, rem64, rem = _near_midpoint(x)
    assert np.array_equal(rem.astype(np.float64), rem64)        # the remainder is exact in f32
    assert near[keys].all()
    assert 0.061 < near.mean() < 0.064
    xd = x[keys]
    for k in (-45, -41, -40, -20, -3, -1, 1, 7, 30, 62):
        xs = (xd.astype(np.float64) * 4.0 ** k).astype(np.float32)
        assert np.isfinite(xs).all() and (xs > 0).all()
        assert _near_midpoint(xs)[0].all(), k
