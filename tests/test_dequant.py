"""CPU tests of the dequantizers (tests/dequant.py) and of the weighted-MSE
tie rule on the reference's golden vectors.

The dequantizers are pinned by what the formats force: on the reference's own
golden bytes every type reconstructs its input with the error level of its bit
width, the least-squares gain of the input on the reconstruction is ~1 (a
wrong scale, nibble order or sign convention breaks one of these), and large
values keep their sign. Q4_0 also has a closed-form known answer."""

from __future__ import annotations

import numpy as np
import pytest

import dequant
import oracle
from golden_data import TYPES, as_f32, block_identical, cases

# relative RMSE bound per type on the ffn-like ("normal") golden case (measured error x ~1.3)
REL_RMSE_MAX = {"q4_0": 0.15, "q2_k": 0.37, "q3_k": 0.21, "q4_k": 0.11, "q5_k": 0.055,
                "q6_k": 0.03, "iq4_xs": 0.125, "iq2_xxs": 0.62, "iq2_xs": 0.52, "iq2_s": 0.46,
                "iq3_xxs": 0.30, "iq3_s": 0.27}
# gain of x on xhat, weighted like the quantizers' objective; the IQ formats
# reconstruct a few percent large by design (grid magnitudes 8/25/43 for levels
# 1/3/5 x 8, d x 1.0125 / 1.033 for IQ3)
GAIN = {t: (0.99, 1.01) for t in TYPES} | {"iq2_xxs": (0.9, 0.97), "iq2_xs": (0.9, 0.97),
                                           "iq2_s": (0.92, 0.98), "iq3_xxs": (0.93, 0.99),
                                           "iq3_s": (0.93, 0.99), "q2_k": (0.96, 1.01)}


@pytest.mark.parametrize("qtype", sorted(TYPES))
def test_dequantized_golden_bytes_reconstruct_the_input(qtype):
    for key, x, qw, expect in cases(qtype):
        if not key.startswith("normal"):
            continue
        xf = as_f32(x).astype(np.float64)
        xh = dequant.dequantize(qtype, expect, xf.shape[0])
        assert np.isfinite(xh).all()
        rel = np.sqrt(((xf - xh) ** 2).mean() / (xf ** 2).mean())
        assert rel < REL_RMSE_MAX[qtype], f"{key}: relative RMSE {rel:.4f}"
        w = np.ones(xf.shape[1]) if qw is None else qw[: xf.shape[1]].astype(np.float64)
        w = w[None, :] * np.sqrt(2 * (xf ** 2).mean(1, keepdims=True) + xf ** 2)
        gain = (w * xf * xh).sum() / (w * xh * xh).sum()
        lo, hi = GAIN[qtype]
        assert lo <= gain <= hi, f"{key}: gain {gain:.4f}"
        big = np.abs(xf) > 2.5 * xf.std()
        assert (np.sign(xh[big]) == np.sign(xf[big])).mean() > 0.99


def test_q4_0_known_answer():
    # d = -8 * ... : block [-8..7] * 0.5 packs to d = 0.5 (the max-magnitude value is -4 = -8d)
    x = (np.arange(-8, 8, dtype=np.float32) * 0.5).repeat(2)
    q = oracle.quantize("q4_0", x[None, :], None)
    np.testing.assert_array_equal(dequant.dequantize("q4_0", q, 1)[0], x.astype(np.float64))


@pytest.mark.parametrize("qtype", sorted(TYPES))
def test_tie_rule_on_golden_vectors(qtype):
    """Blocks that differ from the reference's bytes must not have a larger
    imatrix-weighted squared error. The oracle (which the GPU matches bit for
    bit) differs on no golden block, so the rule holds trivially; with plain
    IEEE sqrt it would not (one IQ2_S block, see test_oracle.py)."""
    for key, x, qw, expect in cases(qtype):
        xf = as_f32(x)
        got = oracle.quantize(qtype, xf, qw, n_threads=4)
        diff = ~block_identical(got, expect, qtype)
        if diff.any():
            e_got = dequant.block_weighted_mse(qtype, got, xf, qw)
            e_ref = dequant.block_weighted_mse(qtype, expect, xf, qw)
            assert (e_got[diff] <= e_ref[diff]).all(), f"{key}: {np.nonzero(diff)[0]}"


def test_ieee_sqrt_block_has_larger_weighted_error():
    """The one golden block IEEE sqrt would change is not a tie in the rule's
    sense: its weighted error is larger than the reference's -- why the kernels
    reproduce torch's square root instead."""
    oracle.use_ieee_sqrt(True)
    try:
        worse = 0
        for key, x, qw, expect in cases("iq2_s"):
            xf = as_f32(x)
            got = oracle.quantize("iq2_s", xf, qw, n_threads=4)
            diff = ~block_identical(got, expect, "iq2_s")
            if diff.any():
                e_got = dequant.block_weighted_mse("iq2_s", got, xf, qw)[diff]
                e_ref = dequant.block_weighted_mse("iq2_s", expect, xf, qw)[diff]
                worse += int((e_got > e_ref).sum())
    finally:
        oracle.use_ieee_sqrt(False)
    assert worse >= 1
