"""An independent numpy restatement of the five formats the reference has no
module for (Q4_1, Q5_0, Q5_1, Q8_0, IQ4_NL), vectorised over blocks, one
float32 operation per step of ggml's reference quantizers
(quantize_row_q4_1_ref / _q5_0_ref / _q5_1_ref / _q8_0_ref and
quantize_row_iq4_nl_impl with one block of 32 per call) in the conventions of
the reference's Q4_0 (q4_0.py:14-33: first-index signed absmax, IEEE division,
one rounding per operation) and its IQ4_XS search (iq4_xs.py:35-76). Used by
tests/test_extra_types.py to pin the C oracle bit for bit. Square roots are
IEEE here: the comparison runs the oracle in its IEEE square-root mode."""

from __future__ import annotations

import numpy as np

F = np.float32
KVALUES = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], F)


def _f16(v: np.ndarray) -> np.ndarray:
    """fp16 bytes (round to nearest even), little-endian, per block: (n, 2)."""
    return v.astype(np.float16).view(np.uint8).reshape(-1, 2)


def _nibbles(q: np.ndarray) -> np.ndarray:
    """16 bytes per block: q[j] | q[j + 16] << 4 (low nibbles only)."""
    return ((q[:, :16] & 15) | ((q[:, 16:] & 15) << 4)).astype(np.uint8)


def _high_bits(q: np.ndarray) -> np.ndarray:
    """4 bytes per block: bit i of the u32 = bit 4 of q[i]."""
    bits = ((q >> 4) & 1).astype(np.uint64) << np.arange(32, dtype=np.uint64)
    return bits.sum(1).astype(np.uint32).view(np.uint8).reshape(-1, 4)


def _inv(d: np.ndarray) -> np.ndarray:
    """1/d (IEEE, float32; infinite below 2^-128), 0 where d == 0."""
    with np.errstate(divide="ignore", over="ignore"):
        return np.where(d != 0, F(1) / np.where(d != 0, d, F(1)), F(0)).astype(F)


def _signed_absmax(b: np.ndarray) -> np.ndarray:
    """Per block the value of largest |x|, the first one among equals."""
    return b[np.arange(b.shape[0]), np.argmax(np.abs(b), axis=1)]


def q_1(b: np.ndarray, nmax: int) -> np.ndarray:
    """Q4_1 (nmax 15) / Q5_1 (nmax 31): d = (max - min) / nmax, m = min,
    q = min(trunc((x - m) * (1/d) + 0.5), nmax)."""
    mn, mx = b.min(1), b.max(1)
    d = ((mx - mn) / F(nmax)).astype(F)
    t = (b - mn[:, None]).astype(F) * _inv(d)[:, None]
    t = (t + F(0.5)).astype(F)
    q = np.fmin(np.fmax(np.trunc(t), F(0)), F(nmax)).astype(np.uint8)     # NaN -> 0, as fmaxf
    parts = [_f16(d), _f16(mn)]
    if nmax == 31:
        parts.append(_high_bits(q))
    return np.concatenate(parts + [_nibbles(q)], axis=1)


def q5_0(b: np.ndarray) -> np.ndarray:
    """d = (signed absmax) / -16, q = clamp(floor(x * (1/d) + 16.5), 0, 31)."""
    d = (_signed_absmax(b) / F(-16)).astype(F)
    t = (b * _inv(d)[:, None]).astype(F)
    t = (t + F(16.5)).astype(F)
    q = np.fmin(np.fmax(np.floor(t), F(0)), F(31)).astype(np.uint8)
    return np.concatenate([_f16(d), _high_bits(q), _nibbles(q)], axis=1)


def _round_half_away(v: np.ndarray) -> np.ndarray:
    """C roundf, exactly: the integer part, plus one away from zero when the
    fraction (exact for |v| < 2^23) is at least one half."""
    r = np.trunc(v)
    with np.errstate(invalid="ignore"):
        frac = (v - r).astype(F)
    return r + np.where(np.abs(frac) >= F(0.5), np.sign(v), F(0))


def q8_0(b: np.ndarray) -> np.ndarray:
    """d = max|x| / 127, q = roundf(x * (1/d)) as int8."""
    d = (np.abs(b).max(1) / F(127)).astype(F)
    t = (b * _inv(d)[:, None]).astype(F)
    r = _round_half_away(t)
    # an infinite 1/d (d below 127 * 2^-128): saturate to [-128, 127], NaN -> 0
    q = np.where(np.isnan(r), F(0), np.clip(r, F(-128), F(127))).astype(np.int32)
    return np.concatenate([_f16(d), q.astype(np.int8).view(np.uint8)], axis=1)


def _best_index(al: np.ndarray) -> np.ndarray:
    """Nearest IQ4 LUT index (iq4_xs.py:35-39): the bracket of
    searchsorted(right), clamped to 1..15, then `al - lo < hi - al`."""
    # C's scan `while (V[mu] <= al) mu++` stops at once on NaN (mu 0 -> 1)
    mu = np.where(np.isnan(al), 1, np.clip(np.searchsorted(KVALUES, al, side="right"), 1, 15))
    lo, hi = KVALUES[mu - 1], KVALUES[mu]
    with np.errstate(invalid="ignore"):
        return np.where((al - lo).astype(F) < (hi - al).astype(F), mu - 1, mu)


def _seq_sum(t: np.ndarray) -> np.ndarray:
    s = t[:, 0].copy()
    for i in range(1, t.shape[1]):
        s = (s + t[:, i]).astype(F)
    return s


def _cascade8_32(v: np.ndarray) -> np.ndarray:
    """torch's `.sum(-1)` over 32 values: 8 lanes of ((v0 + v8) + v16) + v24,
    then added left to right from +0."""
    lanes = (((v[:, 0:8] + v[:, 8:16]).astype(F) + v[:, 16:24]).astype(F) + v[:, 24:32]).astype(F)
    s = np.zeros(v.shape[0], F)
    for l in range(8):
        s = (s + lanes[:, l]).astype(F)
    return s


def _search_scale(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """The IQ4_XS block search (iq4_xs.py:52-76) on blocks of 32."""
    am = _signed_absmax(x)
    live = np.abs(am) >= F(1e-15)
    mxs = np.where(live, am, F(1)).astype(F)
    d0 = (-mxs / F(-127)).astype(F)

    def sums(inv):
        q = KVALUES[_best_index((inv[:, None] * x).astype(F))]
        wq = (w * q).astype(F)
        return _seq_sum((wq * x).astype(F)), _seq_sum((wq * q).astype(F))

    sqx, sq2 = sums((F(1) / d0).astype(F))
    with np.errstate(divide="ignore", invalid="ignore"):
        d = np.where(sq2 > 0, sqx / np.where(sq2 > 0, sq2, F(1)), F(0)).astype(F)
    best = (d * sqx).astype(F)
    for itry in range(-7, 8):
        inv = ((F(1) / mxs).astype(F) * F(itry - 127)).astype(F)      # torch: c / t = (1/t) * c
        sqx, sq2 = sums(inv)
        acc = (sq2 > 0) & ((sqx * sqx).astype(F) > (best * sq2).astype(F))
        nd = (sqx / np.where(sq2 > 0, sq2, F(1))).astype(F)
        d = np.where(acc, nd, d)
        best = np.where(acc, (nd * sqx).astype(F), best)
    return np.where(live, d, F(0)).astype(F)


def iq4_nl(b: np.ndarray, qw: np.ndarray | None) -> np.ndarray:
    """IQ4_NL, one block of 32 per superblock: weights x^2, or
    qw * sqrt(2 * sum(x^2) / 32 + x^2) with the `.sum(-1)` cascade; the IQ4_XS
    search; levels at 1/d."""
    x2 = (b * b).astype(F)
    if qw is None:
        w = x2
    else:
        sigma2 = ((F(2) * _cascade8_32(x2)).astype(F) / F(32)).astype(F)
        w = (qw * np.sqrt((sigma2[:, None] + x2).astype(F))).astype(F)
    d = _search_scale(b, w)
    idx = _best_index((b * _inv(d)[:, None]).astype(F)).astype(np.uint8)
    return np.concatenate([_f16(d), _nibbles(idx)], axis=1)


def quantize(qtype: str, x: np.ndarray, qw: np.ndarray | None = None) -> np.ndarray:
    """Rows of x (n, k) -> packed bytes (n, k/32 * block bytes)."""
    n, k = x.shape
    b = np.ascontiguousarray(x, dtype=F).reshape(-1, 32)
    if qtype == "q4_1":
        out = q_1(b, 15)
    elif qtype == "q5_1":
        out = q_1(b, 31)
    elif qtype == "q5_0":
        out = q5_0(b)
    elif qtype == "q8_0":
        out = q8_0(b)
    elif qtype == "iq4_nl":
        w = None if qw is None else np.tile(np.asarray(qw, F)[:k].reshape(-1, 32), (n, 1))
        out = iq4_nl(b, w)
    else:
        raise ValueError(qtype)
    return out.reshape(n, -1)
