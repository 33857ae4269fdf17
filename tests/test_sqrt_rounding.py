"""The reference's square root rounds differently on different hosts (torch.sqrt
on a CPU tensor goes through the host's MKL): the library reproduces an Intel
host (the default, where the golden vectors were written), an AMD EPYC host
(the host of an MI355X machine) or the IEEE root. These CPU tests pin the embedded AMD map
and prove its lookup band; test_host_sqrt_rounding checks the running host's
torch against the tables."""

from __future__ import annotations

import hashlib

import numpy as np
import pytest

import oracle
import sqrt_hosts

# the map measured on an MI355X machine's host (AMD EPYC, torch 2.10.0+rocm7.0,
# oneAPI MKL 2024.2) by gen_sqrt_table.py
AMD_MAP_SHA256 = "3e49f6e5c17392c0788450ff06ee602787215ebd84301e185ef6ff4e1bd41903"
AMD_COUNTS = {-1: 1239767, 0: 13900284, 1: 1637165}


def test_amd_map_is_the_measured_one():
    blob = sqrt_hosts.AMD_MAP.read_bytes()
    assert hashlib.sha256(blob).hexdigest() == AMD_MAP_SHA256
    d = sqrt_hosts.amd_ulps()
    vals, counts = np.unique(d, return_counts=True)
    assert dict(zip(vals.tolist(), counts.tolist())) == AMD_COUNTS
    # the Intel host's one-ulp-down set is no subset of it: the hosts differ
    intel = sqrt_hosts.intel_ulps()
    assert 0.4 < (d[intel == -1] == -1).mean() < 0.5


def _looked_up(v: np.ndarray, lo: float, hi: float) -> np.ndarray:
    """sqrt_lookup_key of qs_device.h, op for op in float32: is the map read?"""
    r = np.sqrt(v)
    rem64 = v.astype(np.float64) - r.astype(np.float64) ** 2
    rem = rem64.astype(np.float32)
    assert np.array_equal(rem.astype(np.float64), rem64)     # exact, as the kernels' fma
    ulp = ((r.view(np.uint32) & np.uint32(0x7f800000)) - np.uint32(23 << 23)).view(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        lim_lo = (np.float32(lo) * r) * ulp
        lim_hi = (np.float32(hi) * r) * ulp
    return (rem < lim_lo) | (rem > lim_hi) | (v.view(np.uint32) < np.uint32(0x17800000))


def test_amd_band_reads_every_listed_key():
    """The kernels read the AMD maps only where the remainder is outside
    +-0.48 r ulp(r): every key the map moves (down or up) is read, over all
    2^24 classes in [1, 4) and scaled by powers of 4 across the float range;
    about half of all inputs are."""
    d = sqrt_hosts.amd_ulps()
    m = np.arange(1 << 23, dtype=np.uint32)
    x = np.concatenate([(127 << 23) | m, (128 << 23) | m]).astype(np.uint32).view(np.float32)
    look = _looked_up(x, -0.48, 0.48)
    assert look[d != 0].all()
    assert 0.5 < look.mean() < 0.53
    # a band of 0.51 misses keys: the margin is real
    assert not _looked_up(x, -0.51, 0.51)[d != 0].all()
    xd = x[d != 0][::7]
    for k in (-45, -40, -20, -3, 1, 7, 30, 62):
        xs = (xd.astype(np.float64) * 4.0 ** k).astype(np.float32)
        assert _looked_up(xs, -0.48, 0.48).all(), k


def test_oracle_square_root_modes():
    """The oracle's weights take the IEEE root moved by the installed table,
    the plain IEEE root, or (by default) the Intel map; subnormals included."""
    d = sqrt_hosts.amd_ulps()
    rng = np.random.default_rng(1)
    v = np.concatenate([np.exp(rng.uniform(-80, 80, 3000)),
                        rng.integers(1, 1 << 23, 500).astype(np.uint32).view(np.float32)]).astype(np.float32)
    L = oracle.lib()
    ieee = np.sqrt(v.astype(np.float64)).astype(np.float32)
    want_amd = sqrt_hosts.predicted(v, d, subnormal_ieee=True)
    want_intel = sqrt_hosts.predicted(v, sqrt_hosts.intel_ulps())
    assert not np.array_equal(want_amd, ieee) and not np.array_equal(want_intel, ieee)
    # the AMD host's rounding leaves subnormal inputs at the IEEE root; the
    # table alone would move some of them
    assert not np.array_equal(sqrt_hosts.predicted(v, d), want_amd)
    oracle.use_amd_host_sqrt(d)
    try:
        assert np.array_equal(np.array([L.qso_sqrt(float(t)) for t in v], np.float32), want_amd)
    finally:
        oracle.use_sqrt_table(None)
    oracle.use_ieee_sqrt(True)
    try:
        assert np.array_equal(np.array([L.qso_sqrt(float(t)) for t in v], np.float32), ieee)
    finally:
        oracle.use_ieee_sqrt(False)
    assert np.array_equal(np.array([L.qso_sqrt(float(t)) for t in v], np.float32), want_intel)


def test_host_sqrt_rounding():
    """This host's torch.sqrt follows one of the tables (and its other CPU
    operations are the IEEE ones the oracle assumes)."""
    torch = pytest.importorskip("torch")
    name = sqrt_hosts.host_rounding_matches(torch)
    print(f"this host's torch.sqrt: {name}")


@pytest.mark.gpu
def test_gpu_host_sqrt_rounding():
    """The same check on the host CPU of the machine that holds the GPU (an
    AMD EPYC host, whose rounding torch-cpu-amd records)."""
    torch = pytest.importorskip("torch")
    name = sqrt_hosts.host_rounding_matches(torch)
    print(f"GPU host torch.sqrt: {name}", flush=True)
