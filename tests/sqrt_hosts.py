"""The reference's square-root rounding per host: the measured maps the
library embeds, decoded for the tests and the oracle, and a check of the
running host's torch against them."""

from __future__ import annotations

import importlib.util
from pathlib import Path

import numpy as np

CSRC = Path(__file__).resolve().parents[1] / "quant-studio_amd" / "csrc"
AMD_MAP = CSRC / "qs_sqrt_amd.bin"


def gen_module():
    spec = importlib.util.spec_from_file_location("gen_sqrt_table", CSRC / "gen_sqrt_table.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def intel_ulps() -> np.ndarray:
    """Per-key ulp offsets of the Intel-host rounding (qs_sqrt_table.h)."""
    d = np.zeros(1 << 24, np.int8)
    d[gen_module().header_keys()] = -1
    return d


def amd_ulps() -> np.ndarray:
    """Per-key ulp offsets of the AMD-host rounding (qs_sqrt_amd.bin)."""
    return gen_module().decode_map(AMD_MAP.read_bytes())


def key_of(v: np.ndarray) -> np.ndarray:
    """sqrt_key of qs_device.h for positive finite float32 v."""
    b = v.view(np.uint32)
    sub = b < np.uint32(0x00800000)
    bn = b.copy()
    bn[sub] = (v[sub] * np.float32(2.0 ** 64)).view(np.uint32)
    return ((((bn >> np.uint32(23)) & np.uint32(1)) ^ np.uint32(1)) << np.uint32(23)) | (bn & np.uint32(0x7fffff))


def predicted(v: np.ndarray, ulps: np.ndarray, subnormal_ieee: bool = False) -> np.ndarray:
    """The tabulated root of positive finite float32 v: IEEE root + offset
    (with subnormal_ieee, the IEEE root for subnormal v)."""
    r = np.sqrt(v.astype(np.float64)).astype(np.float32)
    off = ulps[key_of(v)].astype(np.int32)
    if subnormal_ieee:
        off[v.view(np.uint32) < np.uint32(0x00800000)] = 0
    return (r.view(np.int32) + off).view(np.float32)


def host_rounding_matches(torch) -> str:
    """Which tabulated rounding this host's torch.sqrt follows ("torch-cpu" or
    "torch-cpu-amd"), checked over all 2^24 key classes in [1, 4), at other
    exponents and on subnormals; also checks the other torch CPU operations the
    oracle takes as IEEE on this host (reciprocal, division, round half-even,
    the `.sum(-1)` cascade). Raises AssertionError otherwise."""
    import oracle
    gen = gen_module()
    census = gen.rounding_census()
    here = np.zeros(1 << 24, np.int8)
    for v, k in census["keys"].items():
        here[k] = v
    name = None
    # the Intel host's map covers subnormal inputs by their scaled keys; the
    # AMD host returns the IEEE root for every subnormal input
    for cand, table, sub_ieee in (("torch-cpu", intel_ulps(), False),
                                  ("torch-cpu-amd", amd_ulps(), True)):
        if np.array_equal(here, table):
            name, ulps, subnormal_ieee = cand, table, sub_ieee
    assert name is not None, f"torch.sqrt on this host follows neither table: {census['counts']}"
    rng = np.random.default_rng(5)
    for lo, hi in ((2.0 ** -126, 2.0 ** -100), (1e-30, 1e-10), (1e-6, 1e3), (1e10, 1e30)):
        v = np.exp(rng.uniform(np.log(lo), np.log(hi), 1 << 18)).astype(np.float32)
        got = torch.sqrt(torch.from_numpy(v)).numpy()
        assert np.array_equal(got.view(np.int32),
                              predicted(v, ulps, subnormal_ieee).view(np.int32)), (lo, hi)
    sub = np.arange(1, 1 << 23, dtype=np.uint32).view(np.float32)      # every subnormal
    got = torch.sqrt(torch.from_numpy(sub)).numpy()
    assert np.array_equal(got.view(np.int32),
                          predicted(sub, ulps, subnormal_ieee).view(np.int32)), "subnormals"
    # the other operations are IEEE / exact on this host as on the golden host
    a = (rng.standard_normal(1 << 18) * 0.02).astype(np.float32)
    b = np.exp(rng.standard_normal(1 << 18)).astype(np.float32)
    ta, tb = torch.from_numpy(a), torch.from_numpy(b)
    assert np.array_equal(torch.reciprocal(tb).numpy(), np.float32(1.0) / b)
    assert np.array_equal((ta / tb).numpy(), a / b)
    assert np.array_equal(torch.round(ta * 1000).numpy(), np.rint(a * np.float32(1000)))
    for n in (8, 16, 32, 256):
        rows = a[: (a.size // n) * n].reshape(-1, n)[:3000]
        want = np.array([oracle.sum_cascade8(r) for r in rows], np.float32)
        assert np.array_equal(torch.from_numpy(rows).sum(-1).numpy(), want), n
    return name
