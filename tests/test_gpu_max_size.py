"""GPU: one C call at the per-call maximum of 2^34 values (a 4,194,304 x 4096
bf16 tensor, 32 GiB) for one kernel of every launch shape. Offsets of the
input pass 2^31 values and 2^32 bytes and the outputs pass 4 GiB, so a 32-bit
index anywhere in a kernel, its grid or the launcher would show here; rows on
both sides of each such boundary are compared with the oracle byte for byte.
The reference has no size limit of its own (its torch path takes any tensor);
this checks the limit include/quant_studio.h documents."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

K = 4096
ROWS = (1 << 34) // K            # 4,194,304 rows: exactly 2^34 values


@pytest.fixture(scope="module")
def big():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(34)
    print(f"generating {ROWS}x{K} bf16 (32 GiB)", flush=True)
    x = torch.empty((ROWS, K), dtype=torch.bfloat16, device=dev)
    x.normal_(0.0, 0.02, generator=g)
    qw = torch.empty(K, dtype=torch.float32, device=dev).log_normal_(0.0, 1.0, generator=g)
    torch.cuda.synchronize()
    held = [x, qw]
    del x
    yield held
    held.clear()                     # the 32 GiB go back to the device for later tests
    torch.cuda.empty_cache()


def check_rows(rb: int) -> list[int]:
    """Rows around every 2^31-value, 2^32-byte and 4 GiB-of-output boundary."""
    rows = {0, 1, ROWS - 2, ROWS - 1}
    for v in (1 << 31, 1 << 32, 1 << 33):          # input values (bf16 bytes are 2x)
        r = v // K
        rows |= {r - 1, r}
    for b in (1 << 32, 1 << 33):                    # output bytes
        r = b // rb
        rows |= {r - 1, r, r + 1}
    return sorted(r for r in rows if 0 <= r < ROWS)


def host_rows(x: torch.Tensor, rows: list[int]) -> np.ndarray:
    idx = torch.tensor(rows, device=x.device)
    return x.index_select(0, idx).view(torch.int16).cpu().numpy().view(np.uint16)


# one type per kernel family / launch shape: 256 blocks of 32 per 256-thread
# workgroup (k_b32), 64 blocks per wave (IQ4_NL), 8 / 4 / 2 superblocks per
# one-wave workgroup, and 16 superblocks per four-wave workgroup (IQ2_S)
CASES = [("q4_0", False), ("iq4_nl", True), ("q4_k", True), ("q6_k", True),
         ("iq2_xs", True), ("iq2_s", True), ("iq3_xxs", True)]


@pytest.mark.parametrize("qtype,imat", CASES)
def test_one_call_of_2_pow_34_values(qs, big, qtype, imat):
    x, qw = big
    tid = int(qs.ALL_SPECS[qtype].ggml_type)
    rb = qs.row_bytes(tid, K)
    L = qs.library()
    print(f"{qtype} imat={imat}: one call, {ROWS}x{K} ({ROWS * rb / 2**30:.2f} GiB out)", flush=True)
    out = torch.empty((ROWS, rb), dtype=torch.uint8, device=x.device)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    qptr = qw.data_ptr() if imat else None
    rc = L.qs_quantize(int(tid), 30, x.data_ptr(), ROWS, K, K * 2, qptr, out.data_ptr(), out.numel(), stream)
    assert rc == 0, qs.last_error()
    torch.cuda.synchronize()
    rows = check_rows(rb)
    got = out.index_select(0, torch.tensor(rows, device=x.device)).cpu().numpy()
    del out
    ref = oracle.quantize(qtype, host_rows(x, rows), qw.cpu().numpy() if imat else None)
    bad = [r for r, g_, e in zip(rows, got, ref) if not np.array_equal(g_, e)]
    assert not bad, f"{qtype}: rows {bad} differ from the oracle"


def test_strided_rows_past_2_pow_31(qs, big):
    """Q4_0 on a strided view (row stride 4096, 3840 columns): the padded-row
    path of the 32-value kernel, whose row/column split is 64-bit."""
    x, _ = big
    kk = 3840
    tid = int(qs.ALL_SPECS["q4_0"].ggml_type)
    rb = qs.row_bytes(tid, kk)
    print(f"q4_0 strided {ROWS}x{kk} of {K}", flush=True)
    out = torch.empty((ROWS, rb), dtype=torch.uint8, device=x.device)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    rc = qs.library().qs_quantize(int(tid), 30, x.data_ptr(), ROWS, kk, K * 2, None, out.data_ptr(),
                                  out.numel(), stream)
    assert rc == 0, qs.last_error()
    torch.cuda.synchronize()
    rows = check_rows(rb)
    got = out.index_select(0, torch.tensor(rows, device=x.device)).cpu().numpy()
    del out
    ref = oracle.quantize("q4_0", np.ascontiguousarray(host_rows(x, rows)[:, :kk]), None)
    assert np.array_equal(got, ref)


def test_one_row_past_the_limit_is_refused(qs, big):
    """2^34 + 4096 values in one call: QS_EINVAL before any launch (the
    pointers are real, nothing is read)."""
    x, _ = big
    out = torch.empty(16, dtype=torch.uint8, device=x.device)
    L = qs.library()
    rc = L.qs_quantize(2, 30, x.data_ptr(), ROWS + 1, K, K * 2, None, out.data_ptr(), ctypes.c_int64(1 << 40),
                       torch.cuda.current_stream(x.device).cuda_stream)
    assert rc != 0 and "2^34" in qs.last_error()
