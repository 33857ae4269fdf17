"""Q8_0: a ggml format the reference has no module for (its command line stops
on it, quant-studio.py:396-399), in the shape of the reference's per-type
modules: quantize_q8_0(x, qw) and a SPECS entry, computed by the HIP kernel
k_b32 through the C ABI."""

from . import ALL_SPECS, quantize


def quantize_q8_0(x, qw=None):
    """x: (n_rows, k) float32 / float16 / bfloat16 on a ROCm device or the CPU,
    k % 32 == 0; qw: accepted and ignored (the 32-value integer formats take no imatrix,
    as the reference's Q4_0).
    Returns (n_rows, k//32 * 34) uint8 on x's device."""
    return quantize(int(ALL_SPECS['q8_0'].ggml_type), x, None)


SPECS = {'q8_0': ALL_SPECS['q8_0']}
