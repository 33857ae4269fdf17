"""IQ4_NL: a ggml format the reference has no module for (its command line stops
on it, quant-studio.py:396-399), in the shape of the reference's per-type
modules: quantize_iq4_nl(x, qw) and a SPECS entry, computed by the HIP kernel
k_iq4_nl through the C ABI."""

from . import ALL_SPECS, quantize


def quantize_iq4_nl(x, qw=None):
    """x: (n_rows, k) float32 / float16 / bfloat16 on a ROCm device or the CPU,
    k % 32 == 0; qw: (k,) float32 imatrix weights on x's device, or None.
    Returns (n_rows, k//32 * 18) uint8 on x's device."""
    return quantize(int(ALL_SPECS['iq4_nl'].ggml_type), x, qw)


SPECS = {'iq4_nl': ALL_SPECS['iq4_nl']}
