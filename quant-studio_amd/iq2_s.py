"""IQ2_S: the reference module's quantizer and SPECS entry (kernels/iq2_s.py:21,
:70-73), computed by the HIP kernel k_iq2_xs_s through the C ABI."""

from . import ALL_SPECS, quantize


def quantize_iq2_s(x, qw):
    """x: (n_rows, k) float32 / float16 / bfloat16 on a ROCm device or the CPU,
    k % 256 == 0; qw: (k,) float32 imatrix weights on x's device (required).
    Returns (n_rows, k//256 * 82) uint8 on x's device (a CPU x is staged
    through the current ROCm device)."""
    return quantize(int(ALL_SPECS['iq2_s'].ggml_type), x, qw)


SPECS = {'iq2_s': ALL_SPECS['iq2_s']}
