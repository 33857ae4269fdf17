"""IQ3_S: the reference module's quantizer and SPECS entry (kernels/iq3_s.py:31,
:148-151), computed by the HIP kernel k_iq3 through the C ABI."""

from . import ALL_SPECS, quantize


def quantize_iq3_s(x, qw):
    """x: (n_rows, k) float32 / float16 / bfloat16 on a ROCm device or the CPU,
    k % 256 == 0; qw: (k,) float32 imatrix weights on x's device, or None.
    Returns (n_rows, k//256 * 110) uint8 on x's device (a CPU x is staged
    through the current ROCm device)."""
    return quantize(int(ALL_SPECS['iq3_s'].ggml_type), x, qw)


SPECS = {'iq3_s': ALL_SPECS['iq3_s']}
