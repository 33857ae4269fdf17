"""IQ4_XS: the reference module's quantizer and SPECS entry (kernels/iq4_xs.py:149,
:195-198), computed by the HIP kernel k_iq4_xs through the C ABI."""

from . import ALL_SPECS, quantize


def quantize_iq4_xs(x, qw):
    """x: (n_rows, k) float32 / float16 / bfloat16 on a ROCm device or the CPU,
    k % 256 == 0; qw: (k,) float32 imatrix weights on x's device, or None.
    Returns (n_rows, k//256 * 136) uint8 on x's device (a CPU x is staged
    through the current ROCm device)."""
    return quantize(int(ALL_SPECS['iq4_xs'].ggml_type), x, qw)


SPECS = {'iq4_xs': ALL_SPECS['iq4_xs']}
