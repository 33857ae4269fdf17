"""IQ3_XXS: the reference module's quantizer and SPECS entry (kernels/iq3_xxs.py:31,
:142-146), computed by the HIP kernel k_iq3 through the C ABI.

Without qw the weights are x^2 (iq3_xxs.py:41-42); the type's SPECS entry
still sets needs_imatrix, so the command line refuses to plan it without one."""

from . import ALL_SPECS, quantize


def quantize_iq3_xxs(x, qw):
    """x: (n_rows, k) float32 / float16 / bfloat16 on a ROCm device or the CPU,
    k % 256 == 0; qw: (k,) float32 imatrix weights on x's device, or None.
    Returns (n_rows, k//256 * 98) uint8 on x's device (a CPU x is staged
    through the current ROCm device)."""
    return quantize(int(ALL_SPECS['iq3_xxs'].ggml_type), x, qw)


SPECS = {'iq3_xxs': ALL_SPECS['iq3_xxs']}
