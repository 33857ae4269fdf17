"""IQ2_XXS: the reference module's quantizer and SPECS entry (kernels/iq2.py:418,
:506-509), computed by the HIP kernel k_iq2_xxs through the C ABI."""

from . import ALL_SPECS, quantize


def quantize_iq2_xxs(x, qw, T=None):
    """x: (n_rows, k) float32 / float16 / bfloat16 on a ROCm device or the CPU,
    k % 256 == 0; qw: (k,) float32 imatrix weights on x's device (required);
    T: accepted for the reference's signature and unused (the grid tables
    live in the library, uploaded once per device).
    Returns (n_rows, k//256 * 66) uint8 on x's device (a CPU x is staged
    through the current ROCm device)."""
    return quantize(int(ALL_SPECS['iq2_xxs'].ggml_type), x, qw)


SPECS = {'iq2_xxs': ALL_SPECS['iq2_xxs']}
