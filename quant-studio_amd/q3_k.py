"""Q3_K: the reference module's quantizer and SPECS entry (kernels/q3_k.py:23,
:85-88), computed by the HIP kernel k_q3_k through the C ABI."""

from . import ALL_SPECS, quantize


def quantize_q3_k(x, qw):
    """x: (n_rows, k) float32 / float16 / bfloat16 on a ROCm device or the CPU,
    k % 256 == 0; qw: (k,) float32 imatrix weights on x's device, or None.
    Returns (n_rows, k//256 * 110) uint8 on x's device (a CPU x is staged
    through the current ROCm device)."""
    return quantize(int(ALL_SPECS['q3_k'].ggml_type), x, qw)


SPECS = {'q3_k': ALL_SPECS['q3_k']}
