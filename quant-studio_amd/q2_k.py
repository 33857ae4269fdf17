"""Q2_K: the reference module's quantizer and SPECS entry (kernels/q2_k.py:25,
:88-91), computed by the HIP kernel k_q2_k through the C ABI."""

from . import ALL_SPECS, quantize


def quantize_q2_k(x, qw):
    """x: (n_rows, k) float32 / float16 / bfloat16 on a ROCm device or the CPU,
    k % 256 == 0; qw: (k,) float32 imatrix weights on x's device, or None.
    Returns (n_rows, k//256 * 84) uint8 on x's device (a CPU x is staged
    through the current ROCm device)."""
    return quantize(int(ALL_SPECS['q2_k'].ggml_type), x, qw)


SPECS = {'q2_k': ALL_SPECS['q2_k']}
