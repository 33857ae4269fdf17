"""Q6_K: the reference module's quantizer and SPECS entry (kernels/q6_k.py:22,
:72-75), computed by the HIP kernel k_q6_k through the C ABI."""

from . import ALL_SPECS, quantize


def quantize_q6_k(x, qw):
    """x: (n_rows, k) float32 / float16 / bfloat16 on a ROCm device or the CPU,
    k % 256 == 0; qw: (k,) float32 imatrix weights on x's device, or None.
    Returns (n_rows, k//256 * 210) uint8 on x's device (a CPU x is staged
    through the current ROCm device)."""
    return quantize(int(ALL_SPECS['q6_k'].ggml_type), x, qw)


SPECS = {'q6_k': ALL_SPECS['q6_k']}
