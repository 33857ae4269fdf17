"""Q4_K: the reference module's quantizer and SPECS entry (kernels/q4_k.py:25,
:86-89), computed by the HIP kernel k_q45_k through the C ABI."""

from . import ALL_SPECS, quantize


def quantize_q4_k(x, qw):
    """x: (n_rows, k) float32 / float16 / bfloat16 on a ROCm device or the CPU,
    k % 256 == 0; qw: (k,) float32 imatrix weights on x's device, or None.
    Returns (n_rows, k//256 * 144) uint8 on x's device (a CPU x is staged
    through the current ROCm device)."""
    return quantize(int(ALL_SPECS['q4_k'].ggml_type), x, qw)


SPECS = {'q4_k': ALL_SPECS['q4_k']}
