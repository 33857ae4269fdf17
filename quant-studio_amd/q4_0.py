"""Q4_0: the reference module's quantizer and SPECS entry (kernels/q4_0.py:14,
:40-43), computed by the HIP kernel k_b32 (256 blocks of 32 per workgroup) through the C ABI.

The reference's Q4_0 takes no imatrix (q4_0.py:36-37)."""

from . import ALL_SPECS, quantize


def quantize_q4_0(x):
    """x: (n_rows, k) float32 / float16 / bfloat16 on a ROCm device or the CPU,
    k % 32 == 0.
    Returns (n_rows, k//32 * 18) uint8 on x's device (a CPU x is staged
    through the current ROCm device)."""
    return quantize(int(ALL_SPECS['q4_0'].ggml_type), x, None)


SPECS = {'q4_0': ALL_SPECS['q4_0']}
