// Measurement aid, not part of the quantizer ABI: a kernel whose waves issue
// nothing but independent f32 multiplies and adds on VGPR operands, giving the
// VALU issue rate (wave instructions per second) that the quantizer kernels
// are compared with. With enough resident waves gfx950 issues about two such
// instructions per CU per clock; an SGPR operand in every instruction halves
// that, so the operands here are per-lane values. Built into its own library
// (libqs_calib.so) and used only by bench.py.
#include <hip/hip_runtime.h>

namespace {

constexpr int kChains = 16;     // independent mul/add chains per lane

__global__ __launch_bounds__(256) void k_valu_issue(float* out, int iters, float b0, float c0) {
    float a[kChains];
#pragma unroll
    for (int j = 0; j < kChains; j++) a[j] = (float)threadIdx.x * 0.001f + (float)j;
    // per-lane multiplier and addend (VGPRs), close to b0 and c0
    const float b = b0 + (float)threadIdx.x * 1e-9f, c = c0 + (float)threadIdx.x * 1e-9f;
    for (int i = 0; i < iters; i++) {
#pragma unroll
        for (int j = 0; j < kChains; j++) {
            a[j] = a[j] * b;
            a[j] = a[j] + c;
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kChains; j++) s = s + a[j];
    if (s == 1234.5f) out[0] = s;     // keeps the chains live; never true for these inputs
}

}  // namespace

extern "C" {

// VALU wave instructions one launch of (grid x 256 threads, iters) issues in
// its loop (2 per chain per iteration per wave).
double qs_calib_valu_insts(int grid, int iters) { return (double)grid * 4.0 * iters * 2.0 * kChains; }

// Launch the issue-rate kernel on hip_stream; out is a device float.
int qs_calib_valu(int grid, int iters, float* out, void* hip_stream) {
    if (grid <= 0 || iters <= 0 || !out) return -22;
    hipLaunchKernelGGL(k_valu_issue, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(hip_stream), out,
                       iters, 0.999f, 0.001f);
    return hipGetLastError() == hipSuccess ? 0 : -5;
}

}  // extern "C"
