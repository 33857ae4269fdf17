// Measurement aids, not part of the quantizer ABI. k_valu_issue: a kernel whose waves issue
// nothing but independent f32 multiplies and adds on VGPR operands, giving the
// VALU issue rate (wave instructions per second) that the quantizer kernels
// are compared with. With enough resident waves gfx950 issues about two such
// instructions per CU per clock; an SGPR operand in every instruction halves
// that, so the operands here are per-lane values. k_copy_stream: a streaming
// copy, the HBM rate the 32-value formats are compared with. Built into their
// own library (libqs_calib.so) and used only by bench.py.
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

// A streaming copy in the shape of the 32-value quantizer kernel: 256 threads,
// four 16-byte non-temporal loads per thread issued before any store, one
// workgroup per 16 KB, non-temporal 16-byte stores. Its rate is the measured
// copy peak the HBM-bound kernels are set against (read + written bytes).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void k_copy_stream(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                     long long n16) {
    constexpr int kPer = 4;
    const long long base = (long long)blockIdx.x * (256 * kPer) + threadIdx.x;
    u32x4 v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; u++) {
        const long long i = base + u * 256;
        if (i < n16) v[u] = __builtin_nontemporal_load(src + i);
    }
#pragma unroll
    for (int u = 0; u < kPer; u++) {
        const long long i = base + u * 256;
        if (i < n16) __builtin_nontemporal_store(v[u], dst + i);
    }
}

}  // namespace

extern "C" {

// Copy nbytes (a multiple of 16; both pointers 16-byte aligned) on hip_stream.
int qs_calib_copy(const void* src, void* dst, long long nbytes, void* hip_stream) {
    if (!src || !dst || nbytes <= 0 || nbytes % 16 || (reinterpret_cast<unsigned long long>(src) % 16) ||
        (reinterpret_cast<unsigned long long>(dst) % 16))
        return -22;
    const long long n16 = nbytes / 16;
    const long long grid = (n16 + 1023) / 1024;
    if (grid > 0x7fffffffLL) return -22;
    hipLaunchKernelGGL(k_copy_stream, dim3((unsigned)grid), dim3(256), 0, static_cast<hipStream_t>(hip_stream),
                       static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), n16);
    return hipGetLastError() == hipSuccess ? 0 : -5;
}

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
