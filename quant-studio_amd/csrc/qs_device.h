// Device-side numerics shared by every quantizer kernel (gfx950 only).
//
// The kernels must reproduce the reference's eager torch CPU arithmetic bit for
// bit, so this file pins the few operations whose rounding matters:
//   - the library is compiled with -ffp-contract=off: a*b+c stays a v_mul_f32
//     followed by a v_add_f32, as torch evaluates it op by op;
//   - `/` and sqrtf are IEEE correctly rounded (-fhip-fp32-correctly-rounded-
//     divide-sqrt, hipcc's default);
//   - torch's `python_float / tensor` is `tensor.reciprocal() * float`
//     (two roundings), which rdiv() restates;
//   - torch.round is round-half-even: rintf -> v_rndne_f32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define QS_DEV __device__ __forceinline__

namespace qs {

constexpr int QK_K = 256;
constexpr float GROUP_MAX_EPS = 1e-15f;
constexpr float F32_TINY = 1.17549435e-38f;

// source element encodings (ggml type ids)
enum : int { SRC_F32 = 0, SRC_F16 = 1, SRC_BF16 = 30 };

QS_DEV float rdiv(float c, float t) {
    float r = 1.0f / t;
    return r * c;
}
QS_DEV float clampf(float v, float lo, float hi) { return fminf(fmaxf(v, lo), hi); }

// f32 -> fp16 bits, round to nearest even (v_cvt_f16_f32 under the default mode)
QS_DEV uint32_t f16_bits(float v) {
    _Float16 h = (_Float16)v;
    return (uint32_t)__builtin_bit_cast(uint16_t, h);
}
QS_DEV float f16_round(float v) { return (float)(_Float16)v; }

// Load n consecutive source elements starting at element offset `off` and
// widen them to f32 (exact for f16 and bf16). VEC: 16-byte aligned vector loads.
template <int SRC, bool VEC, int N>
QS_DEV void load_elems(const void* base, int64_t off, float (&out)[N]) {
    if constexpr (SRC == SRC_BF16) {
        const uint16_t* p = static_cast<const uint16_t*>(base) + off;
        if constexpr (VEC) {
#pragma unroll
            for (int j = 0; j < N / 8; j++) {
                uint4 u = reinterpret_cast<const uint4*>(p)[j];
                uint32_t v[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    out[8 * j + 2 * t] = __builtin_bit_cast(float, v[t] << 16);
                    out[8 * j + 2 * t + 1] = __builtin_bit_cast(float, v[t] & 0xffff0000u);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < N; i++) out[i] = __builtin_bit_cast(float, (uint32_t)p[i] << 16);
        }
    } else if constexpr (SRC == SRC_F16) {
        const uint16_t* p = static_cast<const uint16_t*>(base) + off;
        if constexpr (VEC) {
#pragma unroll
            for (int j = 0; j < N / 8; j++) {
                uint4 u = reinterpret_cast<const uint4*>(p)[j];
                uint32_t v[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    out[8 * j + 2 * t] = (float)__builtin_bit_cast(_Float16, (uint16_t)(v[t] & 0xffffu));
                    out[8 * j + 2 * t + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(v[t] >> 16));
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < N; i++) out[i] = (float)__builtin_bit_cast(_Float16, p[i]);
        }
    } else {
        const float* p = static_cast<const float*>(base) + off;
        if constexpr (VEC) {
#pragma unroll
            for (int j = 0; j < N / 4; j++) {
                float4 u = reinterpret_cast<const float4*>(p)[j];
                out[4 * j] = u.x;
                out[4 * j + 1] = u.y;
                out[4 * j + 2] = u.z;
                out[4 * j + 3] = u.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < N; i++) out[i] = p[i];
        }
    }
}

// ---- reduction orders (all within one lane) ----

// adjacent-pair tree (kq_common.py:38-43); N a power of two
template <int N>
QS_DEV float tree_sum(const float (&v)[N]) {
    float t[N / 2];
#pragma unroll
    for (int i = 0; i < N / 2; i++) t[i] = v[2 * i] + v[2 * i + 1];
#pragma unroll
    for (int m = N / 2; m > 1; m >>= 1) {
#pragma unroll
        for (int i = 0; i < m / 2; i++) t[i] = t[2 * i] + t[2 * i + 1];
    }
    return t[0];
}

// left-to-right (qx_common.py:37-44)
template <int N>
QS_DEV float seq_sum(const float (&v)[N]) {
    float s = v[0];
#pragma unroll
    for (int i = 1; i < N; i++) s = s + v[i];
    return s;
}

// torch CPU `.sum(-1)` of a contiguous row of N <= 32 elements: the 8-lane
// vector cascade. N=32: lane l sums ((v[l]+v[8+l])+v[16+l])+v[24+l];
// N=16: (v[l]+v[8+l]); N=8: v[l]; then a scalar pass over the 8 lanes from +0.
template <int N>
QS_DEV float cascade8_sum(const float (&v)[N]) {
    static_assert(N == 8 || N == 16 || N == 32, "cascade8_sum: N in {8,16,32}");
    float fin = 0.0f;
#pragma unroll
    for (int l = 0; l < 8; l++) {
        float p;
        if constexpr (N == 32) {
            p = v[l] + v[8 + l];
            p = p + v[16 + l];
            p = p + v[24 + l];
        } else if constexpr (N == 16) {
            p = 0.0f + v[l];
            p = p + v[8 + l];
        } else {
            p = 0.0f + v[l];
        }
        fin = fin + p;
    }
    return fin;
}

// first index of the largest |v| (qx_common.py:26-34); returns the signed value
template <int N>
QS_DEV float absmax_first(const float (&v)[N], float& amax) {
    float am = fabsf(v[0]), mv = v[0];
#pragma unroll
    for (int i = 1; i < N; i++) {
        float a = fabsf(v[i]);
        bool gt = a > am;
        am = gt ? a : am;
        mv = gt ? v[i] : mv;
    }
    amax = am;
    return mv;
}

}  // namespace qs
