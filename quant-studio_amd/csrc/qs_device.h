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
//   - torch.round is round-half-even: rintf -> v_rndne_f32;
//   - torch.sqrt on a CPU tensor is not correctly rounded, and how it rounds
//     depends on the host's MKL: sqrt_ref<SQ>() is the IEEE root adjusted by
//     one ulp on the tabulated keys of the selected host (or left IEEE).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define QS_DEV __device__ __forceinline__

namespace qs {

constexpr int QK_K = 256;
constexpr float GROUP_MAX_EPS = 1e-15f;
constexpr float F32_TINY = 1.17549435e-38f;

// native 4 x u32 vector (nontemporal loads need a builtin vector type)
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Streaming 16-byte load: the source is read exactly once, so it is fetched
// non-temporally and does not push the kernels' constant tables (imatrix,
// square-root map, IQ lists) out of L2.
QS_DEV u32x4 load_stream16(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// source element encodings (ggml type ids)
enum : int { SRC_F32 = 0, SRC_F16 = 1, SRC_BF16 = 30 };

QS_DEV float rdiv(float c, float t) {
    float r = 1.0f / t;
    return r * c;
}
QS_DEV float clampf(float v, float lo, float hi) { return fminf(fmaxf(v, lo), hi); }

// Register-allocation hints (no instructions): the value is taken to change
// here, so the compiler can neither recompute it later from its inputs (which
// would keep those live instead) nor hoist work that uses it out of a loop.
QS_DEV void keep_in_register(float& v) { asm volatile("" : "+v"(v)); }
// pred holds on some active lane of the wave
QS_DEV bool wave_any(bool pred) { return __builtin_amdgcn_ballot_w64(pred) != 0; }

template <int N>
QS_DEV void keep_in_registers(float (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; i++) keep_in_register(v[i]);
}

// The reference's square root (torch.sqrt, kernels/q4_k.py:34, :51,
// iq2.py:431, :436 and the other weight sites), whose rounding depends on the
// host it ran on. The kernels take the host as a template parameter SQ, so
// each compiles only the lookups its rounding needs (a runtime choice kept a
// second map's words live in every kernel and spilled the tightest ones):
//   SQ_IEEE   the correctly rounded root (torch.sqrt on a GPU tensor, sqrtf);
//   SQ_INTEL  torch.sqrt on an Intel host's CPU: the IEEE root, one ulp lower
//             where the input's key is set in the `down` map; subnormal
//             inputs follow the key of their value scaled by 2^64;
//   SQ_AMD    torch.sqrt on an AMD EPYC host's CPU: one ulp lower where the
//             key is set in `down`, one ulp higher where it is set in `up`;
//             subnormal inputs keep the IEEE root (measured on all 2^23 - 1).
// The key is (exponent parity << 23 | mantissa); the 2^24-bit maps are built
// per device from the measured tables. BAND variants read the maps only where
// the exact root s can lie on the flipped side: with r the IEEE root and
// rem = v - r^2 (exact, fma(-r, r, v)), s - r = rem / (s + r), and every
// tabulated key has rem below lo * r * ulp(r) (down) or above hi * r * ulp(r)
// (up), with (lo, hi) = (-0.875, none) on the Intel host and (-0.48, 0.48) on
// the AMD host, both checked over all 2^24 keys on the host; below 2^-80 the
// products lose precision and the maps are always read. Zero, negative,
// infinite and NaN inputs keep the IEEE result. Lanes that need no lookup
// read word 0 (one shared cache line).
enum : int { SQ_IEEE = 0, SQ_INTEL = 1, SQ_AMD = 2 };

struct SqrtMap {
    const uint32_t* down;
    const uint32_t* up;
};

// true for inputs the maps apply to: positive finite (Intel), positive
// normal finite (AMD)
template <int SQ>
QS_DEV bool sqrt_mapped(uint32_t b) {
    constexpr uint32_t lo = SQ == SQ_AMD ? 0x00800000u : 1u;
    return b - lo < 0x7f800000u - lo;
}

QS_DEV uint32_t sqrt_key(float v) {
    const uint32_t b = __float_as_uint(v);
    const uint32_t bn = b < 0x00800000u ? __float_as_uint(v * 18446744073709551616.0f) : b;
    return ((((bn >> 23) & 1u) ^ 1u) << 23) | (bn & 0x7fffffu);     // always < 2^24
}

// The map key with bit 31 set when the maps must be read for v (root r), else 0.
template <int SQ>
QS_DEV uint32_t sqrt_lookup_key(float v, float r) {
    const float rem = __builtin_fmaf(-r, r, v);
    const float ulp = __uint_as_float((__float_as_uint(r) & 0x7f800000u) - (23u << 23));
    const uint32_t b = __float_as_uint(v);
    bool outside;
    if constexpr (SQ == SQ_AMD) {
        const float lim = (0.48f * r) * ulp;
        outside = rem < -lim || rem > lim;
    } else {
        outside = rem < (-0.875f * r) * ulp;
    }
    const bool look = sqrt_mapped<SQ>(b) && (outside || b < 0x17800000u);
    return look ? (sqrt_key(v) | 0x80000000u) : 0u;
}

// r adjusted by the looked-up map bits (kn from sqrt_lookup_key)
template <int SQ>
QS_DEV float sqrt_fix(float r, uint32_t kn, uint32_t wdown, uint32_t wup) {
    const uint32_t sh = kn & 31u, on = kn >> 31;
    const uint32_t dn = on & (wdown >> sh);
    if constexpr (SQ == SQ_AMD) {
        const uint32_t up = on & (wup >> sh);
        return __uint_as_float(__float_as_uint(r) - (dn & 1u) + (up & 1u));
    } else {
        return __uint_as_float(__float_as_uint(r) - (dn & 1u));
    }
}

QS_DEV uint32_t sqrt_word(const uint32_t* __restrict__ map, uint32_t kn) {
    return map[(kn & 0x00ffffffu) >> 5];
}

// r = sqrtf(v) adjusted by the key's bits when every input reads its own words
template <int SQ>
QS_DEV float sqrt_fix_plain(float v, uint32_t key, uint32_t wdown, uint32_t wup) {
    const float r = sqrtf(v);
    const bool on = sqrt_mapped<SQ>(__float_as_uint(v));
    const bool dn = on && ((wdown >> (key & 31u)) & 1u);
    if constexpr (SQ == SQ_AMD) {
        const bool up = on && ((wup >> (key & 31u)) & 1u);
        return __uint_as_float(__float_as_uint(r) - (dn ? 1u : 0u) + (up ? 1u : 0u));
    } else {
        return dn ? __uint_as_float(__float_as_uint(r) - 1u) : r;
    }
}

template <int SQ>
QS_DEV float sqrt_ref(float v, const SqrtMap& m) {
    if constexpr (SQ == SQ_IEEE) {
        return sqrtf(v);
    } else {
        const uint32_t key = sqrt_key(v);
        return sqrt_fix_plain<SQ>(v, key, m.down[key >> 5], SQ == SQ_AMD ? m.up[key >> 5] : 0u);
    }
}

// sqrt_ref over a lane's N values, every map load issued before any is used.
// BAND reads the maps only where sqrt_lookup_key asks (every kernel uses it:
// 2-17% faster where the map loads were on the critical path, as fast for
// Q4_K/Q5_K); without it every value reads its own words.
template <int N, bool BAND, int SQ>
QS_DEV void sqrt_ref_n(const float (&v)[N], const SqrtMap& m, float (&out)[N]) {
    if constexpr (SQ == SQ_IEEE) {
#pragma unroll
        for (int i = 0; i < N; i++) out[i] = sqrtf(v[i]);
        return;
    }
    constexpr bool UP = SQ == SQ_AMD;
    uint32_t kn[N], wd[N], wu[N];
    if constexpr (BAND) {
#pragma unroll
        for (int i = 0; i < N; i++) {
            out[i] = sqrtf(v[i]);
            kn[i] = sqrt_lookup_key<SQ>(v[i], out[i]);
        }
#pragma unroll
        for (int i = 0; i < N; i++) wd[i] = sqrt_word(m.down, kn[i]);
#pragma unroll
        for (int i = 0; i < N; i++) wu[i] = UP ? sqrt_word(m.up, kn[i]) : 0u;
#pragma unroll
        for (int i = 0; i < N; i++) out[i] = sqrt_fix<SQ>(out[i], kn[i], wd[i], wu[i]);
    } else {
#pragma unroll
        for (int i = 0; i < N; i++) kn[i] = sqrt_key(v[i]);
#pragma unroll
        for (int i = 0; i < N; i++) wd[i] = m.down[kn[i] >> 5];
#pragma unroll
        for (int i = 0; i < N; i++) wu[i] = UP ? m.up[kn[i] >> 5] : 0u;
#pragma unroll
        for (int i = 0; i < N; i++) out[i] = sqrt_fix_plain<SQ>(v[i], kn[i], wd[i], wu[i]);
    }
}

// imatrix weights w[i] = qw[i] * sqrt_ref(sigma2 + x[i]^2) (e.g. q4_k.py:51),
// with the imatrix and map loads of CH values issued together (CH < N bounds
// the registers the phase holds, for kernels whose occupancy it would set)
template <int N, bool BAND, int SQ, int CH = N>
QS_DEV void imatrix_weights(const float* __restrict__ qw, float sigma2, const float (&x)[N],
                            const SqrtMap& m, float (&w)[N]) {
    static_assert(N % CH == 0, "chunks tile the group");
#pragma unroll
    for (int c = 0; c < N; c += CH) {
        float v[CH], q[CH];
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const float t = x[c + i] * x[c + i];
            v[i] = sigma2 + t;
            q[i] = qw[c + i];
        }
        float r[CH];
        sqrt_ref_n<CH, BAND, SQ>(v, m, r);
#pragma unroll
        for (int i = 0; i < CH; i++) {
            w[c + i] = q[i] * r[i];
            if constexpr (CH < N) keep_in_register(w[c + i]);
        }
    }
}

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
                const u32x4 u = load_stream16(p + 8 * j);
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
                const u32x4 u = load_stream16(p + 8 * j);
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
                const u32x4 u = load_stream16(p + 4 * j);
                // copy the lanes out before reinterpreting them: hipcc narrows
                // the load to one dword when __builtin_bit_cast is applied to
                // an ext_vector element directly
                const uint32_t v[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int t = 0; t < 4; t++) out[4 * j + t] = __builtin_bit_cast(float, v[t]);
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
// cascade8_of takes the values as f(0) .. f(N-1), each computed where the sum
// needs it, so no array of N values is ever live.
template <int N, typename F>
QS_DEV float cascade8_of(F&& f) {
    static_assert(N == 8 || N == 16 || N == 32, "cascade8_of: N in {8,16,32}");
    float fin = 0.0f;
#pragma unroll
    for (int l = 0; l < 8; l++) {
        float p;
        if constexpr (N == 32) {
            p = f(l) + f(8 + l);
            p = p + f(16 + l);
            p = p + f(24 + l);
        } else if constexpr (N == 16) {
            p = 0.0f + f(l);
            p = p + f(8 + l);
        } else {
            p = 0.0f + f(l);
        }
        fin = fin + p;
    }
    return fin;
}

template <int N>
QS_DEV float cascade8_sum(const float (&v)[N]) {
    return cascade8_of<N>([&](int i) { return v[i]; });
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
