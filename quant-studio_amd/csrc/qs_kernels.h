// Quantizer kernels for the 32-value block formats (Q4_0, Q4_1, Q5_0, Q5_1,
// Q8_0), Q2_K..Q6_K, IQ4_XS and IQ4_NL on gfx950.
//
// The 32-value formats are HBM-bound: four lanes per block, 16-byte coalesced
// loads, cross-lane absmax / min / max, output staged through LDS and stored
// with coalesced words.
//
// The K-quants and IQ4_XS are VALU-bound (their scale searches cost hundreds of
// f32 ops per value): one lane per 16/32-value group keeps the group and its
// sequential candidate chain in registers, one 64-lane workgroup covers 4 or 8
// superblocks, and the superblock-level steps (sums over 256 values, the
// sub-scale fits) exchange data through LDS.
#pragma once

#include "qs_fits.h"
#include "qs_wave.h"

namespace qs {

struct KArgs {
    const void* src;      // source rows (F32 / F16 / BF16)
    int64_t n_units;      // superblocks (or Q4_0 blocks)
    int64_t units_per_row;
    int64_t stride;       // source row stride in elements
    const float* qw;      // k imatrix weights or nullptr
    uint8_t* dst;         // packed output, n_units * block bytes
    SqrtMap sqrt;         // square-root rounding of the weights (sqrt_ref)
};

struct QpSteps {
    float v[8];
};

// ------------------------------------------------------------------
// 32-value block formats: Q4_0 (q4_0.py:14-33) and the ggml formats the
// reference has no module for (its command line stops on them,
// quant-studio.py:396-399): Q4_1, Q5_0, Q5_1, Q8_0. Those follow ggml's block
// layouts and reference quantizers (quantize_row_q4_1_ref ... _q8_0_ref) with
// the conventions of the reference's Q4_0: first-index signed absmax, IEEE
// division, one rounding per operation. The imatrix is not used by any of
// them (as for the reference's Q4_0, q4_0.py:36-37).
// ------------------------------------------------------------------
enum class B32 { Q4_0, Q4_1, Q5_0, Q5_1, Q8_0 };

template <B32 T>
constexpr int b32_bytes() {
    return T == B32::Q4_0 ? 18 : T == B32::Q4_1 ? 20 : T == B32::Q5_0 ? 22 : T == B32::Q5_1 ? 24 : 34;
}

constexpr int Q40_TILE = 64;                   // blocks per 256-thread tile (4 lanes per block)
constexpr int Q40_TILES = 4;                   // tiles per workgroup, loaded before any compute
constexpr int Q40_BLOCKS_PER_WG = Q40_TILE * Q40_TILES;

// Lane (lane ^ M) of the lane's group of four (M = 1 or 2): a DPP quad
// permute, a VALU move with no LDS round trip (a width-4 __shfl_xor compiles
// to ds_bpermute and a wait on LDS). Every lane of the group must be active.
template <int M>
QS_DEV uint32_t quad_xor(uint32_t v) {
    static_assert(M == 1 || M == 2, "quad lanes");
    constexpr int ctrl = M == 1 ? 0xB1 : 0x4E;     // quad_perm:[1,0,3,2] / [2,3,0,1]
    // bound_ctrl: a quad permute never reads outside the row, so no lane keeps
    // the (unused) old value
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, ctrl, 0xF, 0xF, true);
}
template <int M>
QS_DEV float quad_xor(float v) {
    return __builtin_bit_cast(float, quad_xor<M>(__builtin_bit_cast(uint32_t, v)));
}

// Magnitude of v as an ordered key: the float order for finite and infinite
// values, every NaN one above Inf and equal to every other NaN, so the first
// NaN of a block is its maximum, as torch's argmax of |x| takes it
// (q4_0.py:21-22)
QS_DEV uint32_t mag_key(float v) {
    return min(__float_as_uint(v) & 0x7fffffffu, 0x7f800001u);
}

// one round of the quarters' absmax merge: take the partner's (max, value)
// when its max is larger, or equal and the partner is the lower quarter
template <int M>
QS_DEV void quad_absmax_round(uint32_t& am, float& mv, int q) {
    const uint32_t pam = quad_xor<M>(am);
    const float pmv = quad_xor<M>(mv);
    const bool take = (pam > am) | ((pam == am) & ((q ^ M) < q));
    am = take ? pam : am;
    mv = take ? pmv : mv;
}

// signed value of the largest |x| of the block, first index wins (argmax of
// abs, a NaN above everything): the lane's max key, then its first value of
// that key, then the lowest quarter holding the block's max
QS_DEV float quad_absmax_first(const float (&x)[8], int q) {
    uint32_t key[8];
#pragma unroll
    for (int i = 0; i < 8; i++) key[i] = mag_key(x[i]);
    uint32_t am = key[0];
#pragma unroll
    for (int i = 1; i < 8; i++) am = max(am, key[i]);
    float mv = x[7];
#pragma unroll
    for (int i = 6; i >= 0; i--) mv = key[i] == am ? x[i] : mv;
    quad_absmax_round<1>(am, mv, q);
    quad_absmax_round<2>(am, mv, q);
    return mv;
}

QS_DEV void quad_min_max(const float (&x)[8], float& mn, float& mx) {
    mn = x[0];
    mx = x[0];
#pragma unroll
    for (int i = 1; i < 8; i++) {
        mn = fminf(mn, x[i]);
        mx = fmaxf(mx, x[i]);
    }
    mn = fminf(mn, quad_xor<1>(mn));
    mx = fmaxf(mx, quad_xor<1>(mx));
    mn = fminf(mn, quad_xor<2>(mn));
    mx = fmaxf(mx, quad_xor<2>(mx));
}

// The lane's 8 levels (each < 256) as bytes: w[0] = L0..L3, w[1] = L4..L7
QS_DEV void bytes_of(const uint32_t (&l)[8], uint32_t (&w)[2]) {
#pragma unroll
    for (int h = 0; h < 2; h++)
        w[h] = l[4 * h] | (l[4 * h + 1] << 8) | (l[4 * h + 2] << 16) | (l[4 * h + 3] << 24);
}

// qs[j] = L[j] & 15 | (L[j+16] & 15) << 4 from the lanes' level bytes:
// quarters 0/1 hold the low halves and take the high nibbles of quarters 2/3
// (one exchange per word); writes 8 bytes at o (q < 2), o 2-byte aligned
QS_DEV void quad_store_nibbles(const uint32_t (&w)[2], int q, uint8_t* o) {
    const uint32_t hi0 = quad_xor<2>(w[0]), hi1 = quad_xor<2>(w[1]);
    if (q < 2) {
        const uint32_t w0 = (w[0] & 0x0f0f0f0fu) | ((hi0 & 0x0f0f0f0fu) << 4);
        const uint32_t w1 = (w[1] & 0x0f0f0f0fu) | ((hi1 & 0x0f0f0f0fu) << 4);
        uint16_t* o16 = reinterpret_cast<uint16_t*>(o + 8 * q);
        o16[0] = (uint16_t)w0;
        o16[1] = (uint16_t)(w0 >> 16);
        o16[2] = (uint16_t)w1;
        o16[3] = (uint16_t)(w1 >> 16);
    }
}

// one block, four lanes: lane quarter q holds values 8q..8q+7 and writes its
// share of the block's bytes at o (LDS, block start, 2-byte aligned)
template <B32 T>
QS_DEV void b32_block(const float (&x)[8], int q, uint8_t* o) {
    uint16_t* o16 = reinterpret_cast<uint16_t*>(o);
    if constexpr (T == B32::Q4_0 || T == B32::Q5_0) {
        // d = max / -8 (q4_0.py:24) or max / -16: exact scalings by a power of two
        const float mv = quad_absmax_first(x, q);
        const float d = T == B32::Q4_0 ? mv * -0.125f : mv * -0.0625f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        constexpr float OFF = T == B32::Q4_0 ? 8.5f : 16.5f;
        constexpr float TOP = T == B32::Q4_0 ? 15.5f : 31.5f;
        uint32_t l[8], w[2], h5 = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float t = x[i] * id;
            t = t + OFF;
            // clamp(floor(t), 0, top) == trunc(clamp(t, 0, top + 0.5)): truncation
            // is floor on [0, top + 0.5] (NaN clamps to 0 either way)
            l[i] = (uint32_t)clampf(t, 0.0f, TOP);
            if constexpr (T == B32::Q5_0) h5 |= (l[i] >> 4) << i;
        }
        bytes_of(l, w);
        if (q == 0) o16[0] = (uint16_t)f16_bits(d);
        if constexpr (T == B32::Q4_0) {
            quad_store_nibbles(w, q, o + 2);
        } else {
            o[2 + q] = (uint8_t)h5;                 // qh: bit j is bit 4 of L[j]
            quad_store_nibbles(w, q, o + 6);
        }
    } else if constexpr (T == B32::Q4_1 || T == B32::Q5_1) {
        // d = (max - min) / nmax, m = min; L = min(nmax, trunc((x - min) * id + 0.5))
        constexpr float NMAX = T == B32::Q4_1 ? 15.0f : 31.0f;
        float mn, mx;
        quad_min_max(x, mn, mx);
        const float d = (mx - mn) / NMAX;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint32_t l[8], w[2], h5 = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float t = x[i] - mn;
            t = t * id;
            t = t + 0.5f;
            l[i] = (uint32_t)clampf(t, 0.0f, NMAX);
            if constexpr (T == B32::Q5_1) h5 |= (l[i] >> 4) << i;
        }
        bytes_of(l, w);
        if (q == 0) {
            o16[0] = (uint16_t)f16_bits(d);
            o16[1] = (uint16_t)f16_bits(mn);
        }
        if constexpr (T == B32::Q4_1) {
            quad_store_nibbles(w, q, o + 4);
        } else {
            o[4 + q] = (uint8_t)h5;
            quad_store_nibbles(w, q, o + 8);
        }
    } else {
        // Q8_0: d = amax / 127, q = round half away from zero (C roundf)
        float am = fabsf(x[0]);
#pragma unroll
        for (int i = 1; i < 8; i++) am = fmaxf(am, fabsf(x[i]));
        am = fmaxf(am, quad_xor<1>(am));
        am = fmaxf(am, quad_xor<2>(am));
        const float d = am / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint32_t w[2] = {0u, 0u};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            // where 1/d overflowed (d below 127 * 2^-128) x * id is infinite or
            // NaN: saturate to [-128, 127], NaN to 0, instead of an undefined
            // conversion
            const float r = roundf(x[i] * id);
            const int v = r == r ? (int)clampf(r, -128.0f, 127.0f) : 0;
            w[i >> 2] |= ((uint32_t)v & 0xffu) << (8 * (i & 3));
        }
        if (q == 0) o16[0] = (uint16_t)f16_bits(d);
        uint16_t* p = reinterpret_cast<uint16_t*>(o + 2 + 8 * q);
        p[0] = (uint16_t)w[0];
        p[1] = (uint16_t)(w[0] >> 16);
        p[2] = (uint16_t)w[1];
        p[3] = (uint16_t)(w[1] >> 16);
    }
}

// HBM-bound: four lanes per 32-value block, four tiles of 16-byte loads in
// flight per lane, output staged through LDS and stored with 16-byte words
template <int SRC, B32 T>
__global__ __launch_bounds__(256) void k_b32(KArgs a) {
    constexpr int BYTES = b32_bytes<T>();
    __shared__ __attribute__((aligned(16))) uint8_t stage[Q40_BLOCKS_PER_WG * BYTES];
    const int tid = threadIdx.x;
    const int q = tid & 3;                       // quarter of the block: values 8q..8q+7
    const int64_t b0 = (int64_t)blockIdx.x * Q40_BLOCKS_PER_WG;
    float x[Q40_TILES][8];
    // issue every tile's 16-byte loads first: 16 KB of bf16 in flight per workgroup.
    // Rows stored back to back (the usual case) index the source flat; only
    // padded rows pay for the 64-bit division into row and column.
    const bool flat = a.stride == a.units_per_row * 32;
#pragma unroll
    for (int u = 0; u < Q40_TILES; u++) {
        int64_t b = b0 + u * Q40_TILE + (tid >> 2);
        b = b < a.n_units ? b : a.n_units - 1;
        int64_t e;
        if (flat) {
            e = b * 32 + 8 * q;
        } else {
            const int64_t row = b / a.units_per_row;
            e = row * a.stride + (b - row * a.units_per_row) * 32 + 8 * q;
        }
        load_elems<SRC, true, 8>(a.src, e, x[u]);
    }
#pragma unroll
    for (int u = 0; u < Q40_TILES; u++) b32_block<T>(x[u], q, stage + (u * Q40_TILE + (tid >> 2)) * BYTES);
    __syncthreads();
    const int64_t nvalid = min((int64_t)Q40_BLOCKS_PER_WG, a.n_units - b0);
    const int nbytes = (int)nvalid * BYTES;
    uint8_t* dbase = a.dst + b0 * BYTES;
    if ((reinterpret_cast<uintptr_t>(dbase) & 15) == 0) {
        const int n16 = nbytes >> 4;
        const uint4* s16 = reinterpret_cast<const uint4*>(stage);
        uint4* d16 = reinterpret_cast<uint4*>(dbase);
        // streamed out with non-temporal stores: 8-12% faster on 33-50 MB
        // tensors than plain stores, which keep the output in L2
        for (int t = tid; t < n16; t += 256)
            __builtin_nontemporal_store(reinterpret_cast<const u32x4*>(s16)[t], reinterpret_cast<u32x4*>(d16) + t);
        for (int t = (n16 << 4) + tid; t < nbytes; t += 256) dbase[t] = stage[t];
    } else if ((reinterpret_cast<uintptr_t>(dbase) & 3) == 0) {
        const int nw = nbytes >> 2;
        const uint32_t* s4 = reinterpret_cast<const uint32_t*>(stage);
        uint32_t* d4 = reinterpret_cast<uint32_t*>(dbase);
        for (int t = tid; t < nw; t += 256) d4[t] = s4[t];
        for (int t = (nw << 2) + tid; t < nbytes; t += 256) dbase[t] = stage[t];
    } else {
        for (int t = tid; t < nbytes; t += 256) dbase[t] = stage[t];
    }
}

// ------------------------------------------------------------------
// shared LDS layout of the superblock kernels
// ------------------------------------------------------------------
// The x^2 staging of the weight phase (v, tmp) and the levels and packed
// blocks of the final phase (L, out) are never live together (every kernel
// passes several wave_syncs between them), so they share storage: less LDS
// per workgroup, more resident waves.
template <int SPW, int BYTES, int VSB = SPW>
struct alignas(16) SbLds {
    union {
        struct {
            float v[VSB][QK_K];      // per-value staging for superblock sums (VSB at a time)
            float tmp[VSB][40];
        };
        struct {
            uint8_t L[SPW][QK_K];
            uint8_t out[SPW * BYTES + 16];
        };
    };
    float sc[SPW][16], mn[SPW][16], sw[SPW][16];
    float hdr[SPW][4];
    int ls[SPW][16], lm[SPW][16];
};

// finish: every valid superblock of the wave has its bytes in s.out
template <int SPW, int BYTES, int VSB>
QS_DEV void sb_store(const SbLds<SPW, BYTES, VSB>& s, const KArgs& a) {
    const int64_t first = (int64_t)blockIdx.x * SPW;
    const int64_t nvalid = min((int64_t)SPW, a.n_units - first);
    store_staged(s.out, a.dst, first * BYTES, (int)nvalid * BYTES);
}

// sb_cascade8_256 of x^2 over each superblock of the wave, staged half the
// wave's superblocks at a time (half the LDS). Every lane takes part in both
// rounds, the wave barriers included; lanes of the other half compute the
// same sums from the same staged values and discard them.
template <int LPS, int SPW, int GROUP, bool WL = false>
QS_DEV float sb_sumsq_halves(float (*v)[QK_K], float (*tmp)[40], const float (&x)[GROUP], int slot, int g) {
    static_assert(GROUP * LPS == QK_K, "the lanes of a superblock cover its values");
    constexpr int H = SPW / 2;
    const int hs = slot % H;
    float sum = 0.0f;
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const bool mine = slot / H == r;
        if (mine) {
#pragma unroll
            for (int i = 0; i < GROUP; i++) v[hs][GROUP * g + i] = x[i] * x[i];
        }
        wave_sync<WL>();
        const float t = sb_cascade8_256<LPS, WL>(v[hs], tmp[hs], g);
        sum = mine ? t : sum;
        wave_sync<WL>();                          // the next round restages v and tmp
    }
    return sum;
}

// ------------------------------------------------------------------
// Q4_K / Q5_K  (q4_k.py:25-79, q5_k.py:25-82)
// ------------------------------------------------------------------
template <int SRC, bool IMAT, int NMAX, int SQ>
// SQ: the host whose square-root rounding the weights take (SQ_*).
// Occupancy: the imatrix variant (143 VGPRs) runs 3 waves per SIMD; the other
// (131) is held to 128 for a fourth wave: its 6 spilled registers cost one
// scratch store on an accepted candidate and reloads after the candidate
// loop (measured 5% faster). Held to 128, the imatrix variant spills inside
// the loop and is 7% slower.
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(IMAT ? 3 : 4))) void k_q45_k(KArgs a, Steps steps, QpSteps qps) {
    constexpr int LPS = 8, SPW = 8, BYTES = NMAX == 15 ? 144 : 176;
    constexpr float FMAX = (float)NMAX;
    // the imatrix path stages x^2 of all 8 superblocks for sigma2; the other
    // keeps no per-value staging (its weights need only the lane's own sum)
    __shared__ SbLds<SPW, BYTES, IMAT ? SPW : 1> s;
    const SbPos p = sb_pos<LPS, 32>(a.n_units, a.units_per_row, a.stride);
    const int slot = p.slot, g = p.g;
    float x[32], w[32];
    load_elems<SRC, true, 32>(a.src, p.elem, x);

    if constexpr (IMAT) {
#pragma unroll
        for (int i = 0; i < 32; i++) s.v[slot][32 * g + i] = x[i] * x[i];
        wave_sync();
        const float sum = sb_cascade8_256<LPS>(s.v[slot], s.tmp[slot], g);
        const float sigma2 = (2.0f * sum) / 256.0f;
        imatrix_weights<32, true, SQ>(a.qw + p.col, sigma2, x, a.sqrt, w);
    } else {
        float t[32];
#pragma unroll
        for (int i = 0; i < 32; i++) t[i] = x[i] * x[i];
        const float av = sqrt_ref<SQ>(cascade8_sum(t) / 32.0f, a.sqrt);
#pragma unroll
        for (int i = 0; i < 32; i++) w[i] = av + fabsf(x[i]);
    }

    const QkxResult r = qkx_fit<32, false, IMAT>(x, w, steps, FMAX);
    s.sc[slot][g] = r.scale;
    s.mn[slot][g] = r.the_min;
    if constexpr (IMAT) s.sw[slot][g] = cascade8_sum(w);
    wave_sync();

    int ls, lm;
    float d16, m16;
    if constexpr (IMAT) {
        // make_qp over the 8 scales (lanes 0-3 of the superblock) and the 8
        // mins (lanes 4-7), each fit's trials spread over its four lanes;
        // the exchange reuses the sigma2 scratch
        const int f = g >> 2, c = g & 3;
        {
            float xv[8], wv[8], L[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                xv[i] = f == 0 ? s.sc[slot][i] : s.mn[slot][i];
                wv[i] = s.sw[slot][i];
            }
            const float sc = qp_fit_spread<8, 4>(xv, wv, 63, qps.v, L, c, s.tmp[slot] + 18 * f);
            if (c == 0) {
                s.hdr[slot][f] = sc;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const int li = (int)L[i] & 0xFF;
                    if (f == 0) s.ls[slot][i] = li;
                    else s.lm[slot][i] = li;
                }
            }
        }
        wave_sync();
        d16 = f16_round(s.hdr[slot][0]);
        m16 = f16_round(s.hdr[slot][1]);
        ls = s.ls[slot][g];
        lm = s.lm[slot][g];
    } else {
        float ms = s.sc[slot][0], mm = s.mn[slot][0];
#pragma unroll
        for (int j = 1; j < 8; j++) {
            ms = fmaxf(ms, s.sc[slot][j]);
            mm = fmaxf(mm, s.mn[slot][j]);
        }
        const float inv_s = ms > 0 ? rdiv(63.0f, ms) : 0.0f;
        const float inv_m = mm > 0 ? rdiv(63.0f, mm) : 0.0f;
        const int la = (int)rintf(inv_s * r.scale) & 0xFF, lb = (int)rintf(inv_m * r.the_min) & 0xFF;
        ls = la > 63 ? 63 : la;
        lm = lb > 63 ? 63 : lb;
        d16 = f16_round(ms / 63.0f);
        m16 = f16_round(mm / 63.0f);
        wave_sync();
        s.ls[slot][g] = ls;
        s.lm[slot][g] = lm;
    }

    const float dg = d16 * (float)(ls & 63), mg = m16 * (float)(lm & 63);
#pragma unroll
    for (int i = 0; i < 32; i++) {
        float v;
        if (dg != 0.0f) {
            const float t = x[i] + mg;
            v = clampf(rintf(t / dg), 0.0f, FMAX);
        } else {
            v = qkx_level(r, x[i], FMAX);
        }
        s.L[slot][32 * g + i] = (uint8_t)(int)v;
    }
    if (g == 0) {
        s.hdr[slot][2] = __builtin_bit_cast(float, f16_bits(d16));
        s.hdr[slot][3] = __builtin_bit_cast(float, f16_bits(m16));
    }
    wave_sync();

    // pack (q4_k.py:70-78, q5_k.py:70-81)
    const uint8_t* L = s.L[slot];
    const int* LS = s.ls[slot];
    const int* LM = s.lm[slot];
    uint8_t* o = s.out + slot * BYTES;
    const uint32_t dbits = __builtin_bit_cast(uint32_t, s.hdr[slot][2]);
    const uint32_t mbits = __builtin_bit_cast(uint32_t, s.hdr[slot][3]);
    for (int bi = g; bi < BYTES; bi += LPS) {
        uint32_t v;
        if (bi < 2) v = dbits >> (8 * bi);
        else if (bi < 4) v = mbits >> (8 * (bi - 2));
        else if (bi < 8) { const int j = bi - 4; v = LS[j] | ((LS[4 + j] >> 4) << 6); }
        else if (bi < 12) { const int j = bi - 8; v = LM[j] | ((LM[4 + j] >> 4) << 6); }
        else if (bi < 16) { const int j = bi - 12; v = (LS[4 + j] & 15) | ((LM[4 + j] & 15) << 4); }
        else if (NMAX == 31 && bi < 48) {
            const int l = bi - 16;
            v = 0;
#pragma unroll
            for (int sb = 0; sb < 8; sb++) v |= ((L[32 * sb + l] >> 4) & 1u) << sb;
        } else {
            const int t = bi - (NMAX == 31 ? 48 : 16), j = t >> 5, l = t & 31;
            v = (L[64 * j + l] & 15u) | ((L[64 * j + 32 + l] & 15u) << 4);
        }
        o[bi] = (uint8_t)v;
    }
    wave_sync();
    sb_store(s, a);
}

// ------------------------------------------------------------------
// Q6_K  (q6_k.py:22-65)
// ------------------------------------------------------------------
template <int SRC, bool IMAT>
__global__ __launch_bounds__(64) void k_q6_k(KArgs a, Steps steps) {
    constexpr int LPS = 16, SPW = 4, BYTES = 210;
    __shared__ SbLds<SPW, BYTES> s;
    const SbPos p = sb_pos<LPS, 16>(a.n_units, a.units_per_row, a.stride);
    const int slot = p.slot, g = p.g;
    float x[16], w[16];
    load_elems<SRC, true, 16>(a.src, p.elem, x);
#pragma unroll
    for (int i = 0; i < 16; i++) w[i] = IMAT ? a.qw[p.col + i] : x[i] * x[i];

    const QxResult r = qx_fit<16>(x, w, 32, steps);
    s.sc[slot][g] = r.scale;
    wave_sync();
    float sc16[16];
#pragma unroll
    for (int j = 0; j < 16; j++) sc16[j] = s.sc[slot][j];
    float amax;
    const float max_scale = absmax_first(sc16, amax);
    const bool live = amax >= GROUP_MAX_EPS;
    const float iscale = rdiv(-128.0f, live ? max_scale : 1.0f);
    const float d16 = f16_round(live ? 1.0f / iscale : 0.0f);
    int sc8 = (int)fminf(rintf(iscale * r.scale), 127.0f);
    sc8 = ((sc8 & 0xFF) ^ 0x80) - 0x80;
    const float dq = d16 * (float)sc8;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        float v;
        if (dq != 0.0f) v = clampf(rintf(x[i] / dq), -32.0f, 31.0f) + 32.0f;
        else v = qx_level(r, x[i], 32.0f);
        s.L[slot][16 * g + i] = live ? (uint8_t)(int)v : (uint8_t)0;
    }
    s.ls[slot][g] = live ? sc8 : 0;
    if (g == 0) s.hdr[slot][0] = __builtin_bit_cast(float, f16_bits(d16));
    wave_sync();

    // pack (q6_k.py:55-64)
    const uint8_t* L = s.L[slot];
    uint8_t* o = s.out + slot * BYTES;
    const uint32_t dbits = __builtin_bit_cast(uint32_t, s.hdr[slot][0]);
    for (int bi = g; bi < BYTES; bi += LPS) {
        uint32_t v;
        if (bi < 128) {
            const int h = bi >> 6, rr = bi & 63;
            const uint8_t* q = L + 128 * h + (rr & 31) + (rr >= 32 ? 32 : 0);
            v = (q[0] & 15u) | ((q[64] & 15u) << 4);
        } else if (bi < 192) {
            const int t = bi - 128, h = t >> 5, l = t & 31;
            const uint8_t* q = L + 128 * h + l;
            v = (q[0] >> 4) | ((q[32] >> 4) << 2) | ((q[64] >> 4) << 4) | ((q[96] >> 4) << 6);
        } else if (bi < 208) {
            v = (uint32_t)s.ls[slot][bi - 192] & 0xFFu;
        } else {
            v = dbits >> (8 * (bi - 208));
        }
        o[bi] = (uint8_t)v;
    }
    wave_sync();
    sb_store(s, a);
}

// ------------------------------------------------------------------
// Q3_K  (q3_k.py:23-78)
// ------------------------------------------------------------------
template <int SRC, bool IMAT, int SQ>
__global__ __launch_bounds__(64) void k_q3_k(KArgs a, Steps steps4, Steps steps32) {
    constexpr int LPS = 16, SPW = 4, BYTES = 110;
    __shared__ SbLds<SPW, BYTES> s;
    const SbPos p = sb_pos<LPS, 16>(a.n_units, a.units_per_row, a.stride);
    const int slot = p.slot, g = p.g;
    float x[16];
    load_elems<SRC, true, 16>(a.src, p.elem, x);

    float Lg[16];
    int ls6;
    float d16;
    if constexpr (!IMAT) {
        const float scale = q3_fit<16>(x, 4, Lg);
        s.sc[slot][g] = scale;
        wave_sync();
        float sc16[16];
#pragma unroll
        for (int j = 0; j < 16; j++) sc16[j] = s.sc[slot][j];
        float amax;
        const float max_scale = absmax_first(sc16, amax);
        const bool has = max_scale != 0.0f;
        const float iscale = rdiv(-32.0f, has ? max_scale : 1.0f);
        int l = (int)rintf(iscale * scale);
        l = ((l & 0xFF) ^ 0x80) - 0x80;
        l = l < -32 ? -32 : (l > 31 ? 31 : l);
        ls6 = has ? l + 32 : 0;
        d16 = f16_round(has ? 1.0f / iscale : 0.0f);
    } else {
        float w[16];
#pragma unroll
        for (int i = 0; i < 16; i++) s.v[slot][16 * g + i] = x[i] * x[i];
        wave_sync();
        const float sigma2 = (2.0f * sb_seq_256(s.v[slot])) / 256.0f;
        imatrix_weights<16, true, SQ>(a.qw + p.col, sigma2, x, a.sqrt, w);
        const QxResult r = qx_fit<16>(x, w, 4, steps4);
#pragma unroll
        for (int i = 0; i < 16; i++) Lg[i] = qx_level(r, x[i], 4.0f);
        s.sc[slot][g] = r.scale;
        s.sw[slot][g] = seq_sum(w);
        wave_sync();
        {
            // make_qx over the 16 sub-block scales, its 19 trials spread over
            // the superblock's 16 lanes; the exchange reuses the x^2 staging
            float sc16[16], sw16[16];
#pragma unroll
            for (int j = 0; j < 16; j++) {
                sc16[j] = s.sc[slot][j];
                sw16[j] = s.sw[slot][j];
            }
            const QxResult r2 = qx_fit_spread<16, 16, 18>(sc16, sw16, 32, steps32, g, s.v[slot]);
            if (g == 0) s.hdr[slot][0] = r2.scale;
            s.ls[slot][g] = (int)qx_level(r2, s.sc[slot][g], 32.0f);
        }
        wave_sync();
        ls6 = s.ls[slot][g];
        d16 = f16_round(s.hdr[slot][0]);
    }

    const float dq = d16 * (float)(ls6 - 32);
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float v = dq != 0.0f ? clampf(rintf(x[i] / dq), -4.0f, 3.0f) + 4.0f : Lg[i];
        s.L[slot][16 * g + i] = (uint8_t)(int)v;
    }
    wave_sync();
    s.ls[slot][g] = ls6;
    if (g == 0) s.hdr[slot][1] = __builtin_bit_cast(float, f16_bits(d16));
    wave_sync();

    // pack (q3_k.py:61-77)
    const uint8_t* L = s.L[slot];
    const int* LS = s.ls[slot];
    uint8_t* o = s.out + slot * BYTES;
    const uint32_t dbits = __builtin_bit_cast(uint32_t, s.hdr[slot][1]);
    for (int bi = g; bi < BYTES; bi += LPS) {
        uint32_t v = 0;
        if (bi < 32) {
#pragma unroll
            for (int b = 0; b < 8; b++) v |= (L[32 * b + bi] > 3 ? 1u : 0u) << b;
        } else if (bi < 96) {
            const int t = bi - 32, h = t >> 5, l = t & 31;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint32_t q = L[128 * h + 32 * i + l];
                q = q > 3 ? q - 4 : q;
                v |= q << (2 * i);
            }
        } else if (bi < 104) {
            const int j = bi - 96;
            v = (LS[j] & 15) | ((LS[j + 8] & 15) << 4);
        } else if (bi < 108) {
            const int i = bi - 104;
            v = (LS[i] >> 4) | ((LS[4 + i] >> 4) << 2) | ((LS[8 + i] >> 4) << 4) | ((LS[12 + i] >> 4) << 6);
        } else {
            v = dbits >> (8 * (bi - 108));
        }
        o[bi] = (uint8_t)v;
    }
    wave_sync();
    sb_store(s, a);
}

// ------------------------------------------------------------------
// Q2_K  (q2_k.py:25-81)
// ------------------------------------------------------------------
template <int SRC, bool IMAT, int SQ>
__global__ __launch_bounds__(64) void k_q2_k(KArgs a, Steps steps, QpSteps qps) {
    constexpr int LPS = 16, SPW = 4, BYTES = 84;
    __shared__ SbLds<SPW, BYTES> s;
    const SbPos p = sb_pos<LPS, 16>(a.n_units, a.units_per_row, a.stride);
    const int slot = p.slot, g = p.g;
    float x[16], w[16];
    load_elems<SRC, true, 16>(a.src, p.elem, x);

    QkxResult r;
    int ls, lm;
    float d16, m16;
    if constexpr (!IMAT) {
#pragma unroll
        for (int i = 0; i < 16; i++) w[i] = fabsf(x[i]);
        r = qkx_fit<16, true>(x, w, steps, 3.0f);
        s.sc[slot][g] = r.scale;
        s.mn[slot][g] = r.the_min;
        wave_sync();
        float ms = s.sc[slot][0], mm = s.mn[slot][0];
#pragma unroll
        for (int j = 1; j < 16; j++) {
            ms = fmaxf(ms, s.sc[slot][j]);
            mm = fmaxf(mm, s.mn[slot][j]);
        }
        const bool pos_s = ms > 0, pos_m = mm > 0;
        const float inv_s = pos_s ? 15.0f / ms : 0.0f;
        const float inv_m = pos_m ? 15.0f / mm : 0.0f;
        ls = (int)rintf(inv_s * r.scale) & 0xFF;
        lm = (int)rintf(inv_m * r.the_min) & 0xFF;
        d16 = f16_round(pos_s ? ms / 15.0f : 0.0f);
        m16 = f16_round(pos_m ? mm / 15.0f : 0.0f);
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) s.v[slot][16 * g + i] = x[i] * x[i];
        wave_sync();
        const float sigma2 = sb_cascade8_256<LPS>(s.v[slot], s.tmp[slot], g) / 256.0f;
        imatrix_weights<16, true, SQ>(a.qw + p.col, sigma2, x, a.sqrt, w);
        r = qkx_fit<16, false>(x, w, steps, 3.0f);
        s.sc[slot][g] = r.scale;
        s.mn[slot][g] = r.the_min;
        s.sw[slot][g] = cascade8_sum(w);
        wave_sync();
        {
            // the 16 scales on lanes 0-7 of the superblock, the 16 mins on
            // lanes 8-15, each fit's trials spread over its eight lanes
            const int f = g >> 3, c = g & 7;
            float xv[16], wv[16], L[16];
#pragma unroll
            for (int i = 0; i < 16; i++) {
                xv[i] = f == 0 ? s.sc[slot][i] : s.mn[slot][i];
                wv[i] = s.sw[slot][i];
            }
            const float sc = qp_fit_spread<16, 8>(xv, wv, 15, qps.v, L, c, s.tmp[slot] + 18 * f);
            if (c == 0) {
                s.hdr[slot][f] = sc;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int li = (int)L[i] & 0xFF;
                    if (f == 0) s.ls[slot][i] = li;
                    else s.lm[slot][i] = li;
                }
            }
        }
        wave_sync();
        d16 = f16_round(s.hdr[slot][0]);
        m16 = f16_round(s.hdr[slot][1]);
        ls = s.ls[slot][g];
        lm = s.lm[slot][g];
    }
    const int scb = (ls | (lm << 4)) & 0xFF;
    const float dg = d16 * (float)(scb & 15), mg = m16 * (float)(scb >> 4);
#pragma unroll
    for (int i = 0; i < 16; i++) {
        float v;
        if (dg != 0.0f) {
            const float t = x[i] + mg;
            v = clampf(rintf(t / dg), 0.0f, 3.0f);
        } else {
            v = qkx_level(r, x[i], 3.0f);
        }
        s.L[slot][16 * g + i] = (uint8_t)(int)v;
    }
    wave_sync();
    s.ls[slot][g] = scb;
    if (g == 0) {
        s.hdr[slot][2] = __builtin_bit_cast(float, f16_bits(d16));
        s.hdr[slot][3] = __builtin_bit_cast(float, f16_bits(m16));
    }
    wave_sync();

    // pack (q2_k.py:74-80)
    const uint8_t* L = s.L[slot];
    uint8_t* o = s.out + slot * BYTES;
    const uint32_t dbits = __builtin_bit_cast(uint32_t, s.hdr[slot][2]);
    const uint32_t mbits = __builtin_bit_cast(uint32_t, s.hdr[slot][3]);
    for (int bi = g; bi < BYTES; bi += LPS) {
        uint32_t v = 0;
        if (bi < 16) v = (uint32_t)s.ls[slot][bi];
        else if (bi < 80) {
            const int t = bi - 16, h = t >> 5, l = t & 31;
#pragma unroll
            for (int i = 0; i < 4; i++) v |= (uint32_t)L[128 * h + 32 * i + l] << (2 * i);
        } else if (bi < 82) v = dbits >> (8 * (bi - 80));
        else v = mbits >> (8 * (bi - 82));
        o[bi] = (uint8_t)v;
    }
    wave_sync();
    sb_store(s, a);
}

// ------------------------------------------------------------------
// IQ4_XS  (iq4_xs.py:149-188)
// ------------------------------------------------------------------
template <int SRC, bool IMAT, int SQ>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(3))) void k_iq4_xs(KArgs a) {
    constexpr int LPS = 8, SPW = 8, BYTES = 136;
    // LDS is what limits this kernel's residency: the imatrix path stages x^2
    // for sigma2 half the wave's superblocks at a time, the other stages none
    __shared__ SbLds<SPW, BYTES, IMAT ? SPW / 2 : 1> s;
    __shared__ float2 iq4tab[256];
    __shared__ uint8_t iq4mu[256];
    iq4_build_table(iq4tab, iq4mu);
    const SbPos p = sb_pos<LPS, 32>(a.n_units, a.units_per_row, a.stride);
    const int slot = p.slot, g = p.g;
    float x[32], w[32];
    load_elems<SRC, true, 32>(a.src, p.elem, x);
    if constexpr (IMAT) {
        const float sigma2 = (2.0f * sb_sumsq_halves<LPS, SPW, 32>(s.v, s.tmp, x, slot, g)) / 256.0f;
        imatrix_weights<32, true, SQ, 8>(a.qw + p.col, sigma2, x, a.sqrt, w);
    } else {
#pragma unroll
        for (int i = 0; i < 32; i++) w[i] = x[i] * x[i];
    }
    if constexpr (!IMAT) wave_sync();          // iq4tab ready (the imatrix path synced above)
    const float scale = iq4_scale_search<IMAT ? 16 : 32>(x, w, iq4tab);
    s.sc[slot][g] = scale;
    wave_sync();
    float sc8[8];
#pragma unroll
    for (int j = 0; j < 8; j++) sc8[j] = s.sc[slot][j];
    float amax;
    const float max_scale = absmax_first(sc8, amax);
    const float d = -max_scale / 32.0f;
    const float idq = d != 0.0f ? 1.0f / d : 0.0f;
    const float lsf = clampf(rintf(idq * scale), -32.0f, 31.0f);
    const float dl = d * lsf;
    const float idl = dl != 0.0f ? 1.0f / dl : 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) s.L[slot][32 * g + i] = (uint8_t)iq4_project_index(idl * x[i], iq4tab, iq4mu);
    s.ls[slot][g] = (int)(lsf + 32.0f);
    if (g == 0) s.hdr[slot][0] = __builtin_bit_cast(float, f16_bits(d));
    wave_sync();

    const uint8_t* L = s.L[slot];
    const int* LS = s.ls[slot];
    uint8_t* o = s.out + slot * BYTES;
    const uint32_t dbits = __builtin_bit_cast(uint32_t, s.hdr[slot][0]);
    for (int bi = g; bi < BYTES; bi += LPS) {
        uint32_t v;
        if (bi < 2) v = dbits >> (8 * bi);
        else if (bi < 4) {
            uint32_t hb = 0;
#pragma unroll
            for (int b = 0; b < 8; b++) hb |= (uint32_t)(LS[b] >> 4) << (2 * b);
            v = hb >> (8 * (bi - 2));
        } else if (bi < 8) {
            const int j = bi - 4;
            v = (LS[2 * j] & 15) | ((LS[2 * j + 1] & 15) << 4);
        } else {
            const int t = bi - 8, blk = t >> 4, j = t & 15;
            v = L[32 * blk + j] | (L[32 * blk + 16 + j] << 4);
        }
        o[bi] = (uint8_t)v;
    }
    wave_sync();
    sb_store(s, a);
}

// ------------------------------------------------------------------
// IQ4_NL: no module in the reference (its command line stops on the type,
// quant-studio.py:396-399). ggml's quantize_row_iq4_nl_impl with one block
// per superblock, restated with the reference's IQ4_XS conventions: weights
// x^2 or qw*sqrt(2*sum(x^2)/32 + x^2) (the `.sum(-1)` cascade over the block,
// as iq4_xs.py:158-160 over 256), the IQ4_XS block search (iq4_xs.py:52-76),
// d = fp16(scale), levels reprojected at 1/scale with the same LUT rule.
// One lane per block, 64 blocks per workgroup.
// ------------------------------------------------------------------
template <int SRC, bool IMAT, int SQ>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(3))) void k_iq4_nl(KArgs a) {
    constexpr int BYTES = 18;
    __shared__ __attribute__((aligned(16))) uint8_t stage[64 * BYTES];
    __shared__ float2 iq4tab[256];
    __shared__ uint8_t iq4mu[256];
    iq4_build_table(iq4tab, iq4mu);
    const int lane = threadIdx.x;
    const int64_t b0 = (int64_t)blockIdx.x * 64;
    int64_t b = b0 + lane;
    b = b < a.n_units ? b : a.n_units - 1;
    const int64_t row = b / a.units_per_row;
    const int64_t col = (b - row * a.units_per_row) * 32;
    float x[32], w[32];
    load_elems<SRC, true, 32>(a.src, row * a.stride + col, x);
    if constexpr (IMAT) {
        const float sigma2 = (2.0f * cascade8_of<32>([&](int i) { return x[i] * x[i]; })) / 32.0f;
        imatrix_weights<32, true, SQ, 8>(a.qw + col, sigma2, x, a.sqrt, w);
    } else {
#pragma unroll
        for (int i = 0; i < 32; i++) w[i] = x[i] * x[i];
    }
    wave_sync();                                 // iq4tab ready
    const float scale = iq4_scale_search<IMAT ? 16 : 32>(x, w, iq4tab);
    const float id = scale != 0.0f ? 1.0f / scale : 0.0f;
    uint8_t* o = stage + lane * BYTES;
    const uint32_t h = f16_bits(scale);
    o[0] = (uint8_t)h;
    o[1] = (uint8_t)(h >> 8);
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const int lo = iq4_project_index(id * x[j], iq4tab, iq4mu);
        const int hi = iq4_project_index(id * x[j + 16], iq4tab, iq4mu);
        o[2 + j] = (uint8_t)(lo | (hi << 4));
    }
    wave_sync();
    const int64_t nvalid = min((int64_t)64, a.n_units - b0);
    const int nbytes = (int)nvalid * BYTES;
    uint8_t* dbase = a.dst + b0 * BYTES;
    if ((reinterpret_cast<uintptr_t>(dbase) & 3) == 0) {
        const int nw = nbytes >> 2;
        const uint32_t* s4 = reinterpret_cast<const uint32_t*>(stage);
        uint32_t* d4 = reinterpret_cast<uint32_t*>(dbase);
        for (int t = lane; t < nw; t += 64) d4[t] = s4[t];
        for (int t = (nw << 2) + lane; t < nbytes; t += 64) dbase[t] = stage[t];
    } else {
        for (int t = lane; t < nbytes; t += 64) dbase[t] = stage[t];
    }
}

}  // namespace qs
