/*
 * CPU oracle for the GGUF block quantizers -- TEST INFRASTRUCTURE ONLY
 * (the expected bytes for tests/, smoke() and the CPU-baseline leg of bench.py;
 * never linked into the product library).
 *
 * Restates the reference's eager torch CPU path type by type. Conventions that
 * recur (pinned against torch 2.10 CPU and against the golden vectors written
 * from the reference itself, tests/golden/):
 *   - every torch elementwise op rounds once; a*b+c is two roundings (no FMA);
 *   - `python_float / tensor` is `tensor.reciprocal() * float` (RDIV below);
 *     `tensor / tensor` and `tensor / python_float` are IEEE division;
 *   - `.sum(-1)` over a contiguous row uses torch's 8-lane cascade
 *     (sum_c8), tree_sum is the adjacent-pair tree (kq_common.py:38-43) and
 *     seq_sum the left-to-right sum (qx_common.py:37-44);
 *   - torch.round is round-half-even (rintf), argmax/argmin pick the first index.
 */
#include "qs_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define QK_K 256
#define GROUP_MAX_EPS 1e-15f
#define F32_TINY 1.17549435e-38f

/* Planted-mistake switch for the tests that show the golden vectors pin each
 * convention (0 = the faithful restatement). */
static int g_mut = 0;
void qso_set_mutation(int m) { g_mut = m; }
enum { MUT_IEEE_RDIV = 1, MUT_SEQ_CASCADE = 2, MUT_SEQ_TREE = 3, MUT_DROP_STEP = 4,
       MUT_ROUND_AWAY = 5, MUT_ACCEPT_GE = 6,
       /* the 32-value formats without a reference module: d = a * (1/n) instead of
        * the IEEE a / n, and x / d instead of x * (1/d) */
       MUT_D_BY_RECIP = 7, MUT_X_DIV_D = 8,
       /* slips that only zero imatrix weights expose (every distance or error
        * ties at 0, a sum of squares is exactly 0): the last of equal neighbour
        * distances kept, make_qp's candidate accept with <=, make_qx's first
        * scale divided without its zero guard, IQ2_XXS active without
        * scale0*3 > 0 */
       MUT_IQ_LAST_MIN = 9, MUT_QP_ACCEPT_LE = 10, MUT_QX_NO_GUARD = 11, MUT_IQ2XXS_NO_EFF = 12 };

/* torch: python_float / tensor  ->  tensor.reciprocal() * python_float */
static inline float RDIV(float c, float t) {
    if (g_mut == MUT_IEEE_RDIV) return c / t;
    float r = 1.0f / t;
    return r * c;
}
static inline float RINT(float v) { return g_mut == MUT_ROUND_AWAY ? roundf(v) : rintf(v); }

/* Square root of the reference: torch.sqrt on a CPU tensor (MKL's vectorised
 * routine), which returns the float just below the IEEE root for 0.59% of
 * inputs, a set that depends only on the mantissa and the exponent's parity
 * (qs_sqrt_table.h, generated from torch.sqrt itself). sqrt_ref = IEEE sqrtf,
 * minus one ulp on that set. A test can install another routine (e.g. torch's,
 * called live) with qso_set_sqrt_hook, or plain IEEE sqrtf with
 * qso_set_sqrt_ieee. */
#include "../quant-studio_amd/csrc/qs_sqrt_table.h"

static uint32_t g_sqrt_down[1 << 19];     /* 2^24-bit map, built once */
static int g_sqrt_ready = 0;
static void sqrt_table_init(void) {
    if (g_sqrt_ready) return;
    uint32_t key = 0;
    for (int i = 0; i < QS_SQRT_DOWN_N; i++) {
        key += QS_SQRT_DOWN_GAPS[i];
        g_sqrt_down[key >> 5] |= 1u << (key & 31);
    }
    g_sqrt_ready = 1;
}

float qso_sqrt_ref(float v) {
    sqrt_table_init();
    float r = sqrtf(v);
    uint32_t b;
    memcpy(&b, &v, 4);
    if (b - 1u < 0x7f7fffffu) {                      /* 0 < v < inf */
        if (b < 0x00800000u) {                        /* subnormal: scale by 2^64 (exact) */
            float n = v * 18446744073709551616.0f;
            memcpy(&b, &n, 4);
        }
        uint32_t key = ((((b >> 23) & 1u) ^ 1u) << 23) | (b & 0x7fffffu);
        if ((g_sqrt_down[key >> 5] >> (key & 31)) & 1u) {
            uint32_t rb;
            memcpy(&rb, &r, 4);
            rb -= 1u;
            memcpy(&r, &rb, 4);
        }
    }
    return r;
}

/* Another host's torch.sqrt rounding, given as a per-key offset in ulps from
 * the IEEE root (2^24 int8 entries, same keys as above): the rounding measured
 * on a host whose MKL takes a different code path (tests only). With
 * subnormal_ieee set, subnormal inputs keep the IEEE root (the AMD EPYC host's
 * torch.sqrt does on all 2^23 - 1 of them). */
static const int8_t *g_sqrt_ulps = 0;
static int g_sqrt_sub_ieee = 0;
void qso_set_sqrt_table(const int8_t *ulps, int subnormal_ieee) {
    g_sqrt_ulps = ulps;
    g_sqrt_sub_ieee = subnormal_ieee;
}
static float sqrt_table_ulps(float v) {
    float r = sqrtf(v);
    uint32_t b;
    memcpy(&b, &v, 4);
    if (b - 1u < 0x7f7fffffu && !(g_sqrt_sub_ieee && b < 0x00800000u)) {
        if (b < 0x00800000u) {
            float n = v * 18446744073709551616.0f;
            memcpy(&b, &n, 4);
        }
        uint32_t key = ((((b >> 23) & 1u) ^ 1u) << 23) | (b & 0x7fffffu), rb;
        memcpy(&rb, &r, 4);
        rb = (uint32_t)((int32_t)rb + g_sqrt_ulps[key]);
        memcpy(&r, &rb, 4);
    }
    return r;
}

static float (*g_sqrt_hook)(float) = 0;
static int g_sqrt_ieee = 0;
void qso_set_sqrt_hook(float (*fn)(float)) { g_sqrt_hook = fn; }
void qso_set_sqrt_ieee(int on) { g_sqrt_ieee = on; }
static inline float SQRT(float v) {
    if (g_sqrt_hook) return g_sqrt_hook(v);
    if (g_sqrt_ulps) return sqrt_table_ulps(v);
    return g_sqrt_ieee ? sqrtf(v) : qso_sqrt_ref(v);
}
float qso_sqrt(float v) { return SQRT(v); }
static inline float clampf(float v, float lo, float hi) { return fminf(fmaxf(v, lo), hi); }

/* ------------------------------------------------------------------ */
/* fp16 <-> f32, round to nearest even (torch .to(float16))             */
/* ------------------------------------------------------------------ */
uint16_t qso_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u)
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u | ((ax >> 13) & 0x3ffu) : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);     /* rounds to inf */
    if (ax >= 0x38800000u) {                                       /* normal half */
        uint32_t h = ((((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13));
        uint32_t rem = ax & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (ax < 0x33000000u) return (uint16_t)sign;                   /* < 2^-25 */
    uint32_t e = ax >> 23, mant = (ax & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e;                                     /* units of 2^-24 */
    uint32_t h = mant >> shift, rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float qso_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu, x;
    if (e == 0) {
        if (m == 0) x = sign;
        else {                                                     /* subnormal: normalise */
            int s = 0;
            while (!(m & 0x400u)) { m <<= 1; s++; }
            x = sign | ((uint32_t)(113 - s) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) x = sign | 0x7f800000u | (m << 13);
    else x = sign | ((e + 112u) << 23) | (m << 13);
    float f;
    memcpy(&f, &x, 4);
    return f;
}

static inline void put_f16(uint8_t *p, float v) {
    uint16_t h = qso_f32_to_f16(v);
    p[0] = (uint8_t)(h & 0xff);
    p[1] = (uint8_t)(h >> 8);
}
static inline float f16_round(float v) { return qso_f16_to_f32(qso_f32_to_f16(v)); }

/* ------------------------------------------------------------------ */
/* reduction orders                                                    */
/* ------------------------------------------------------------------ */

/* torch 2.10 CPU `.sum(-1)` of a contiguous row (used at e.g. q4_k.py:34,
 * :49, :53; kq_common.py:109-120): 8-lane vectors, 4 lane-wise accumulators
 * fed round-robin, leftover vectors into accumulator 0, accumulators combined
 * ((a0+a1)+a2)+a3, then a scalar pass over the tail and the 8 lanes. */
float qso_sum_cascade8(const float *v, int n) {
    if (g_mut == MUT_SEQ_CASCADE) {
        float s = 0.0f;
        for (int i = 0; i < n; i++) s += v[i];
        return s;
    }
    int nv = n / 8, full = nv / 4;
    float acc[4][8];
    for (int a = 0; a < 4; a++)
        for (int l = 0; l < 8; l++) acc[a][l] = 0.0f;
    for (int i = 0; i < full; i++)
        for (int a = 0; a < 4; a++)
            for (int l = 0; l < 8; l++) acc[a][l] += v[(4 * i + a) * 8 + l];
    for (int j = 4 * full; j < nv; j++)
        for (int l = 0; l < 8; l++) acc[0][l] += v[j * 8 + l];
    float fin = 0.0f;
    for (int t = 8 * nv; t < n; t++) fin += v[t];
    for (int l = 0; l < 8; l++) {
        float p = acc[0][l] + acc[1][l];
        p = p + acc[2][l];
        p = p + acc[3][l];
        fin += p;
    }
    return fin;
}

/* tree_sum kq_common.py:38-43 (twins iq2xs_common.py:33-38, iq3_common.py:71-75) */
float qso_sum_tree(const float *v, int n) {
    if (g_mut == MUT_SEQ_TREE) {
        float s = v[0];
        for (int i = 1; i < n; i++) s += v[i];
        return s;
    }
    float t[256];
    for (int i = 0; i < n; i++) t[i] = v[i];
    for (int m = n; m > 1; m >>= 1)
        for (int i = 0; i < m / 2; i++) t[i] = t[2 * i] + t[2 * i + 1];
    return t[0];
}

/* seq_sum qx_common.py:37-44 / _seq_sum iq4_xs.py:42-49 */
static float sum_seq(const float *v, int n) {
    float s = v[0];
    for (int i = 1; i < n; i++) s = s + v[i];
    return s;
}

/* Magnitude of v as an ordered key: the float order for finite and infinite
 * values, every NaN one above Inf and equal to every other NaN. torch's
 * argmax of |x| (q4_0.py:21-22) takes the first NaN as the maximum. */
static uint32_t mag_key(float v) {
    uint32_t b;
    memcpy(&b, &v, sizeof b);
    b &= 0x7fffffffu;
    return b < 0x7f800001u ? b : 0x7f800001u;
}

/* the first index of the largest magnitude, a NaN above everything */
static int argmax_abs_nan(const float *b, int n) {
    int im = 0;
    uint32_t am = mag_key(b[0]);
    for (int i = 1; i < n; i++)
        if (mag_key(b[i]) > am) { am = mag_key(b[i]); im = i; }
    return im;
}

/* absmax_first qx_common.py:26-34: value with the largest |x|, first index wins */
static int absmax_first(const float *x, int n, float *amax) {
    int im = 0;
    float am = fabsf(x[0]);
    for (int i = 1; i < n; i++)
        if (fabsf(x[i]) > am) { am = fabsf(x[i]); im = i; }
    *amax = am;
    return im;
}

/* ------------------------------------------------------------------ */
/* candidate numerators                                                */
/* ------------------------------------------------------------------ */

/* qkx_steps kq_common.py:21-24: (rmin + rdelta*s) + nmax in f32 */
static int qkx_steps(float rmin, float rdelta, int nstep, int nmax, float *out) {
    for (int s = 0; s <= nstep; s++) {
        float t = rdelta * (float)s;
        t = rmin + t;
        out[s] = t + (float)nmax;
    }
    return nstep + 1;
}

/* qp_steps kq_common.py:27-30: 0.1*s + nmax, s in -4..4, s != 0 */
static int qp_steps(int nmax, float *out) {
    int n = 0;
    for (int s = -4; s <= 4; s++) {
        if (s == 0) continue;
        float t = 0.1f * (float)s;
        out[n++] = t + (float)nmax;
    }
    return n;
}

/* qx_steps qx_common.py:20-23: nmax + 0.1*s, s in -9..9, s != 0 */
static int qx_steps(int nmax, float *out) {
    int n = 0;
    for (int s = -9; s <= 9; s++) {
        if (s == 0) continue;
        float t = 0.1f * (float)s;
        out[n++] = (float)nmax + t;
    }
    return n;
}

/* ------------------------------------------------------------------ */
/* group fits                                                          */
/* ------------------------------------------------------------------ */

/* make_qkx_quants_eager kq_common.py:51-96 (n = 16 or 32) */
static void make_qkx(const float *x, const float *w, int n, const float *steps, int nsteps,
                     int nmax, int use_mad, float *scale_out, float *the_min_out, float *Lout) {
    float fmax = (float)nmax, tmp[32], Laux[32], L[32];
    float mn = x[0], mx = x[0];
    for (int i = 1; i < n; i++) { mn = fminf(mn, x[i]); mx = fmaxf(mx, x[i]); }
    mn = fminf(mn, 0.0f);
    int degen = (mx == mn);
    float sum_w = qso_sum_tree(w, n);
    for (int i = 0; i < n; i++) tmp[i] = w[i] * x[i];
    float sum_x = qso_sum_tree(tmp, n);

    float den = degen ? 1.0f : mx - mn;
    float iscale = fmax / den;
    float scale = 1.0f / iscale;
    for (int i = 0; i < n; i++) L[i] = clampf(RINT(iscale * (x[i] - mn)), 0.0f, fmax);
    for (int i = 0; i < n; i++) {
        float d = scale * L[i];
        d = d + mn;
        d = d - x[i];
        tmp[i] = w[i] * (use_mad ? fabsf(d) : d * d);
    }
    float best = qso_sum_tree(tmp, n);

    if (g_mut == MUT_DROP_STEP) nsteps--;
    for (int s = 0; s < nsteps; s++) {
        den = degen ? 1.0f : mx - mn;
        float isc = steps[s] / den;
        float wl[32], t2[32], t3[32];
        for (int i = 0; i < n; i++) {
            Laux[i] = clampf(RINT(isc * (x[i] - mn)), 0.0f, fmax);
            wl[i] = w[i] * Laux[i];
            t2[i] = wl[i] * Laux[i];
            t3[i] = wl[i] * x[i];
        }
        float sum_l = qso_sum_tree(wl, n), sum_l2 = qso_sum_tree(t2, n), sum_xl = qso_sum_tree(t3, n);
        float D = sum_w * sum_l2 - sum_l * sum_l;
        float Dsafe = D > 0 ? D : 1.0f;
        float this_scale = (sum_w * sum_xl - sum_x * sum_l) / Dsafe;
        float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / Dsafe;
        if (this_min > 0) {
            this_scale = sum_xl / fmaxf(sum_l2, F32_TINY);
            this_min = 0.0f;
        }
        for (int i = 0; i < n; i++) {
            float d = this_scale * Laux[i];
            d = d + this_min;
            d = d - x[i];
            tmp[i] = w[i] * (use_mad ? fabsf(d) : d * d);
        }
        float cur = qso_sum_tree(tmp, n);
        if (D > 0 && cur < best && !degen) {
            scale = this_scale;
            mn = this_min;
            best = cur;
            memcpy(L, Laux, sizeof(float) * n);
        }
    }
    if (degen) {
        scale = 0.0f;
        for (int i = 0; i < n; i++) L[i] = 0.0f;
    }
    *scale_out = scale;
    *the_min_out = (mn == 0.0f) ? 0.0f : -mn;
    memcpy(Lout, L, sizeof(float) * n);
}

/* make_qp_quants_eager kq_common.py:99-141 (n = 8 or 16); also the n = 32,
 * nmax = 4 twin _make_qp_quants iq2.py:375-415, whose candidate numerators
 * (0.1*step + 4.0) are computed in f64 and then rounded once to f32. */
static void make_qp(const float *x, const float *w, int n, int nmax, int f64_steps,
                    float *scale_out, float *Lout) {
    float fmax = (float)nmax, tmp[32], L[32], steps[8];
    float mx = x[0];
    for (int i = 1; i < n; i++) mx = fmaxf(mx, x[i]);
    int dead = mx < GROUP_MAX_EPS;
    float mxs = dead ? 1.0f : mx;

    if (f64_steps) {
        int c = 0;
        for (int s = -4; s <= 4; s++)
            if (s) steps[c++] = (float)(0.1 * s + (double)nmax);
    } else {
        qp_steps(nmax, steps);
    }

    float iscale = RDIV(fmax, mxs);
    for (int i = 0; i < n; i++) {
        float l0 = RINT(iscale * x[i]);                 /* first pass: no clamp */
        float r = (1.0f / iscale) * l0;
        float d = x[i] - r;
        tmp[i] = w[i] * (d * d);
    }
    float best_mse = qso_sum_cascade8(tmp, n);
    for (int s = 0; s < 8; s++) {
        float isc = RDIV(steps[s], mxs);
        float ri = 1.0f / isc;
        for (int i = 0; i < n; i++) {
            float l = fminf(RINT(isc * x[i]), fmax);
            float d = x[i] - ri * l;
            tmp[i] = w[i] * (d * d);
        }
        float mse = qso_sum_cascade8(tmp, n);
        if (mse < best_mse || (g_mut == MUT_QP_ACCEPT_LE && mse == best_mse)) { best_mse = mse; iscale = isc; }
    }
    for (int i = 0; i < n; i++) L[i] = fminf(RINT(iscale * x[i]), fmax);
    float t2[32];
    for (int i = 0; i < n; i++) { tmp[i] = (w[i] * x[i]) * L[i]; t2[i] = (w[i] * L[i]) * L[i]; }
    float sumlx = qso_sum_cascade8(tmp, n), suml2 = qso_sum_cascade8(t2, n);
    for (int pass = 0; pass < 5; pass++) {
        for (int i = 0; i < n; i++) {
            float xi = x[i], wi = w[i], Li = L[i];
            float slx = sumlx - (wi * xi) * Li;
            float sl2 = suml2 - (wi * Li) * Li;
            int ok = slx > 0 && sl2 > 0;
            float newl = fminf(RINT((xi * sl2) / (ok ? slx : 1.0f)), fmax);
            float slx2 = slx + (wi * xi) * newl;
            float sl22 = sl2 + (wi * newl) * newl;
            if (ok && newl != Li && (slx2 * slx2) * suml2 > (sumlx * sumlx) * sl22) {
                L[i] = newl;
                sumlx = slx2;
                suml2 = sl22;
            }
        }
    }
    float scale = suml2 > 0 ? sumlx / fmaxf(suml2, F32_TINY) : 0.0f;
    if (dead) {
        scale = 0.0f;
        for (int i = 0; i < n; i++) L[i] = 0.0f;
    }
    *scale_out = scale;
    if (Lout) memcpy(Lout, L, sizeof(float) * n);
}

/* make_qx_quants_eager qx_common.py:52-82 (n = 16) */
static void make_qx(const float *x, const float *w, int n, int nmax, float *scale_out, float *Lout) {
    float fmax = (float)nmax, tmp[16], t2[16], L[16], La[16], steps[18];
    float amax;
    float mx = x[absmax_first(x, n, &amax)];
    int live = amax >= GROUP_MAX_EPS;
    float mxs = live ? mx : 1.0f;
    qx_steps(nmax, steps);

    float iscale = RDIV(-fmax, mxs);
    for (int i = 0; i < n; i++) L[i] = clampf(RINT(iscale * x[i]), -fmax, fmax - 1.0f);
    for (int i = 0; i < n; i++) { tmp[i] = (w[i] * x[i]) * L[i]; t2[i] = (w[i] * L[i]) * L[i]; }
    float sumlx = sum_seq(tmp, n), suml2 = sum_seq(t2, n);
    float scale = (suml2 != 0 || g_mut == MUT_QX_NO_GUARD) ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int s = 0; s < 18; s++) {
        float isc = RDIV(-steps[s], mxs);
        for (int i = 0; i < n; i++) {
            La[i] = clampf(RINT(isc * x[i]), -fmax, fmax - 1.0f);
            tmp[i] = (w[i] * x[i]) * La[i];
            t2[i] = (w[i] * La[i]) * La[i];
        }
        float slx = sum_seq(tmp, n), sl2 = sum_seq(t2, n);
        if (sl2 > 0 && (g_mut == MUT_ACCEPT_GE ? slx * slx >= best * sl2 : slx * slx > best * sl2)) {
            float cand = slx / sl2;
            scale = cand;
            best = cand * slx;
            memcpy(L, La, sizeof(float) * n);
        }
    }
    *scale_out = live ? scale : 0.0f;
    for (int i = 0; i < n; i++) Lout[i] = live ? L[i] + fmax : 0.0f;
}

/* make_q3_quants_eager qx_common.py:85-121 (n = 16) */
static void make_q3(const float *x, int n, int nmax, float *scale_out, float *Lout) {
    float fmax = (float)nmax, w[16], tmp[16], t2[16], L[16];
    for (int i = 0; i < n; i++) w[i] = x[i] * x[i];
    float amax;
    float mx = x[absmax_first(x, n, &amax)];
    int live = amax >= GROUP_MAX_EPS;
    float mxs = live ? mx : 1.0f;
    float iscale = RDIV(-fmax, mxs);
    for (int i = 0; i < n; i++) L[i] = clampf(RINT(iscale * x[i]), -fmax, fmax - 1.0f);
    for (int i = 0; i < n; i++) { tmp[i] = (w[i] * x[i]) * L[i]; t2[i] = (w[i] * L[i]) * L[i]; }
    float sumlx = sum_seq(tmp, n), suml2 = sum_seq(t2, n);
    for (int pass = 0; pass < 5; pass++) {
        for (int i = 0; i < n; i++) {
            float xi = x[i], wi = w[i], Li = L[i];
            float slx = sumlx - (wi * xi) * Li;
            int ok = slx > 0;
            float sl2 = suml2 - (wi * Li) * Li;
            float newl = clampf(RINT((xi * sl2) / (ok ? slx : 1.0f)), -fmax, fmax - 1.0f);
            float slx2 = slx + (wi * xi) * newl;
            float sl22 = sl2 + (wi * newl) * newl;
            if (ok && newl != Li && sl22 > 0 && (slx2 * slx2) * suml2 > (sumlx * sumlx) * sl22) {
                L[i] = newl;
                sumlx = slx2;
                suml2 = sl22;
            }
        }
    }
    float scale = suml2 > 0 ? sumlx / suml2 : 0.0f;
    *scale_out = live ? scale : 0.0f;
    for (int i = 0; i < n; i++) Lout[i] = live ? L[i] + fmax : 0.0f;
}

/* imatrix weights qw*sqrt(sigma2 + x^2) shared by the K-quants and IQ types */
static void imat_weights(const float *x, const float *qw, float sigma2, float *w) {
    for (int i = 0; i < QK_K; i++) {
        float t = x[i] * x[i];
        w[i] = qw[i] * SQRT(sigma2 + t);
    }
}

static float sumsq_c8(const float *x, int n) {
    float t[QK_K];
    for (int i = 0; i < n; i++) t[i] = x[i] * x[i];
    return qso_sum_cascade8(t, n);
}

/* ------------------------------------------------------------------ */
/* Q4_0  q4_0.py:14-33                                                 */
/* ------------------------------------------------------------------ */
static void q4_0_block(const float *b, uint8_t *out) {
    const int im = argmax_abs_nan(b, 32);          /* b.abs().argmax() q4_0.py:21 */
    float d = b[im] / -8.0f;
    float id = d != 0 ? 1.0f / d : 0.0f;
    uint8_t q[32];
    for (int i = 0; i < 32; i++) {
        float t = b[i] * id;
        t = t + 8.5f;
        q[i] = (uint8_t)clampf(floorf(t), 0.0f, 15.0f);
    }
    put_f16(out, d);
    for (int j = 0; j < 16; j++) out[2 + j] = (uint8_t)(q[j] | (q[j + 16] << 4));
}

/* ------------------------------------------------------------------ */
/* Q2_K  q2_k.py:25-81                                                 */
/* ------------------------------------------------------------------ */
static void q2_k_block(const float *x, const float *qw, uint8_t *out) {
    float w[QK_K], sc[16], mn[16], L[QK_K], steps[40];
    int64_t ls[16], lm[16];
    float d16, m16;
    if (!qw) {
        int ns = qkx_steps(-0.5f, 0.1f, 15, 3, steps);
        for (int i = 0; i < QK_K; i++) w[i] = fabsf(x[i]);
        for (int g = 0; g < 16; g++)
            make_qkx(x + 16 * g, w + 16 * g, 16, steps, ns, 3, 1, &sc[g], &mn[g], L + 16 * g);
        float max_scale = sc[0], max_min = mn[0];
        for (int g = 1; g < 16; g++) { max_scale = fmaxf(max_scale, sc[g]); max_min = fmaxf(max_min, mn[g]); }
        int pos_s = max_scale > 0, pos_m = max_min > 0;
        float inv_s = pos_s ? 15.0f / max_scale : 0.0f;
        float inv_m = pos_m ? 15.0f / max_min : 0.0f;
        for (int g = 0; g < 16; g++) {
            ls[g] = (int64_t)RINT(inv_s * sc[g]) & 0xFF;
            lm[g] = (int64_t)RINT(inv_m * mn[g]) & 0xFF;
        }
        d16 = f16_round(pos_s ? max_scale / 15.0f : 0.0f);
        m16 = f16_round(pos_m ? max_min / 15.0f : 0.0f);
    } else {
        int ns = qkx_steps(-0.9f, 0.05f, 36, 3, steps);
        float sigma2 = sumsq_c8(x, QK_K) / (float)QK_K;
        imat_weights(x, qw, sigma2, w);
        float sw[16], Ls[16], Lm[16], db, mb;
        for (int g = 0; g < 16; g++) {
            make_qkx(x + 16 * g, w + 16 * g, 16, steps, ns, 3, 0, &sc[g], &mn[g], L + 16 * g);
            sw[g] = qso_sum_cascade8(w + 16 * g, 16);
        }
        make_qp(sc, sw, 16, 15, 0, &db, Ls);
        make_qp(mn, sw, 16, 15, 0, &mb, Lm);
        for (int g = 0; g < 16; g++) { ls[g] = (int64_t)Ls[g] & 0xFF; lm[g] = (int64_t)Lm[g] & 0xFF; }
        d16 = f16_round(db);
        m16 = f16_round(mb);
    }
    int64_t scb[16];
    int Lf[QK_K];
    for (int g = 0; g < 16; g++) {
        scb[g] = (ls[g] | (lm[g] << 4)) & 0xFF;
        float dg = d16 * (float)(scb[g] & 0xF), mg = m16 * (float)(scb[g] >> 4);
        for (int i = 0; i < 16; i++) {
            float v;
            if (dg != 0) {
                float t = x[16 * g + i] + mg;
                v = clampf(RINT(t / dg), 0.0f, 3.0f);
            } else v = L[16 * g + i];
            Lf[16 * g + i] = (int)v;
        }
    }
    for (int g = 0; g < 16; g++) out[g] = (uint8_t)scb[g];
    for (int h = 0; h < 2; h++)
        for (int l = 0; l < 32; l++) {
            const int *q = Lf + 128 * h + l;
            out[16 + 32 * h + l] = (uint8_t)(q[0] | (q[32] << 2) | (q[64] << 4) | (q[96] << 6));
        }
    put_f16(out + 80, d16);
    put_f16(out + 82, m16);
}

/* ------------------------------------------------------------------ */
/* Q3_K  q3_k.py:23-78                                                 */
/* ------------------------------------------------------------------ */
static void q3_k_block(const float *x, const float *qw, uint8_t *out) {
    float sc[16], L[QK_K], d16;
    int64_t ls6[16];
    if (!qw) {
        for (int g = 0; g < 16; g++) make_q3(x + 16 * g, 16, 4, &sc[g], L + 16 * g);
        float amax;
        float max_scale = sc[absmax_first(sc, 16, &amax)];
        int has = max_scale != 0;
        float iscale = RDIV(-32.0f, has ? max_scale : 1.0f);
        for (int g = 0; g < 16; g++) {
            int64_t l = (int64_t)RINT(iscale * sc[g]);
            l = ((l & 0xFF) ^ 0x80) - 0x80;
            l = l < -32 ? -32 : (l > 31 ? 31 : l);
            ls6[g] = has ? l + 32 : 0;
        }
        d16 = f16_round(has ? 1.0f / iscale : 0.0f);
    } else {
        float w[QK_K], sw[16], Ls[16], db, sq[QK_K];
        for (int i = 0; i < QK_K; i++) sq[i] = x[i] * x[i];
        float sigma2 = (2.0f * sum_seq(sq, QK_K)) / (float)QK_K;
        imat_weights(x, qw, sigma2, w);
        for (int g = 0; g < 16; g++) {
            make_qx(x + 16 * g, w + 16 * g, 16, 4, &sc[g], L + 16 * g);
            sw[g] = sum_seq(w + 16 * g, 16);
        }
        make_qx(sc, sw, 16, 32, &db, Ls);
        for (int g = 0; g < 16; g++) ls6[g] = (int64_t)Ls[g];
        d16 = f16_round(db);
    }
    int Lf[QK_K];
    for (int g = 0; g < 16; g++) {
        float dq = d16 * (float)(ls6[g] - 32);
        for (int i = 0; i < 16; i++) {
            float v;
            if (dq != 0) v = clampf(RINT(x[16 * g + i] / dq), -4.0f, 3.0f) + 4.0f;
            else v = L[16 * g + i];
            Lf[16 * g + i] = (int)v;
        }
    }
    uint8_t *hmask = out, *qs = out + 32, *scb = out + 96;
    for (int l = 0; l < 32; l++) {
        int m = 0;
        for (int b = 0; b < 8; b++) m |= (Lf[32 * b + l] > 3) << b;
        hmask[l] = (uint8_t)m;
    }
    for (int h = 0; h < 2; h++)
        for (int l = 0; l < 32; l++) {
            int q[4];
            for (int i = 0; i < 4; i++) {
                int v = Lf[128 * h + 32 * i + l];
                q[i] = v > 3 ? v - 4 : v;
            }
            qs[32 * h + l] = (uint8_t)(q[0] | (q[1] << 2) | (q[2] << 4) | (q[3] << 6));
        }
    for (int j = 0; j < 8; j++) scb[j] = (uint8_t)((ls6[j] & 0xF) | ((ls6[j + 8] & 0xF) << 4));
    for (int i = 0; i < 4; i++)
        scb[8 + i] = (uint8_t)((ls6[i] >> 4) | ((ls6[4 + i] >> 4) << 2) | ((ls6[8 + i] >> 4) << 4) |
                               ((ls6[12 + i] >> 4) << 6));
    put_f16(out + 108, d16);
}

/* ------------------------------------------------------------------ */
/* Q4_K / Q5_K  q4_k.py:25-79, q5_k.py:25-82                           */
/* ------------------------------------------------------------------ */
static void q45_k_block(const float *x, const float *qw, uint8_t *out, int nmax) {
    float w[QK_K], sc[8], mn[8], L[QK_K], steps[40];
    int64_t ls[8], lm[8];
    float d16, m16;
    if (!qw) {
        int ns = nmax == 15 ? qkx_steps(-1.0f, 0.1f, 20, 15, steps) : qkx_steps(-0.5f, 0.1f, 15, 31, steps);
        for (int g = 0; g < 8; g++) {
            float av_x = SQRT(sumsq_c8(x + 32 * g, 32) / 32.0f);
            for (int i = 0; i < 32; i++) w[32 * g + i] = av_x + fabsf(x[32 * g + i]);
            make_qkx(x + 32 * g, w + 32 * g, 32, steps, ns, nmax, 0, &sc[g], &mn[g], L + 32 * g);
        }
        float max_scale = sc[0], max_min = mn[0];
        for (int g = 1; g < 8; g++) { max_scale = fmaxf(max_scale, sc[g]); max_min = fmaxf(max_min, mn[g]); }
        float inv_s = max_scale > 0 ? RDIV(63.0f, max_scale) : 0.0f;
        float inv_m = max_min > 0 ? RDIV(63.0f, max_min) : 0.0f;
        for (int g = 0; g < 8; g++) {
            int64_t a = (int64_t)RINT(inv_s * sc[g]) & 0xFF, b = (int64_t)RINT(inv_m * mn[g]) & 0xFF;
            ls[g] = a > 63 ? 63 : a;
            lm[g] = b > 63 ? 63 : b;
        }
        d16 = f16_round(max_scale / 63.0f);
        m16 = f16_round(max_min / 63.0f);
    } else {
        int ns = qkx_steps(-0.9f, 0.05f, 36, nmax, steps);
        float sigma2 = (2.0f * sumsq_c8(x, QK_K)) / (float)QK_K;
        imat_weights(x, qw, sigma2, w);
        float sw[8], Ls[8], Lm[8], db, mb;
        for (int g = 0; g < 8; g++) {
            make_qkx(x + 32 * g, w + 32 * g, 32, steps, ns, nmax, 0, &sc[g], &mn[g], L + 32 * g);
            sw[g] = qso_sum_cascade8(w + 32 * g, 32);
        }
        make_qp(sc, sw, 8, 63, 0, &db, Ls);
        make_qp(mn, sw, 8, 63, 0, &mb, Lm);
        for (int g = 0; g < 8; g++) { ls[g] = (int64_t)Ls[g] & 0xFF; lm[g] = (int64_t)Lm[g] & 0xFF; }
        d16 = f16_round(db);
        m16 = f16_round(mb);
    }
    int Lf[QK_K];
    for (int g = 0; g < 8; g++) {
        float dg = d16 * (float)(ls[g] & 63), mg = m16 * (float)(lm[g] & 63);
        for (int i = 0; i < 32; i++) {
            float v;
            if (dg != 0) {
                float t = x[32 * g + i] + mg;
                v = clampf(RINT(t / dg), 0.0f, (float)nmax);
            } else v = L[32 * g + i];
            Lf[32 * g + i] = (int)v;
        }
    }
    put_f16(out, d16);
    put_f16(out + 2, m16);
    uint8_t *scb = out + 4;
    for (int j = 0; j < 4; j++) {
        scb[j] = (uint8_t)(ls[j] | ((ls[4 + j] >> 4) << 6));
        scb[4 + j] = (uint8_t)(lm[j] | ((lm[4 + j] >> 4) << 6));
        scb[8 + j] = (uint8_t)((ls[4 + j] & 0xF) | ((lm[4 + j] & 0xF) << 4));
    }
    uint8_t *qs = out + 16;
    if (nmax == 31) {
        uint8_t *qh = out + 16;
        qs = out + 48;
        for (int l = 0; l < 32; l++) {
            int m = 0;
            for (int s = 0; s < 8; s++) m |= ((Lf[32 * s + l] >> 4) & 1) << s;
            qh[l] = (uint8_t)m;
        }
    }
    for (int j = 0; j < 4; j++)
        for (int l = 0; l < 32; l++)
            qs[32 * j + l] = (uint8_t)((Lf[64 * j + l] & 0xF) | ((Lf[64 * j + 32 + l] & 0xF) << 4));
}

/* ------------------------------------------------------------------ */
/* Q6_K  q6_k.py:22-65                                                 */
/* ------------------------------------------------------------------ */
static void q6_k_block(const float *x, const float *qw, uint8_t *out) {
    float w[QK_K], sc[16], L[QK_K];
    if (!qw) for (int i = 0; i < QK_K; i++) w[i] = x[i] * x[i];
    else memcpy(w, qw, sizeof(w));
    for (int g = 0; g < 16; g++) make_qx(x + 16 * g, w + 16 * g, 16, 32, &sc[g], L + 16 * g);
    float amax;
    float max_scale = sc[absmax_first(sc, 16, &amax)];
    int live = amax >= GROUP_MAX_EPS;
    float iscale = RDIV(-128.0f, live ? max_scale : 1.0f);
    float d16 = f16_round(live ? 1.0f / iscale : 0.0f);
    int64_t sc8[16];
    int Lf[QK_K];
    for (int g = 0; g < 16; g++) {
        int64_t s = (int64_t)fminf(RINT(iscale * sc[g]), 127.0f);
        s = ((s & 0xFF) ^ 0x80) - 0x80;
        float dq = d16 * (float)s;
        for (int i = 0; i < 16; i++) {
            float v;
            if (dq != 0) v = clampf(RINT(x[16 * g + i] / dq), -32.0f, 31.0f) + 32.0f;
            else v = L[16 * g + i];
            Lf[16 * g + i] = live ? (int)v : 0;
        }
        sc8[g] = live ? s : 0;
    }
    uint8_t *ql = out, *qh = out + 128, *scb = out + 192;
    for (int h = 0; h < 2; h++)
        for (int l = 0; l < 32; l++) {
            const int *q = Lf + 128 * h + l;
            ql[64 * h + l] = (uint8_t)((q[0] & 0xF) | ((q[64] & 0xF) << 4));
            ql[64 * h + 32 + l] = (uint8_t)((q[32] & 0xF) | ((q[96] & 0xF) << 4));
            qh[32 * h + l] = (uint8_t)((q[0] >> 4) | ((q[32] >> 4) << 2) | ((q[64] >> 4) << 4) | ((q[96] >> 4) << 6));
        }
    for (int g = 0; g < 16; g++) scb[g] = (uint8_t)(sc8[g] & 0xFF);
    put_f16(out + 208, d16);
}

/* ------------------------------------------------------------------ */
/* IQ4_XS  iq4_xs.py:23-76, 149-188                                    */
/* ------------------------------------------------------------------ */
static const float KVALUES_IQ4NL[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                         1, 13, 25, 38, 53, 69, 89, 113};

/* _best_index iq4_xs.py:35-39: searchsorted(right) bracket, strict midpoint compare */
static int iq4_best_index(float al) {
    int mu = 0;
    while (mu < 16 && KVALUES_IQ4NL[mu] <= al) mu++;
    mu = mu < 1 ? 1 : (mu > 15 ? 15 : mu);
    float lo = KVALUES_IQ4NL[mu - 1], hi = KVALUES_IQ4NL[mu];
    return (al - lo < hi - al) ? mu - 1 : mu;
}

/* _search_scales_eager iq4_xs.py:52-76 */
static float iq4_search_scale(const float *xb, const float *w) {
    float amax;
    float mx = xb[absmax_first(xb, 32, &amax)];
    int live = fabsf(mx) >= GROUP_MAX_EPS;
    float mxs = live ? mx : 1.0f;
    float d0 = -mxs / KVALUES_IQ4NL[0];
    float id0 = 1.0f / d0, t1[32], t2[32];
    for (int i = 0; i < 32; i++) {
        float q = KVALUES_IQ4NL[iq4_best_index(id0 * xb[i])];
        t1[i] = (w[i] * q) * xb[i];
        t2[i] = (w[i] * q) * q;
    }
    float sumqx = sum_seq(t1, 32), sumq2 = sum_seq(t2, 32);
    float d = sumq2 > 0 ? sumqx / sumq2 : 0.0f;
    float best = d * sumqx;
    for (int itry = -7; itry <= 7; itry++) {
        float idv = RDIV((float)(itry - 127), mxs);
        for (int i = 0; i < 32; i++) {
            float q = KVALUES_IQ4NL[iq4_best_index(idv * xb[i])];
            t1[i] = (w[i] * q) * xb[i];
            t2[i] = (w[i] * q) * q;
        }
        sumqx = sum_seq(t1, 32);
        sumq2 = sum_seq(t2, 32);
        if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
            float nd = sumqx / sumq2;
            d = nd;
            best = nd * sumqx;
        }
    }
    return live ? d : 0.0f;
}

static void iq4_xs_block(const float *x, const float *qw, uint8_t *out) {
    float w[QK_K], sc[8];
    if (!qw) for (int i = 0; i < QK_K; i++) w[i] = x[i] * x[i];
    else imat_weights(x, qw, (2.0f * sumsq_c8(x, QK_K)) / (float)QK_K, w);
    for (int b = 0; b < 8; b++) sc[b] = iq4_search_scale(x + 32 * b, w + 32 * b);
    float amax;
    float max_scale = sc[absmax_first(sc, 8, &amax)];
    float d = -max_scale / 32.0f;
    float idq = d != 0 ? 1.0f / d : 0.0f;
    int lsq[8], L[QK_K];
    for (int b = 0; b < 8; b++) {
        float ls = clampf(RINT(idq * sc[b]), -32.0f, 31.0f);
        float dl = d * ls;
        float idl = dl != 0 ? 1.0f / dl : 0.0f;
        for (int i = 0; i < 32; i++) L[32 * b + i] = iq4_best_index(idl * x[32 * b + i]);
        lsq[b] = (int)(ls + 32.0f);
    }
    put_f16(out, d);
    int hb = 0;
    for (int b = 0; b < 8; b++) hb |= (lsq[b] >> 4) << (2 * b);
    out[2] = (uint8_t)(hb & 0xFF);
    out[3] = (uint8_t)(hb >> 8);
    for (int j = 0; j < 4; j++) out[4 + j] = (uint8_t)((lsq[2 * j] & 0xF) | ((lsq[2 * j + 1] & 0xF) << 4));
    for (int b = 0; b < 8; b++)
        for (int j = 0; j < 16; j++) out[8 + 16 * b + j] = (uint8_t)(L[32 * b + j] | (L[32 * b + 16 + j] << 4));
}

/* ------------------------------------------------------------------ */
/* Q4_1, Q5_0, Q5_1, Q8_0, IQ4_NL: ggml formats the reference has no     */
/* module for (quant-studio.py:396-399 stops on them). PARITY UNPINNED   */
/* against the reference, which cannot produce these types. Written from  */
/* ggml's block layouts and reference quantizers (quantize_row_q4_1_ref,   */
/* _q5_0_ref, _q5_1_ref, _q8_0_ref; quantize_row_iq4_nl_impl with one     */
/* block per superblock) in the conventions of the reference's Q4_0       */
/* (q4_0.py:14-33: first-index signed absmax, IEEE division, one rounding */
/* per operation) and IQ4_XS (iq4_xs.py:52-76, 149-188: the block search, */
/* the `.sum(-1)` cascade for sigma2). Pinned instead by known answers,   */
/* dequantisation bounds and special blocks (tests/test_oracle.py), and   */
/* IQ4_NL's search by the IQ4_XS golden vectors it shares.               */
/* ------------------------------------------------------------------ */
/* planted-slip helpers (tests only): a / n and x * id as written, or slipped */
static inline float DIV_N(float a, float n) { return g_mut == MUT_D_BY_RECIP ? a * (1.0f / n) : a / n; }
static inline float MUL_ID(float x, float id, float d) { return g_mut == MUT_X_DIV_D && d != 0 ? x / d : x * id; }

static void q8_0_block(const float *b, uint8_t *out) {
    /* fmaxf from the first value: a NaN is passed over unless every value is one */
    float am = fabsf(b[0]);
    for (int i = 1; i < 32; i++) am = fmaxf(am, fabsf(b[i]));
    float d = DIV_N(am, 127.0f);
    float id = d != 0 ? 1.0f / d : 0.0f;
    put_f16(out, d);
    /* half away from zero (C roundf). A d below 127 * 2^-128 makes 1/d infinite
     * and x * id infinite or NaN, where C's conversion is undefined: such values
     * saturate to [-128, 127] and NaN gives 0 (the kernels do the same). */
    for (int i = 0; i < 32; i++) {
        float r = roundf(MUL_ID(b[i], id, d));
        out[2 + i] = (uint8_t)(int8_t)(r != r ? 0 : (int)clampf(r, -128.0f, 127.0f));
    }
}

/* Q4_1 (nmax 15) and Q5_1 (nmax 31): d = (max - min) / nmax, m = min */
static void q_1_block(const float *b, uint8_t *out, int nmax) {
    float mn = b[0], mx = b[0];
    for (int i = 1; i < 32; i++) { mn = fminf(mn, b[i]); mx = fmaxf(mx, b[i]); }
    float d = DIV_N(mx - mn, (float)nmax);
    float id = d != 0 ? 1.0f / d : 0.0f;
    uint8_t q[32];
    for (int i = 0; i < 32; i++) {
        float t = b[i] - mn;
        t = MUL_ID(t, id, d);
        t = t + 0.5f;
        /* clamp to [0, nmax] (t >= 0.5 unless 1/d overflowed; NaN gives 0) */
        q[i] = (uint8_t)clampf(truncf(t), 0.0f, (float)nmax);
    }
    put_f16(out, d);
    put_f16(out + 2, mn);
    int qs = 4;
    if (nmax == 31) {
        uint32_t qh = 0;
        for (int i = 0; i < 32; i++) qh |= (uint32_t)(q[i] >> 4) << i;
        for (int j = 0; j < 4; j++) out[4 + j] = (uint8_t)(qh >> (8 * j));
        qs = 8;
    }
    for (int j = 0; j < 16; j++) out[qs + j] = (uint8_t)((q[j] & 15) | ((q[j + 16] & 15) << 4));
}

static void q5_0_block(const float *b, uint8_t *out) {
    const int im = argmax_abs_nan(b, 32);          /* as Q4_0 */
    float d = b[im] / -16.0f;
    float id = d != 0 ? 1.0f / d : 0.0f;
    uint8_t q[32];
    for (int i = 0; i < 32; i++) {
        float t = MUL_ID(b[i], id, d);
        t = t + 16.5f;
        q[i] = (uint8_t)clampf(floorf(t), 0.0f, 31.0f);
    }
    put_f16(out, d);
    uint32_t qh = 0;
    for (int i = 0; i < 32; i++) qh |= (uint32_t)(q[i] >> 4) << i;
    for (int j = 0; j < 4; j++) out[2 + j] = (uint8_t)(qh >> (8 * j));
    for (int j = 0; j < 16; j++) out[6 + j] = (uint8_t)((q[j] & 15) | ((q[j + 16] & 15) << 4));
}

static void iq4_nl_block(const float *x, const float *qw, uint8_t *out) {
    float w[32];
    if (!qw) {
        for (int i = 0; i < 32; i++) w[i] = x[i] * x[i];
    } else {
        float sigma2 = (2.0f * sumsq_c8(x, 32)) / 32.0f;
        for (int i = 0; i < 32; i++) {
            float t = x[i] * x[i];
            w[i] = qw[i] * SQRT(sigma2 + t);
        }
    }
    float d = iq4_search_scale(x, w);
    float id = d != 0 ? 1.0f / d : 0.0f;
    put_f16(out, d);
    for (int j = 0; j < 16; j++)
        out[2 + j] = (uint8_t)(iq4_best_index(MUL_ID(x[j], id, d)) |
                               (iq4_best_index(MUL_ID(x[j + 16], id, d)) << 4));
}

/* ------------------------------------------------------------------ */
/* dispatch                                                            */
/* ------------------------------------------------------------------ */
#include "qs_oracle_iq.c"

static int block_info(int type, int *blk, int *bytes) {
    switch (type) {
    case QSO_Q4_0: *blk = 32; *bytes = 18; return 0;
    case QSO_Q2_K: *blk = 256; *bytes = 84; return 0;
    case QSO_Q3_K: *blk = 256; *bytes = 110; return 0;
    case QSO_Q4_K: *blk = 256; *bytes = 144; return 0;
    case QSO_Q5_K: *blk = 256; *bytes = 176; return 0;
    case QSO_Q6_K: *blk = 256; *bytes = 210; return 0;
    case QSO_IQ4_XS: *blk = 256; *bytes = 136; return 0;
    case QSO_IQ2_XXS: *blk = 256; *bytes = 66; return 0;
    case QSO_IQ2_XS: *blk = 256; *bytes = 74; return 0;
    case QSO_IQ2_S: *blk = 256; *bytes = 82; return 0;
    case QSO_IQ3_XXS: *blk = 256; *bytes = 98; return 0;
    case QSO_IQ3_S: *blk = 256; *bytes = 110; return 0;
    case QSO_Q4_1: *blk = 32; *bytes = 20; return 0;
    case QSO_Q5_0: *blk = 32; *bytes = 22; return 0;
    case QSO_Q5_1: *blk = 32; *bytes = 24; return 0;
    case QSO_Q8_0: *blk = 32; *bytes = 34; return 0;
    case QSO_IQ4_NL: *blk = 32; *bytes = 18; return 0;
    default: return -1;
    }
}

int64_t qso_row_bytes(int type, int64_t k) {
    int blk, bytes;
    if (block_info(type, &blk, &bytes) || k <= 0 || k % blk) return -1;
    return k / blk * bytes;
}

int qso_quantize(int type, const float *x, int64_t n_rows, int64_t k, const float *qw,
                 uint8_t *out, int n_threads) {
    int blk, bytes;
    if (block_info(type, &blk, &bytes) || k <= 0 || k % blk || n_rows < 0) return -1;
    int64_t nb = k / blk, total = n_rows * nb;
    int bad = 0;
    if (n_threads < 1) n_threads = 1;
    sqrt_table_init();                   /* before the worker threads read it */
#pragma omp parallel for schedule(dynamic, 64) num_threads(n_threads) reduction(| : bad)
    for (int64_t b = 0; b < total; b++) {
        int64_t r = b / nb, c = b % nb;
        const float *xb = x + r * k + c * blk;
        const float *qb = qw ? qw + c * blk : NULL;
        uint8_t *ob = out + b * bytes;
        switch (type) {
        case QSO_Q4_0: q4_0_block(xb, ob); break;
        case QSO_Q2_K: q2_k_block(xb, qb, ob); break;
        case QSO_Q3_K: q3_k_block(xb, qb, ob); break;
        case QSO_Q4_K: q45_k_block(xb, qb, ob, 15); break;
        case QSO_Q5_K: q45_k_block(xb, qb, ob, 31); break;
        case QSO_Q6_K: q6_k_block(xb, qb, ob); break;
        case QSO_IQ4_XS: iq4_xs_block(xb, qb, ob); break;
        case QSO_Q4_1: q_1_block(xb, ob, 15); break;
        case QSO_Q5_0: q5_0_block(xb, ob); break;
        case QSO_Q5_1: q_1_block(xb, ob, 31); break;
        case QSO_Q8_0: q8_0_block(xb, ob); break;
        case QSO_IQ4_NL: iq4_nl_block(xb, qb, ob); break;
        default: bad |= qs_oracle_iq(type, xb, qb, ob); break;
        }
    }
    return bad ? -1 : 0;
}
