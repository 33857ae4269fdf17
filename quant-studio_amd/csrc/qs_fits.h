// Per-group scale/min searches of the K-quants and IQ4_XS, one lane per group.
//
// Each function keeps a whole group (16 or 32 values) in registers and walks
// the reference's sequential candidate chain for it; parallelism comes from
// running one group per lane. The candidate order, the accept tests and every
// reduction order follow the reference's eager torch path line by line (cited
// per function), so the chosen levels and scales are bit-identical to it.
#pragma once

#include "qs_device.h"
#include "qs_wave.h"

namespace qs {

// Candidate numerators. Computed on the host in f32 exactly as the reference's
// numpy f32 chains (kq_common.py:21-30, qx_common.py:20-23) and passed in.
struct Steps {
    float v[40];
    int n;
};

// Result of the make_qkx2/qkx3 search: the levels are regenerated from
// (isc, mn) of the accepted candidate instead of being carried in registers.
struct QkxResult {
    float scale, the_min, isc, mn;
    bool degen;
};

// make_qkx_quants_eager kq_common.py:51-96 for one group of N values.
// SPEC: divide the next candidate's inverse scale during the error pass (below).
template <int N, bool MAD, bool SPEC = false>
QS_DEV QkxResult qkx_fit(const float (&x)[N], const float (&w)[N], const Steps& steps, float fmax) {
    float mn = x[0], mx = x[0];
#pragma unroll
    for (int i = 1; i < N; i++) {
        mn = fminf(mn, x[i]);
        mx = fmaxf(mx, x[i]);
    }
    mn = fminf(mn, 0.0f);
    const bool degen = (mx == mn);
    float t[N];
    const float sum_w = tree_sum(w);
#pragma unroll
    for (int i = 0; i < N; i++) t[i] = w[i] * x[i];
    const float sum_x = tree_sum(t);

    float den = degen ? 1.0f : mx - mn;
    const float iscale = fmax / den;
    float scale = 1.0f / iscale;
    float best_isc = iscale, best_mn = mn;
#pragma unroll
    for (int i = 0; i < N; i++) {
        float L = clampf(rintf(iscale * (x[i] - mn)), 0.0f, fmax);
        float d = scale * L;
        d = d + mn;
        d = d - x[i];
        t[i] = w[i] * (MAD ? fabsf(d) : d * d);
    }
    float best = tree_sum(t);

    // 16-value groups load each step one candidate ahead, so the scalar
    // load's latency is not waited for at the top of every candidate (Q2_K
    // 2-6% faster). With SPEC the next candidate's inverse scale is divided
    // both ways while this candidate's error pass runs, for a kept min
    // (mx - mn) and for this candidate's min should it be accepted
    // (mx - this_min), so no division heads the next candidate; the quotients
    // are the ones dividing after the accept gives. Q4_K / Q5_K with imatrix
    // (37 candidates) run 1.4-1.9% faster that way; without imatrix they ran
    // 1.4-2.3% slower and 16-value groups 5-9% slower (one more division per
    // candidate weighs more there), so only the former use it.
    static_assert(!SPEC || N == 32, "SPEC is timed for 32-value groups only");
    constexpr bool AHEAD = N == 16;
    float step_next = steps.v[0];
    float isc_keep = SPEC ? step_next / den : 0.0f, isc_acc = isc_keep;
    bool accepted = false;
#pragma unroll 1
    for (int s = 0; s < steps.n; s++) {
        float isc;
        if constexpr (SPEC) {
            isc = accepted ? isc_acc : isc_keep;
        } else {
            const float step = AHEAD ? step_next : steps.v[s];
            if constexpr (AHEAD) step_next = steps.v[s + 1 < 40 ? s + 1 : 39];
            den = degen ? 1.0f : mx - mn;
            isc = step / den;
        }
        // the three tree sums are formed 8 values at a time (the tree over N
        // is the trees over its 8-value blocks, then the tree over the block
        // sums), so only one block of products is live at once
        constexpr int NB = N / 8;
        float La[N], sa[NB], sb[NB], sc[NB];
#pragma unroll
        for (int k = 0; k < NB; k++) {
            float a[8], b[8], c[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int i = 8 * k + j;
                La[i] = clampf(rintf(isc * (x[i] - mn)), 0.0f, fmax);
                a[j] = w[i] * La[i];
                b[j] = a[j] * La[i];
                c[j] = a[j] * x[i];
            }
            sa[k] = tree_sum(a);
            sb[k] = tree_sum(b);
            sc[k] = tree_sum(c);
        }
        const float sum_l = tree_sum(sa), sum_l2 = tree_sum(sb), sum_xl = tree_sum(sc);
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        const float Dsafe = D > 0 ? D : 1.0f;
        float this_scale = (sum_w * sum_xl - sum_x * sum_l) / Dsafe;
        float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / Dsafe;
        if (this_min > 0) {
            this_scale = sum_xl / fmaxf(sum_l2, F32_TINY);
            this_min = 0.0f;
        }
        float next_keep = 0.0f, next_acc = 0.0f;
        if constexpr (SPEC) {
            const float step = steps.v[s + 1 < 40 ? s + 1 : 39];
            next_keep = step / (degen ? 1.0f : mx - mn);
            next_acc = step / (degen ? 1.0f : mx - this_min);
        }
        float se[NB];
#pragma unroll
        for (int k = 0; k < NB; k++) {
            float e8[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int i = 8 * k + j;
                float d = this_scale * La[i];
                d = d + this_min;
                d = d - x[i];
                e8[j] = w[i] * (MAD ? fabsf(d) : d * d);
            }
            se[k] = tree_sum(e8);
        }
        const float cur = tree_sum(se);
        accepted = D > 0 && cur < best && !degen;
        isc_keep = next_keep;
        isc_acc = next_acc;
        if (accepted) {
            best_isc = isc;
            best_mn = mn;
            scale = this_scale;
            mn = this_min;
            best = cur;
        }
    }
    QkxResult r;
    r.scale = degen ? 0.0f : scale;
    r.the_min = (mn == 0.0f) ? 0.0f : -mn;
    r.isc = best_isc;
    r.mn = best_mn;
    r.degen = degen;
    return r;
}

// level i of the accepted make_qkx candidate
QS_DEV float qkx_level(const QkxResult& r, float x, float fmax) {
    return r.degen ? 0.0f : clampf(rintf(r.isc * (x - r.mn)), 0.0f, fmax);
}

// make_qp_quants_eager kq_common.py:99-141, in three parts: qp_trial (one
// trial's weighted error), qp_finish (levels, sums and refinement passes for
// the chosen iscale) and the choice between them, made by qp_fit on one lane
// or by qp_fit_spread over several.

// The weighted error of the levels rint(isc * x), clamped to fmax unless
// `clamp` is false: the first pass (kq_common.py:107-109) does not clamp.
template <int N>
QS_DEV float qp_trial(const float (&x)[N], const float (&w)[N], float isc, float fmax, bool clamp) {
    const float r = 1.0f / isc;
    return cascade8_of<N>([&](int i) {
        float l = rintf(isc * x[i]);
        l = clamp ? fminf(l, fmax) : l;
        float d = x[i] - r * l;
        return w[i] * (d * d);
    });
}

// kq_common.py:118-141 for the chosen iscale: writes the levels to L and
// returns the scale.
template <int N>
QS_DEV float qp_finish(const float (&x)[N], const float (&w)[N], float fmax, float iscale, bool dead,
                       float (&L)[N]) {
#pragma unroll
    for (int i = 0; i < N; i++) L[i] = fminf(rintf(iscale * x[i]), fmax);
    float sumlx = cascade8_of<N>([&](int i) { return (w[i] * x[i]) * L[i]; });
    float suml2 = cascade8_of<N>([&](int i) { return (w[i] * L[i]) * L[i]; });
#pragma unroll 1
    for (int pass = 0; pass < 5; pass++) {
        bool changed = false;
#pragma unroll
        for (int i = 0; i < N; i++) {
            const float xi = x[i], Li = L[i];
            float wi = w[i];
            // keeps wi * xi inside the pass: hoisting the N products out of
            // the loop would hold N more registers for the whole fit
            keep_in_register(wi);
            const float slx = sumlx - (wi * xi) * Li;
            const float sl2 = suml2 - (wi * Li) * Li;
            const bool ok = slx > 0 && sl2 > 0;
            const float newl = fminf(rintf((xi * sl2) / (ok ? slx : 1.0f)), fmax);
            const float slx2 = slx + (wi * xi) * newl;
            const float sl22 = sl2 + (wi * newl) * newl;
            if (ok && newl != Li && (slx2 * slx2) * suml2 > (sumlx * sumlx) * sl22) {
                L[i] = newl;
                sumlx = slx2;
                suml2 = sl22;
                changed = true;
            }
        }
        // a pass that commits nothing leaves L, sumlx and suml2 as they were,
        // so every later pass repeats it (the C loop's early break, which the
        // reference's five passes stand for, kq_common.py:121-136): the wave stops
        // once none of its lanes committed
        if (!wave_any(changed)) break;
    }
    float scale = suml2 > 0 ? sumlx / fmaxf(suml2, F32_TINY) : 0.0f;
    if (dead) {
        scale = 0.0f;
#pragma unroll
        for (int i = 0; i < N; i++) L[i] = 0.0f;
    }
    return scale;
}


template <int N>
QS_DEV float qp_max(const float (&x)[N]) {
    float mx = x[0];
#pragma unroll
    for (int i = 1; i < N; i++) mx = fmaxf(mx, x[i]);
    return mx;
}

// make_qp_quants_eager on one lane (N = 8, 16, 32). Writes the levels to L
// and returns the scale.
template <int N>
QS_DEV float qp_fit(const float (&x)[N], const float (&w)[N], int nmax, const float (&steps)[8], float (&L)[N]) {
    const float fmax = (float)nmax;
    const float mx = qp_max(x);
    const bool dead = mx < GROUP_MAX_EPS;
    const float mxs = dead ? 1.0f : mx;

    float iscale = rdiv(fmax, mxs);
    float best_mse = qp_trial<N>(x, w, iscale, fmax, false);
#pragma unroll 1
    for (int s = 0; s < 8; s++) {
        const float isc = rdiv(steps[s], mxs);
        const float mse = qp_trial<N>(x, w, isc, fmax, true);
        if (mse < best_mse) {
            best_mse = mse;
            iscale = isc;
        }
    }
    return qp_finish<N>(x, w, fmax, iscale, dead, L);
}

// make_qp_quants_eager for one superblock's N sub-block scales (or mins),
// spread over P consecutive lanes (c = 0..P-1) that all hold x and w. The
// nine trials (the first pass, then the eight candidates) do not depend on
// each other, only the choice among them does, so lane c runs trials c,
// c + P, ...; their (error, iscale) pairs meet in xch (18 floats of LDS) and
// every lane makes the reference's choice in trial order (the first strict
// minimum) and finishes the fit. Every lane of the wave must call it (it
// holds a wave barrier); all P lanes return the same scale and levels.
template <int N, int P, bool WL = false>
QS_DEV float qp_fit_spread(const float (&x)[N], const float (&w)[N], int nmax, const float (&steps)[8],
                           float (&L)[N], int c, float* xch) {
    static_assert(P >= 1 && P <= 9, "one to nine lanes share the trials");
    const float fmax = (float)nmax;
    const float mx = qp_max(x);
    const bool dead = mx < GROUP_MAX_EPS;
    const float mxs = dead ? 1.0f : mx;
#pragma unroll
    for (int k = 0; k < (9 + P - 1) / P; k++) {
        const int e = c + k * P;
        if (e < 9) {
            float num = fmax;        // trial 0: nmax / max; trial e: candidate e - 1
#pragma unroll
            for (int j = 0; j < 8; j++) num = e == j + 1 ? steps[j] : num;
            const float isc = rdiv(num, mxs);
            xch[2 * e] = qp_trial<N>(x, w, isc, fmax, e != 0);
            xch[2 * e + 1] = isc;
        }
    }
    wave_sync<WL>();
    float best_mse = xch[0], iscale = xch[1];
#pragma unroll
    for (int e = 1; e < 9; e++) {
        const float mse = xch[2 * e];
        if (mse < best_mse) {
            best_mse = mse;
            iscale = xch[2 * e + 1];
        }
    }
    return qp_finish<N>(x, w, fmax, iscale, dead, L);
}

// make_qx_quants_eager qx_common.py:52-82 for one group of 16 values.
// Returns the scale; the levels are regenerated from (isc) by qx_level.
struct QxResult {
    float scale, isc;
    bool live;
};

// sums of one make_qx trial: the levels clamp(rint(isc * x), -nmax, nmax - 1)
// and their seq-sums sum w x L, sum w L^2 (qx_common.py:61-63, :68-70)
template <int N>
QS_DEV float2 qx_trial(const float (&x)[N], const float (&w)[N], float isc, float fmax) {
    float t[N], u[N];
#pragma unroll
    for (int i = 0; i < N; i++) {
        float La = clampf(rintf(isc * x[i]), -fmax, fmax - 1.0f);
        t[i] = (w[i] * x[i]) * La;
        u[i] = (w[i] * La) * La;
    }
    return make_float2(seq_sum(t), seq_sum(u));
}

template <int N>
QS_DEV QxResult qx_fit(const float (&x)[N], const float (&w)[N], int nmax, const Steps& steps) {
    const float fmax = (float)nmax;
    float amax;
    const float mx = absmax_first(x, amax);
    const bool live = amax >= GROUP_MAX_EPS;
    const float mxs = live ? mx : 1.0f;
    const float iscale = rdiv(-fmax, mxs);
    const float2 s0 = qx_trial<N>(x, w, iscale, fmax);
    const float sumlx = s0.x, suml2 = s0.y;
    float scale = suml2 != 0 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx, best_isc = iscale;
    float step_next = steps.v[0];      // loaded one candidate ahead (Q3_K 4%, Q6_K 2% faster)
#pragma unroll 1
    for (int s = 0; s < steps.n; s++) {
        const float step = step_next;
        step_next = steps.v[s + 1 < 40 ? s + 1 : 39];
        const float isc = rdiv(-step, mxs);
        const float2 sc = qx_trial<N>(x, w, isc, fmax);
        const float slx = sc.x, sl2 = sc.y;
        if (sl2 > 0 && slx * slx > best * sl2) {
            const float cand = slx / sl2;
            scale = cand;
            best = cand * slx;
            best_isc = isc;
        }
    }
    QxResult r;
    r.scale = live ? scale : 0.0f;
    r.isc = best_isc;
    r.live = live;
    return r;
}

// make_qx_quants_eager for one superblock's N sub-block scales, spread over
// P consecutive lanes (c = 0..P-1) that all hold x and w, for NS candidates
// (the host's steps.n). A trial's levels and sums depend only on its iscale,
// not on earlier accepts, so lane c forms the sums of trials c, c + P, ...
// (trial 0: the first pass; trial e: candidate e - 1); they meet in xch
// (3 (NS + 1) floats of LDS) and every lane runs the accept chain in
// candidate order. Every lane of the wave must call it (it holds a wave
// barrier); all P lanes return the same result.
template <int N, int P, int NS, bool WL = false>
QS_DEV QxResult qx_fit_spread(const float (&x)[N], const float (&w)[N], int nmax, const Steps& steps,
                              int c, float* xch) {
    const float fmax = (float)nmax;
    float amax;
    const float mx = absmax_first(x, amax);
    const bool live = amax >= GROUP_MAX_EPS;
    const float mxs = live ? mx : 1.0f;
#pragma unroll
    for (int k = 0; k < (NS + 1 + P - 1) / P; k++) {
        const int e = c + k * P;
        if (e <= NS) {
            float num = fmax;
#pragma unroll
            for (int j = 0; j < NS; j++) num = e == j + 1 ? steps.v[j] : num;
            const float isc = rdiv(-num, mxs);
            const float2 sc = qx_trial<N>(x, w, isc, fmax);
            xch[3 * e] = sc.x;
            xch[3 * e + 1] = sc.y;
            xch[3 * e + 2] = isc;
        }
    }
    wave_sync<WL>();
    const float sumlx = xch[0], suml2 = xch[1];
    float scale = suml2 != 0 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx, best_isc = xch[2];
#pragma unroll 1
    for (int e = 1; e <= NS; e++) {
        const float slx = xch[3 * e], sl2 = xch[3 * e + 1];
        if (sl2 > 0 && slx * slx > best * sl2) {
            const float cand = slx / sl2;
            scale = cand;
            best = cand * slx;
            best_isc = xch[3 * e + 2];
        }
    }
    QxResult r;
    r.scale = live ? scale : 0.0f;
    r.isc = best_isc;
    r.live = live;
    return r;
}

// level (0 .. 2*nmax-1) of the accepted make_qx candidate
QS_DEV float qx_level(const QxResult& r, float x, float fmax) {
    return r.live ? clampf(rintf(r.isc * x), -fmax, fmax - 1.0f) + fmax : 0.0f;
}

// make_q3_quants_eager qx_common.py:85-121 for one group of 16 (w = x*x).
// Writes levels (0 .. 2*nmax-1) and returns the scale.
template <int N>
QS_DEV float q3_fit(const float (&x)[N], int nmax, float (&L)[N]) {
    const float fmax = (float)nmax;
    float w[N], t[N], u[N];
#pragma unroll
    for (int i = 0; i < N; i++) w[i] = x[i] * x[i];
    float amax;
    const float mx = absmax_first(x, amax);
    const bool live = amax >= GROUP_MAX_EPS;
    const float mxs = live ? mx : 1.0f;
    const float iscale = rdiv(-fmax, mxs);
#pragma unroll
    for (int i = 0; i < N; i++) {
        L[i] = clampf(rintf(iscale * x[i]), -fmax, fmax - 1.0f);
        t[i] = (w[i] * x[i]) * L[i];
        u[i] = (w[i] * L[i]) * L[i];
    }
    float sumlx = seq_sum(t), suml2 = seq_sum(u);
#pragma unroll 1
    for (int pass = 0; pass < 5; pass++) {
        bool changed = false;
#pragma unroll
        for (int i = 0; i < N; i++) {
            const float xi = x[i], wi = w[i], Li = L[i];
            const float slx = sumlx - (wi * xi) * Li;
            const bool ok = slx > 0;
            const float sl2 = suml2 - (wi * Li) * Li;
            const float newl = clampf(rintf((xi * sl2) / (ok ? slx : 1.0f)), -fmax, fmax - 1.0f);
            const float slx2 = slx + (wi * xi) * newl;
            const float sl22 = sl2 + (wi * newl) * newl;
            if (ok && newl != Li && sl22 > 0 && (slx2 * slx2) * suml2 > (sumlx * sumlx) * sl22) {
                L[i] = newl;
                sumlx = slx2;
                suml2 = sl22;
                changed = true;
            }
        }
        if (!wave_any(changed)) break;        // as in qp_fit (qx_common.py:100-114)
    }
    const float scale = suml2 > 0 ? sumlx / suml2 : 0.0f;
#pragma unroll
    for (int i = 0; i < N; i++) L[i] = live ? L[i] + fmax : 0.0f;
    return live ? scale : 0.0f;
}

// ---- IQ4_XS (iq4_xs.py:23-76) ----

// Bracket table of _best_index (iq4_xs.py:35-39): the LUT values are integers,
// so #{V <= al} = #{V <= floor(al)}; entry k + 128 (k = -128..127) holds the
// bracket (V[mu-1], V[mu]) with mu = clamp(#{V <= k}, 1, 15), and mu itself in
// `mus`. Built by the workgroup in LDS.
QS_DEV void iq4_build_table(float2* tab, uint8_t* mus) {
    constexpr float V[16] = {-127.f, -104.f, -83.f, -65.f, -49.f, -35.f, -22.f, -10.f,
                             1.f,    13.f,   25.f,  38.f,  53.f,  69.f,  89.f,  113.f};
    for (int e = threadIdx.x; e < 256; e += blockDim.x) {
        const float k = (float)(e - 128);
        int mu = 0;
#pragma unroll
        for (int i = 0; i < 16; i++) mu += (V[i] <= k) ? 1 : 0;
        mu = mu < 1 ? 1 : (mu > 15 ? 15 : mu);
        float lo = V[0], hi = V[1];
#pragma unroll
        for (int i = 2; i < 16; i++) {
            lo = (mu == i) ? V[i - 1] : lo;
            hi = (mu == i) ? V[i] : hi;
        }
        tab[e] = make_float2(lo, hi);
        mus[e] = (uint8_t)mu;
    }
}

// LUT value of _best_index(al): the bracket from the table, then the C
// midpoint compare `al - lo < hi - al` (strict; NaN takes hi, as the scan)
QS_DEV float iq4_project(float al, const float2* tab) {
    const float f = clampf(floorf(al), -128.0f, 127.0f);
    const float2 e = tab[(int)f + 128];
    const float d1 = al - e.x, d2 = e.y - al;
    return d1 < d2 ? e.x : e.y;
}

// LUT index of _best_index(al), from the same table
QS_DEV int iq4_project_index(float al, const float2* tab, const uint8_t* mus) {
    const int k = (int)clampf(floorf(al), -128.0f, 127.0f) + 128;
    const float2 e = tab[k];
    const int mu = mus[k];
    const float d1 = al - e.x, d2 = e.y - al;
    return d1 < d2 ? mu - 1 : mu;
}

// _search_scales_eager iq4_xs.py:52-76 for one block of 32. The two sums of
// a candidate run left to right (seq_sum's order) over terms staged CH values
// at a time: CH = 16 holds 121-126 VGPRs instead of 140-168, which with the
// imatrix weights taken 8 at a time gives the imatrix kernels a fourth wave
// per SIMD (6-7% faster); the kernels without imatrix were 4% slower at 4
// waves and stage all 32 (CH = 32, 3 waves).
template <int CH>
QS_DEV float iq4_scale_search(const float (&x)[32], const float (&w)[32], const float2* tab) {
    float amax;
    const float mx = absmax_first(x, amax);
    const bool live = fabsf(mx) >= GROUP_MAX_EPS;
    const float mxs = live ? mx : 1.0f;
    const float d0 = -mxs / -127.0f;
    const float id0 = 1.0f / d0;
    auto sums = [&](float iv, float& sqx, float& sq2) {
#pragma unroll
        for (int c = 0; c < 32; c += CH) {
            float t[CH], u[CH];
#pragma unroll
            for (int i = 0; i < CH; i++) {
                const float q = iq4_project(iv * x[c + i], tab);
                const float wq = w[c + i] * q;
                t[i] = wq * x[c + i];
                u[i] = wq * q;
            }
#pragma unroll
            for (int i = 0; i < CH; i++) {
                sqx = c + i == 0 ? t[i] : sqx + t[i];
                sq2 = c + i == 0 ? u[i] : sq2 + u[i];
            }
        }
    };
    float sumqx, sumq2;
    sums(id0, sumqx, sumq2);
    float d = sumq2 > 0 ? sumqx / sumq2 : 0.0f;
    float best = d * sumqx;
#pragma unroll 1
    for (int itry = -7; itry <= 7; itry++) {
        const float idv = rdiv((float)(itry - 127), mxs);
        sums(idv, sumqx, sumq2);
        if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
            const float nd = sumqx / sumq2;
            d = nd;
            best = nd * sumqx;
        }
    }
    return live ? d : 0.0f;
}

}  // namespace qs
