// IQ2_XXS / IQ2_XS / IQ2_S / IQ3_XXS / IQ3_S quantizer kernels (gfx950).
//
// One lane per group (32 values for IQ2_XXS and IQ3, 16 for IQ2_XS/S); the
// group's candidate-scale sweep runs in registers, each step projecting the
// group's subgroups onto the E8/3-bit grid: levels -> code -> kmap hit, or a
// first-minimum weighted search over the code's neighbour list. Grid codes
// (and the IQ3 kmap) are staged in LDS; the IQ2 kmaps and every neighbour
// list are read through L1/L2 (at most 250 KB per table). Superblock scales
// and the packed block go through LDS like the K-quant kernels.
#pragma once

#include <type_traits>

#include "qs_fits.h"
#include "qs_kernels.h"
#include "qs_wave.h"

namespace qs {

// Device copy of one grid's tables (built once per device on the host).
// cinfo packs everything a projection needs about a code:
//   on-grid:  bit 31 set, bits 0..15 = grid index;
//   off-grid: bits 12..30 = first neighbour / CH, bits 0..11 = list length;
// each list starts on a CH-entry boundary of nbr and is padded to a multiple
// of CH, so a lane fetches a chunk of CH candidates with one vector load
// (CH = 8 for the IQ2 grids, 4 for the IQ3 grids, whose lists are short).
//
// cinfo_red has the same layout and points at each list's reduced copy: the
// list without the entries that change a proper superset of an earlier
// entry's changed values (against the code's levels) and agree with it on
// those. A search may read it when the code's level is the best level of
// every value for its distance terms (iq_codes<..., PRUNE>): every left-out
// entry then has each term >= that earlier entry's, so a distance >= it and
// can never be the first minimum; the reduced list keeps the list's order, so
// its first minimum is the list's. cinfo_red2 points at a second reduced
// copy, which leaves an entry out only when the earlier entry also makes
// every raise from the code's clamped top level (IQ2: level 2) to the grid's
// level 3 that the left-out entry makes: it stays valid where the code's
// level is every value's best level except at values on level 2 whose
// level-3 term is lower (there level 2 still beats levels 0 and 1, so only a
// raise to 3 lowers the term). Grids built without the second copy point
// cinfo_red2 at the reduced lists, grids without reduced lists point both at
// the full lists.
struct IqTabDev {
    const uint16_t* grid;     // grid codes (BITS-bit levels per value)
    // code -> packed kmap / list position / length: the full lists' entries,
    // then (at +ncodes) the reduced lists', then (at +2 ncodes) the
    // clamp-tolerant reduced lists' (cinfo_red, cinfo_red2 above)
    const uint32_t* cinfo;
    int ncodes;
    const uint16_t* nbr;      // neighbour grid indices, (distance, index) order
    int code0;                // grid index of the all-zero code (0 if off-grid)
};

constexpr uint32_t CI_ON_GRID = 0x80000000u;

// candidates per chunk, and the most chunks in one neighbour list of each
// grid (longest lists: IQ2 150 / 292 / 70, IQ3 36 / 38 entries; checked when
// the tables are built)
constexpr int IQ2_CH = 8, IQ3_CH = 4;
constexpr int IQ2_256_MAXCH = 19, IQ2_512_MAXCH = 37, IQ2_1024_MAXCH = 9;
constexpr int IQ3_256_MAXCH = 9, IQ3_512_MAXCH = 10;

// LDS of the IQ kernels: x^2 staging for the superblock sum (half the wave's
// superblocks at a time), sharing its storage with the packed output blocks
// written at the end, and the per-group scales.
template <int SPW, int BYTES>
struct alignas(16) IqLds {
    union {                      // the weight phase's staging, then the packed blocks
        struct {
            float v[SPW / 2][QK_K];      // x^2 of half the wave's superblocks at a time
            float tmp[SPW / 2][40];
        };
        uint8_t out[SPW * BYTES + 16];
    };
    float sc[SPW][16];
};

// (a workgroup of several waves may hold waves past the last superblock:
// they store nothing)
template <int SPW, int BYTES, int WPG = 1>
QS_DEV void sb_store(const IqLds<SPW, BYTES>& s, const KArgs& a) {
    const int64_t first = grid_wave<WPG>() * SPW;
    const int64_t nvalid = min((int64_t)SPW, a.n_units - first);
    if (WPG == 1 || nvalid > 0) store_staged<(WPG > 1)>(s.out, a.dst, first * BYTES, (int)nvalid * BYTES);
}

template <int I, int END, typename F>
QS_DEV void static_for(F&& f) {
    if constexpr (I < END) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, END>(f);
    }
}

// Grid levels staged in LDS as bytes 2l+1 (4 per word, NV/4 words per grid
// point), so a level is one byte-to-float conversion.
template <int BITS, int NV, int GS, int THREADS = 64>
QS_DEV void stage_levels(const uint16_t* grid, uint32_t* glv) {
    constexpr int W = NV / 4;
    for (int i = threadIdx.x; i < GS * W; i += THREADS) {
        const uint32_t code = grid[i / W];
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int e = 4 * (i % W) + b;
            word |= (2u * ((code >> (BITS * e)) & ((1u << BITS) - 1u)) + 1u) << (8 * b);
        }
        glv[i] = word;
    }
}

template <int NV>
struct Levels {
    uint32_t w[NV / 4];
};

template <int NV>
QS_DEV Levels<NV> grid_levels(const uint32_t* glv, int gi) {
    Levels<NV> L;
    if constexpr (NV == 8) {
        const uint2 q = reinterpret_cast<const uint2*>(glv)[gi];
        L.w[0] = q.x;
        L.w[1] = q.y;
    } else {
        L.w[0] = glv[gi];
    }
    return L;
}

template <int NV>
QS_DEV float level(const Levels<NV>& L, int e) {
    return (float)((L.w[e >> 2] >> (8 * (e & 3))) & 0xffu);
}


// Project every lane's subgroups at its candidate scale
// (iq2.py:347-372, iq2xs_common.py:222-271, iq3_common.py:209-256): levels
// clamp(round(0.5*(inv*x - 1)), 0, LMAX) -> code -> kmap hit (iq_codes), or
// the reference's d2.argmin(-1) over the code's neighbour list (iq_search,
// one call per subgroup OFF..OFF+NV-1). IQ2 distances are a left-to-right sum
// of 8 terms from +0; IQ3's are ((t0+t1)+t2)+t3, with t = (wv*diff)*diff and
// diff = sc*g - x. torch's argmin takes the first NaN as the minimum, else
// the first minimum (the first entry when every distance is +inf).
//
// The search is wave-balanced: the off-grid lanes' lists are cut into chunks
// of CH candidates and the wave's chunks are dealt to all 64 lanes in turn, so
// one long list no longer holds the whole wave. A chunk's lane fetches the
// owner's values and scale with ds_bpermute, evaluates its candidates in list
// order and merges its first minimum into the owner's LDS slot as a 64-bit key
// (distance bits, list position, grid index); the least key is the list's
// first finite minimum. Every lane of the wave calls this together; lanes
// with want == false take part but search nothing (their result is grid
// index 0 and unused).
//   cmap: LDS, 64 * MAXCH bytes (chunk -> owner lane)
//   res:  LDS, 64 keys
//
// NaN terms. A term is NaN only for a NaN weight or value, for w = +inf at
// d = 0, or for w = +-0 at an infinite d. With the reference's weights
// (qw*sqrt(sigma2 + x^2), or x^2 without an imatrix) a NaN distance never sits
// next to a finite one: an infinite d needs |x| or sc (at most about max |x|)
// near 1e37, where x^2 and sigma2 overflow, so every searched subgroup then
// holds a +inf or NaN weight (a subgroup off the all-zero code has a value at
// level >= 1, within a factor ~10 of max |x|); and a +inf or NaN weight makes
// that value's term +inf or NaN for every candidate. So when no distance is
// finite, iq_search hands the list back (iq_search_miss) and iq_rescan scans
// it in order for the first NaN, else takes the first entry; otherwise the
// least key is the argmin.
//
// PRUNE: the search of subgroup s (scale sc, the very operand of its
// distance terms) reads the code's reduced list when the code's level
// is a best level in each of its values (no level's term below its term). A
// term is t(v) = (w*d)*d with d = sc*v - x, computed in f32. For a finite
// w >= 0 it is a non-decreasing function of |d| (rounding is monotone and
// sign-symmetric), and for sc > 0, d is non-decreasing in v. So when the code
// level's |d| is strictly below both neighbouring levels' (the grid's levels
// are 0..3 for IQ2 and 0..7 for IQ3; at an end the missing neighbour is not
// needed), d changes sign there, every other level's |d| is at least the
// code level's, and so is its term: the check takes two instructions a
// level instead of the four a term takes. The weights are square roots
// (>= 0, -0 or NaN). A NaN weight makes every distance NaN (the first entry
// wins, and no reduced list leaves it out); at a +inf weight only the code's
// level can have d = 0, so an entry left out for an earlier one that keeps
// every level it keeps is NaN only when that earlier one is: the first NaN
// and the first entry are the same in either list. With PRUNE 2, where the
// check fails only in values at the clamped top level 2 (IQ2) whose level-3
// |d| is strictly below the level-2 |d| (so d < 0 at level 2 and levels 0 and
// 1 have terms no smaller), the clamp-tolerant reduced list is read (an entry
// it leaves out also shares every raise to level 3 with the earlier one). A
// NaN or infinite d at the code level, a tie or sc <= 0 reads the full
// list. PRUNE 0 reads the full lists.
template <int BITS, int NV, int NSUB, int PRUNE = 0, int N>
QS_DEV void iq_codes(const IqTabDev& T, const float (&xv)[N], float inv, uint32_t (&ci)[NSUB], float sc) {
    // all subgroups' codes first, so their cinfo loads are in flight together
    constexpr float LMAX = BITS == 2 ? 2.0f : 7.0f;
    constexpr float GMAX = BITS == 2 ? 3.0f : 7.0f;     // the grid's largest level
    // per subgroup, PRUNE 1: whether the code's level is every value's best
    // level, a bool (a lane mask: its updates take no VALU instructions);
    // PRUNE 2: an int with bit 0 set when a value's code level is not its
    // best level and bit 1 when the clamp-tolerant list does not hold either
    // (two bools per subgroup spill in the IQ2_XXS search)
    int code[NSUB], miss[NSUB];
    bool best[NSUB];
    const bool prune = PRUNE > 0 && sc > 0.0f;
#pragma unroll
    for (int s = 0; s < NSUB; s++) {
        code[s] = 0;
        best[s] = prune;
        miss[s] = prune ? 0 : 3;
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const float x = xv[NV * s + j];
            float t = inv * x;
            t = t - 1.0f;
            t = 0.5f * t;
            const float lf = clampf(rintf(t), 0.0f, LMAX);
            code[s] |= (int)lf << (BITS * j);
            if constexpr (PRUNE > 0) {
                const float v = 2.0f * lf + 1.0f;
                auto dist = [&](float lv) {
                    float d = sc * lv;
                    d = d - x;
                    return fabsf(d);
                };
                const float du = dist(v), dm = dist(v - 2.0f), dp = dist(v + 2.0f);
                const bool ok = (lf == 0.0f || du < dm) && (lf == GMAX || du < dp);
                if constexpr (PRUNE == 2) {
                    // the clamped top level with the grid's level 3 strictly closer
                    const bool up = LMAX < GMAX && lf == LMAX && dp < du;
                    miss[s] |= ok ? 0 : up ? 1 : 3;
                } else {
                    best[s] = best[s] && ok;
                }
            }
        }
    }
#pragma unroll
    for (int s = 0; s < NSUB; s++) {
        int tab = best[s] ? 1 : 0;
        if constexpr (PRUNE == 2) tab = miss[s] == 0 ? 1 : miss[s] == 1 ? 2 : 0;
        ci[s] = T.cinfo[code[s] + tab * T.ncodes];
    }
}

// The values and distance weights of one subgroup, passed by value.
template <int NV>
struct IqSub {
    float x[NV], w[NV];
};

// torch's argmin over one neighbour list, entry by entry, with the distance
// arithmetic of iq_chunk_best: the first NaN distance, else the first
// minimum (the list's first entry when every distance is +inf). It runs
// only for lists with no finite distance; iq_argmin_scan_call keeps one copy
// out of line per kernel.
template <int NV, int CH>
QS_DEV int iq_argmin_scan(const uint16_t* nbr, const uint32_t* glds, uint32_t ci, const IqSub<NV>& v, float sc) {
    const uint16_t* list = nbr + (size_t)((ci >> 12) & 0x7ffffu) * CH;
    const int n = (int)(ci & 0xfffu);
    int best_gi = list[0];
    float best = 0.0f;
    for (int k = 0; k < n; k++) {
        const int gi = list[k];
        const Levels<NV> gl = grid_levels<NV>(glds, gi);
        float d2 = 0.0f;
#pragma unroll
        for (int e = 0; e < NV; e++) {
            float diff = sc * level<NV>(gl, e);
            diff = diff - v.x[e];
            const float t = (v.w[e] * diff) * diff;
            d2 = (e == 0) ? t : d2 + t;
        }
        if (d2 != d2) return gi;
        if (k == 0 || d2 < best) {
            best = d2;
            best_gi = gi;
        }
    }
    return best_gi;
}

template <int NV, int CH>
__device__ __attribute__((noinline)) int iq_argmin_scan_call(const uint16_t* nbr, const uint32_t* glds, uint32_t ci,
                                                             IqSub<NV> v, float sc) {
    return iq_argmin_scan<NV, CH>(nbr, glds, ci, v, sc);
}

// First minimum of one chunk (CH list slots from slot CH*kc) as a 64-bit key
// (distance bits, list position, grid index); slots past the list end (o_n)
// are masked out. Every slot is evaluated (padding holds index 0, a valid
// grid point), without branches. IQ2: slots are visited in list order, so a
// strict `d2 < best` keeps the first minimum and the key is built once per
// chunk (4-7% faster); a chunk with no finite distance returns ~0 (as if it
// held no candidate: with no finite distance anywhere in the list the search
// hands the list to iq_rescan either way). IQ3 compares
// the 64-bit key per slot (its 4-slot chunks measured 1-2% faster that way).
template <int BITS, int NV, int CH>
QS_DEV unsigned long long iq_chunk_best(const uint32_t* glds, const uint32_t (&wd)[CH / 2], int kc, int o_n,
                                        float o_sc, const float (&xs)[NV], const float (&ws)[NV]) {
    unsigned long long best = ~0ull;     // IQ3
    float best_d2 = __builtin_inff();    // IQ2
    int best_j = -1;
    // every slot's grid levels are read from LDS before any is used, so the
    // chunk waits for LDS once instead of once per slot
    int gi[CH];
    Levels<NV> gl[CH];
#pragma unroll
    for (int j = 0; j < CH; j++) {
        gi[j] = (int)((wd[j >> 1] >> (16 * (j & 1))) & 0xffffu);
        gl[j] = grid_levels<NV>(glds, gi[j]);
    }
#pragma unroll
    for (int j = 0; j < CH; j++) {
        const int pos = CH * kc + j;
        float d2 = 0.0f;
#pragma unroll
        for (int e = 0; e < NV; e++) {
            float diff = o_sc * level<NV>(gl[j], e);
            diff = diff - xs[e];
            // IQ2's sum runs from +0 (iq2.py) and IQ3's from its first term;
            // t = (w*d)*d is -0 only for w = -0, and a subgroup whose weights
            // are all -0 has -0 (or NaN) for every candidate, so starting
            // from the first term decides no different minimum
            const float t = (ws[e] * diff) * diff;
            d2 = (e == 0) ? t : d2 + t;
        }
        if constexpr (BITS == 3) {
            const unsigned long long key = ((unsigned long long)__float_as_uint(d2) << 32) |
                                           ((unsigned long long)pos << 16) | (unsigned)gi[j];
            best = (pos < o_n && key < best) ? key : best;
        } else {
            const bool take = pos < o_n && d2 < best_d2;
            best_d2 = take ? d2 : best_d2;
            best_j = take ? j : best_j;
        }
    }
    if constexpr (BITS == 3) return best;
    if (best_j < 0) return ~0ull;
    int best_gi = gi[0];
#pragma unroll
    for (int j = 1; j < CH; j++) best_gi = best_j == j ? gi[j] : best_gi;
    return ((unsigned long long)__float_as_uint(best_d2) << 32) |
           ((unsigned long long)(CH * kc + best_j) << 16) | (unsigned)best_gi;
}

template <int CH>
QS_DEV void iq_load_chunk(const IqTabDev& T, size_t chunk, uint32_t (&wd)[CH / 2]) {
    if constexpr (CH == 8) {
        const uint4 q = reinterpret_cast<const uint4*>(T.nbr)[chunk];
        wd[0] = q.x; wd[1] = q.y; wd[2] = q.z; wd[3] = q.w;
    } else {
        const uint2 q = reinterpret_cast<const uint2*>(T.nbr)[chunk];
        wd[0] = q.x; wd[1] = q.y;
    }
}

// The result of a search with no finite distance: its list's cinfo word
// (off-grid, so bit 31 is free) with bit 31 set, a negative int.
QS_DEV int iq_search_miss(uint32_t ci) { return (int)(ci | CI_ON_GRID); }

template <int BITS, int NV, int OFF, int CH, int MAXCH, bool WL = false, int N>
QS_DEV int iq_search(const IqTabDev& T, const uint32_t* glds, uint8_t* cmap, unsigned long long* res,
                     const float (&xv)[N], const float (&wv)[N], float sc, uint32_t ci, bool want,
                     bool& on) {
    static_assert(CH == 4 || CH == 8, "chunks are one 8- or 16-byte load");
    const int lane = WL ? lane_id() : (int)threadIdx.x;
    on = (ci & CI_ON_GRID) != 0;
    const int n = (on || !want) ? 0 : (int)(ci & 0xfffu);
    // IQ3: the list's first chunk is evaluated by its own lane, loaded here,
    // before the scan, with no lane exchange, and only chunks 1.. are dealt
    // (IQ3's lists are a chunk or two: 2-6% faster). IQ2 deals every chunk
    // (its own-chunk variant measured up to 7% slower).
    constexpr int FIRST = BITS == 3 ? 1 : 0;     // chunks the owner evaluates itself
    uint32_t own[CH / 2];
#pragma unroll
    for (int i = 0; i < CH / 2; i++) own[i] = 0;
    if (FIRST && n > 0) iq_load_chunk<CH>(T, (ci >> 12) & 0x7ffffu, own);
    const int nch = (n + CH - 1) / CH;
    const int nd = nch > FIRST ? nch - FIRST : 0;
    // exclusive prefix sum of the lanes' dealt chunk counts, a DPP scan (VALU
    // only; against a shuffle scan: IQ3 5-8%, IQ2_XXS 5%, IQ2_S 2% faster)
    const int incl = wave_incl_scan(nd);
    const int excl = incl - nd;
    // the wave's dealt chunk count, read from lane 63 into a scalar register
    // so the round loop is scalar-controlled
    const int total = __builtin_amdgcn_readlane(incl, 63);
    for (int i = 0; i < nd; i++) cmap[excl + i] = (uint8_t)lane;
    res[lane] = ~0ull;
    unsigned long long best_own = ~0ull;
    if (FIRST && n > 0) {
        float xs[NV], ws[NV];
#pragma unroll
        for (int e = 0; e < NV; e++) {
            xs[e] = xv[OFF + e];
            ws[e] = wv[OFF + e];
        }
        best_own = iq_chunk_best<BITS, NV, CH>(glds, own, 0, n, sc, xs, ws);
    }
    wave_sync<WL>();
    for (int base = 0; base < total; base += 64) {
        const int c = base + lane;
        const bool have = c < total;
        const int owner = have ? (int)cmap[c] : lane;
        const int o_excl = __shfl(excl, owner);
        const uint32_t o_ci = (uint32_t)__shfl((int)ci, owner);
        const float o_sc = __shfl(sc, owner);
        float xs[NV], ws[NV];
#pragma unroll
        for (int e = 0; e < NV; e++) {
            xs[e] = __shfl(xv[OFF + e], owner);
            ws[e] = __shfl(wv[OFF + e], owner);
        }
        const int kc = FIRST + c - o_excl;
        const int o_n = (int)(o_ci & 0xfffu);
        if (have && kc >= FIRST && CH * kc < o_n) {    // a dealt chunk lies inside its owner's list
            uint32_t wd[CH / 2];
            iq_load_chunk<CH>(T, ((o_ci >> 12) & 0x7ffffu) + (size_t)kc, wd);
            atomicMin(&res[owner], iq_chunk_best<BITS, NV, CH>(glds, wd, kc, o_n, o_sc, xs, ws));
        }
    }
    wave_sync<WL>();
    if (on) return (int)(ci & 0xffffu);
    const unsigned long long r0 = res[lane];
    const unsigned long long r = r0 < best_own ? r0 : best_own;
    // a finite first minimum (-0, every distance of a subgroup whose weights
    // are all -0, counts as one), else the list for iq_rescan
    const bool fin = ((uint32_t)(r >> 32) & 0x7fffffffu) < 0x7f800000u;
    return !want ? 0 : fin ? (int)(r & 0xffffu) : iq_search_miss(ci);     // off-grid: n > 0 iff want
}

// Every subgroup whose search found no finite distance (rare: an infinite
// or NaN weight, value or scale) gets torch's argmin from an in-order scan
// of its list; the wave skips this when none did. OUTLINE calls the scan
// out of line, which leaves the kernel's search code as it was: IQ2_XXS ran
// 3.4%, IQ2_S 2.0% and IQ3_XXS 0.6% faster that way (IQ3_S alike), IQ2_XS
// 2.8% slower.
template <int NV, int CH, bool OUTLINE, int NSUB, int N>
QS_DEV void iq_rescan(const IqTabDev& T, const uint32_t* glds, const float (&xv)[N], const float (&wv)[N],
                      float sc, int (&gi)[NSUB]) {
    bool miss = false;
#pragma unroll
    for (int s = 0; s < NSUB; s++) miss = miss || gi[s] < 0;
    if (!wave_any(miss)) return;
    static_for<0, NSUB>([&](auto S) {
        if (gi[S] < 0) {
            IqSub<NV> v;
#pragma unroll
            for (int e = 0; e < NV; e++) {
                v.x[e] = xv[NV * S + e];
                v.w[e] = wv[NV * S + e];
            }
            const uint32_t ci = (uint32_t)gi[S] & ~CI_ON_GRID;
            if constexpr (OUTLINE) gi[S] = iq_argmin_scan_call<NV, CH>(T.nbr, glds, ci, v, sc);
            else gi[S] = iq_argmin_scan<NV, CH>(T.nbr, glds, ci, v, sc);
        }
    });
}

// sign-parity fold of 8 values (iq2.py:438-450): |x|, the smallest (w*x)*x
// entry negated when the sign count is odd; returns the 7 stored sign bits
template <int OFF, int N>
QS_DEV int parity_fold8(const float (&x)[N], const float (&w)[N], float (&xval)[N]) {
    int s = 0, nneg = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        xval[OFF + j] = fabsf(x[OFF + j]);
        const bool neg = x[OFF + j] < 0;
        s |= neg ? (1 << j) : 0;
        nneg += neg ? 1 : 0;
    }
    float m = (w[OFF] * x[OFF]) * x[OFF];
    int imin = 0;
#pragma unroll
    for (int j = 1; j < 8; j++) {
        const float v = (w[OFF + j] * x[OFF + j]) * x[OFF + j];
        const bool lt = v < m;
        m = lt ? v : m;
        imin = lt ? j : imin;
    }
    const bool odd = nneg & 1;
#pragma unroll
    for (int j = 0; j < 8; j++)
        if (odd && imin == j) xval[OFF + j] = -xval[OFF + j];
    s ^= odd ? (1 << imin) : 0;
    return s & 127;
}

template <int OFF, int N>
QS_DEV int sign_bits8(const float (&x)[N], float (&xval)[N]) {
    int s = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        xval[OFF + j] = fabsf(x[OFF + j]);
        s |= x[OFF + j] < 0 ? (1 << j) : 0;
    }
    return s;
}

// sums of (w*xval)*q and (w*q)*q over the lane's group for grid winners gi[],
// reduced as tree_sum over the whole group: NV is a power
// of two, so the group's pairwise tree is each subgroup's own tree followed by
// a tree over the NSUB subgroup sums; reducing per subgroup keeps 2*NSUB
// partials live instead of 2*N products
template <int BITS, int NV, int NSUB, int N>
QS_DEV void iq_tree_sums(const uint32_t* glds, const int (&gi)[NSUB], const float (&w)[N], const float (&xval)[N],
                         float& sumqx, float& sumq2) {
    static_assert(NV * NSUB == N && (NV & (NV - 1)) == 0, "subgroups must tile the group");
    float sa[NSUB], sb[NSUB];
#pragma unroll
    for (int s = 0; s < NSUB; s++) {
        const Levels<NV> gl = grid_levels<NV>(glds, gi[s]);
        float a[NV], b[NV];
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const float q = level<NV>(gl, j);
            a[j] = (w[NV * s + j] * xval[NV * s + j]) * q;
            b[j] = (w[NV * s + j] * q) * q;
        }
        sa[s] = tree_sum(a);
        sb[s] = tree_sum(b);
    }
    if constexpr (NSUB == 1) {
        sumqx = sa[0];
        sumq2 = sb[0];
    } else {
        sumqx = tree_sum(sa);
        sumq2 = tree_sum(sb);
    }
}

// The same two sums reduced as cascade8_sum<32> (torch's `.sum(-1)` over 32):
// lane l of the 8-wide accumulator is ((v[l] + v[8+l]) + v[16+l]) + v[24+l],
// i.e. the four 8-value subgroups added in order, then +0 + p[0] + ... + p[7];
// accumulating subgroup by subgroup keeps 16 partials live instead of 64
// products.
QS_DEV void iq_cascade_sums_32(const uint32_t* glds, const int (&gi)[4], const float (&w)[32],
                               const float (&xval)[32], float& sumqx, float& sumq2) {
    float pa[8], pb[8];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const Levels<8> gl = grid_levels<8>(glds, gi[s]);
#pragma unroll
        for (int l = 0; l < 8; l++) {
            const float q = level<8>(gl, l);
            float wl = w[8 * s + l];
            keep_in_register(wl);          // w * xval stays in the loop, not 32 hoisted products
            const float a = (wl * xval[8 * s + l]) * q;
            const float b = (wl * q) * q;
            pa[l] = s == 0 ? a : pa[l] + a;
            pb[l] = s == 0 ? b : pb[l] + b;
        }
    }
    float fa = 0.0f, fb = 0.0f;
#pragma unroll
    for (int l = 0; l < 8; l++) {
        fa = fa + pa[l];
        fb = fb + pb[l];
    }
    sumqx = fa;
    sumq2 = fb;
}

// superblock scale nibbles: d = max/31, l = clamp(round(0.5*(sc/d - 1)), 0, 15)
// (iq2.py:92-96, iq2xs_common.py:345-355, iq3_xxs.py:115-121)
template <int NG>
QS_DEV void iq_scale_nibbles(const float* sc, float& d, bool& has, int (&l)[NG]) {
    float mx = sc[0];
#pragma unroll
    for (int i = 1; i < NG; i++) mx = fmaxf(mx, sc[i]);
    has = mx > 0;
    d = mx / 31.0f;
    const float inv_d = 1.0f / (has ? d : 1.0f);
#pragma unroll
    for (int i = 0; i < NG; i++) {
        float t = inv_d * sc[i];
        t = t - 1.0f;
        t = 0.5f * t;
        l[i] = (int)clampf(rintf(t), 0.0f, 15.0f);
    }
}

struct IqSteps {
    float v[32];
    int n;
};

template <int SRC, int LPS, int GROUP, int SQ, bool WL = false>
QS_DEV void iq_load_weights(const KArgs& a, const SbPos& p, float (*vlds)[QK_K], float (*tmp)[40],
                            float sig_mult, bool use_x2, float (&x)[GROUP], float (&w)[GROUP]) {
    constexpr int SPW = 64 / LPS;
    load_elems<SRC, true, GROUP>(a.src, p.elem, x);
    if (use_x2) {
#pragma unroll
        for (int i = 0; i < GROUP; i++) w[i] = x[i] * x[i];
        return;
    }
    const float sum = sb_sumsq_halves<LPS, SPW, GROUP, WL>(vlds, tmp, x, p.slot, p.g);
    const float sigma2 = (sig_mult == 2.0f ? 2.0f * sum : sum) / 256.0f;
    imatrix_weights<GROUP, true, SQ>(a.qw + p.col, sigma2, x, a.sqrt, w);
}

// ------------------------------------------------------------------
// IQ2_XXS  quantize_iq2_xxs iq2.py:418-498 (+ _finalize :87-108)
// ------------------------------------------------------------------
template <int SRC, int SQ>
// 3 waves per SIMD (168 VGPRs, some spills): 9% faster than 2 waves unspilled
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(3))) void k_iq2_xxs(KArgs a, IqTabDev T, QpSteps qp4, IqSteps sweep) {
    constexpr int LPS = 8, SPW = 8, BYTES = 66;
    __shared__ IqLds<SPW, BYTES> s;
    __shared__ __align__(16) uint32_t glds[256 * 2];
    __shared__ uint8_t cmap[64 * IQ2_256_MAXCH];
    __shared__ unsigned long long res[64];
    stage_levels<2, 8, 256>(T.grid, glds);
    const SbPos p = sb_pos<LPS, 32>(a.n_units, a.units_per_row, a.stride);
    const int slot = p.slot, g = p.g;
    float x[32], w[32], waux[32], xval[32];
    iq_load_weights<SRC, LPS, 32, SQ>(a, p, s.v, s.tmp, 1.0f, false, x, w);
    sqrt_ref_n<32, true, SQ>(w, a.sqrt, waux);
    keep_in_registers(waux);
    int signs[4];
    static_for<0, 4>([&](auto S) { signs[S] = parity_fold8<8 * S>(x, w, xval); });
    float gmax = xval[0];
#pragma unroll
    for (int i = 1; i < 32; i++) gmax = fmaxf(gmax, xval[i]);
    bool active = gmax >= GROUP_MAX_EPS;
    float Lq[32];
    const float scale0 = qp_fit<32>(xval, w, 4, qp4.v, Lq);
    const float eff = scale0 * 3.0f;
    active = active && eff > 0;
    const float eff_safe = active ? eff : 1.0f;
    float scale = scale0, best = 0.0f;
    const int zero_gi = T.code0;
    int L[4] = {zero_gi, zero_gi, zero_gi, zero_gi};
#pragma unroll 1
    for (int st = 0; st < sweep.n; st++) {
        const float inv = rdiv(sweep.v[st], eff_safe);
        const float sc = 1.0f / inv;
        int gi[4];
        bool on;
        uint32_t ci[4];
        iq_codes<2, 8, 4, 2>(T, xval, inv, ci, sc);
        static_for<0, 4>([&](auto S) {
            gi[S] = iq_search<2, 8, 8 * S, IQ2_CH, IQ2_256_MAXCH>(T, glds, cmap, res, xval, waux, sc, ci[S], true, on);
        });
        iq_rescan<8, IQ2_CH, true>(T, glds, xval, waux, sc, gi);
        float sumqx, sumq2;
        iq_cascade_sums_32(glds, gi, w, xval, sumqx, sumq2);
        if (active && sumq2 > 0 && sumqx * sumqx > best * sumq2) {
            const float ns = sumqx / fmaxf(sumq2, F32_TINY);
            scale = ns;
            best = ns * sumqx;
#pragma unroll
            for (int k = 0; k < 4; k++) L[k] = gi[k];
        }
    }
    const bool proj = active && scale > 0;
    {
        const float inv = 1.0f / (proj ? scale : 1.0f);
        int gp[4];
        bool on;
        uint32_t ci[4];
        iq_codes<2, 8, 4, 2>(T, xval, inv, ci, scale);
        static_for<0, 4>([&](auto S) {
            gp[S] = iq_search<2, 8, 8 * S, IQ2_CH, IQ2_256_MAXCH>(T, glds, cmap, res, xval, waux, scale, ci[S], proj, on);
        });
        iq_rescan<8, IQ2_CH, true>(T, glds, xval, waux, scale, gp);
        float sumqx, sumq2;
        iq_cascade_sums_32(glds, gp, w, xval, sumqx, sumq2);
        if (proj && sumq2 > 0) scale = sumqx / fmaxf(sumq2, F32_TINY);
        if (proj) {
#pragma unroll
            for (int k = 0; k < 4; k++) L[k] = gp[k];
        }
    }
    if (active && scale < 0) {
        scale = -scale;
#pragma unroll
        for (int k = 0; k < 4; k++) signs[k] = (~signs[k]) & 127;
    }
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        lo |= (uint32_t)L[k] << (8 * k);
        hi |= (uint32_t)signs[k] << (7 * k);
    }
    s.sc[slot][g] = active ? scale : 0.0f;
    wave_sync();
    float d;
    bool has;
    int l[8];
    iq_scale_nibbles<8>(s.sc[slot], d, has, l);
    const uint32_t wlo = (active && has) ? lo : 0u;
    const uint32_t whi = has ? ((active ? hi : 0u) | ((uint32_t)l[g] << 28)) : 0u;
    uint8_t* o = s.out + slot * BYTES;
    if (g == 0) {
        const uint32_t h = f16_bits(has ? d : 0.0f);
        o[0] = (uint8_t)h;
        o[1] = (uint8_t)(h >> 8);
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        o[2 + 8 * g + k] = (uint8_t)(wlo >> (8 * k));
        o[2 + 8 * g + 4 + k] = (uint8_t)(whi >> (8 * k));
    }
    wave_sync();
    sb_store(s, a);
}

// ------------------------------------------------------------------
// IQ2_XS / IQ2_S  scale_search iq2xs_common.py:280-342; quantize_iq2_xs
// iq2_xs.py:20-69; quantize_iq2_s iq2_s.py:21-62
// ------------------------------------------------------------------
template <int SRC, bool IS_S, int SQ, int WPG>
// WPG waves per workgroup share one staged grid (4 / 8 KB) and keep their own
// search and output buffers; each wave quantizes its own superblocks and
// syncs only with itself once the grid is staged. IQ2_S (8 KB of grid, 12.4
// KB of LDS per one-wave workgroup, 156 VGPRs: 3 waves per SIMD) runs 4
// waves per workgroup at 6.3 KB of LDS and 128 VGPRs per wave (4 waves per
// SIMD, 20 spilled): 6% faster. IQ2_XS fits 4 waves per SIMD in one-wave
// workgroups already (127 VGPRs, 10.1 KB) and stays there (1% slower with 4)
__global__ __launch_bounds__(64 * WPG) __attribute__((amdgpu_waves_per_eu(IS_S && WPG == 1 ? 3 : 4))) void k_iq2_xs_s(KArgs a, IqTabDev T, IqSteps sweep) {
    constexpr int LPS = 16, SPW = 4, BYTES = IS_S ? 82 : 74, GS = IS_S ? 1024 : 512;
    constexpr int MAXCH = IS_S ? IQ2_1024_MAXCH : IQ2_512_MAXCH;
    __shared__ IqLds<SPW, BYTES> s_w[WPG];
    __shared__ __align__(16) uint32_t glds[GS * 2];
    __shared__ int wlds_w[WPG][SPW][16][2];
    __shared__ uint8_t cmap_w[WPG][64 * MAXCH];
    __shared__ unsigned long long res_w[WPG][64];
    const int wave = (int)(threadIdx.x >> 6);
    IqLds<SPW, BYTES>& s = s_w[wave];
    int (*wlds)[16][2] = wlds_w[wave];
    uint8_t* cmap = cmap_w[wave];
    unsigned long long* res = res_w[wave];
    constexpr bool WL = WPG > 1;
    stage_levels<2, 8, GS, 64 * WPG>(T.grid, glds);
    if constexpr (WL) __syncthreads();            // the grid is every wave's
    const SbPos p = sb_pos<LPS, 16, WPG>(a.n_units, a.units_per_row, a.stride);
    const int slot = p.slot, g = p.g;
    float x[16], w[16], waux[16], xval[16];
    iq_load_weights<SRC, LPS, 16, SQ, WL>(a, p, s.v, s.tmp, IS_S ? 2.0f : 1.0f, false, x, w);
    sqrt_ref_n<16, true, SQ>(w, a.sqrt, waux);
    int signs[2];
    if constexpr (IS_S) {
        signs[0] = sign_bits8<0>(x, xval);
        signs[1] = sign_bits8<8>(x, xval);
    } else {
        signs[0] = parity_fold8<0>(x, w, xval);
        signs[1] = parity_fold8<8>(x, w, xval);
    }
    float gmax = xval[0];
#pragma unroll
    for (int i = 1; i < 16; i++) gmax = fmaxf(gmax, xval[i]);
    const bool active = IS_S ? gmax >= 1e-8f : gmax >= GROUP_MAX_EPS;
    const float gsafe = active ? gmax : 1.0f;
    const int code0 = T.code0;
    float scale = active ? gmax / 5.0f : 0.0f, best = 0.0f;
    int win[2] = {code0, code0};
    bool og[2] = {true, true};
#pragma unroll 1
    for (int st = 0; st < sweep.n; st++) {
        const float inv = rdiv(sweep.v[st], gsafe), sc = 1.0f / inv;
        int gi[2];
        bool on[2];
        uint32_t ci[2];
        iq_codes<2, 8, 2, IS_S ? 0 : 1>(T, xval, inv, ci, sc);
        gi[0] = iq_search<2, 8, 0, IQ2_CH, MAXCH, WL>(T, glds, cmap, res, xval, waux, sc, ci[0], true, on[0]);
        gi[1] = iq_search<2, 8, 8, IQ2_CH, MAXCH, WL>(T, glds, cmap, res, xval, waux, sc, ci[1], true, on[1]);
        iq_rescan<8, IQ2_CH, IS_S>(T, glds, xval, waux, sc, gi);
        float sumqx, sumq2;
        iq_tree_sums<2, 8, 2>(glds, gi, w, xval, sumqx, sumq2);
        if (active && sumq2 > 0 && sumqx * sumqx > best * sumq2) {
            const float ns = sumqx / fmaxf(sumq2, F32_TINY);
            scale = ns;
            best = ns * sumqx;
            win[0] = gi[0];
            win[1] = gi[1];
            og[0] = on[0];
            og[1] = on[1];
        }
    }
    const bool need = active && scale > 0 && !(og[0] && og[1]);
    {
        // every lane takes part in the wave search; only off-grid winners of
        // lanes that need it are searched and replaced
        const float inv = 1.0f / (need ? scale : 1.0f);
        bool on;
        uint32_t ci[2];
        iq_codes<2, 8, 2, IS_S ? 0 : 1>(T, xval, inv, ci, scale);
        int r[2];
        r[0] = iq_search<2, 8, 0, IQ2_CH, MAXCH, WL>(T, glds, cmap, res, xval, waux, scale, ci[0],
                                                     need && !og[0], on);
        r[1] = iq_search<2, 8, 8, IQ2_CH, MAXCH, WL>(T, glds, cmap, res, xval, waux, scale, ci[1],
                                                     need && !og[1], on);
        iq_rescan<8, IQ2_CH, IS_S>(T, glds, xval, waux, scale, r);
        if (need && !og[0]) win[0] = r[0];
        if (need && !og[1]) win[1] = r[1];
    }
    if (need) {
        float sumqx, sumq2;
        iq_tree_sums<2, 8, 2>(glds, win, w, xval, sumqx, sumq2);
        if (sumq2 > 0) scale = sumqx / fmaxf(sumq2, F32_TINY);
    }
    if (active && scale < 0) {
        scale = -scale;
        signs[0] = (~signs[0]) & (IS_S ? 255 : 127);
        signs[1] = (~signs[1]) & (IS_S ? 255 : 127);
    }
    s.sc[slot][g] = active ? scale : 0.0f;
    wlds[slot][g][0] = active ? win[0] : 0;
    wlds[slot][g][1] = active ? win[1] : 0;
    wave_sync<WL>();
    float d;
    bool has;
    int l[16];
    iq_scale_nibbles<16>(s.sc[slot], d, has, l);
    uint8_t* o = s.out + slot * BYTES;
    if constexpr (!IS_S) {
        if (g == 0) {
            const uint32_t h = f16_bits(has ? d : 0.0f);
            o[0] = (uint8_t)h;
            o[1] = (uint8_t)(h >> 8);
        }
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const uint32_t q2 = (active && has) ? ((uint32_t)win[k] | ((uint32_t)signs[k] << 9)) : 0u;
            o[2 + 4 * g + 2 * k] = (uint8_t)q2;
            o[2 + 4 * g + 2 * k + 1] = (uint8_t)(q2 >> 8);
        }
        if (g < 8) o[66 + g] = (uint8_t)(has ? (l[2 * g] | (l[2 * g + 1] << 4)) : 0);
    } else {
        if (g == 0) {
            const uint32_t h = f16_bits(has ? d * 0.9875f : 0.0f);
            o[0] = (uint8_t)h;
            o[1] = (uint8_t)(h >> 8);
        }
#pragma unroll
        for (int k = 0; k < 2; k++) {
            o[2 + 2 * g + k] = (uint8_t)((active ? win[k] : 0) & 255);
            o[34 + 2 * g + k] = (uint8_t)(active ? signs[k] : 0);
        }
        if (g < 8) {
            int v = 0;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int sub = 4 * g + t;
                v |= (wlds[slot][sub >> 1][sub & 1] >> 8) << (2 * t);
            }
            o[66 + g] = (uint8_t)v;
            o[74 + g] = (uint8_t)(has ? (l[2 * g] | (l[2 * g + 1] << 4)) : 0);
        }
    }
    wave_sync<WL>();
    sb_store<SPW, BYTES, WPG>(s, a);
}

// ------------------------------------------------------------------
// IQ3_XXS / IQ3_S  quantize_iq3_xxs iq3_xxs.py:31-134, quantize_iq3_s
// iq3_s.py:31-140
// ------------------------------------------------------------------



// IQ3_XXS / IQ3_S (iq3_common.py:209-256, iq3_xxs.py:31-134, iq3_s.py:31-140)
// with LPG lanes per 32-value group: each lane holds 32/LPG values (its
// subgroups of 4), a wave takes 8/LPG superblocks and each subgroup pass
// searches one list per lane. The group's sums are the lanes' trees joined
// by a butterfly of lane exchanges: the reference's tree over the 8 subgroup
// sums is ((s0+s1)+(s2+s3)) + ((s4+s5)+(s6+s7)), each exchange level joins
// two adjacent subtrees, and fl(a + b) = fl(b + a), so every lane of the
// group holds the same bits and takes the same accept and re-projection
// decisions (the maximum, the off-grid flag and the packed sign and high-bit
// words are joined the same way). Measured against one lane per group (168
// VGPRs with 59-64 spilled at 3 waves per SIMD; IQ3_S with imatrix at 2):
// LPG = 2 (125-128 VGPRs, 4 waves) IQ3_XXS 15%, IQ3_S 17%, IQ3_S with
// imatrix 25% faster; LPG = 4 (80 VGPRs, 6 waves) another 5-6.5%; same bytes.
template <int SRC, bool IS_S, bool IMAT, int SQ, int LPG>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(LPG == 4 ? 6 : 4))) void k_iq3(KArgs a, IqTabDev T, IqSteps steps) {
    constexpr int VPL = 32 / LPG, NSL = VPL / 4, NCH = VPL / 8;
    constexpr int LPS = 8 * LPG, SPW = 64 / LPS, BYTES = IS_S ? 110 : 98, GS = IS_S ? 512 : 256;
    constexpr int SMASK = IS_S ? 255 : 127;
    __shared__ IqLds<SPW, BYTES> s;
    __shared__ __align__(16) uint32_t glds[GS];
    __shared__ int act_lds[SPW][8];
    constexpr int MAXCH = IS_S ? IQ3_512_MAXCH : IQ3_256_MAXCH;
    __shared__ uint8_t cmap[64 * MAXCH];
    __shared__ unsigned long long res[64];
    stage_levels<3, 4, GS>(T.grid, glds);
    const SbPos p = sb_pos<LPS, VPL>(a.n_units, a.units_per_row, a.stride);
    const int slot = p.slot, grp = p.g / LPG, q = p.g % LPG;
    float x[VPL], w[VPL], waux[VPL], xval[VPL];
    iq_load_weights<SRC, LPS, VPL, SQ>(a, p, s.v, s.tmp, 2.0f, !IMAT, x, w);
    sqrt_ref_n<VPL, true, SQ>(w, a.sqrt, waux);
    keep_in_registers(waux);
    int signs[NCH];
    if constexpr (IS_S) {
        static_for<0, NCH>([&](auto S) { signs[S] = sign_bits8<8 * S>(x, xval); });
    } else {
        static_for<0, NCH>([&](auto S) { signs[S] = parity_fold8<8 * S>(x, w, xval); });
    }
    float gmax = xval[0];
#pragma unroll
    for (int i = 1; i < VPL; i++) gmax = fmaxf(gmax, xval[i]);
#pragma unroll
    for (int m = 1; m < LPG; m <<= 1) gmax = fmaxf(gmax, __shfl_xor(gmax, m));
    const bool active = IS_S ? gmax > 0 : gmax >= 1e-8f;
    const float gsafe = active ? gmax : 1.0f;
    float scale = gmax / 15.0f, best = 0.0f;
    int Wg[NSL];
    bool og[NSL];
#pragma unroll
    for (int k = 0; k < NSL; k++) {
        Wg[k] = 0;
        og[k] = !IS_S;
    }
    auto group_sums = [&](const int (&gi)[NSL], float& sumqx, float& sumq2) {
        float hx, h2;
        iq_tree_sums<3, 4, NSL>(glds, gi, w, xval, hx, h2);
#pragma unroll
        for (int m = 1; m < LPG; m <<= 1) {
            hx = hx + __shfl_xor(hx, m);
            h2 = h2 + __shfl_xor(h2, m);
        }
        sumqx = hx;
        sumq2 = h2;
    };
    wave_sync();   // glds ready
#pragma unroll 1
    for (int st = 0; st < steps.n; st++) {
        const float inv = rdiv(steps.v[st], gsafe), sc = 1.0f / inv;
        int gi[NSL];
        bool on[NSL];
        uint32_t ci[NSL];
        iq_codes<3, 4, NSL, 1>(T, xval, inv, ci, sc);
        static_for<0, NSL>([&](auto S) {
            gi[S] = iq_search<3, 4, 4 * S, IQ3_CH, MAXCH>(T, glds, cmap, res, xval, waux, sc, ci[S], true, on[S]);
        });
        iq_rescan<4, IQ3_CH, true>(T, glds, xval, waux, sc, gi);
        float sumqx, sumq2;
        group_sums(gi, sumqx, sumq2);
        if (active && sumq2 > 0 && sumqx * sumqx > best * sumq2) {
            const float ns = sumqx / fmaxf(sumq2, F32_TINY);
            scale = ns;
            best = ns * sumqx;
#pragma unroll
            for (int k = 0; k < NSL; k++) {
                Wg[k] = gi[k];
                og[k] = on[k];
            }
        }
    }
    int anyoff = 0;
#pragma unroll
    for (int k = 0; k < NSL; k++) anyoff |= og[k] ? 0 : 1;
#pragma unroll
    for (int m = 1; m < LPG; m <<= 1) anyoff |= __shfl_xor(anyoff, m);
    const bool redo = active && anyoff && scale > 0;
    {
        const float inv2 = 1.0f / (redo ? scale : 1.0f);
        int w2[NSL];
        bool on[NSL];
        uint32_t ci[NSL];
        iq_codes<3, 4, NSL, 1>(T, xval, inv2, ci, scale);
        static_for<0, NSL>([&](auto S) {
            w2[S] = iq_search<3, 4, 4 * S, IQ3_CH, MAXCH>(T, glds, cmap, res, xval, waux, scale, ci[S],
                                                          redo && (IS_S || !og[S]), on[S]);
        });
        iq_rescan<4, IQ3_CH, true>(T, glds, xval, waux, scale, w2);
#pragma unroll
        for (int k = 0; k < NSL; k++)
            if (redo && (IS_S || !og[k])) Wg[k] = w2[k];
        float sumqx, sumq2;
        group_sums(Wg, sumqx, sumq2);
        if (redo && sumq2 > 0) scale = sumqx / fmaxf(sumq2, F32_TINY);
    }
    if (active && scale < 0) {
        scale = -scale;
#pragma unroll
        for (int k = 0; k < NCH; k++) signs[k] = (~signs[k]) & SMASK;
    }
    if (q == 0) {
        s.sc[slot][grp] = active ? scale : 0.0f;
        act_lds[slot][grp] = active ? 1 : 0;
    }
    uint8_t* o = s.out + slot * BYTES;
    for (int t = p.g; t < BYTES; t += LPS) o[t] = 0;
    wave_sync();
    float d;
    bool has;
    int l[8];
    iq_scale_nibbles<8>(s.sc[slot], d, has, l);
    if constexpr (!IS_S) {
        if (p.g == 0) {
            const uint32_t h = f16_bits(has ? d * 1.0125f : 0.0f);
            o[0] = (uint8_t)h;
            o[1] = (uint8_t)(h >> 8);
        }
        uint32_t word = 0;
#pragma unroll
        for (int k = 0; k < NCH; k++) word |= (uint32_t)(active ? signs[k] : 0) << (7 * (NCH * q + k));
#pragma unroll
        for (int m = 1; m < LPG; m <<= 1) word |= (uint32_t)__shfl_xor((int)word, m);
        word |= (uint32_t)l[grp] << 28;
        if (!has) word = 0;
#pragma unroll
        for (int k = 0; k < NSL; k++) o[2 + 8 * grp + NSL * q + k] = (uint8_t)((has && active) ? Wg[k] : 0);
        constexpr int WB = 4 / LPG;
#pragma unroll
        for (int k = 0; k < WB; k++) o[66 + 4 * grp + WB * q + k] = (uint8_t)(word >> (8 * (WB * q + k)));
    } else {
        if (p.g == 0) {
            const uint32_t h = f16_bits(has ? d * 1.033f : 0.0f);
            o[0] = (uint8_t)h;
            o[1] = (uint8_t)(h >> 8);
        }
        int hb = 0;
#pragma unroll
        for (int k = 0; k < NSL; k++) hb |= (Wg[k] >> 8) << (NSL * q + k);
#pragma unroll
        for (int m = 1; m < LPG; m <<= 1) hb |= __shfl_xor(hb, m);
        if (q == 0) o[66 + grp] = (uint8_t)(active ? hb : 0);
        if (active) {
            int slot_idx = 0;                  // live groups compact to the front (iq3_s.py:113-122)
            for (int j = 0; j < grp; j++) slot_idx += act_lds[slot][j];
#pragma unroll
            for (int k = 0; k < NSL; k++) o[2 + 8 * slot_idx + NSL * q + k] = (uint8_t)(Wg[k] & 255);
#pragma unroll
            for (int k = 0; k < NCH; k++) o[74 + 4 * slot_idx + NCH * q + k] = (uint8_t)signs[k];
        }
        if (p.g < 4) o[106 + p.g] = (uint8_t)(has ? (l[2 * p.g] | (l[2 * p.g + 1] << 4)) : 0);
    }
    wave_sync();
    sb_store(s, a);
}

}  // namespace qs
