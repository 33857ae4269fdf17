// C ABI of the gfx950 quantizer library: argument checks, per-type launch
// geometry and template dispatch. Declarations and the reference interfaces
// they replace are in include/quant_studio.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <system_error>
#include <thread>
#include <tuple>
#include <utility>
#include <vector>

#include <zlib.h>

#include "quant_studio.h"
#include "qs_grids.h"
#include "qs_host.h"
#include "qs_iq.h"
#include "qs_kernels.h"
#include "qs_launch.h"
#include "qs_sqrt_table.h"

namespace {
thread_local std::string g_err;
}  // namespace

// The AMD-host square-root map (qs_sqrt_amd.bin: zlib-compressed, 2 bits per
// key, written by gen_sqrt_table.py --write-map on an AMD EPYC host),
// embedded at build time. Host code only.
#ifndef QS_SQRT_AMD_BIN
#error "build with -DQS_SQRT_AMD_BIN=<path of qs_sqrt_amd.bin> (quant-studio_amd/build.py)"
#endif
#if !defined(__HIP_DEVICE_COMPILE__)
__asm__(".section .rodata\n"
        ".balign 16\n"
        ".global qs_sqrt_amd_blob\n"
        ".hidden qs_sqrt_amd_blob\n"
        "qs_sqrt_amd_blob:\n"
        ".incbin \"" QS_SQRT_AMD_BIN "\"\n"
        ".global qs_sqrt_amd_blob_end\n"
        ".hidden qs_sqrt_amd_blob_end\n"
        "qs_sqrt_amd_blob_end:\n"
        ".previous\n");
#endif
extern "C" const unsigned char qs_sqrt_amd_blob[], qs_sqrt_amd_blob_end[];

namespace qs_host {

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

void clear_error() { g_err.clear(); }

}  // namespace qs_host

namespace {

using qs_host::fail;

struct TypeInfo {
    int id;
    const char* name;
    int blk, bytes;
    bool needs_imatrix, uses_imatrix;
    // the reference's quantizer function has no path without an imatrix
    // (IQ2_XXS / IQ2_XS / IQ2_S: iq2.py:418-431, iq2_xs.py:20-29, iq2_s.py:21-30
    // index qw unconditionally); IQ3_XXS's needs_imatrix is the command line's
    // policy only, its function takes None (iq3_xxs.py:41-42)
    bool fn_requires_imatrix;
};

// block sizes and type sizes: BLOCK_BYTES of each reference module
// (q4_0.py:11/:30-32, q2_k.py:19, q3_k.py:20, q4_k.py:19, q5_k.py:19,
// q6_k.py:19, iq4_xs.py:20, iq2.py:27, ...); imatrix flags from the SPECS
// entries (q4_0.py:40-43, q2_k.py:88-91, ..., iq3_s.py:148-151).
constexpr TypeInfo kTypes[] = {
    {QS_TYPE_Q4_0, "q4_0", 32, 18, false, false, false},
    {QS_TYPE_Q2_K, "q2_k", 256, 84, false, true, false},
    {QS_TYPE_Q3_K, "q3_k", 256, 110, false, true, false},
    {QS_TYPE_Q4_K, "q4_k", 256, 144, false, true, false},
    {QS_TYPE_Q5_K, "q5_k", 256, 176, false, true, false},
    {QS_TYPE_Q6_K, "q6_k", 256, 210, false, true, false},
    {QS_TYPE_IQ4_XS, "iq4_xs", 256, 136, false, true, false},
    {QS_TYPE_IQ2_XXS, "iq2_xxs", 256, 66, true, true, true},
    {QS_TYPE_IQ2_XS, "iq2_xs", 256, 74, true, true, true},
    {QS_TYPE_IQ2_S, "iq2_s", 256, 82, true, true, true},
    {QS_TYPE_IQ3_XXS, "iq3_xxs", 256, 98, true, true, false},
    {QS_TYPE_IQ3_S, "iq3_s", 256, 110, false, true, false},
    // ggml formats without a reference module (quant-studio.py:396-399 stops
    // on them): block layouts from the GGUF format; the imatrix is used by
    // IQ4_NL only (the 32-value integer formats ignore it, as Q4_0 does)
    {QS_TYPE_Q4_1, "q4_1", 32, 20, false, false, false},
    {QS_TYPE_Q5_0, "q5_0", 32, 22, false, false, false},
    {QS_TYPE_Q5_1, "q5_1", 32, 24, false, false, false},
    {QS_TYPE_Q8_0, "q8_0", 32, 34, false, false, false},
    {QS_TYPE_IQ4_NL, "iq4_nl", 32, 18, false, true, false},
};

const TypeInfo* find_type(int id) {
    for (const auto& t : kTypes)
        if (t.id == id) return &t;
    return nullptr;
}

bool has_kernel(int id) { return find_type(id) != nullptr; }

}  // namespace

bool qs_host::quantizer_requires_imatrix(int ggml_type) {
    const TypeInfo* t = find_type(ggml_type);
    return t && t->fn_requires_imatrix;
}

namespace {

// ---- IQ grid tables: built once per process, uploaded once per device ----

using namespace qs_launch;      // IqTabId, launch_src

struct HostTab {
    std::vector<uint16_t> grid, nbr;
    std::vector<uint32_t> cinfo;       // IQ2 layout described at qs::IqTabDev
    std::vector<uint32_t> cinfo_red;   // the same for the reduced lists (qs::IqTabDev)
    std::vector<uint32_t> cinfo_red2;  // and for the lists reduced for a clamped level (qs::IqTabDev)
    int code0 = 0;
    bool ok = true;
};

// kmap plus, for every off-grid code the level projection can produce (IQ2:
// levels 0..2, IQ3: 0..7), the grid points within its nwant smallest distinct
// squared distances in (distance, index) order -- the neighbour tables of
// iq2.py:31-74, iq2xs_common.py:41-95, iq3_common.py:29-68. The codes are
// split over host threads in contiguous ranges; each range's lists are
// appended in code order and the ranges joined in order, so the tables are
// the sequential build's byte for byte.
//
// With reduce >= 1, every list also gets a reduced copy (cinfo_red, stored after
// all full lists): an entry is left out when an earlier entry of the list
// changes a proper subset of the values it changes (against the code's
// levels) and agrees with it on those. When the code's level is the best
// level of every value for the search's distance terms, the left-out entry
// has every term >= the earlier entry's, so it can never be the list's first
// minimum (qs::iq_codes decides which list a search reads). With reduce 2, a
// second reduced copy (cinfo_red2, after the first) leaves an entry out only
// when that earlier entry also makes every raise from the code's clamped top
// level (IQ2: level 2) to the grid's level 3 that it makes: it stays valid
// where such a value's level-3 term is below its level-2 term.
HostTab build_host_tab(const uint16_t* grid, int gs, int bits, int nwant, int ch, int maxch, int reduce) {
    const int nsub = bits == 2 ? 8 : 4, lmask = (1 << bits) - 1, lmax = bits == 2 ? 2 : 7;
    const int ksize = bits == 2 ? 43692 : 4096;
    HostTab t;
    t.grid.assign(grid, grid + gs);
    t.cinfo.assign(ksize, 0);
    std::vector<int> kmap(ksize, -1);
    for (int i = 0; i < gs; i++) {
        kmap[grid[i]] = i;
        t.cinfo[grid[i]] = qs::CI_ON_GRID | (uint32_t)i;
    }
    t.code0 = kmap[0] >= 0 ? kmap[0] : 0;
    std::vector<int> gl(gs * nsub);
    for (int i = 0; i < gs; i++)
        for (int j = 0; j < nsub; j++) gl[i * nsub + j] = 2 * ((grid[i] >> (bits * j)) & lmask) + 1;
    // lists of codes [c0, c1): cinfo entries with starts relative to the range
    struct Part {
        std::vector<uint16_t> nbr, red, red2;
        bool ok = true;
    };
    t.cinfo_red.assign(ksize, 0);
    t.cinfo_red2.assign(ksize, 0);
    const int vclamp = 2 * lmax + 1, vtop = 2 * lmask + 1;     // values of the code's and the grid's top levels
    auto build_range = [&](int c0, int c1, Part& part) {
        std::vector<int> d2(gs);
        for (int c = c0; c < c1; c++) {
            if (kmap[c] >= 0) continue;
            int p[8];
            bool ok = true;
            for (int j = 0; j < nsub; j++) {
                const int l = (c >> (bits * j)) & lmask;
                ok = ok && l <= lmax;
                p[j] = 2 * l + 1;
            }
            if (!ok) continue;
            // the nwant smallest distinct distances (ascending), then every grid
            // point within the largest of them, in (distance, index) order
            int small[4];
            int nd = 0;
            for (int i = 0; i < gs; i++) {
                int v = 0;
                for (int j = 0; j < nsub; j++) v += (p[j] - gl[i * nsub + j]) * (p[j] - gl[i * nsub + j]);
                d2[i] = v;
                int pos = 0;
                while (pos < nd && small[pos] < v) pos++;
                if ((pos < nd && small[pos] == v) || pos >= nwant) continue;
                for (int q = std::min(nd, nwant - 1); q > pos; q--) small[q] = small[q - 1];
                small[pos] = v;
                nd = std::min(nd + 1, nwant);
            }
            const size_t start = part.nbr.size();     // a multiple of ch: one aligned vector per chunk
            for (int r = 0; r < nd; r++)
                for (int i = 0; i < gs; i++)
                    if (d2[i] == small[r]) part.nbr.push_back((uint16_t)i);
            const size_t len = part.nbr.size() - start;
            if (reduce > 0) {
                // changed values of each entry (bit j: its level differs from the code's)
                std::vector<uint32_t> chg(len);
                for (size_t k = 0; k < len; k++) {
                    const int gi = part.nbr[start + k];
                    uint32_t m = 0;
                    for (int j = 0; j < nsub; j++)
                        if (gl[gi * nsub + j] != p[j]) m |= 1u << j;
                    chg[k] = m;
                }
                // values where an entry raises the code's clamped top level to the grid's top
                std::vector<uint32_t> up(len);
                for (size_t k = 0; k < len && reduce == 2; k++) {
                    const int gi = part.nbr[start + k];
                    uint32_t m = 0;
                    for (int j = 0; j < nsub; j++)
                        if (vclamp != vtop && p[j] == vclamp && gl[gi * nsub + j] == vtop) m |= 1u << j;
                    up[k] = m;
                }
                const size_t rstart = part.red.size(), rstart2 = part.red2.size();
                for (size_t jj = 0; jj < len; jj++) {
                    const int gj = part.nbr[start + jj];
                    bool drop = false, drop2 = false;
                    for (size_t ii = 0; ii < jj && !(reduce == 2 ? drop2 : drop); ii++) {
                        if ((chg[ii] & ~chg[jj]) || chg[ii] == chg[jj]) continue;   // not a proper subset
                        const int gi = part.nbr[start + ii];
                        bool agree = true;
                        for (int j = 0; j < nsub; j++)
                            if ((chg[ii] >> j) & 1u) agree = agree && gl[gi * nsub + j] == gl[gj * nsub + j];
                        if (!agree) continue;
                        drop = true;
                        drop2 = !(up[jj] & ~chg[ii]);
                    }
                    if (!drop) part.red.push_back((uint16_t)gj);
                    if (!drop2 && reduce == 2) part.red2.push_back((uint16_t)gj);
                }
                const size_t rlen = part.red.size() - rstart, rlen2 = part.red2.size() - rstart2;
                part.red.resize((part.red.size() + ch - 1) / ch * ch, 0);
                part.red2.resize((part.red2.size() + ch - 1) / ch * ch, 0);
                t.cinfo_red[c] = (uint32_t)((rstart / ch) << 12) | (uint32_t)rlen;
                t.cinfo_red2[c] = (uint32_t)((rstart2 / ch) << 12) | (uint32_t)rlen2;
            }
            part.nbr.resize((part.nbr.size() + ch - 1) / ch * ch, 0);
            t.cinfo[c] = (uint32_t)((start / ch) << 12) | (uint32_t)len;
            part.ok = part.ok && len < 4096 && len <= (size_t)ch * maxch;
        }
    };
    const int nthr = (int)std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    std::vector<Part> parts(nthr);
    std::vector<std::thread> threads;
    int started = 0;
    try {
        for (; started < nthr; started++)
            threads.emplace_back(build_range, (int)((int64_t)ksize * started / nthr),
                                 (int)((int64_t)ksize * (started + 1) / nthr), std::ref(parts[started]));
    } catch (const std::system_error&) {
        // no more threads (a process limit, a sandbox): this thread builds the
        // remaining ranges; the ranges and their join are the same either way
    }
    for (int k = started; k < nthr; k++)
        build_range((int)((int64_t)ksize * k / nthr), (int)((int64_t)ksize * (k + 1) / nthr), parts[k]);
    for (auto& th : threads) th.join();
    // join the ranges in code order, moving each range's starts by the lists
    // before it; the reduced lists follow all full lists
    size_t base = 0, total = 0, total_red = 0;
    for (int k = 0; k < nthr; k++) {
        total += parts[k].nbr.size();
        total_red += parts[k].red.size();
    }
    size_t rbase = total, rbase2 = total + total_red;
    for (int k = 0; k < nthr; k++) {
        const int c0 = (int)((int64_t)ksize * k / nthr), c1 = (int)((int64_t)ksize * (k + 1) / nthr);
        for (int c = c0; c < c1; c++) {
            if (kmap[c] >= 0 || !(t.cinfo[c] & 0xfffu)) continue;
            const size_t start = ((t.cinfo[c] >> 12) & 0x7ffffu) + base / ch;
            t.ok = t.ok && start < (1u << 19);
            t.cinfo[c] = (uint32_t)(start << 12) | (t.cinfo[c] & 0xfffu);
            if (reduce > 0) {
                const size_t rstart = ((t.cinfo_red[c] >> 12) & 0x7ffffu) + rbase / ch;
                t.ok = t.ok && rstart < (1u << 19) && (t.cinfo_red[c] & 0xfffu) > 0;
                t.cinfo_red[c] = (uint32_t)(rstart << 12) | (t.cinfo_red[c] & 0xfffu);
            }
            if (reduce == 2) {
                const size_t rstart2 = ((t.cinfo_red2[c] >> 12) & 0x7ffffu) + rbase2 / ch;
                t.ok = t.ok && rstart2 < (1u << 19) && (t.cinfo_red2[c] & 0xfffu) > 0;
                t.cinfo_red2[c] = (uint32_t)(rstart2 << 12) | (t.cinfo_red2[c] & 0xfffu);
            }
        }
        t.nbr.insert(t.nbr.end(), parts[k].nbr.begin(), parts[k].nbr.end());
        base += parts[k].nbr.size();
        rbase += parts[k].red.size();
        rbase2 += parts[k].red2.size();
        t.ok = t.ok && parts[k].ok;
    }
    for (int k = 0; k < nthr; k++) t.nbr.insert(t.nbr.end(), parts[k].red.begin(), parts[k].red.end());
    for (int k = 0; k < nthr; k++) t.nbr.insert(t.nbr.end(), parts[k].red2.begin(), parts[k].red2.end());
    // on-grid codes, codes without a list and tables without reduced lists
    // read the full entry; tables without the second reduced copy read the
    // first in its place
    for (int c = 0; c < ksize; c++) {
        if (reduce == 0 || kmap[c] >= 0 || !(t.cinfo[c] & 0xfffu)) t.cinfo_red[c] = t.cinfo[c];
        if (reduce < 2 || kmap[c] >= 0 || !(t.cinfo[c] & 0xfffu)) t.cinfo_red2[c] = t.cinfo_red[c];
    }
    return t;
}

// one grid's host tables, built on first use of that grid
const HostTab& host_tab(int id) {
    static std::array<std::once_flag, IQT_N> once;
    static std::array<HostTab, IQT_N> tabs;
    std::call_once(once[id], [id] {
        switch (id) {
        // IQ2_S's lists (one distance) have no entry whose changes contain
        // another's, so its grid keeps only the full lists; the second
        // reduced copy is read by the IQ2_XXS search only (qs::iq_codes
        // PRUNE 2: on IQ2_XS its bookkeeping cost more than it saved, and
        // the IQ3 grids' top level is the code's)
        case IQT_G2_256: tabs[id] = build_host_tab(QS_GRID2_256, 256, 2, 2, qs::IQ2_CH, qs::IQ2_256_MAXCH, 2); break;
        case IQT_G2_512: tabs[id] = build_host_tab(QS_GRID2_512, 512, 2, 2, qs::IQ2_CH, qs::IQ2_512_MAXCH, 1); break;
        case IQT_G2_1024: tabs[id] = build_host_tab(QS_GRID2_1024, 1024, 2, 1, qs::IQ2_CH, qs::IQ2_1024_MAXCH, 0); break;
        case IQT_G3_256: tabs[id] = build_host_tab(QS_GRID3_256, 256, 3, 2, qs::IQ3_CH, qs::IQ3_256_MAXCH, 1); break;
        default: tabs[id] = build_host_tab(QS_GRID3_512, 512, 3, 3, qs::IQ3_CH, qs::IQ3_512_MAXCH, 1); break;
        }
    });
    return tabs[id];
}

// grid table used by an IQ type (-1 for the other types)
int iq_table_of(int ggml_type) {
    switch (ggml_type) {
    case QS_TYPE_IQ2_XXS: return IQT_G2_256;
    case QS_TYPE_IQ2_XS: return IQT_G2_512;
    case QS_TYPE_IQ2_S: return IQT_G2_1024;
    case QS_TYPE_IQ3_XXS: return IQT_G3_256;
    case QS_TYPE_IQ3_S: return IQT_G3_512;
    default: return -1;
    }
}

std::mutex g_dev_mutex;

// Square-root maps (2^24 bits each, see qs::SqrtMap): the Intel-host set that
// torch.sqrt rounds one ulp down (qs_sqrt_table.h), and the AMD-host sets
// rounded one ulp down and one ulp up (qs_sqrt_amd.bin).
enum SqrtMapId { SQM_INTEL_DOWN, SQM_AMD_DOWN, SQM_AMD_UP, SQM_N };

// Per-device constant tables: the IQ grids and neighbour lists, and the
// square-root maps.
struct DevTables {
    std::array<qs::IqTabDev, IQT_N> iq{};
    std::array<const uint32_t*, SQM_N> sqrt{};
};

// one map's bits, expanded on the host once per process: the Intel set from
// its key gaps, the AMD pair from the embedded 2-bit map only when an AMD
// mode first runs (false if that map is corrupt)
bool sqrt_map_bits(int id, const std::vector<uint32_t>*& out) {
    static std::once_flag intel_once, amd_once;
    static std::array<std::vector<uint32_t>, SQM_N> bits;
    static bool amd_ok = false;
    out = &bits[id];
    if (id == SQM_INTEL_DOWN) {
        std::call_once(intel_once, [] {
            auto& b = bits[SQM_INTEL_DOWN];
            b.assign(1u << 19, 0u);
            uint32_t key = 0;
            for (int i = 0; i < QS_SQRT_DOWN_N; i++) {
                key += QS_SQRT_DOWN_GAPS[i];
                b[key >> 5] |= 1u << (key & 31u);
            }
        });
        return true;
    }
    std::call_once(amd_once, [] {
        bits[SQM_AMD_DOWN].assign(1u << 19, 0u);
        bits[SQM_AMD_UP].assign(1u << 19, 0u);
        std::vector<unsigned char> packed(1u << 22);
        uLongf len = (uLongf)packed.size();
        const uLong clen = (uLong)(qs_sqrt_amd_blob_end - qs_sqrt_amd_blob);
        if (uncompress(packed.data(), &len, qs_sqrt_amd_blob, clen) != Z_OK || len != packed.size())
            return;
        for (uint32_t k = 0; k < (1u << 24); k++) {
            const uint32_t code = (packed[k >> 2] >> (2 * (k & 3u))) & 3u;
            if (code == 3) return;
            if (code) bits[code == 1 ? SQM_AMD_DOWN : SQM_AMD_UP][k >> 5] |= 1u << (k & 31u);
        }
        amd_ok = true;
    });
    return amd_ok;
}

template <typename T>
const T* upload(const std::vector<T>& v) {
    void* p = nullptr;
    const size_t n = std::max<size_t>(1, v.size()) * sizeof(T);
    if (hipMalloc(&p, n) != hipSuccess) return nullptr;
    if (!v.empty() && hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(p);
        return nullptr;
    }
    return static_cast<const T*>(p);
}

// Tables of each device, uploaded on first use (an IQ grid's tables when a
// type using that grid first runs, or all of them by qs_init) and kept until
// the process ends.
std::map<int, DevTables> g_dev_state;

// square-root rounding of the weights (QS_SQRT_*), process-wide
std::atomic<int> g_sqrt_mode{QS_SQRT_TORCH_CPU};

// the maps a square-root mode reads
std::array<bool, SQM_N> maps_of(int mode) {
    return {mode == QS_SQRT_TORCH_CPU, mode == QS_SQRT_TORCH_CPU_AMD, mode == QS_SQRT_TORCH_CPU_AMD};
}

bool device_tables_locked(int dev, int iq_table, const std::array<bool, SQM_N>& maps, DevTables& out) {
    DevTables& d = g_dev_state[dev];
    for (int m = 0; m < SQM_N; m++) {
        if (!maps[m] || d.sqrt[m]) continue;
        const std::vector<uint32_t>* bits = nullptr;
        if (!sqrt_map_bits(m, bits)) return false;
        d.sqrt[m] = upload(*bits);
        if (!d.sqrt[m]) return false;
    }
    if (iq_table >= 0 && !d.iq[iq_table].grid) {
        const HostTab& h = host_tab(iq_table);
        qs::IqTabDev g{};
        g.grid = upload(h.grid);
        // the three code tables back to back (qs::IqTabDev::cinfo)
        std::vector<uint32_t> ci(h.cinfo);
        ci.insert(ci.end(), h.cinfo_red.begin(), h.cinfo_red.end());
        ci.insert(ci.end(), h.cinfo_red2.begin(), h.cinfo_red2.end());
        g.cinfo = upload(ci);
        g.ncodes = (int)h.cinfo.size();
        g.nbr = upload(h.nbr);
        g.code0 = h.code0;
        if (!h.ok || !g.grid || !g.cinfo || !g.nbr) {
            // nothing is kept from a failed upload; the next call tries again
            for (const void* q : {(const void*)g.grid, (const void*)g.cinfo, (const void*)g.nbr})
                if (q) (void)hipFree(const_cast<void*>(q));
            return false;
        }
        d.iq[iq_table] = g;
    }
    out = d;
    return true;
}

// tables of the current device (uploaded under the lock when missing)
bool device_tables(int iq_table, int sqrt_mode, DevTables& out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    std::lock_guard<std::mutex> lock(g_dev_mutex);
    return device_tables_locked(dev, iq_table, maps_of(sqrt_mode), out);
}

// the kernels' view of a square-root mode: the maps, and the template kind
qs::SqrtMap sqrt_map(int mode, const DevTables& t) {
    if (mode == QS_SQRT_TORCH_CPU) return {t.sqrt[SQM_INTEL_DOWN], nullptr};
    if (mode == QS_SQRT_TORCH_CPU_AMD) return {t.sqrt[SQM_AMD_DOWN], t.sqrt[SQM_AMD_UP]};
    return {nullptr, nullptr};      // QS_SQRT_IEEE
}

int sqrt_kind(int mode) {
    return mode == QS_SQRT_TORCH_CPU ? qs::SQ_INTEL : mode == QS_SQRT_TORCH_CPU_AMD ? qs::SQ_AMD : qs::SQ_IEEE;
}

}  // namespace

extern "C" {

int qs_abi_version(void) { return QS_ABI_VERSION; }

int qs_type_supported(int ggml_type) { return has_kernel(ggml_type) ? 1 : 0; }

int qs_type_needs_imatrix(int ggml_type) {
    const TypeInfo* t = find_type(ggml_type);
    if (!t) return fail(QS_ENOTSUP, "unknown ggml type %d", ggml_type);
    return t->needs_imatrix ? 1 : 0;
}

int qs_type_uses_imatrix(int ggml_type) {
    const TypeInfo* t = find_type(ggml_type);
    if (!t) return fail(QS_ENOTSUP, "unknown ggml type %d", ggml_type);
    return t->uses_imatrix ? 1 : 0;
}

int64_t qs_row_bytes(int ggml_type, int64_t k) {
    const TypeInfo* t = find_type(ggml_type);
    if (!t) return fail(QS_ENOTSUP, "unknown ggml type %d", ggml_type);
    if (k <= 0 || k % t->blk)
        return fail(QS_EINVAL, "%s: row length %lld is not a positive multiple of %d", t->name,
                    (long long)k, t->blk);
    return k / t->blk * t->bytes;
}

const char* qs_last_error(void) { return g_err.c_str(); }

int qs_quantize(int ggml_type, int src_type, const void* src, int64_t n_rows, int64_t k,
                int64_t src_row_stride_bytes, const float* imatrix, void* dst, int64_t dst_bytes,
                void* hip_stream) {
    g_err.clear();
    const TypeInfo* t = find_type(ggml_type);
    if (!t) return fail(QS_ENOTSUP, "unknown ggml type %d", ggml_type);
    if (!has_kernel(ggml_type)) return fail(QS_ENOTSUP, "%s: no HIP quantizer in this build", t->name);
    const int esz = src_type == QS_SRC_F32 ? 4 : (src_type == QS_SRC_F16 || src_type == QS_SRC_BF16) ? 2 : 0;
    if (!esz) return fail(QS_EINVAL, "unsupported source type %d (F32=0, F16=1, BF16=30)", src_type);
    if (n_rows < 0) return fail(QS_EINVAL, "n_rows %lld < 0", (long long)n_rows);
    if (k <= 0 || k % t->blk)
        return fail(QS_EINVAL, "%s: row length %lld is not a positive multiple of %d", t->name,
                    (long long)k, t->blk);
    // size limits, checked by division so no product below can wrap: at most
    // 2^34 values per call (64 GiB of f32; every launch's grid then stays
    // below 2^32 work-items) and a source span below 2^62 bytes
    constexpr int64_t kMaxValues = INT64_C(1) << 34, kMaxSpan = INT64_C(1) << 62;
    if (k > kMaxValues || n_rows > kMaxValues / k)
        return fail(QS_EINVAL, "%lld x %lld values exceed the 2^34 per call", (long long)n_rows,
                    (long long)k);
    const int64_t rb = k / t->blk * t->bytes;
    if (n_rows == 0) return 0;
    if (!src || !dst) return fail(QS_EINVAL, "null src or dst");
    if (src_row_stride_bytes < k * esz || src_row_stride_bytes % 16)
        return fail(QS_EINVAL, "row stride %lld must be >= %lld and a multiple of 16",
                    (long long)src_row_stride_bytes, (long long)(k * esz));
    if (n_rows > kMaxSpan / src_row_stride_bytes)
        return fail(QS_EINVAL, "%lld rows of stride %lld bytes exceed a 2^62-byte span",
                    (long long)n_rows, (long long)src_row_stride_bytes);
    if (reinterpret_cast<uintptr_t>(src) % 16) return fail(QS_EINVAL, "src must be 16-byte aligned");
    if (dst_bytes < n_rows * rb)
        return fail(QS_EINVAL, "dst holds %lld bytes, %lld needed", (long long)dst_bytes,
                    (long long)(n_rows * rb));
    if (t->fn_requires_imatrix && !imatrix) return fail(QS_EINVAL, "%s requires an imatrix", t->name);
    const bool imat = t->uses_imatrix && imatrix != nullptr;

    qs::KArgs a;
    a.src = src;
    a.units_per_row = k / t->blk;
    a.n_units = n_rows * a.units_per_row;
    a.stride = src_row_stride_bytes / esz;
    a.qw = imat ? imatrix : nullptr;
    a.dst = static_cast<uint8_t*>(dst);
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    DevTables tabs;
    const int mode = g_sqrt_mode.load(std::memory_order_relaxed);
    if (!device_tables(iq_table_of(ggml_type), mode, tabs))
        return fail(QS_EIO, "%s: cannot upload constant tables to the device", t->name);
    a.sqrt = sqrt_map(mode, tabs);
    hipError_t e;
    switch (src_type) {
    case QS_SRC_F32: e = launch_src<qs::SRC_F32>(sqrt_kind(mode), ggml_type, imat, a, st, tabs.iq); break;
    case QS_SRC_F16: e = launch_src<qs::SRC_F16>(sqrt_kind(mode), ggml_type, imat, a, st, tabs.iq); break;
    default: e = launch_src<qs::SRC_BF16>(sqrt_kind(mode), ggml_type, imat, a, st, tabs.iq); break;
    }
    if (e != hipSuccess) return fail(QS_EIO, "%s: launch failed: %s", t->name, hipGetErrorString(e));
    return 0;
}

int qs_init(int device) {
    g_err.clear();
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n)
        return fail(QS_EINVAL, "device %d not present (%d ROCm devices)", device, n);
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess) return fail(QS_EIO, "hipGetDevice failed");
    if (hipSetDevice(device) != hipSuccess) return fail(QS_EIO, "hipSetDevice(%d) failed", device);
    bool ok = true;
    {
        std::lock_guard<std::mutex> lock(g_dev_mutex);
        DevTables d;
        const std::array<bool, SQM_N> all{true, true, true};
        for (int id = 0; id < IQT_N && ok; id++) ok = device_tables_locked(device, id, all, d);
    }
    // the uploads are blocking copies: nothing of this library is pending on
    // the device when qs_init returns
    const bool restored = hipSetDevice(prev) == hipSuccess;
    if (!ok) return fail(QS_EIO, "cannot upload constant tables to device %d", device);
    if (!restored) return fail(QS_EIO, "hipSetDevice(%d) failed", prev);
    return 0;
}

int qs_set_sqrt_rounding(int mode) {
    if (mode != QS_SQRT_TORCH_CPU && mode != QS_SQRT_IEEE && mode != QS_SQRT_TORCH_CPU_AMD)
        return fail(QS_EINVAL, "square-root mode %d (torch CPU Intel = %d, IEEE = %d, torch CPU AMD = %d)",
                    mode, QS_SQRT_TORCH_CPU, QS_SQRT_IEEE, QS_SQRT_TORCH_CPU_AMD);
    g_sqrt_mode.store(mode, std::memory_order_relaxed);
    return 0;
}

int qs_get_sqrt_rounding(void) { return g_sqrt_mode.load(std::memory_order_relaxed); }

}  // extern "C"
