// Per-type launch geometry and template dispatch of the quantizer kernels.
// Built once per source element type (-DQS_LAUNCH_SRC=<qs::SRC_* value>), so
// the three instantiation sets compile in parallel.
#include <hip/hip_runtime.h>

#include <tuple>
#include <utility>

#include "quant_studio.h"
#include "qs_launch.h"

#ifndef QS_LAUNCH_SRC
#error "build with -DQS_LAUNCH_SRC=<source type id> (quant-studio_amd/build.py)"
#endif

namespace qs_launch {
namespace {

// Launch through hipLaunchKernel so its status comes back as the return
// value: the caller's pending hipGetLastError() state is neither read nor
// reset by this library.
template <typename... P, typename... A>
hipError_t launch(void (*kernel)(P...), dim3 grid, dim3 block, hipStream_t st, A&&... args) {
    static_assert(sizeof...(P) == sizeof...(A), "kernel argument count");
    std::tuple<P...> vals(std::forward<A>(args)...);
    void* argv[sizeof...(P)];
    std::apply([&](auto&... v) {
        int i = 0;
        ((argv[i++] = static_cast<void*>(&v)), ...);
    }, vals);
    return hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, argv, 0, st);
}

qs::IqSteps iq_steps(float base, float delta, int lo, int hi) {
    qs::IqSteps s{};
    s.n = 0;
    for (int i = lo; i <= hi; i++) {
        float t = (float)i * delta;
        s.v[s.n++] = base + t;
    }
    return s;
}

// candidate numerators, f32 chains as kq_common.py:21-30 and qx_common.py:20-23
qs::Steps qkx_steps(float rmin, float rdelta, int nstep, int nmax) {
    qs::Steps s{};
    for (int i = 0; i <= nstep; i++) {
        float t = rdelta * (float)i;
        t = rmin + t;
        s.v[i] = t + (float)nmax;
    }
    s.n = nstep + 1;
    return s;
}

qs::QpSteps qp_steps(int nmax) {
    qs::QpSteps s{};
    int n = 0;
    for (int i = -4; i <= 4; i++) {
        if (!i) continue;
        float t = 0.1f * (float)i;
        s.v[n++] = t + (float)nmax;
    }
    return s;
}

qs::Steps qx_steps(int nmax) {
    qs::Steps s{};
    int n = 0;
    for (int i = -9; i <= 9; i++) {
        if (!i) continue;
        float t = 0.1f * (float)i;
        s.v[n++] = (float)nmax + t;
    }
    s.n = n;
    return s;
}

template <int SRC, qs::B32 T>
hipError_t launch_b32(const qs::KArgs& a, hipStream_t st) {
    const unsigned g = (unsigned)((a.n_units + qs::Q40_BLOCKS_PER_WG - 1) / qs::Q40_BLOCKS_PER_WG);
    return launch(qs::k_b32<SRC, T>, dim3(g), dim3(256), st, a);
}

// SQ: the host whose square-root rounding the weights take (qs::SQ_*);
// kernels whose weights take no square root are instantiated once (SQ_IEEE).
template <int SRC, int SQ>
hipError_t launch_type(int type, bool imat, const qs::KArgs& a, hipStream_t st,
                       const IqTabs& tabs) {
    using namespace qs;
    const dim3 wave(64);
    const dim3 sb8((unsigned)((a.n_units + 7) / 8)), sb4((unsigned)((a.n_units + 3) / 4));
    switch (type) {
    case QS_TYPE_Q4_0: return launch_b32<SRC, B32::Q4_0>(a, st);
    case QS_TYPE_Q4_1: return launch_b32<SRC, B32::Q4_1>(a, st);
    case QS_TYPE_Q5_0: return launch_b32<SRC, B32::Q5_0>(a, st);
    case QS_TYPE_Q5_1: return launch_b32<SRC, B32::Q5_1>(a, st);
    case QS_TYPE_Q8_0: return launch_b32<SRC, B32::Q8_0>(a, st);
    case QS_TYPE_IQ4_NL: {
        const dim3 g((unsigned)((a.n_units + 63) / 64));
        return imat ? launch(k_iq4_nl<SRC, true, SQ>, g, wave, st, a)
                    : launch(k_iq4_nl<SRC, false, SQ_IEEE>, g, wave, st, a);
    }
    case QS_TYPE_Q4_K:
        return imat ? launch(k_q45_k<SRC, true, 15, SQ>, sb8, wave, st, a, qkx_steps(-0.9f, 0.05f, 36, 15),
                             qp_steps(63))
                    : launch(k_q45_k<SRC, false, 15, SQ>, sb8, wave, st, a, qkx_steps(-1.0f, 0.1f, 20, 15),
                             qp_steps(63));
    case QS_TYPE_Q5_K:
        return imat ? launch(k_q45_k<SRC, true, 31, SQ>, sb8, wave, st, a, qkx_steps(-0.9f, 0.05f, 36, 31),
                             qp_steps(63))
                    : launch(k_q45_k<SRC, false, 31, SQ>, sb8, wave, st, a, qkx_steps(-0.5f, 0.1f, 15, 31),
                             qp_steps(63));
    case QS_TYPE_Q6_K:
        return imat ? launch(k_q6_k<SRC, true>, sb4, wave, st, a, qx_steps(32))
                    : launch(k_q6_k<SRC, false>, sb4, wave, st, a, qx_steps(32));
    case QS_TYPE_Q3_K:
        return imat ? launch(k_q3_k<SRC, true, SQ>, sb4, wave, st, a, qx_steps(4), qx_steps(32))
                    : launch(k_q3_k<SRC, false, SQ_IEEE>, sb4, wave, st, a, qx_steps(4), qx_steps(32));
    case QS_TYPE_Q2_K:
        return imat ? launch(k_q2_k<SRC, true, SQ>, sb4, wave, st, a, qkx_steps(-0.9f, 0.05f, 36, 3),
                             qp_steps(15))
                    : launch(k_q2_k<SRC, false, SQ_IEEE>, sb4, wave, st, a, qkx_steps(-0.5f, 0.1f, 15, 3),
                             qp_steps(15));
    case QS_TYPE_IQ4_XS:
        return imat ? launch(k_iq4_xs<SRC, true, SQ>, sb8, wave, st, a)
                    : launch(k_iq4_xs<SRC, false, SQ_IEEE>, sb8, wave, st, a);
    case QS_TYPE_IQ2_XXS: {
        // candidate numerators computed in f64 and rounded once (iq2.py:387, :470)
        QpSteps qp4{};
        IqSteps sweep{};
        int n = 0;
        for (int i = -4; i <= 4; i++)
            if (i) qp4.v[n++] = (float)(0.1 * i + 4.0);
        for (int i = -6; i <= 6; i++) sweep.v[sweep.n++] = (float)(5.0 + 0.1 * i);
        return launch(k_iq2_xxs<SRC, SQ>, sb8, wave, st, a, tabs[IQT_G2_256], qp4, sweep);
    }
    case QS_TYPE_IQ2_XS:      // SWEEP_CS iq2xs_common.py:21
        return launch(k_iq2_xs_s<SRC, false, SQ, 1>, sb4, wave, st, a, tabs[IQT_G2_512],
                      iq_steps(5.0f, 0.1f, -9, 9));
    case QS_TYPE_IQ2_S: {     // four waves per workgroup share the 1024-entry grid
        constexpr int WPG = 4;
        const dim3 g((unsigned)((a.n_units + 4 * WPG - 1) / (4 * WPG)));
        return launch(k_iq2_xs_s<SRC, true, SQ, WPG>, g, dim3(64 * WPG), st, a, tabs[IQT_G2_1024],
                      iq_steps(5.0f, 0.1f, -9, 9));
    }
    case QS_TYPE_IQ3_XXS: {    // _STEPS iq3_xxs.py:22
        const dim3 sb2((unsigned)((a.n_units + 1) / 2));
        return imat ? launch(k_iq3<SRC, false, true, SQ, 4>, sb2, wave, st, a, tabs[IQT_G3_256],
                             iq_steps(15.0f, 0.2f, -15, 15))
                    : launch(k_iq3<SRC, false, false, SQ, 4>, sb2, wave, st, a, tabs[IQT_G3_256],
                             iq_steps(15.0f, 0.2f, -15, 15));
    }
    case QS_TYPE_IQ3_S: {      // _STEPS iq3_s.py:22
        const dim3 sb2((unsigned)((a.n_units + 1) / 2));
        return imat ? launch(k_iq3<SRC, true, true, SQ, 4>, sb2, wave, st, a, tabs[IQT_G3_512],
                             iq_steps(15.0f, 0.2f, -9, 9))
                    : launch(k_iq3<SRC, true, false, SQ, 4>, sb2, wave, st, a, tabs[IQT_G3_512],
                             iq_steps(15.0f, 0.2f, -9, 9));
    }
    default:
        return hipErrorInvalidValue;
    }
}

}  // namespace

template <int SRC>
hipError_t launch_src(int sq, int type, bool imat, const qs::KArgs& a, hipStream_t st, const IqTabs& tabs) {
    switch (sq) {
    case qs::SQ_INTEL: return launch_type<SRC, qs::SQ_INTEL>(type, imat, a, st, tabs);
    case qs::SQ_AMD: return launch_type<SRC, qs::SQ_AMD>(type, imat, a, st, tabs);
    default: return launch_type<SRC, qs::SQ_IEEE>(type, imat, a, st, tabs);
    }
}


template hipError_t launch_src<QS_LAUNCH_SRC>(int, int, bool, const qs::KArgs&, hipStream_t, const IqTabs&);

}  // namespace qs_launch
