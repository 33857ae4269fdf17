// Kernel dispatch of the quantizer library, shared by the C ABI (qs_api.hip)
// and the launch translation units (qs_launch.hip, built once per source
// element type so the three compile in parallel).
#pragma once

#include <hip/hip_runtime.h>

#include <array>

#include "qs_iq.h"
#include "qs_kernels.h"

namespace qs_launch {

// the IQ grids whose tables live on each device
enum IqTabId { IQT_G2_256, IQT_G2_512, IQT_G2_1024, IQT_G3_256, IQT_G3_512, IQT_N };

using IqTabs = std::array<qs::IqTabDev, IQT_N>;

// Launch the kernel of ggml type `type` over `a` on stream `st`: SRC is the
// source element type (qs::SRC_*), sq the host whose square-root rounding the
// weights take (qs::SQ_*). Returns the launch status.
template <int SRC>
hipError_t launch_src(int sq, int type, bool imat, const qs::KArgs& a, hipStream_t st, const IqTabs& tabs);

extern template hipError_t launch_src<qs::SRC_F32>(int, int, bool, const qs::KArgs&, hipStream_t, const IqTabs&);
extern template hipError_t launch_src<qs::SRC_F16>(int, int, bool, const qs::KArgs&, hipStream_t, const IqTabs&);
extern template hipError_t launch_src<qs::SRC_BF16>(int, int, bool, const qs::KArgs&, hipStream_t, const IqTabs&);

}  // namespace qs_launch
