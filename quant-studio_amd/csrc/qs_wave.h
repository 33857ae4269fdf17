// Wave-level plumbing shared by the superblock kernels: one 64-lane workgroup
// quantizes SB_PER_WAVE superblocks, LPS lanes per superblock. Cross-lane
// reductions of a superblock go through LDS in the exact order the reference's
// sums use; the packed output is staged in LDS and written with coalesced
// dword stores.
#pragma once

#include "qs_device.h"

namespace qs {

// Orders LDS traffic between the lanes of one wave. One-wave workgroups use
// the workgroup barrier (WL = false: measured 1-10% faster for them than the
// fence below). Kernels whose workgroup holds several waves that do not wait
// for each other pass WL = true: the wave's LDS instructions execute in
// order, so a fence at wavefront scope is enough; they sync the whole
// workgroup with __syncthreads() only where its waves share data.
template <bool WL = false>
QS_DEV void wave_sync() {
    if constexpr (WL) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    } else {
        __syncthreads();
    }
}

// lane within the wave, and the wave's index over the whole grid for
// workgroups of WPG waves
QS_DEV int lane_id() { return (int)(threadIdx.x & 63u); }
template <int WPG = 1>
QS_DEV int64_t grid_wave() {
    if constexpr (WPG == 1) return (int64_t)blockIdx.x;
    return (int64_t)blockIdx.x * WPG + (threadIdx.x >> 6);
}

// Inclusive prefix sum of x over the wave's 64 lanes, in VALU only: DPP row
// shifts 1, 2, 4, 8 scan each row of 16 lanes, then row broadcasts carry lane
// 15's and lane 31's totals into the rows above (no LDS round trips).
QS_DEV int wave_incl_scan(int x) {
    int v = x;
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);   // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);   // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);   // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);   // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);   // row_bcast:15 -> rows 1, 3
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);   // row_bcast:31 -> rows 2, 3
    return v;
}

// Superblock position of this lane.
struct SbPos {
    int64_t sb;      // global superblock index (clamped copy used for loads)
    bool valid;      // sb < n_sb
    int slot;        // superblock slot within the wave
    int g;           // group index within the superblock (lane's group)
    int64_t elem;    // element offset of the lane's group in the source
    int64_t col;     // column of the lane's group start within its row
};

template <int LPS, int GROUP, int WPG = 1>
QS_DEV SbPos sb_pos(int64_t n_sb, int64_t sb_per_row, int64_t stride) {
    constexpr int SPW = 64 / LPS;
    SbPos p;
    const int lane = WPG > 1 ? lane_id() : (int)threadIdx.x;
    p.slot = lane / LPS;
    p.g = lane % LPS;
    const int64_t sb = grid_wave<WPG>() * SPW + p.slot;
    p.valid = sb < n_sb;
    p.sb = p.valid ? sb : n_sb - 1;
    const int64_t row = p.sb / sb_per_row;
    p.col = (p.sb % sb_per_row) * QK_K + (int64_t)p.g * GROUP;
    p.elem = row * stride + p.col;
    return p;
}

// torch CPU `.sum(-1)` over one superblock's 256 values (8-lane cascade):
// acc[a][l] = sum over i=0..7 (in order) of v[32i + 8a + l], p[l] =
// ((acc0+acc1)+acc2)+acc3, result = +0 + p[0] + ... + p[7].
// `v` is the superblock's 256 values in LDS; `tmp` holds 40 floats.
template <int LPS, bool WL = false>
QS_DEV float sb_cascade8_256(const float* v, float* tmp, int g) {
    constexpr int PER = 32 / LPS;
#pragma unroll
    for (int t = 0; t < PER; t++) {
        const int j = g * PER + t;             // j = 8a + l
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) acc = acc + v[32 * i + j];
        tmp[j] = acc;
    }
    wave_sync<WL>();
    if (g < 8) {
        float p = tmp[g] + tmp[8 + g];
        p = p + tmp[16 + g];
        p = p + tmp[24 + g];
        tmp[32 + g] = p;
    }
    wave_sync<WL>();
    float fin = 0.0f;
#pragma unroll
    for (int l = 0; l < 8; l++) fin = fin + tmp[32 + l];
    return fin;
}

// strict left-to-right sum of a superblock's 256 values held in LDS
QS_DEV float sb_seq_256(const float* v) {
    const float4* v4 = reinterpret_cast<const float4*>(v);
    float s = v[0];
    float4 q = v4[0];
    s = s + q.y;
    s = s + q.z;
    s = s + q.w;
#pragma unroll 8
    for (int j = 1; j < 64; j++) {
        q = v4[j];
        s = s + q.x;
        s = s + q.y;
        s = s + q.z;
        s = s + q.w;
    }
    return s;
}

// Copy the wave's staged output (nbytes at `stage`) to dst + off with
// coalesced dword stores when the destination is 4-byte aligned.
template <bool WL = false>
QS_DEV void store_staged(const uint8_t* stage, uint8_t* dst, int64_t off, int nbytes) {
    const int lane = WL ? lane_id() : (int)threadIdx.x;
    uint8_t* d = dst + off;
    if ((reinterpret_cast<uintptr_t>(d) & 3) == 0) {
        const int nw = nbytes >> 2;
        const uint32_t* s4 = reinterpret_cast<const uint32_t*>(stage);
        uint32_t* d4 = reinterpret_cast<uint32_t*>(d);
        for (int t = lane; t < nw; t += 64) d4[t] = s4[t];
        for (int t = (nw << 2) + lane; t < nbytes; t += 64) d[t] = stage[t];
    } else {
        for (int t = lane; t < nbytes; t += 64) d[t] = stage[t];
    }
}

}  // namespace qs
