// Device helpers of the heads' Linear layers, shared by the heads kernel
// (azh_kernels.hip) and the small-board pass (azh_small_tower.hip), so both
// compute every output with the same instructions in the same order.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>

namespace azh {

typedef float HeadVec4 __attribute__((ext_vector_type(4)));

__host__ __device__ constexpr int headPad16(int x) { return (x + 15) / 16 * 16; }

// One 16 x 16 block of a head Linear: positions 0..15 (LDS rows of stride
// RS) x columns n0..n0+15 of W^T [KPAD][ld]. Lane (m, kk) ends holding
// (position 4*kk + r, column n0 + m). A step is 16 K values: one LDS read
// and four MFMAs, in K order. Steps go in groups of eight whose 32 weight
// loads are issued a whole group ahead: group g + 1's loads are in flight
// while group g multiplies, so the block waits for one load round trip, not
// one per group (a group's MFMAs are far shorter than a round trip).
template <int KPAD, int RS>
__device__ __forceinline__ HeadVec4 fcBlock(const HeadVec4* xs4, int m, int kk, int n0, int ld, const float* wt) {
    constexpr int kGroup = 8;
    constexpr int kSteps = KPAD / 16;
    constexpr int kGroups = (kSteps + kGroup - 1) / kGroup;
    HeadVec4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    float bv[2][kGroup][4];
    // The scheduling groups pin that order (left free, the scheduler sinks
    // each weight load next to its MFMA and hoists the LDS reads).
    // A step's weights: W^T rows k0 + 4*kk + j, column n0 + m; the row base
    // wt + k0*ld is uniform, the lane's part one of four fixed offsets.
    int laneOff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) laneOff[j] = (4 * kk + j) * ld + n0 + m;
    auto loadGroup = [&](int g, float (&dst)[kGroup][4]) {
#pragma unroll
        for (int u = 0; u < kGroup; ++u) {
            const int k0 = (g * kGroup + u) * 16;
            if (k0 < KPAD) {   // KPAD is a multiple of 16
                const float* row = wt + (size_t)k0 * ld;
#pragma unroll
                for (int j = 0; j < 4; ++j) dst[u][j] = row[laneOff[j]];
                __builtin_amdgcn_sched_group_barrier(0x020, 4, 0);
            }
        }
    };
    // The positions' values of a step are read from LDS a step ahead.
    HeadVec4 av[2];
    av[0] = xs4[(m * RS) / 4 + kk];
    loadGroup(0, bv[0]);
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
        if (g + 1 < kGroups) loadGroup(g + 1, bv[(g + 1) & 1]);
#pragma unroll
        for (int u = 0; u < kGroup; ++u) {
            const int step = g * kGroup + u;
            if (step < kSteps) {
                if (step + 1 < kSteps) {
                    av[(step + 1) & 1] = xs4[(m * RS + (step + 1) * 16) / 4 + kk];
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[step & 1][j], bv[g & 1][u][j], acc, 0, 0, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
            }
        }
    }
    return acc;
}

} // namespace azh
