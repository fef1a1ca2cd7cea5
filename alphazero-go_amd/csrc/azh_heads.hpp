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
// and four MFMAs, in K order. Steps go in groups of eight: the group's 32
// weight loads are issued before its first MFMA, so a group waits for one
// load round trip instead of eight (one step is far shorter than a load's
// round trip).
template <int KPAD, int RS>
__device__ __forceinline__ HeadVec4 fcBlock(const HeadVec4* xs4, int m, int kk, int n0, int ld, const float* wt) {
    constexpr int kGroup = 8;
    HeadVec4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
    for (int g0 = 0; g0 < KPAD; g0 += 16 * kGroup) {
        float bv[kGroup][4];
#pragma unroll
        for (int u = 0; u < kGroup; ++u) {
            const int k0 = g0 + 16 * u;
            if (k0 < KPAD) {
                const float* wr = wt + (size_t)(k0 + 4 * kk) * ld + n0 + m;
#pragma unroll
                for (int j = 0; j < 4; ++j) bv[u][j] = wr[(size_t)j * ld];
            }
        }
#pragma unroll
        for (int u = 0; u < kGroup; ++u) {
            const int k0 = g0 + 16 * u;
            if (k0 < KPAD) {
                const HeadVec4 av = xs4[(m * RS + k0) / 4 + kk];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j], bv[u][j], acc, 0, 0, 0);
            }
        }
    }
    return acc;
}

} // namespace azh
