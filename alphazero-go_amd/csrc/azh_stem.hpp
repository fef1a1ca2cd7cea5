// The stem convolution's last chunk of input planes (device code shared by
// the per-layer stem kernel, azh_conv.hpp, and the one-launch small-board
// pass, azh_small_tower.hip, so both sum in one order).
#pragma once
#include <hip/hip_runtime.h>

namespace azh {

namespace stem_detail {
typedef float f4 __attribute__((ext_vector_type(4)));
}

// The stem's last chunk of input planes, when cin is not a multiple of 16.
// The stem's other chunks run as every convolution's (lane group k supplies
// channel quad k, the four MFMAs of a tap take the quad's elements in turn:
// 36 MFMAs per chunk of 16 channels). The last one holds only
// rem = cin - 16 (nq - 1) planes (2 of the 18), so its 9 rem (channel, tap)
// pairs are packed four to an MFMA instead: step s takes pair 4 s + k from
// lane group k, pair i being channel i % rem at tap i / rem of the chunk.
// That is ceil(9 rem / 4) MFMAs (5 for 18 planes, where the quad order
// spends 36 on a chunk that is 7/8 zeros). The pairs of the last step past
// 9 rem read channel 15's tap 0: a zero weight on a zero plane (channel 15
// is past cin, and the staging writes a chunk's planes past cin as zeros).
// Every tiling and the one-launch small-board pass sum in this order. The
// fragments need no other packing: the weight of output channel i, input
// channel c of the chunk, tap t is element c % 4 of lane i + 16 (c / 4)'s
// fragment of tap t.
//
// rem = 2 (the network's 2H + 2 planes when H is a multiple of 8: 18 at
// H = 8) runs as straight-line code (a lane's pairs are channel k % 2 at
// taps 2 s + k / 2, its operand offsets one select between two constants
// per step), with its five weights per block fetched apart (fetch), so a
// caller can fetch them early; any other rem runs a step at a time
// (multiply alone).
//
// wl: the chunk's fragment floats of block cb0 with the lane's row added
// (n16 floats of 4: block c at c * blockStride floats, tap t at t * 256,
// lane group g at g * 64); acc: the lane's COW x PPW accumulators; bq: the
// chunk's staged quads as floats (quad g at g * GC cells); cell[j] - bias:
// the lane's top-left tap cell of column group j (a caller's read positions
// may carry a per-lane offset, bias). Global or LDS fragments alike (wl may
// point into LDS).
template <int COW, int GC, int H>
struct StemTail {
    static constexpr int tapOff(int t) { return (t / 3) * H + (t % 3); }
    // A pad pair's offsets: channel 15 (quad 3, element 3) at tap 0.
    static constexpr int kPadW = (16 * 3) * 4 + 3, kPadB = (3 * GC) * 4 + 3;

    float a[COW][5];
    int bofs[5];

    __device__ __forceinline__ void fetch(const float* wl, size_t blockStride, int k, int rem) {
        if (rem != 2) return;
        const int c = k & 1;
        const bool odd = (k >> 1) != 0;
#pragma unroll
        for (int s = 0; s < 5; ++s) {
            const bool pad = s == 4 && odd;
            const int t0 = 2 * s, t1 = 2 * s + 1 < 9 ? 2 * s + 1 : 0;
            const int wofs = pad ? kPadW : (odd ? t1 * 256 : t0 * 256) + c;
            bofs[s] = pad ? kPadB : (odd ? tapOff(t1) * 4 : tapOff(t0) * 4) + c;
#pragma unroll
            for (int cc = 0; cc < COW; ++cc) a[cc][s] = wl[cc * blockStride + wofs];
        }
    }

    template <int PPW>
    __device__ __forceinline__ void multiply(stem_detail::f4 (&acc)[COW][PPW], const float* wl, size_t blockStride,
                                             const float* bq, const int (&cell)[PPW], int bias, int k,
                                             int rem) const {
        if (rem == 2) {
#pragma unroll
            for (int s = 0; s < 5; ++s)
#pragma unroll
                for (int j = 0; j < PPW; ++j) {
                    const float bv = bq[(cell[j] - bias) * 4 + bofs[s]];
#pragma unroll
                    for (int cc = 0; cc < COW; ++cc)
                        acc[cc][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[cc][s], bv, acc[cc][j], 0, 0, 0);
                }
            return;
        }
        const int pairs = 9 * rem, steps = (pairs + 3) / 4;
        for (int s = 0; s < steps; ++s) {
            const int pi = 4 * s + k;
            const bool live = pi < pairs;
            const int c = pi % rem, t = pi / rem;
            const int wofs = live ? (t * 64 + 16 * (c >> 2)) * 4 + (c & 3) : kPadW;
            const int bofs1 = live ? ((c >> 2) * GC + tapOff(t)) * 4 + (c & 3) : kPadB;
            float a1[COW];
#pragma unroll
            for (int cc = 0; cc < COW; ++cc) a1[cc] = wl[cc * blockStride + wofs];
#pragma unroll
            for (int j = 0; j < PPW; ++j) {
                const float bv = bq[(cell[j] - bias) * 4 + bofs1];
#pragma unroll
                for (int cc = 0; cc < COW; ++cc)
                    acc[cc][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[cc], bv, acc[cc][j], 0, 0, 0);
            }
        }
    }
};

// Fetch and multiply in one call.
template <int COW, int PPW, int GC, int H>
__device__ __forceinline__ void stemTail(stem_detail::f4 (&acc)[COW][PPW], const float* wl, size_t blockStride,
                                         const float* bq, const int (&cell)[PPW], int bias, int k, int rem) {
    StemTail<COW, GC, H> st;
    st.fetch(wl, blockStride, k, rem);
    st.multiply(acc, wl, blockStride, bq, cell, bias, k, rem);
}

} // namespace azh
