// The gfx950 3x3 convolution (template body; instantiated per board size
// and workgroup shape by azh_conv_inst.hip).
//
// conv3x3: the stem and residual-tower convolutions as an implicit GEMM on
// fp32 MFMA (v_mfma_f32_16x16x4_f32), no im2col buffer. A workgroup owns one
// position (board) and a tile of output channels. For each chunk of 16
// input channels it stages the board's planes in LDS with a one-point zero
// halo ((n+2) x (n+2) per channel, four channels interleaved per point so a
// lane fetches four K values with one ds_read_b128, as the trunk's channel
// quads already hold them in global memory); the nine taps are then
// constant offsets into that tile, so the inner loop is LDS reads with
// immediate offsets and MFMAs, and the im2col matrix never exists. The
// chunks are double-buffered: the next chunk's global loads are in flight
// while the current one is multiplied. Weights come pre-packed in MFMA
// fragment order straight from global memory (one coalesced dwordx4 per lane
// per fragment quad; every workgroup reads the same 0.6 MB per layer, which
// stays in L2). BN (scale, shift), the residual add and ReLU are applied to
// the accumulators before the single store of each channel quad.
//
// MFMA operand layout (16x16x4 f32, wave64): A[i][k] comes from lane
// i + 16k, B[k][j] from lane j + 16k, and lane j + 16g holds D[4g + r][j] in
// accumulator element r.
#pragma once
#include "azh_conv_iface.hpp"

#include <hip/hip_runtime.h>

namespace azh {

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

template <int N>
struct Geo {
    static constexpr int A = N * N;            // points per plane
    static constexpr int H = N + 2;            // haloed row length
    static constexpr int HA = H * H;           // haloed plane (float4 units per group)
    static constexpr int NPG = (A + 15) / 16;  // 16-point MFMA column groups
    static constexpr int BUF = 4 * HA;         // float4 units of one LDS buffer (4 groups)
};

// The epilogue: y = relu?(scale * acc + shift (+ skip)), each operation
// rounded on its own, for a lane's COW x PPW accumulators (channels cb0..,
// column groups pg0..). A lane's four accumulators of a block are the four
// channels of one quad at one point, so each output (and each residual
// value) moves as one 16-byte access in the channel-quad layout; channels
// past cout in the last quad are written as zeros. The residual input may be
// the output buffer itself (the block's second convolution writes over its
// input), so the compiler cannot move a residual read above an earlier
// store: all of a lane's residual quads are read first, in one batch, then
// combined and stored.
template <int N, int COW, int PPW>
__device__ __forceinline__ void storeOutputs(const f4 (&acc)[COW][PPW], const float* __restrict__ scale,
                                             const float* __restrict__ shift, const float* skip, float* y, int b,
                                             int cout, int cb0, int pg0, int k, int n16, int relu) {
    using G = Geo<N>;
    const int quads = (cout + 3) / 4;
    const size_t board = (size_t)b * quads * G::A;   // in float4 units
    const f4* skipq = skip ? reinterpret_cast<const f4*>(skip) + board : nullptr;
    f4* yq = reinterpret_cast<f4*>(y) + board;
    float sc[COW][4], sh[COW][4];
#pragma unroll
    for (int c = 0; c < COW; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int co = min((cb0 + c) * 16 + 4 * k + r, cout - 1);
            sc[c][r] = scale[co];
            sh[c][r] = shift[co];
        }
    f4 res[COW][PPW];
    if (skipq) {
#pragma unroll
        for (int c = 0; c < COW; ++c)
#pragma unroll
            for (int j = 0; j < PPW; ++j) {
                // Lanes past the board or past cout read a valid quad; their
                // values are never stored.
                const int g = min((cb0 + c) * 4 + k, quads - 1);
                const int p = min((pg0 + j) * 16 + n16, G::A - 1);
                res[c][j] = skipq[(size_t)g * G::A + p];
            }
    }
#pragma unroll
    for (int c = 0; c < COW; ++c) {
        const int g = (cb0 + c) * 4 + k;
        if (g >= quads) continue;
#pragma unroll
        for (int j = 0; j < PPW; ++j) {
            const int p = (pg0 + j) * 16 + n16;
            f4 o;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                o[r] = 4 * g + r < cout ? epilogue(acc[c][j][r], sc[c][r], sh[c][r], skipq != nullptr, res[c][j][r],
                                                   relu != 0)
                                        : 0.0f;
            if (p < G::A) yq[(size_t)g * G::A + p] = o;
        }
    }
}

// A workgroup computes one board's output channels [co tile] at column
// groups [pixel tile]: WCO x WPG waves, wave (c, g) owning COW blocks of 16
// channels and PPW column groups (PPW = 0: all of them). PLANAR: x is the
// network's input planes [B][cin][A] (the stem), read a channel at a time;
// otherwise x is a trunk activation in channel quads, read a quad at a time.
// Either way input channels past cin are read as zeros.
template <int N, int COW, int WCO, int WPG, int PPW0, bool PLANAR>
__device__ __forceinline__ void conv3x3Body(const float* __restrict__ x, const f4* __restrict__ wp,
                                            const float* __restrict__ scale, const float* __restrict__ shift,
                                            const float* skip, float* y, int cin, int cout, int nq, int coTiles,
                                            int pixTiles, int relu) {
    using G = Geo<N>;
    constexpr int PPW = PPW0 == 0 ? G::NPG : PPW0;
    constexpr int WAVES = WCO * WPG;
    constexpr int THREADS = WAVES * 64;
    // A workgroup that covers part of the board (a pixel tile of SPAN
    // points) stages only the board rows its points and their 3x3
    // neighbourhoods touch: at most (SPAN - 1) / N + 2 rows plus a halo row
    // on each side.
    constexpr int SPAN = WPG * PPW * 16;
    constexpr int ROWS = PPW0 == 0 ? N : ((SPAN - 1) / N + 4 < N ? (SPAN - 1) / N + 4 : N);
    constexpr int ITEMS = 4 * ROWS * N;   // (channel group, point) pairs per chunk, at most
    constexpr int PER = (ITEMS + THREADS - 1) / THREADS;
    // Small pixel tiles on the larger boards (the small batches' shapes at
    // 13x13 and 19x19): a tap is only 4 x PPW MFMAs there, far shorter than
    // a global load's round trip, so the A fragments are fetched a whole
    // chunk ahead (the nine taps of chunk q+1 during chunk q) instead of one
    // tap ahead, and the board planes two chunks ahead instead of one.
    constexpr bool SMALL = PPW0 != 0 && PPW0 <= 2 && N >= 13;
    __shared__ f4 lds[2 * G::BUF];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Workgroups are dealt to the 8 XCDs round-robin; renumber so that the
    // co tiles of one board run on the same XCD and share its L2.
    const int total = gridDim.x;
    const int wg = blockIdx.x;
    const int logical = (total % 8 == 0) ? (wg % 8) * (total / 8) + wg / 8 : wg;
    const int tilesPerBoard = coTiles * pixTiles;
    const int b = logical / tilesPerBoard, tile = logical % tilesPerBoard;
    const int ct = tile / pixTiles, pt = tile % pixTiles;
    const int cb0 = (ct * WCO + wave / WPG) * COW;
    // This wave's first column group (a constant 0 when every wave covers the board).
    const int pg0 = PPW0 == 0 ? 0 : (pt * WPG + wave % WPG) * PPW;
    const int k = lane >> 4, n16 = lane & 15;

    for (int i = tid; i < 2 * G::BUF; i += THREADS) lds[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    // Each lane's LDS read position per column group (float4 units), taps
    // and buffers added as constants. Points past the board read a valid
    // cell; their outputs are never stored.
    int rofs[PPW];
#pragma unroll
    for (int j = 0; j < PPW; ++j) {
        int p = (pg0 + j) * 16 + n16;
        p = p < G::A ? p : G::A - 1;
        rofs[j] = k * G::HA + (p / N) * G::H + (p % N);
    }

    // The staged rows: all of them for a whole-board workgroup; for a pixel
    // tile, its points' rows and one more on each side (clamped to the
    // board; the halo rows stay zero). Rows outside are never read.
    int rowLo = 0, span = G::A;   // compile-time constants unless the tile is a part of the board
    if (PPW0 != 0 && SPAN < G::A) {
        const int p0 = pt * SPAN;
        const int p1 = min(G::A, p0 + SPAN);
        rowLo = max(0, p0 / N - 1);
        span = (min(N - 1, (p1 - 1) / N + 1) - rowLo + 1) * N;
    }
    const int items = 4 * span, first = rowLo * N;

    const float* xb = x + (size_t)b * cin * G::A;                                  // PLANAR
    const f4* xq = reinterpret_cast<const f4*>(x) + (size_t)b * ((cin + 3) / 4) * G::A;   // channel quads
    f4 stage[PER], stage2[SMALL ? PER : 1];
    auto load = [&](int q, f4* dst) {
#pragma unroll
        for (int r = 0; r < PER; ++r) {
            const int it = tid + r * THREADS;
            f4 v = {0.0f, 0.0f, 0.0f, 0.0f};
            if (it < items) {
                const int g = it / span, p = first + it - g * span;
                const int c0 = q * 16 + 4 * g;
                if (PLANAR) {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        if (c0 + c < cin) v[c] = xb[(size_t)(c0 + c) * G::A + p];
                } else if (c0 < cin) {
                    // A quad's channels past cin are stored zeros.
                    v = xq[(size_t)(c0 / 4) * G::A + p];
                }
            }
            dst[r] = v;
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int r = 0; r < PER; ++r) {
            const int it = tid + r * THREADS;
            if (it < items) {
                const int g = it / span, p = first + it - g * span;
                lds[buf * G::BUF + g * G::HA + (p / N + 1) * G::H + (p % N + 1)] = stage[r];
            }
        }
    };

    f4 acc[COW][PPW];
#pragma unroll
    for (int c = 0; c < COW; ++c)
#pragma unroll
        for (int j = 0; j < PPW; ++j) acc[c][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    load(0, stage);
    __syncthreads();   // the zero fill is complete before any interior store
    store(0);
    // Two chunks ahead: chunk 1 waits in `stage` while chunk 0 is multiplied
    // (with one chunk, chunk 0 again, never stored).
    if (SMALL) load(min(1, nq - 1), stage);
    __syncthreads();

    // The (tap, column group) steps of a chunk run as one unrolled stream:
    // the B operand of step i + kRing is read from LDS while step i's MFMAs
    // run, and each tap's A fragments are fetched from global memory one tap
    // ahead, so neither read's latency stalls the matrix pipe. The sched
    // group hints keep that interleave (a step's MFMAs, then the read kRing
    // steps ahead) and pin each A fetch to the start of the tap before the
    // one that uses it (left free, the scheduler sinks it next to its use
    // to save four registers, and every tap then waits a full round trip).
    constexpr int kRing = 4;
    constexpr int STEPS = 9 * PPW;
    auto tapOffset = [](int t) { return (t / 3) * G::H + (t % 3); };
    auto loadA = [&](int q, int t, f4 (&a)[COW]) {
#pragma unroll
        for (int c = 0; c < COW; ++c) a[c] = wp[((size_t)((cb0 + c) * nq + q) * 9 + t) * 64 + lane];
    };
    f4 aCur[COW], aNext[COW];
    f4 aChunk[SMALL ? 9 : 1][COW], aChunkNext[SMALL ? 9 : 1][COW];
    if (SMALL) {
#pragma unroll
        for (int t = 0; t < 9; ++t) loadA(0, t, aChunk[t]);
    } else {
        loadA(0, 0, aCur);
    }
    for (int q = 0; q < nq; ++q) {
        // The last chunks fetch the last one again in place of chunks that
        // do not exist (never stored), which keeps the step stream free of
        // branches.
        const int qn = q + 1 < nq ? q + 1 : q;
        const int q2 = q + 2 < nq ? q + 2 : nq - 1;
        const f4* buf = lds + (q & 1) * G::BUF;
        f4 ring[kRing];
#pragma unroll
        for (int i = 0; i < kRing && i < STEPS; ++i) ring[i] = buf[rofs[i % PPW] + tapOffset(i / PPW)];
        __builtin_amdgcn_sched_group_barrier(0x100, kRing, 0);   // the ring's first reads
#pragma unroll
        for (int i = 0; i < STEPS; ++i) {
            const int t = i / PPW, pg = i % PPW;
            if (pg == 0) {
                // The next tap's A fragments (tap 8: the next chunk's first;
                // SMALL: this tap's of the next chunk), and at tap 0 after
                // them the board planes of the next chunk (SMALL: the one
                // after it; the next waits in `stage`): the count of
                // outstanding loads drains in issue order, so a tap's wait
                // for its fragments does not wait for the planes.
                if (SMALL)
                    loadA(qn, t, aChunkNext[t]);
                else
                    loadA(t + 1 < 9 ? q : qn, (t + 1) % 9, aNext);
                __builtin_amdgcn_sched_group_barrier(0x020, COW, 0);   // issued here, a tap ahead
                if (t == 0) {
                    if (SMALL)
                        load(q2, stage2);
                    else
                        load(qn, stage);
                }
            }
            const f4 bv = ring[i % kRing];
            if (i + kRing < STEPS)
                ring[i % kRing] = buf[rofs[(i + kRing) % PPW] + tapOffset((i + kRing) / PPW)];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int c = 0; c < COW; ++c)
                    acc[c][pg] = __builtin_amdgcn_mfma_f32_16x16x4f32(SMALL ? aChunk[t][c][j] : aCur[c][j], bv[j],
                                                                      acc[c][pg], 0, 0, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 4 * COW, 0);                   // step i's MFMAs,
            if (i + kRing < STEPS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // then step i+kRing's read
            if (!SMALL && pg == PPW - 1) {
#pragma unroll
                for (int c = 0; c < COW; ++c) aCur[c] = aNext[c];
            }
        }
        if (SMALL) {
#pragma unroll
            for (int t = 0; t < 9; ++t)
#pragma unroll
                for (int c = 0; c < COW; ++c) aChunk[t][c] = aChunkNext[t][c];
        }
        if (q + 1 < nq) store((q + 1) & 1);
        if (SMALL) {
#pragma unroll
            for (int r = 0; r < PER; ++r) stage[r] = stage2[r];
        }
        __syncthreads();
    }

    storeOutputs<N, COW, PPW>(acc, scale, shift, skip, y, b, cout, cb0, pg0, k, n16, relu);
}

// The residual tower's convolutions (input in channel quads) and the
// stem's (input: the network's 2H+2 planes) are separate kernels, so
// profiles tell them apart. Two waves per SIMD are asked for where the whole
// workgroup shape allows it (one 16-channel block per wave).
#define AZH_CONV_KERNEL(NAME, PLANAR)                                                                      \
    template <int N, int COW, int WCO, int WPG, int PPW>                                                  \
    __global__ __launch_bounds__(WCO* WPG * 64)                                                          \
        __attribute__((amdgpu_waves_per_eu(COW == 1 && WCO * WPG >= 4 ? 2 : 1,                           \
                                           COW == 1 && WCO * WPG >= 4 ? 2 : 1))) void                    \
        NAME(const float* __restrict__ x, const f4* __restrict__ wp, const float* __restrict__ scale,      \
             const float* __restrict__ shift, const float* skip, float* y, int cin, int cout, int nq,      \
             int coTiles, int pixTiles, int relu) {                                                        \
        conv3x3Body<N, COW, WCO, WPG, PPW, PLANAR>(x, wp, scale, shift, skip, y, cin, cout, nq, coTiles,   \
                                                   pixTiles, relu);                                        \
    }
AZH_CONV_KERNEL(conv3x3Tower, false)
AZH_CONV_KERNEL(conv3x3Stem, true)
#undef AZH_CONV_KERNEL

} // namespace

template <int N, int COW, int WCO, int WPG, int PPW>
hipError_t launchConvT(const float* x, const float* wp, const float* scale, const float* shift, const float* skip,
                       float* y, int B, int cin, int cout, bool relu, bool planarInput, hipStream_t stream) {
    constexpr int NPG = Geo<N>::NPG;
    constexpr int pgPerWave = PPW == 0 ? NPG : PPW;
    const int coTiles = ceilDiv(cout, 16 * COW * WCO);
    const int pixTiles = ceilDiv(NPG, WPG * pgPerWave);
    const int nq = ceilDiv(cin, kChunk);
    const dim3 grid(B * coTiles * pixTiles), block(WCO * WPG * 64);
    if (!planarInput)
        hipLaunchKernelGGL((conv3x3Tower<N, COW, WCO, WPG, PPW>), grid, block, 0, stream, x,
                           reinterpret_cast<const f4*>(wp), scale, shift, skip, y, cin, cout, nq, coTiles, pixTiles,
                           relu ? 1 : 0);
    else
        hipLaunchKernelGGL((conv3x3Stem<N, COW, WCO, WPG, PPW>), grid, block, 0, stream, x,
                           reinterpret_cast<const f4*>(wp), scale, shift, skip, y, cin, cout, nq, coTiles, pixTiles,
                           relu ? 1 : 0);
    return hipGetLastError();
}

} // namespace azh
