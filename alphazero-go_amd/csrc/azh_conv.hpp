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
#include "azh_stem.hpp"

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
//
// What the epilogue reads besides the accumulators (a lane's BN factors and
// residual quads) does not depend on the convolution, so the small-tile
// body reads it before its first MFMA.
template <int COW, int PPW>
struct EpilogueInputs {
    float sc[COW][4], sh[COW][4];
    f4 res[COW][PPW];
};

template <int N, int COW, int PPW>
__device__ __forceinline__ void loadEpilogue(EpilogueInputs<COW, PPW>& e, const float* __restrict__ scale,
                                             const float* __restrict__ shift, const float* skip, int b, int cout,
                                             int cb0, int pg0, int k, int n16) {
    using G = Geo<N>;
    const int quads = (cout + 3) / 4;
    const f4* skipq = skip ? reinterpret_cast<const f4*>(skip) + (size_t)b * quads * G::A : nullptr;
#pragma unroll
    for (int c = 0; c < COW; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int co = min((cb0 + c) * 16 + 4 * k + r, cout - 1);
            e.sc[c][r] = scale[co];
            e.sh[c][r] = shift[co];
        }
    if (skipq) {
#pragma unroll
        for (int c = 0; c < COW; ++c)
#pragma unroll
            for (int j = 0; j < PPW; ++j) {
                // Lanes past the board or past cout read a valid quad; their
                // values are never stored.
                const int g = min((cb0 + c) * 4 + k, quads - 1);
                const int p = min((pg0 + j) * 16 + n16, G::A - 1);
                e.res[c][j] = skipq[(size_t)g * G::A + p];
            }
    }
    // Without a residual e.res stays unset: writeOutputs then adds nothing
    // and never uses it.
}

template <int N, int COW, int PPW>
__device__ __forceinline__ void writeOutputs(const f4 (&acc)[COW][PPW], const EpilogueInputs<COW, PPW>& e,
                                             bool addSkip, float* y, int b, int cout, int cb0, int pg0, int k,
                                             int n16, int relu) {
    using G = Geo<N>;
    const int quads = (cout + 3) / 4;
    f4* yq = reinterpret_cast<f4*>(y) + (size_t)b * quads * G::A;
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
                o[r] = 4 * g + r < cout ? epilogue(acc[c][j][r], e.sc[c][r], e.sh[c][r], addSkip, e.res[c][j][r],
                                                   relu != 0)
                                        : 0.0f;
            if (p < G::A) yq[(size_t)g * G::A + p] = o;
        }
    }
}

template <int N, int COW, int PPW>
__device__ __forceinline__ void storeOutputs(const f4 (&acc)[COW][PPW], const float* __restrict__ scale,
                                             const float* __restrict__ shift, const float* skip, float* y, int b,
                                             int cout, int cb0, int pg0, int k, int n16, int relu) {
    EpilogueInputs<COW, PPW> e;
    loadEpilogue<N, COW, PPW>(e, scale, shift, skip, b, cout, cb0, pg0, k, n16);
    writeOutputs<N, COW, PPW>(acc, e, skip != nullptr, y, b, cout, cb0, pg0, k, n16, relu);
}

// The small pixel tiles (the shapes of small batches): a workgroup of WPG
// waves owns one board, one block of 16 output channels and WPG x PPW of its
// 16-point column groups, PPW per wave. A tap there is only 4 x PPW MFMAs,
// far shorter than a global load's round trip, so:
//  - everything chunk q needs (its board planes, staged as the general body
//    stages them, and its nine taps' A fragments for the block of 16
//    channels, fetched once per workgroup instead of once per wave) is
//    loaded into registers during chunk q - 3 and stored into LDS during
//    chunk q - 1, whose barrier publishes it;
//  - the loads and stores are spread over the taps of the MFMA stream, one
//    item per tap, on addresses computed once (a chunk adds only a uniform
//    offset), so their few instructions issue between the MFMAs instead of
//    holding them up;
//  - the loads are unconditional (an item past the tile loads a valid
//    element and stores to a spare LDS cell; channels past cin are zeroed
//    at the store): loads under a branch would leave the compiler's count
//    of loads in flight unsure at the merge, and it would wait for all;
//  - the load registers alternate between two sets with the chunks (an
//    item's store reads its set just before the item's next load fills it),
//    and the chunk loop runs in pairs so that each set is fixed at compile
//    time: no register copy waits on a load in flight;
//  - the LDS tile holds only the board rows the workgroup's points touch,
//    with a zero row above and below (the whole haloed board on the wider
//    tiles);
//  - a tap's A fragment is read from LDS one tap ahead, the B operands in
//    the general body's ring;
//  - the epilogue's BN factors and, for a layer with a residual, its
//    residual quads are read before the first MFMA (they do not depend on
//    this convolution).
// The MFMA sequence per output (chunk, tap, channel in chunk) and every
// operand are the general body's, so the bits are too.
template <int N, int WPG, int PPW, bool PLANAR>
__device__ __forceinline__ void conv3x3SmallBody(const float* __restrict__ x, const f4* __restrict__ wp,
                                                 const float* __restrict__ scale, const float* __restrict__ shift,
                                                 const float* skip, float* y, int cin, int cout, int nq, int coTiles,
                                                 int pixTiles, int relu) {
    using G = Geo<N>;
    constexpr int THREADS = WPG * 64;
    constexpr int SPAN = WPG * PPW * 16;
    constexpr int ROWS = (SPAN - 1) / N + 4 < N ? (SPAN - 1) / N + 4 : N;   // staged rows, at most
    constexpr int GC = (ROWS + 2) * G::H;     // one channel group's tile: staged rows and two zero rows
    constexpr int CB = 4 * GC;                // one chunk's tile (float4 cells)
    constexpr int ITEMS = 4 * ROWS * N;       // (channel group, point) pairs per chunk, at most
    constexpr int PER = (ITEMS + THREADS - 1) / THREADS;
    constexpr int AITEMS = 9 * 64;            // one block's A fragments per chunk (float4 units)
    constexpr int APER = (AITEMS + THREADS - 1) / THREADS;
    constexpr int NI = PER + APER;            // a thread's items per chunk
    // Two chunk buffers of board planes and of A fragments, and a spare cell
    // each for stores of items past the tile.
    __shared__ f4 lds[2 * CB + 1];
    __shared__ f4 alds[2 * AITEMS + 1];
    constexpr int kSpare = 2 * CB, kSpareA = 2 * AITEMS;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Co tiles of one board on one XCD (as the general body numbers them).
    const int total = gridDim.x;
    const int wg = blockIdx.x;
    const int logical = (total % 8 == 0) ? (wg % 8) * (total / 8) + wg / 8 : wg;
    const int tilesPerBoard = coTiles * pixTiles;
    const int b = logical / tilesPerBoard, tile = logical % tilesPerBoard;
    const int cb0 = tile / pixTiles, pt = tile % pixTiles;
    const int pg0 = (pt * WPG + wave) * PPW;
    const int k = lane >> 4, n16 = lane & 15;

    for (int i = tid; i < 2 * CB; i += THREADS) lds[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    // The staged rows [rowLo, rowLo + span / N): the tile's points' rows and
    // one more on each side, clamped to the board. Tile row r - rowLo + 1
    // holds board row r; the rows above and below stay zero, and are read
    // only where they are off the board.
    int rowLo = 0, span = G::A;
    if (SPAN < G::A) {
        const int p0 = pt * SPAN;
        const int p1 = min(G::A, p0 + SPAN);
        rowLo = max(0, p0 / N - 1);
        span = (min(N - 1, (p1 - 1) / N + 1) - rowLo + 1) * N;
    }
    const int items = 4 * span, first = rowLo * N;
    int rofs[PPW];   // a lane's B read position per column group (float4 cells; taps added as constants)
#pragma unroll
    for (int j = 0; j < PPW; ++j) {
        int p = (pg0 + j) * 16 + n16;
        p = p < G::A ? p : G::A - 1;   // points past the board read a valid cell; never stored
        rofs[j] = k * GC + (p / N - rowLo) * G::H + (p % N);
    }

    // Per item, computed once: where it loads from (relative to a chunk's
    // first plane or quad, and in the last chunk, where quads past cin
    // fall back to the last quad), which LDS cell of each buffer it goes to,
    // and whether the last chunk zeroes it.
    const int lastQuad = (cin - 1) / 4;
    const int qLast = nq - 1;
    const float* xb = x + (size_t)b * cin * G::A;                                        // PLANAR
    const f4* xq = reinterpret_cast<const f4*>(x) + (size_t)b * ((cin + 3) / 4) * G::A;   // channel quads
    const f4* wb = wp + (size_t)cb0 * nq * AITEMS;   // this block's fragments, [chunk][tap][lane]
    int pOff[PER], pOffLast[PER], pG[PER], pCell0[PER], pCell1[PER];
    bool pZeroLast[PER];
#pragma unroll
    for (int r = 0; r < PER; ++r) {
        const int it = tid + r * THREADS;
        const int itc = min(it, items - 1);
        const int g = itc / span, p = first + itc - g * span;
        pG[r] = g;
        const int gLast = min(g, lastQuad - 4 * qLast);   // >= 0: chunk qLast holds at least one quad
        pOff[r] = PLANAR ? 4 * g * G::A + p : g * G::A + p;
        pOffLast[r] = gLast * G::A + p;
        pZeroLast[r] = 4 * qLast + g > lastQuad;
        const int cell = g * GC + (p / N - rowLo + 1) * G::H + (p % N + 1);
        pCell0[r] = it < items ? cell : kSpare;
        pCell1[r] = it < items ? CB + cell : kSpare;
    }
    int aSrc[APER], aCell0[APER], aCell1[APER];
#pragma unroll
    for (int r = 0; r < APER; ++r) {
        const int it = tid + r * THREADS;
        const bool in = AITEMS % THREADS == 0 || it < AITEMS;
        aSrc[r] = min(it, AITEMS - 1);
        aCell0[r] = in ? it : kSpareA;
        aCell1[r] = in ? AITEMS + it : kSpareA;
    }
    // Item i (planes first, then fragments) of chunk q into a register set,
    // and from it into LDS buffer `buf`.
    auto loadItem = [&](int i, int q, f4 (&sp)[PER], f4 (&sa)[APER]) {
        if (i < PER) {
            const int r = i;
            if (PLANAR) {
                // plane q*16 + 4g + c at xb + plane * A + p
                const int c0 = q * 16 + 4 * pG[r];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int ch = min(c0 + c, cin - 1);
                    sp[r][c] = xb[pOff[r] + (ch - 4 * pG[r]) * G::A];
                }
            } else {
                sp[r] = (xq + (size_t)q * 4 * G::A)[q == qLast ? pOffLast[r] : pOff[r]];
            }
        } else {
            const int r = i - PER;
            sa[r] = (wb + (size_t)q * AITEMS)[aSrc[r]];
        }
    };
    auto storeItem = [&](int i, int buf, int q, const f4 (&sp)[PER], const f4 (&sa)[APER]) {
        if (i < PER) {
            const int r = i;
            f4 v = sp[r];
            if (PLANAR) {
                const int c0 = q * 16 + 4 * pG[r];
#pragma unroll
                for (int c = 0; c < 4; ++c) v[c] = c0 + c < cin ? v[c] : 0.0f;
            } else {
                // a quad past cin is zeros (a quad's own channels past cin are stored zeros)
                v = q == qLast && pZeroLast[r] ? f4{0.0f, 0.0f, 0.0f, 0.0f} : v;
            }
            lds[buf ? pCell1[r] : pCell0[r]] = v;
        } else {
            const int r = i - PER;
            alds[buf ? aCell1[r] : aCell0[r]] = sa[r];
        }
    };

    // The epilogue's inputs; residual quads only for a layer that adds one
    // (a uniform branch: the count of loads in flight after it, which the
    // chunks' waits use, is exact either way).
    EpilogueInputs<1, PPW> ep;
    loadEpilogue<N, 1, PPW>(ep, scale, shift, skip, b, cout, cb0, pg0, k, n16);

    f4 acc[1][PPW];
#pragma unroll
    for (int j = 0; j < PPW; ++j) acc[0][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    // Chunks 1 and 2 in flight in the two register sets; chunk 0 published
    // (through a third set, live only here). A chunk past the last is
    // loaded as the last one again, stored into a buffer nobody reads
    // afterwards, and not multiplied.
    f4 p0[PER], a0[APER], p1[PER], a1[APER];
    {
        f4 pz[PER], az[APER];
#pragma unroll
        for (int i = 0; i < NI; ++i) loadItem(i, 0, pz, az);
#pragma unroll
        for (int i = 0; i < NI; ++i) loadItem(i, min(1, qLast), p0, a0);
#pragma unroll
        for (int i = 0; i < NI; ++i) loadItem(i, min(2, qLast), p1, a1);
        __syncthreads();   // the zero fill is complete before any interior store
#pragma unroll
        for (int i = 0; i < NI; ++i) storeItem(i, 0, 0, pz, az);
    }
    __syncthreads();

    constexpr int kRing = 4;
    constexpr int STEPS = 9 * PPW;
    auto tapOffset = [](int t) { return (t / 3) * G::H + (t % 3); };
    // Chunk q from LDS buffer `buf` (q & 1): tap t stores items [t*NI/9,
    // (t+1)*NI/9) of chunk q + 1 from the register set (ps, as), where they
    // were loaded during chunk q - 2, into the other buffer (free since the
    // barrier that ended chunk q - 1), and then loads the same items of
    // chunk q + 3 into the registers the store has just read. A chunk's loads
    // so have two chunks of MFMAs to arrive in (at small batches a chunk is
    // shorter than a load's round trip), and the two register sets
    // alternate with the chunks. The last chunks store copies of the last
    // one there, never read.
    auto chunk = [&](int q, int buf, f4 (&ps)[PER], f4 (&as)[APER]) {
        const int qs = min(q + 1, qLast), ql = min(q + 3, qLast);
        const f4* bb = lds + buf * CB;
        const f4* ab = alds + buf * AITEMS + lane;
        f4 ring[kRing];
#pragma unroll
        for (int i = 0; i < kRing && i < STEPS; ++i) ring[i] = bb[rofs[i % PPW] + tapOffset(i / PPW)];
        f4 aT[2];
        aT[0] = ab[0];
        __builtin_amdgcn_sched_group_barrier(0x100, kRing + 1, 0);   // the ring's first reads, tap 0's fragment
#pragma unroll
        for (int i = 0; i < STEPS; ++i) {
            const int t = i / PPW, pg = i % PPW;
            if (pg == 0) {
                const int i0 = t * NI / 9, i1 = (t + 1) * NI / 9;
#pragma unroll
                for (int it = i0; it < i1; ++it) {
                    storeItem(it, buf ^ 1, qs, ps, as);
                    __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
                }
#pragma unroll
                for (int it = i0; it < i1; ++it) {
                    loadItem(it, ql, ps, as);
                    if (it < PER)
                        __builtin_amdgcn_sched_group_barrier(0x020, PLANAR ? 4 : 1, 0);
                    else
                        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                }
                if (t + 1 < 9) {
                    aT[(t + 1) & 1] = ab[(t + 1) * 64];   // the next tap's fragment, a tap ahead
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
            }
            const f4 bv = ring[i % kRing];
            if (i + kRing < STEPS) ring[i % kRing] = bb[rofs[(i + kRing) % PPW] + tapOffset((i + kRing) / PPW)];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[0][pg] = __builtin_amdgcn_mfma_f32_16x16x4f32(aT[t & 1][j], bv[j], acc[0][pg], 0, 0, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);                         // step i's MFMAs,
            if (i + kRing < STEPS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // then step i+kRing's read
        }
        __syncthreads();
    };
    // The stem's last chunk, unless cin fills it, is multiplied apart
    // (stemTail), after the loop.
    const bool tail = PLANAR && cin % kChunk != 0;
    const int nqQuads = tail ? nq - 1 : nq;
    int q = 0;
    for (; q + 1 < nqQuads; q += 2) {
        chunk(q, 0, p0, a0);
        chunk(q + 1, 1, p1, a1);
    }
    if (q < nqQuads) chunk(q, 0, p0, a0);
    if (tail) {
        const int ql = nq - 1, buf = ql & 1;
        // rofs[j] - k * GC is the lane's top-left cell.
        stemTail<1, PPW, GC, G::H>(acc, reinterpret_cast<const float*>(alds + buf * AITEMS) + n16 * 4, 0,
                                   reinterpret_cast<const float*>(lds + buf * CB), rofs, k * GC, k,
                                   cin - ql * kChunk);
    }

    writeOutputs<N, 1, PPW>(acc, ep, skip != nullptr, y, b, cout, cb0, pg0, k, n16, relu);
}

// A workgroup computes board b's output channels [co tile ct] at column
// groups [pixel tile pt]: WCO x WPG waves, wave (c, g) owning COW blocks of
// 16 channels and PPW column groups (PPW = 0: all of them). PLANAR: x is the
// network's input planes [B][cin][A] (the stem), read a channel at a time;
// otherwise x is a trunk activation in channel quads, read a quad at a time.
// Either way input channels past cin are read as zeros. tid: threadIdx.x.
template <int N, int COW, int WCO, int WPG, int PPW0, bool PLANAR>
__device__ __forceinline__ void conv3x3Body(f4* lds, const float* __restrict__ x, const f4* __restrict__ wp,
                                            const float* __restrict__ scale, const float* __restrict__ shift,
                                            const float* skip, float* y, int cin, int cout, int nq, int b, int ct,
                                            int pt, int relu, int tid) {
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

    const int lane = tid & 63, wave = tid >> 6;
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
    f4 stage[PER];
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
    loadA(0, 0, aCur);
    // The stem's last chunk, unless cin fills it, is multiplied apart
    // (stemTail), after the loop.
    const bool tail = PLANAR && cin % kChunk != 0;
    const int nqQuads = tail ? nq - 1 : nq;
    for (int q = 0; q < nqQuads; ++q) {
        // The last chunk fetches itself again in place of a chunk that does
        // not exist (never stored), which keeps the step stream free of
        // branches.
        const int qn = q + 1 < nq ? q + 1 : q;
        const f4* buf = lds + (q & 1) * G::BUF;
        f4 ring[kRing];
#pragma unroll
        for (int i = 0; i < kRing && i < STEPS; ++i) ring[i] = buf[rofs[i % PPW] + tapOffset(i / PPW)];
        __builtin_amdgcn_sched_group_barrier(0x100, kRing, 0);   // the ring's first reads
#pragma unroll
        for (int i = 0; i < STEPS; ++i) {
            const int t = i / PPW, pg = i % PPW;
            if (pg == 0) {
                // The next tap's A fragments (tap 8: the next chunk's first),
                // and at tap 0 after them the board planes of the next
                // chunk: the count of outstanding loads drains in issue
                // order, so a tap's wait for its fragments does not wait
                // for the planes.
                loadA(t + 1 < 9 ? q : qn, (t + 1) % 9, aNext);
                __builtin_amdgcn_sched_group_barrier(0x020, COW, 0);   // issued here, a tap ahead
                if (t == 0) load(qn, stage);
            }
            const f4 bv = ring[i % kRing];
            if (i + kRing < STEPS)
                ring[i % kRing] = buf[rofs[(i + kRing) % PPW] + tapOffset((i + kRing) / PPW)];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int c = 0; c < COW; ++c)
                    acc[c][pg] = __builtin_amdgcn_mfma_f32_16x16x4f32(aCur[c][j], bv[j], acc[c][pg], 0, 0, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 4 * COW, 0);                   // step i's MFMAs,
            if (i + kRing < STEPS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // then step i+kRing's read
            if (pg == PPW - 1) {
#pragma unroll
                for (int c = 0; c < COW; ++c) aCur[c] = aNext[c];
            }
        }
        if (q + 1 < nq) store((q + 1) & 1);
        __syncthreads();
    }
    if (tail) {
        const int q = nq - 1;
        const float* wl =
            reinterpret_cast<const float*>(wp) + (size_t)cb0 * nq * 9 * 256 + (size_t)q * 9 * 256 + n16 * 4;
        // rofs[j] - k * HA is the lane's top-left cell.
        stemTail<COW, PPW, G::HA, G::H>(acc, wl, (size_t)nq * 9 * 256,
                                        reinterpret_cast<const float*>(lds + (q & 1) * G::BUF), rofs, k * G::HA,
                                        k, cin - q * kChunk);
    }

    storeOutputs<N, COW, PPW>(acc, scale, shift, skip, y, b, cout, cb0, pg0, k, n16, relu);
}

// The stem on whole boards (the shapes of large batches) when its planes
// fit two chunks (cin <= 32: the network's 2H + 2 planes up to H = 15) and
// nothing is added to its outputs (the network's stem adds nothing).
// Both chunks are staged once; then each wave runs its column groups in two
// halves, every K step of a half before its outputs are stored, so the
// first half's stores drain while the second half multiplies (one pass over
// the board would store everything after its last MFMA, with the matrix
// units idle meanwhile), and the stem's last-chunk weights and BN factors
// are fetched before the first MFMA (half the accumulators leave the
// registers for them). The MFMA sequence per output, and so every bit, is
// the general body's. lds: two chunk buffers of the general body's layout;
// the workgroup computes board b's co tile ct; tid: threadIdx.x.
template <int N, int COW, int WCO>
__device__ __forceinline__ void conv3x3StemWhole(f4* lds, const float* __restrict__ x, const f4* __restrict__ wp,
                                                 const float* __restrict__ scale, const float* __restrict__ shift,
                                                 float* y, int cin, int cout, int nq, int b, int ct, int relu,
                                                 int tid) {
    using G = Geo<N>;
    constexpr int THREADS = WCO * 64;
    constexpr int HALF = (G::NPG + 1) / 2;   // column groups per half (the second may hold one fewer)
    constexpr int ITEMS = 4 * G::A;          // (channel group, point) pairs per chunk
    constexpr int PER = (ITEMS + THREADS - 1) / THREADS;

    const int lane = tid & 63, wave = tid >> 6;
    const int cb0 = (ct * WCO + wave) * COW;
    const int k = lane >> 4, n16 = lane & 15;

    for (int i = tid; i < 2 * G::BUF; i += THREADS) lds[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    // Chunk q's planes into buffer q (planes past cin as zeros).
    const float* xb = x + (size_t)b * cin * G::A;
    auto load = [&](int q, f4 (&dst)[PER]) {
#pragma unroll
        for (int r = 0; r < PER; ++r) {
            const int it = tid + r * THREADS;
            f4 v = {0.0f, 0.0f, 0.0f, 0.0f};
            if (it < ITEMS) {
                const int g = it / G::A, p = it - g * G::A;
                const int c0 = q * 16 + 4 * g;
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (c0 + c < cin) v[c] = xb[(size_t)(c0 + c) * G::A + p];
            }
            dst[r] = v;
        }
    };
    auto store = [&](int q, const f4 (&src)[PER]) {
#pragma unroll
        for (int r = 0; r < PER; ++r) {
            const int it = tid + r * THREADS;
            if (it < ITEMS) {
                const int g = it / G::A, p = it - g * G::A;
                lds[q * G::BUF + g * G::HA + (p / N + 1) * G::H + (p % N + 1)] = src[r];
            }
        }
    };
    {
        f4 s0[PER], s1[PER];
        load(0, s0);
        load(1, s1);   // nq == 1: zeros, never read
        __syncthreads();   // the zero fill is complete before any interior store
        store(0, s0);
        store(1, s1);
    }
    __syncthreads();

    const bool tail = cin % kChunk != 0;
    const int nqQuads = tail ? nq - 1 : nq;
    const int qt = nq - 1;
    const float* wl = reinterpret_cast<const float*>(wp) + ((size_t)cb0 * nq + qt) * 9 * 256 + n16 * 4;
    const size_t blockStride = (size_t)nq * 9 * 256;
    StemTail<COW, G::HA, G::H> st;
    if (tail) st.fetch(wl, blockStride, k, cin - qt * kChunk);
    EpilogueInputs<COW, HALF> ep;
    loadEpilogue<N, COW, HALF>(ep, scale, shift, nullptr, b, cout, cb0, 0, k, n16);

    constexpr int kRing = 4;
    constexpr int STEPS = 9 * HALF;
    auto tapOffset = [](int t) { return (t / 3) * G::H + (t % 3); };
    auto loadA = [&](int q, int t, f4 (&a)[COW]) {
#pragma unroll
        for (int c = 0; c < COW; ++c) a[c] = wp[((size_t)((cb0 + c) * nq + q) * 9 + t) * 64 + lane];
    };
    // The stream's A fragments, a tap ahead across chunks and halves.
    f4 aCur[COW], aNext[COW];
    loadA(0, 0, aCur);
    for (int h = 0; h < 2; ++h) {
        const int pg0 = h * HALF;
        int rofs[HALF];
#pragma unroll
        for (int j = 0; j < HALF; ++j) {
            int p = (pg0 + j) * 16 + n16;
            p = p < G::A ? p : G::A - 1;   // points past the board read a valid cell; never stored
            rofs[j] = k * G::HA + (p / N) * G::H + (p % N);
        }
        f4 acc[COW][HALF];
#pragma unroll
        for (int c = 0; c < COW; ++c)
#pragma unroll
            for (int j = 0; j < HALF; ++j) acc[c][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        // The general body's step stream per quad chunk (B operands kRing
        // steps ahead, A fragments a tap ahead).
        for (int q = 0; q < nqQuads; ++q) {
            const f4* buf = lds + q * G::BUF;
            const int qn = q + 1 < nqQuads ? q + 1 : 0;   // whose tap 0 follows tap 8
            f4 ring[kRing];
#pragma unroll
            for (int i = 0; i < kRing; ++i) ring[i] = buf[rofs[i % HALF] + tapOffset(i / HALF)];
            __builtin_amdgcn_sched_group_barrier(0x100, kRing, 0);
#pragma unroll
            for (int i = 0; i < STEPS; ++i) {
                const int t = i / HALF, pg = i % HALF;
                if (pg == 0) {
                    loadA(t + 1 < 9 ? q : qn, (t + 1) % 9, aNext);
                    __builtin_amdgcn_sched_group_barrier(0x020, COW, 0);
                }
                const f4 bv = ring[i % kRing];
                if (i + kRing < STEPS)
                    ring[i % kRing] = buf[rofs[(i + kRing) % HALF] + tapOffset((i + kRing) / HALF)];
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int c = 0; c < COW; ++c)
                        acc[c][pg] = __builtin_amdgcn_mfma_f32_16x16x4f32(aCur[c][j], bv[j], acc[c][pg], 0, 0, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 4 * COW, 0);
                if (i + kRing < STEPS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                if (pg == HALF - 1) {
#pragma unroll
                    for (int c = 0; c < COW; ++c) aCur[c] = aNext[c];
                }
            }
        }
        // rofs[j] - k * HA is the lane's top-left cell.
        if (tail)
            st.multiply(acc, wl, blockStride, reinterpret_cast<const float*>(lds + qt * G::BUF), rofs, k * G::HA, k,
                        cin - qt * kChunk);
        writeOutputs<N, COW, HALF>(acc, ep, false, y, b, cout, cb0, pg0, k, n16, relu);
    }
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
        if constexpr (PPW != 0 && COW * WCO == 1) {                                                         \
            conv3x3SmallBody<N, WPG, PPW, PLANAR>(x, wp, scale, shift, skip, y, cin, cout, nq, coTiles,      \
                                                  pixTiles, relu);                                         \
        } else {                                                                                           \
            __shared__ f4 lds[2 * Geo<N>::BUF];                                                            \
            /* Workgroups are dealt to the 8 XCDs round-robin; renumbered so */                            \
            /* that the tiles of one board run on the same XCD (one L2). */                                \
            const int total = gridDim.x, wg = blockIdx.x;                                                  \
            const int logical = (total % 8 == 0) ? (wg % 8) * (total / 8) + wg / 8 : wg;                   \
            const int b = logical / (coTiles * pixTiles), tile = logical % (coTiles * pixTiles);           \
            const int ct = tile / pixTiles, pt = tile % pixTiles;                                          \
            if constexpr (PLANAR && PPW == 0 && WPG == 1) {                                                \
                if (nq <= 2 && !skip) {                                                                    \
                    conv3x3StemWhole<N, COW, WCO>(lds, x, wp, scale, shift, y, cin, cout, nq, b, ct, relu,     \
                                                  threadIdx.x);                                    \
                    return;                                                                                \
                }                                                                                          \
            }                                                                                              \
            conv3x3Body<N, COW, WCO, WPG, PPW, PLANAR>(lds, x, wp, scale, shift, skip, y, cin, cout, nq, b,  \
                                                       ct, pt, relu, threadIdx.x);                         \
        }                                                                                                  \
    }
AZH_CONV_KERNEL(conv3x3Tower, false)
AZH_CONV_KERNEL(conv3x3Stem, true)
#undef AZH_CONV_KERNEL

// threadIdx.x as a value the compiler cannot see through: the bodies'
// per-lane addresses are then computed again for each layer instead of
// hoisted out of the loops and held across them (which spills).
__device__ __forceinline__ int opaqueThreadIdx() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// The board-resident tower: one workgroup of 8 waves holds a board for the
// stem (when t.in is set) and every layer of the tower, with a workgroup
// barrier between layers in place of a kernel boundary (a board's layer
// reads only that board's previous layer, which the same workgroup wrote).
// Each layer is the general body on the whole board at 128 output channels
// per workgroup (wave w: channels 16w..16w+15), so every output has the
// per-layer launches' MFMA sequence and bits. The workgroup takes boards
// blockIdx.x, + gridDim.x, ...; the layers' activations go through global
// memory (x and mid as the per-layer launches use them), and the
// barrier's workgroup-scope fence orders a layer's stores before the next
// layer's loads. STEM: the launch runs the stem first (t.in set); a kernel
// of its own, apart from the tower alone, so that profiles tell them apart.
template <int N, bool STEM>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void convTowerResident(
    ResidentTower t) {
    __shared__ f4 lds[2 * Geo<N>::BUF];
    const int nq = (t.F + kChunk - 1) / kChunk;
    for (int b = blockIdx.x; b < t.B; b += gridDim.x) {
        if constexpr (STEM) {
            conv3x3StemWhole<N, 1, 8>(lds, t.in, reinterpret_cast<const f4*>(t.stemW), t.stemScale, t.stemShift, t.x,
                                      t.P, t.F, (t.P + kChunk - 1) / kChunk, b, 0, 1, opaqueThreadIdx());
            __syncthreads();
        }
        for (int l = 0; l < t.layers; ++l) {
            const float* w = t.w0 + (size_t)l * t.stride;
            // Even layers: a block's first convolution, x -> mid; odd: its
            // second, mid -> x with x as the residual (in place).
            const bool second = (l & 1) != 0;
            conv3x3Body<N, 1, 8, 1, 0, false>(lds, second ? t.mid : t.x, reinterpret_cast<const f4*>(w),
                                               w + t.scaleOff, w + t.shiftOff, second ? t.x : nullptr,
                                               second ? t.x : t.mid, t.F, t.F, nq, b, 0, 0, 1, opaqueThreadIdx());
            __syncthreads();
        }
    }
}

} // namespace

template <int N>
hipError_t launchResidentTowerT(const ResidentTower& t, int workgroups, hipStream_t stream) {
    if (t.in)
        hipLaunchKernelGGL((convTowerResident<N, true>), dim3(workgroups), dim3(512), 0, stream, t);
    else
        hipLaunchKernelGGL((convTowerResident<N, false>), dim3(workgroups), dim3(512), 0, stream, t);
    return hipGetLastError();
}

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
