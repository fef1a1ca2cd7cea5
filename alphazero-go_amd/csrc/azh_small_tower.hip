// A small board's pass in one launch: one workgroup per board runs the
// stem, every block's two 3x3 convolutions and the heads with the board's
// activations held in LDS (two haloed tiles in channel quads: the block
// input x and the middle activation), so a pass of many short layers is one
// launch instead of one per layer. Boards are independent, so no workgroup
// ever waits for another.
//
// The arithmetic is the per-layer kernels': for the convolutions the tower
// kernel's (azh_conv.hpp) packed A fragments, B values (channel quads with
// zeros past the channel count), order of v_mfma_f32_16x16x4_f32 per output
// (chunk, tap, channel in chunk) and epilogue; for the heads the order of
// headConvKernel's sums and headFcKernel's MFMA blocks. Every output has
// the bits the per-layer launches give it.
#include "azh_kernels.hpp"
#include "azh_heads.hpp"
#include "azh_stem.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>

namespace azh {

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

// 4 waves per board. (8 on 9x9, a channel block's 6 column groups split
// 3 and 3, measured 3% faster up to 256 boards and 9% slower at 512, where
// two 8-wave workgroups no longer fit a CU: a 9x9 board's layer is bound by
// its CU's matrix rate, about 10 us, either way.)
template <int N>
constexpr int smallThreads() { return 256; }

template <int P>
struct Parity {
    static constexpr int value = P;
};

// trunk [B][ceil(F/4)][A] quads, in place; F <= 64, NQ = ceil(F/16) chunks
// (and channel blocks). Layer l's packed weights start at w0 + l *
// layerStride floats, its BN scale and shift at scaleOff and shiftOff floats
// after them (the tower's convolutions sit in the weight arena at one fixed
// stride). Each channel block goes to waves / NQ waves, which share its
// column groups; the A fragments (nine taps) of a wave's next chunk, or of the next
// layer's first, are fetched while the current chunk is multiplied.
// The chunk loop is unrolled with the two fragment buffers assigned at
// compile time (layers come in pairs, so the parity of a chunk's buffer is
// known), which keeps each fetch a whole chunk ahead of its use, and the
// helpers are forced inline (left to the inliner, the 9x9 instances kept
// their arrays in scratch memory).
template <int N, int NQ>
__global__ __launch_bounds__(smallThreads<N>()) void smallTowerKernel(float* __restrict__ trunk, SmallStem stem,
                                                                  SmallHeads heads,
                                                                  const float* __restrict__ w0, size_t layerStride,
                                                                  size_t scaleOff, size_t shiftOff, int layers,
                                                                  int F) {
    constexpr int A = N * N, H = N + 2, HA = H * H, NPG = (A + 15) / 16;
    constexpr int THREADS = smallThreads<N>(), WAVES = THREADS / 64;
    constexpr int G = 4 * NQ;   // channel quads held per tile (whole chunks; the padding stays zero)
    extern __shared__ f4 tile[];
    const int GQ = (F + 3) / 4;   // channel quads stored in the trunk
    // With the stem, the second tile first holds the input planes in
    // channel quads (whole 16-channel chunks, zero past the plane count).
    const int GS = stem.in ? 4 * ((stem.planes + 15) / 16) : 0;
    const int GM = G > GS ? G : GS;
    f4* tx = tile;
    f4* tm = tile + G * HA;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, k = lane >> 4, n16 = lane & 15;
    const int b = blockIdx.x;
    f4* xq = reinterpret_cast<f4*>(trunk) + (size_t)b * GQ * A;

    for (int i = tid; i < (G + GM) * HA; i += THREADS) tile[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    __syncthreads();
    if (stem.in) {
        // The input planes [P][A] of this board, a channel at a time (the
        // stem kernel's staging): channels past P read as zeros.
        const float* in = stem.in + (size_t)b * stem.planes * A;
        for (int i = tid; i < GS * A; i += THREADS) {
            const int g = i / A, p = i - g * A;
            f4 v = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (4 * g + c < stem.planes) v[c] = in[(size_t)(4 * g + c) * A + p];
            tm[g * HA + (p / N + 1) * H + (p % N + 1)] = v;
        }
    } else {
        for (int i = tid; i < GQ * A; i += THREADS) {
            const int g = i / A, p = i - g * A;
            tx[g * HA + (p / N + 1) * H + (p % N + 1)] = xq[i];
        }
    }
    __syncthreads();

    // With fewer channel blocks than waves, a block's column groups are
    // split over WAVES / NQ waves (PGW each), so every wave has work where
    // the board allows (the split decides only which wave computes an
    // output).
    constexpr int WPB = WAVES / NQ;                // waves per channel block
    constexpr int PGW = (NPG + WPB - 1) / WPB;     // column groups per wave
    const int cb = wave / WPB, pg0 = (wave % WPB) * PGW;
    if (cb >= NQ || pg0 >= NPG) {
        if (stem.in) __syncthreads();
        for (int l = 0; l < layers; ++l) __syncthreads();
    } else {
        // Each lane's top-left tap cell per column group; points past the
        // board (and column groups past the board's) read a valid cell and
        // are never stored.
        int base[PGW];
#pragma unroll
        for (int j = 0; j < PGW; ++j) {
            int p = (pg0 + j) * 16 + n16;
            p = p < A ? p : A - 1;
            base[j] = (p / N) * H + (p % N);
        }
        f4 acc[PGW];
        f4 fa[9], fb[9];
        auto load = [&](f4(&f)[9], int l, int q) __attribute__((always_inline)) {
            const f4* w = reinterpret_cast<const f4*>(w0 + (size_t)l * layerStride) + (size_t)((cb * NQ + q) * 9) * 64 +
                          lane;
#pragma unroll
            for (int t = 0; t < 9; ++t) f[t] = w[t * 64];
        };
        auto multiply = [&](const f4(&f)[9], const f4* src, int q) __attribute__((always_inline)) {
#pragma unroll
            for (int t = 0; t < 9; ++t) {
                const f4* s = src + (4 * q + k) * HA + (t / 3) * H + (t % 3);
#pragma unroll
                for (int j = 0; j < PGW; ++j) {
                    const f4 bv = s[base[j]];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(f[t][e], bv[e], acc[j], 0, 0, 0);
                }
            }
        };
        // Lane (n16, k) holds channels 16 cb + 4 k + e of point
        // 16 (pg0 + j) + n16; the second convolution of a block adds the
        // block input it overwrites (the same lane reads and writes each
        // element).
        auto store = [&](const float* sc, const float* sh, f4* dst, bool skip) __attribute__((always_inline)) {
            const int gch = cb * 4 + k;
#pragma unroll
            for (int j = 0; j < PGW; ++j) {
                const int p = (pg0 + j) * 16 + n16;
                if (p < A) {
                    f4* cell = dst + gch * HA + (p / N + 1) * H + (p % N + 1);
                    const f4 sk = skip ? *cell : f4{0.0f, 0.0f, 0.0f, 0.0f};
                    f4 v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int c = gch * 4 + e;
                        v[e] = c < F ? epilogue(acc[j][e], sc[c], sh[c], skip, sk[e], true) : 0.0f;
                    }
                    *cell = v;
                }
            }
        };
        // One layer: chunk q's fragments are in buffer (P + q) & 1 (fa for
        // 0), the next chunk's are fetched into the other before q is
        // multiplied.
        auto layer = [&](int l, auto parity) __attribute__((always_inline)) {
            constexpr int P = decltype(parity)::value;
            const bool second = l & 1;
            const f4* src = second ? tm : tx;
            f4* dst = second ? tx : tm;
#pragma unroll
            for (int j = 0; j < PGW; ++j) acc[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            // Explicit branches, not a select between the two arrays: each
            // branch names its buffers, so they stay in registers.
            auto chunk = [&](f4(&cur)[9], f4(&next)[9], int q) __attribute__((always_inline)) {
                if (q + 1 < NQ)
                    load(next, l, q + 1);
                else if (l + 1 < layers)
                    load(next, l + 1, 0);
                multiply(cur, src, q);
            };
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                if (((P + q) & 1) == 0)
                    chunk(fa, fb, q);
                else
                    chunk(fb, fa, q);
            }
            const float* lw = w0 + (size_t)l * layerStride;
            store(lw + scaleOff, lw + shiftOff, dst, second);
            __syncthreads();   // the layer is complete
        };
        if (layers > 0) load(fa, 0, 0);
        if (stem.in) {
            // The stem: input planes (in tm) -> x, BN and ReLU, no skip; its
            // fragments are fetched a chunk at a time (one layer only).
#pragma unroll
            for (int j = 0; j < PGW; ++j) acc[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            const int nqs = GS / 4;
            // The last chunk, unless the planes fill it, as the stem kernel
            // multiplies it (stemTail).
            const bool tail = stem.planes % kChunk != 0;
            for (int q = 0; q < (tail ? nqs - 1 : nqs); ++q) {
                f4 fs[9];
                const f4* w = reinterpret_cast<const f4*>(stem.w) + (size_t)((cb * nqs + q) * 9) * 64 + lane;
#pragma unroll
                for (int t = 0; t < 9; ++t) fs[t] = w[t * 64];
                multiply(fs, tm, q);
            }
            if (tail) {
                const int q = nqs - 1;
                f4 a1[1][PGW];
#pragma unroll
                for (int j = 0; j < PGW; ++j) a1[0][j] = acc[j];
                const float* wl = stem.w + (size_t)((cb * nqs + q) * 9) * 256 + n16 * 4;
                stemTail<1, PGW, HA, H>(a1, wl, 0, reinterpret_cast<const float*>(tm + 4 * q * HA), base, 0, k,
                                        stem.planes - q * kChunk);
#pragma unroll
                for (int j = 0; j < PGW; ++j) acc[j] = a1[0][j];
            }
            store(stem.scale, stem.shift, tx, false);
            __syncthreads();   // x is complete and the input tile is free
        }
        for (int l = 0; l < layers; l += 2) {
            layer(l, Parity<0>{});
            layer(l + 1, Parity<NQ & 1>{});
        }
    }

    for (int i = tid; i < GQ * A; i += THREADS) {
        const int g = i / A, p = i - g * A;
        xq[i] = tx[g * HA + (p / N + 1) * H + (p % N + 1)];
    }
    if (!heads.logits) return;

    // The heads on the trunk in tx, as headConvKernel and headFcKernel
    // compute them (the same sums in the same order): the 1x1 convolutions
    // per point, then the policy and value Linears as 16-row MFMA blocks
    // whose row 0 is this board (the other 15 rows zero). The second tile is
    // free: the staged rows [16][RS], the value plane [A], the hidden [V].
    constexpr int A1 = A + 1, KP = headPad16(2 * A), KV = headPad16(A), NP = headPad16(A1), RS = KP + 4;
    const HeadWeights& hw = heads.w;
    float* xs = reinterpret_cast<float*>(tm);
    float* valRow = xs + 16 * RS;
    float* hid = valRow + A;
    const int m = lane & 15, kk = lane >> 4;
    for (int i = tid; i < 16 * RS; i += THREADS) xs[i] = 0.0f;
    __syncthreads();
    for (int p = tid; p < A; p += THREADS) {
        const f4* xp = tx + (p / N + 1) * H + (p % N + 1);
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
        for (int c = 0; c < F; ++c) {
            const float x = xp[(c / 4) * HA][c % 4];
            a0 = fmaf(hw.convW[c], x, a0);
            a1 = fmaf(hw.convW[F + c], x, a1);
            a2 = fmaf(hw.convW[2 * F + c], x, a2);
            if (heads.own) a3 = fmaf(hw.convW[3 * F + c], x, a3);
        }
        xs[p] = epilogue(a0, hw.scale[0], hw.shift[0], false, 0.0f, true);       // feature c*A + p
        xs[A + p] = epilogue(a1, hw.scale[1], hw.shift[1], false, 0.0f, true);
        valRow[p] = epilogue(a2, hw.scale[2], hw.shift[2], false, 0.0f, true);
        if (heads.own)
            heads.own[(size_t)b * A + p] = tanhf(epilogue(a3, hw.scale[3], hw.shift[3], false, 0.0f, false));
    }
    __syncthreads();
    const HeadVec4* xs4 = reinterpret_cast<const HeadVec4*>(xs);
    for (int n0 = wave * 16; n0 < NP; n0 += 16 * WAVES) {
        const HeadVec4 acc = fcBlock<KP, RS>(xs4, m, kk, n0, NP, hw.policyWT);
        const int a = n0 + m;
        if (kk == 0 && a < A1) heads.logits[(size_t)b * A1 + a] = __fadd_rn(acc[0], hw.policyB[a]);
    }
    __syncthreads();
    for (int i = tid; i < KV; i += THREADS) xs[i] = i < A ? valRow[i] : 0.0f;
    __syncthreads();
    const int V = heads.V, VP = headPad16(V);
    for (int n0 = wave * 16; n0 < VP; n0 += 16 * WAVES) {
        const HeadVec4 acc = fcBlock<KV, RS>(xs4, m, kk, n0, VP, hw.fc1WT);
        const int v = n0 + m;
        if (kk == 0 && v < V) {
            const float h = __fadd_rn(acc[0], hw.fc1B[v]);
            hid[v] = h > 0.0f ? h : 0.0f;
        }
    }
    __syncthreads();
    if (tid == 0) {
        float s = 0.0f;
        for (int u = 0; u < V; ++u) s = fmaf(hid[u], hw.fc2W[u], s);
        heads.values[b] = tanhf(__fadd_rn(s, hw.fc2B[0]));
    }
}

} // namespace

size_t smallTowerLdsBytes(int n, int F, int planes, bool heads, int V) {
    if (n != 5 && n != 9 && n != 13) return 0;
    const size_t cell = (size_t)(n + 2) * (n + 2) * sizeof(f4);
    const size_t g = 4 * (size_t)((F + 15) / 16), gs = planes > 0 ? 4 * (size_t)((planes + 15) / 16) : 0;
    size_t second = (g > gs ? g : gs) * cell;
    if (heads) {   // the heads' rows, value plane and hidden layer in the second tile
        const size_t A = (size_t)n * n, rows = 16 * (size_t)(headPad16(2 * n * n) + 4) + A + (size_t)V;
        second = std::max(second, rows * sizeof(float));
    }
    return g * cell + second;
}

namespace {

template <int N, int NQ = 1>
hipError_t launchSmallN(float* trunk, const SmallStem& stem, const SmallHeads& heads, const float* w0,
                        size_t layerStride, size_t scaleOff, size_t shiftOff, int layers, int B, int F, size_t lds,
                        hipStream_t stream) {
    if constexpr (NQ <= kSmallTowerMaxChunks) {
        if ((F + 15) / 16 != NQ)
            return launchSmallN<N, NQ + 1>(trunk, stem, heads, w0, layerStride, scaleOff, shiftOff, layers, B, F,
                                           lds, stream);
        hipLaunchKernelGGL((smallTowerKernel<N, NQ>), dim3(B), dim3(smallThreads<N>()), lds, stream, trunk, stem, heads,
                           w0, layerStride, scaleOff, shiftOff, layers, F);
        return hipGetLastError();
    } else {
        return hipErrorInvalidValue;
    }
}

} // namespace

hipError_t launchSmallTower(float* trunk, const SmallStem* stem, const SmallHeads* heads, const float* w0,
                            size_t layerStride, size_t scaleOff, size_t shiftOff, int layers, int B, int n, int F,
                            hipStream_t stream) {
    const SmallStem st = stem ? *stem : SmallStem{};
    const SmallHeads hd = heads ? *heads : SmallHeads{};
    if (st.in && (st.planes < 1 || !st.w || !st.scale || !st.shift)) return hipErrorInvalidValue;
    if (hd.logits && (!hd.values || hd.V < 1 || hd.V > 256)) return hipErrorInvalidValue;
    const size_t lds = smallTowerLdsBytes(n, F, st.in ? st.planes : 0, hd.logits != nullptr, hd.V);
    if (B < 1 || F < 1 || F > 16 * kSmallTowerMaxChunks || layers < 0 || (layers & 1) || lds == 0 ||
        lds > kSmallTowerMaxLds)
        return hipErrorInvalidValue;
    if (n == 5)
        return launchSmallN<5>(trunk, st, hd, w0, layerStride, scaleOff, shiftOff, layers, B, F, lds, stream);
    if (n == 9)
        return launchSmallN<9>(trunk, st, hd, w0, layerStride, scaleOff, shiftOff, layers, B, F, lds, stream);
    return launchSmallN<13>(trunk, st, hd, w0, layerStride, scaleOff, shiftOff, layers, B, F, lds, stream);
}

} // namespace azh
