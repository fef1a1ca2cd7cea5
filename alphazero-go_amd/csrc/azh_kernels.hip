// The gfx950 kernels of the inference pass other than the 3x3 convolution
// (azh_conv.hpp): the heads' 1x1 convolutions and Linear layers and the
// test hooks; plus the convolution's host side (weight packing, the choice
// of workgroup shape, the dispatch to the compiled instances). The
// legal-move softmax is azh_positions.hip's priors kernel without a
// symmetry.
//
// MFMA operand layout (16x16x4 f32, wave64): A[i][k] comes from lane
// i + 16k, B[k][j] from lane j + 16k, and lane j + 16g holds D[4g + r][j] in
// accumulator element r.
#include "azh_kernels.hpp"
#include "azh_heads.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>

namespace azh {

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

// Picks the compiled instance of tiling t for board size N.
template <int N, int I = 0>
hipError_t launchConvN(const float* x, const float* wp, const float* scale, const float* shift, const float* skip,
                       float* y, int B, int cin, int cout, bool relu, bool planarInput, ConvTiling t,
                       hipStream_t stream) {
    if constexpr (I < kConvTilingCount) {
        constexpr ConvTiling c = kConvTilings[I];
        if (t == c)
            return launchConvT<N, c.coPerWave, c.wavesCo, c.wavesPg, c.pgPerWave>(x, wp, scale, shift, skip, y, B,
                                                                                  cin, cout, relu, planarInput,
                                                                                  stream);
        return launchConvN<N, I + 1>(x, wp, scale, shift, skip, y, B, cin, cout, relu, planarInput, t, stream);
    } else {
        return hipErrorInvalidValue;
    }
}

// ------------------------------------------------------------------ heads

// The heads' 1x1 convolutions F -> 2 (policy) and F -> 1 (value), their BN
// and ReLU (src/network.cpp:274-277, 288-291), one point per thread and a
// position's points over gridDim.y workgroups (blockIdx.x the position), the
// trunk read in channel quads (32 16-byte loads per 128 channels) ahead of
// their FMAs:
// act [B][3][A], planes 0-1 the policy's flattened [2A] row (feature c*A + p,
// src/network.cpp:278-285), plane 2 the value's [A] row. With own set, the
// ownership head too: 1x1 conv F -> 1, BN, tanh at every point, no ReLU
// (src/network.cpp:298-308), into own [B][A].
template <int N>
__global__ __launch_bounds__(((N * N + 63) / 64) * 64) void headConvKernel(const float* __restrict__ trunk,
                                                                          HeadWeights w, float* __restrict__ act,
                                                                          float* __restrict__ own, int F) {
    constexpr int A = N * N;
    constexpr int kRound = 128;   // channels per round
    // A round's weights, channel by channel (policy 0, policy 1, value,
    // ownership), staged in LDS and read by every thread at once as one
    // 16-byte broadcast per channel. Channels past F, and the ownership row
    // of a network without one, stage as zeros and their trunk values as
    // zeros: fmaf(0, 0, a) is a for every accumulator a these sums reach
    // (they start at +0 and never become -0), so the straight-line loop
    // rounds exactly as the sum over channels 0..F-1 does.
    __shared__ f4 wsh[kRound];
    const int b = blockIdx.x, p = blockIdx.y * blockDim.x + threadIdx.x;
    const bool withOwn = own != nullptr;
    const int quads = (F + 3) / 4;
    const f4* tq = reinterpret_cast<const f4*>(trunk) + (size_t)b * quads * A + min(p, A - 1);
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    // 128 channels (32 quads) per round: a 128-filter trunk in one load
    // round trip.
    for (int c0 = 0; c0 < F; c0 += kRound) {
        float xv[kRound];
#pragma unroll
        for (int g = 0; g < kRound / 4; ++g) {
            const f4 v = c0 / 4 + g < quads ? tq[(size_t)(c0 / 4 + g) * A] : f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int r = 0; r < 4; ++r) xv[4 * g + r] = c0 + 4 * g + r < F ? v[r] : 0.0f;
        }
        __syncthreads();   // the previous round's weights are no longer read
        for (int c = threadIdx.x; c < kRound; c += blockDim.x) {
            const bool live = c0 + c < F;
            f4 wv;
            wv[0] = live ? w.convW[c0 + c] : 0.0f;
            wv[1] = live ? w.convW[F + c0 + c] : 0.0f;
            wv[2] = live ? w.convW[2 * F + c0 + c] : 0.0f;
            wv[3] = live && withOwn ? w.convW[3 * F + c0 + c] : 0.0f;
            wsh[c] = wv;
        }
        __syncthreads();
        // Eight broadcasts in flight, then their 32 FMAs.
#pragma unroll
        for (int u0 = 0; u0 < kRound; u0 += 8) {
            f4 wv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) wv[j] = wsh[u0 + j];
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                a0 = fmaf(wv[j][0], xv[u0 + j], a0);
                a1 = fmaf(wv[j][1], xv[u0 + j], a1);
                a2 = fmaf(wv[j][2], xv[u0 + j], a2);
                a3 = fmaf(wv[j][3], xv[u0 + j], a3);
            }
            __builtin_amdgcn_sched_group_barrier(0x002, 32, 0);
        }
    }
    if (p >= A) return;
    float* ab = act + (size_t)b * 3 * A;
    ab[p] = epilogue(a0, w.scale[0], w.shift[0], false, 0.0f, true);
    ab[A + p] = epilogue(a1, w.scale[1], w.shift[1], false, 0.0f, true);
    ab[2 * A + p] = epilogue(a2, w.scale[2], w.shift[2], false, 0.0f, true);
    if (withOwn) own[(size_t)b * A + p] = tanhf(epilogue(a3, w.scale[3], w.shift[3], false, 0.0f, false));
}

// The heads' Linear layers as MFMA GEMMs over 16 positions per workgroup
// (one 16 x 16 output block per wave, v_mfma_f32_16x16x4_f32). blockIdx.y <
// policy tiles: 64 policy outputs, logits = flat . W^T + b (Linear::forward,
// src/layers.cpp:169-176); the last y: the value head, fc1 (A -> V) + b,
// ReLU, fc2 (V -> 1) + b, tanh (src/network.cpp:293-296). The positions'
// rows are staged in LDS, zero past the batch and past K; the weights come
// pre-transposed and zero-padded to whole 16 x 16 blocks (HeadWeights).
// Each output is a dot product over its own row only, in a fixed K order.
constexpr int kFcBoards = 16;
constexpr int kFcOutTile = 64;

template <int N>
__global__ __launch_bounds__(256) void headFcKernel(const float* __restrict__ act, HeadWeights w,
                                                    float* __restrict__ logits, float* __restrict__ values, int B,
                                                    int V) {
    constexpr int A = N * N, A1 = A + 1;
    constexpr int KP = headPad16(2 * A);          // policy K, padded
    constexpr int KV = headPad16(A);              // value K, padded
    constexpr int NP = headPad16(A1);             // policy outputs, padded
    constexpr int RS = KP + 4;                    // LDS row stride (floats)
    constexpr int HS = 257;                       // hidden-row stride: fc2's rows in distinct banks
    __shared__ f4 xs4[kFcBoards * RS / 4];
    __shared__ float hid[kFcBoards * HS];
    float* xs = reinterpret_cast<float*>(xs4);
    const int b0 = blockIdx.x * kFcBoards;
    const int nb = min(kFcBoards, B - b0);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int policyTiles = (A1 + kFcOutTile - 1) / kFcOutTile;
    const bool policy = (int)blockIdx.y < policyTiles;
    const int K = policy ? 2 * A : A, KPad = policy ? KP : KV;
    const int src = policy ? 0 : 2 * A;
    // Stage the positions' rows: thread t holds columns t, t + 256, ... of
    // every row, all of its loads in flight at once (one round trip); K
    // padding and the rows past the batch are zeros, written without loads.
    constexpr int KCOLS = (KP + 255) / 256;   // columns per thread (KP >= KV)
    float v[kFcBoards][KCOLS];
#pragma unroll
    for (int bb = 0; bb < kFcBoards; ++bb)
#pragma unroll
        for (int c = 0; c < KCOLS; ++c) {
            const int k = tid + 256 * c;
            v[bb][c] = bb < nb && k < K ? act[(size_t)(b0 + bb) * 3 * A + src + k] : 0.0f;
        }
#pragma unroll
    for (int bb = 0; bb < kFcBoards; ++bb)
#pragma unroll
        for (int c = 0; c < KCOLS; ++c) {
            const int k = tid + 256 * c;
            if (k < KPad) xs[bb * RS + k] = v[bb][c];
        }
    __syncthreads();

    const int m = lane & 15, kk = lane >> 4;
    if (policy) {
        const int n0 = blockIdx.y * kFcOutTile + wave * 16;
        if (n0 >= NP) return;
        const f4 acc = fcBlock<KP, RS>(xs4, m, kk, n0, NP, w.policyWT);
        const int a = n0 + m;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int bb = 4 * kk + r;
            if (bb < nb && a < A1) logits[(size_t)(b0 + bb) * A1 + a] = __fadd_rn(acc[r], w.policyB[a]);
        }
        return;
    }
    const int VP = headPad16(V);
    for (int n0 = wave * 16; n0 < VP; n0 += 64) {
        const f4 acc = fcBlock<KV, RS>(xs4, m, kk, n0, VP, w.fc1WT);
        const int v = n0 + m;
        if (v < V) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float h = __fadd_rn(acc[r], w.fc1B[v]);
                hid[(4 * kk + r) * HS + v] = h > 0.0f ? h : 0.0f;
            }
        }
    }
    __syncthreads();
    if (tid < nb) {
        float s = 0.0f;
        for (int u = 0; u < V; ++u) s = fmaf(hid[tid * HS + u], w.fc2W[u], s);
        values[b0 + tid] = tanhf(__fadd_rn(s, w.fc2B[0]));
    }
}

// ------------------------------------------------------------------ test hooks

__global__ void spinKernel(unsigned long long ticks) {
    const unsigned long long start = wall_clock64();
    unsigned long long spins = 0;
    // Bounded twice over: by the clock, and by a spin count far above any
    // delay a test asks for, so the wave always finishes.
    while (wall_clock64() - start < ticks && spins < (1ull << 34)) ++spins;
}

__global__ void fillKernel(float* data, size_t n, float value) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) data[i] = value;
}

// The matrix units' rate with nothing else in the way: 8 waves per
// workgroup (two per SIMD), each a dependent chain of 4 * chain
// v_mfma_f32_16x16x4_f32 on one accumulator. The SIMD alternates between
// its two waves' chains and so issues one MFMA every 32 cycles (a single
// dependent chain alone on a SIMD issues one only every 44). The operands
// are tiny, so the sums stay finite; one float per thread is written so the
// chain is kept.
__global__ __launch_bounds__(512) void mfmaChainKernel(float* out, int chain) {
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const float a = 1.0f + threadIdx.x * 1e-7f, b = 1e-9f;
    for (int i = 0; i < chain; ++i) {
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
    }
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = acc[0] + acc[1] + acc[2] + acc[3];
}

} // namespace

// ------------------------------------------------------------------ host side

size_t packedConv3x3Floats(int cin, int cout) {
    return (size_t)packedCoBlocks(cout) * ceilDiv(cin, kChunk) * 9 * 64 * 4;
}

std::vector<float> packConv3x3(const float* w, int cin, int cout) {
    const int coBlocks = packedCoBlocks(cout), nq = ceilDiv(cin, kChunk);
    std::vector<float> out(packedConv3x3Floats(cin, cout), 0.0f);
    for (int cb = 0; cb < coBlocks; ++cb)
        for (int q = 0; q < nq; ++q)
            for (int t = 0; t < 9; ++t)
                for (int lane = 0; lane < 64; ++lane)
                    for (int j = 0; j < 4; ++j) {
                        const int co = cb * 16 + (lane & 15);
                        const int ci = q * 16 + 4 * (lane >> 4) + j;
                        const size_t o = ((((size_t)cb * nq + q) * 9 + t) * 64 + lane) * 4 + j;
                        if (co < cout && ci < cin) out[o] = w[((size_t)co * cin + ci) * 9 + t];
                    }
    return out;
}

bool conv3x3Supported(int n) { return n == 5 || n == 9 || n == 13 || n == 19; }

int deviceCUs() {
    static std::atomic<int> cached{0};
    int cus = cached.load();
    if (cus > 0) return cus;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
        cus = 256;   // MI355X
    cached.store(cus);
    return cus;
}

long convWorkgroups(ConvTiling t, int cout, int B, int boardSize) {
    const int groups = ceilDiv(boardSize * boardSize, 16);
    const int groupsPerWorkgroup = t.wavesPg * (t.pgPerWave == 0 ? groups : t.pgPerWave);
    return (long)B * ceilDiv(cout, t.coTile()) * ceilDiv(groups, groupsPerWorkgroup);
}

ConvTiling chooseConvTiling(int cout, int B, int boardSize, bool alone) {
    // From sweeps of every shape over boards 5, 9, 13, 19, 32 to 256
    // channels and batches of 1 to 512 on the MI355X (256 CUs).
    // - Whole-board shapes: a workgroup is one board and 64 output channels
    //   (4 waves of 16; 32 or 16 channels with fewer blocks), two resident
    //   per CU (256 registers per lane, 56 KB of LDS each), one hiding the
    //   other's staging and barriers. On boards up to 13x13 they win as soon
    //   as their waves number about three per CU (two per CU on 5x5, whose
    //   two column groups leave the smaller shapes' waves half idle), taking
    //   the widest channel tile that gets there. At 19x19 a board's
    //   workgroup is long enough that a part-filled round of them costs a
    //   whole one, so they wait for about 40k output tiles (one full round
    //   at 128 channels from 218 boards), or for a batch that gives each
    //   CU one workgroup.
    // - Smaller layers spread a board's column groups over waves and
    //   workgroups instead, so a batch of 1 at 128 channels still runs 48
    //   workgroups at 19x19.
    const int coBlocks = ceilDiv(cout, kCoBlock);
    const int groups = ceilDiv(boardSize * boardSize, 16);
    const long tiles = (long)B * coBlocks * groups;
    const long cus = deviceCUs();
    // Small layers with the GPU to themselves: the shape of one block of 16
    // channels and 3, 6 or 12 column groups per workgroup (3 waves of one
    // group, 6 of one, 6 of two), the first whose workgroups still fit one
    // per CU and, past the first, fill at least 70% of the CUs (a shape that
    // leaves a third of the CUs idle loses: 19x19 at 192 channels, 6 boards,
    // 1.56x the best). The 6-wave shapes need the board's column groups to
    // fill their slots (all but one): on 5x5 and 9x9 boards the rest would
    // idle. One such workgroup per CU beats the 4- and 8-wave shapes by
    // 3-8% per layer (19x19 10x128 at batch 8: 12.95 against 13.59 us; 9x9
    // 6x64 at 64 boards: 7.43 against 7.95) and whole passes by 2.5-8%; over
    // boards 5-19, 32-256 channels and batches 1-192 the layer rule lands
    // within 1.4% of the best of the 13 shapes on average (3.0% with
    // another pass in flight, 4.3% without the three small shapes). With
    // another pass in flight they lose up to 20% of the two passes' rate
    // (both fill every CU), so there only the 3-wave shape is taken, while
    // its workgroups fill at most half the CUs (19x19
    // 10x128 at batch 1 and 2: passes 5-6% shorter, 13-14% more positions/s
    // with two in flight; 19x19 20x256 at batch 1 7% and 21%; 9x9 6x64 at 8
    // and 16 boards 4% and 8-13%).
    if (alone) {
        for (const ConvTiling t : {ConvTiling{1, 1, 3, 1}, ConvTiling{1, 1, 6, 1}, ConvTiling{1, 1, 6, 2}}) {
            if (t.wavesPg > 3 && t.wavesPg * t.pgPerWave > groups + 1) continue;
            const long w = convWorkgroups(t, cout, B, boardSize);
            if (w <= cus && (t.wavesPg == 3 || 10 * w >= 7 * cus)) return t;
        }
    } else {
        const ConvTiling t{1, 1, 3, 1};
        if (2 * convWorkgroups(t, cout, B, boardSize) <= cus) return t;
    }
    if (boardSize >= 19) {
        // One round of one 4-wave workgroup per CU, or nearly: the
        // whole-board shape (128 boards at 128 channels: 104.8 us per layer
        // against 114 for the next best).
        const long wholeWorkgroups = (long)B * ceilDiv(coBlocks, 4);
        if (coBlocks >= 4 && wholeWorkgroups <= cus && 10 * wholeWorkgroups >= 9L * cus)
            return {1, 4, 1, 0};
        if (tiles >= 40000) {
            if (coBlocks >= 4) return {1, 4, 1, 0};
            if (coBlocks >= 2) return {1, 2, 1, 0};
            return {1, 1, 1, 0};
        }
        // 4 waves of 6 column groups cover a 19x19 board's 23 in one workgroup.
        if (tiles >= 3072) return {1, 1, 4, 6};
        if (tiles >= 1536) return {1, 1, 4, 2};
        if (tiles >= 1024) return {1, 1, 8, 1};
        return {1, 1, 4, 1};
    }
    const long need = (long)(groups <= 2 ? 2 : 3) * cus;   // waves
    for (const ConvTiling t : {ConvTiling{1, 4, 1, 0}, ConvTiling{1, 2, 1, 0}, ConvTiling{1, 1, 1, 0}}) {
        if (t.wavesCo > 1 && coBlocks < t.wavesCo) continue;
        const long waves = (long)B * ceilDiv(coBlocks, t.wavesCo) * t.wavesCo;
        if (waves >= need) return t;
    }
    if (groups <= 8 && tiles >= 1024) return {1, 1, 4, 2};
    return {1, 1, 4, 1};
}

ConvTiling chooseStemTiling(ConvTiling tower, int cout, int B) {
    // The stem's whole-board body stages a board's planes once per
    // workgroup: with eight waves (128 channels) instead of four, once per
    // board, as soon as the batch still gives every CU a workgroup (19x19
    // 18 -> 128 planes at 256 boards: 41.7 against 44.2 us; 18 -> 256 at
    // 512: 157.8 against 161.6; at 128 boards, half the CUs idle: 38.6
    // against 26.6).
    if (tower == ConvTiling{1, 4, 1, 0} && ceilDiv(cout, kCoBlock) >= 8 &&
        (long)B * ceilDiv(cout, 8 * kCoBlock) >= deviceCUs())
        return {1, 8, 1, 0};
    return tower;
}

bool residentTowerSupported(int boardSize, int F, int P) {
    // Built for 19x19 (azh_conv_inst.hip); 8 waves of 16 channels, all but
    // the last block of them full; the stem's planes in two chunks.
    return boardSize == 19 && F > 112 && F <= 128 && P >= 1 && P <= 2 * kChunk;
}

hipError_t launchResidentTower(const ResidentTower& t, int boardSize, int workgroups, hipStream_t stream) {
    if (!residentTowerSupported(boardSize, t.F, t.in ? t.P : 1) || t.layers < 0 || workgroups < 1 ||
        workgroups > t.B || !t.x || !t.mid || (t.layers > 0 && !t.w0) ||
        (t.in && (!t.stemW || !t.stemScale || !t.stemShift)))
        return hipErrorInvalidValue;
    return launchResidentTowerT<19>(t, workgroups, stream);
}

hipError_t launchConv3x3(const float* x, const float* wPacked, const float* scale, const float* shift,
                         const float* skip, float* y, int B, int n, int cin, int cout, bool relu, bool planarInput,
                         ConvTiling t, hipStream_t stream) {
    // A launch needs at least one input channel (one K chunk) and one
    // output channel: the kernel reads the weights of chunk 0.
    if (cin < 1 || cout < 1) return hipErrorInvalidValue;
    if (B < 1) return hipSuccess;
    switch (n) {
    case 5: return launchConvN<5>(x, wPacked, scale, shift, skip, y, B, cin, cout, relu, planarInput, t, stream);
    case 9: return launchConvN<9>(x, wPacked, scale, shift, skip, y, B, cin, cout, relu, planarInput, t, stream);
    case 13: return launchConvN<13>(x, wPacked, scale, shift, skip, y, B, cin, cout, relu, planarInput, t, stream);
    case 19: return launchConvN<19>(x, wPacked, scale, shift, skip, y, B, cin, cout, relu, planarInput, t, stream);
    default: return hipErrorInvalidValue;
    }
}

std::vector<float> toChannelQuads(const float* planar, int B, int C, int A) {
    const int Q = channelQuads(C);
    std::vector<float> out(quadFloats(B, C, A), 0.0f);
    for (int b = 0; b < B; ++b)
        for (int c = 0; c < C; ++c)
            for (int p = 0; p < A; ++p)
                out[(((size_t)b * Q + c / 4) * A + p) * 4 + c % 4] = planar[((size_t)b * C + c) * A + p];
    return out;
}

void fromChannelQuads(const float* quads, int B, int C, int A, float* planar) {
    const int Q = channelQuads(C);
    for (int b = 0; b < B; ++b)
        for (int c = 0; c < C; ++c)
            for (int p = 0; p < A; ++p)
                planar[((size_t)b * C + c) * A + p] = quads[(((size_t)b * Q + c / 4) * A + p) * 4 + c % 4];
}

hipError_t launchHeads(const float* trunk, const HeadWeights& w, float* act, float* logits, float* values,
                       float* own, int B, int n, int F, int V, hipStream_t stream) {
    if (B < 1) return hipSuccess;
    if (V > 256) return hipErrorInvalidValue;
    const int A = n * n, A1 = A + 1;
    // A small batch spreads each position's points over up to three
    // workgroups, so more CUs read the trunk (19x19 at batch 1: three of 128
    // threads instead of one of 384); the same per-point arithmetic either way.
    const int slices = std::max(1, std::min(3, (int)(deviceCUs() / (2L * B))));
    const int threads = ceilDiv(ceilDiv(A, slices), 64) * 64;
    const dim3 grid1(B, ceilDiv(A, threads)), grid2(ceilDiv(B, kFcBoards), ceilDiv(A1, kFcOutTile) + 1);
    const dim3 block1(threads), block2(256);
    switch (n) {
#define AZH_HEADS(NN)                                                                                         \
    case NN:                                                                                                  \
        hipLaunchKernelGGL(headConvKernel<NN>, grid1, block1, 0, stream, trunk, w, act, own, F);             \
        hipLaunchKernelGGL(headFcKernel<NN>, grid2, block2, 0, stream, act, w, logits, values, B, V);        \
        break;
        AZH_HEADS(5)
        AZH_HEADS(9)
        AZH_HEADS(13)
        AZH_HEADS(19)
#undef AZH_HEADS
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

size_t headPolicyWTFloats(int n) { return (size_t)headPad16(2 * n * n) * headPad16(n * n + 1); }
size_t headFc1WTFloats(int n, int V) { return (size_t)headPad16(n * n) * headPad16(V); }

hipError_t launchSoftmaxLegal(const float* logits, const uint8_t* legal, float* priors, int B, int actions,
                              hipStream_t stream) {
    return launchPriors(logits, legal, nullptr, nullptr, priors, B, actions, 0, stream);
}

hipError_t launchSpin(unsigned long long nanoseconds, hipStream_t stream) {
    int khz = 0;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev);
    if (e != hipSuccess) return e;
    if (khz <= 0) khz = 100000;
    const unsigned long long ticks = nanoseconds * (unsigned long long)khz / 1000000ull;
    hipLaunchKernelGGL(spinKernel, dim3(1), dim3(1), 0, stream, ticks);
    return hipGetLastError();
}

hipError_t launchMfmaChains(float* out, int workgroups, int chain, hipStream_t stream) {
    if (workgroups < 1 || chain < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mfmaChainKernel, dim3(workgroups), dim3(kMfmaChainThreads), 0, stream, out, chain);
    return hipGetLastError();
}

hipError_t launchFill(float* data, size_t n, float value, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(fillKernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, data, n, value);
    return hipGetLastError();
}

} // namespace azh
