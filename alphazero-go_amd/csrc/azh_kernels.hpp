// Kernel interface of the MI355X (gfx950) inference pass: launchers for the
// fused 3x3 convolution, the fused heads and the legal-move softmax, plus
// the host-side weight packing the convolution reads.
//
// Activations live in HBM board-major: [B][C][n*n] fp32, one contiguous
// plane of n*n points per (position, channel). The network input arrives in
// exactly that layout ([B][planes][n*n], Evaluator::evaluate's input,
// include/azgo/evaluator.hpp:24), so the stem reads it in place.
#pragma once
#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>
#include <vector>

namespace azh {

// Channels per K chunk of the convolution: 4 groups of 4 channels.
constexpr int kChunk = 16;
// Output channels per MFMA block (v_mfma_f32_16x16x4_f32: 16 x 16 outputs).
constexpr int kCoBlock = 16;

inline int ceilDiv(int a, int b) { return (a + b - 1) / b; }

// Output-channel blocks of packed weights: ceil(cout/16) rounded up to whole
// 128-channel workgroup tiles, so no workgroup shape reads past them.
inline int packedCoBlocks(int cout) { return ceilDiv(ceilDiv(cout, kCoBlock), 8) * 8; }

// A 3x3 convolution's weights w [cout][cin][3][3] (Conv2d::w,
// include/azgo/layers.hpp:32, row (c*3 + dy)*3 + dx) packed as the MFMA A
// fragments the kernel loads: [co block][chunk q][tap t][lane 0..63][j 0..3],
// value w[cb*16 + (lane & 15)][q*16 + 4*(lane >> 4) + j][t], zero where the
// output or input channel is padding. co blocks = packedCoBlocks(cout),
// chunks = ceil(cin/16).
std::vector<float> packConv3x3(const float* w, int cin, int cout);
size_t packedConv3x3Floats(int cin, int cout);

// How a convolution launch is cut: output channels per workgroup (a
// multiple of 16) and the resulting number of co tiles. The cut only
// decides which workgroup computes an output, never how: every output
// channel sums its inputs in one fixed order (chunk, tap, channel-in-chunk),
// so results are bitwise independent of the cut and of the batch.
struct ConvTiling {
    int coPerWave;   // MFMA blocks of 16 output channels per wave: 1 or 2
    int wavesCo;     // waves along the output channels (at most 128 channels per workgroup)
    int wavesPg;     // waves along the board's 16-point column groups
    int pgPerWave;   // column groups per wave; 0: all of the board's
    int waves() const { return wavesCo * wavesPg; }
    int coTile() const { return 16 * coPerWave * wavesCo; }
};
ConvTiling chooseConvTiling(int cout, int B, int boardSize);
inline constexpr bool operator==(const ConvTiling& a, const ConvTiling& b) {
    return a.coPerWave == b.coPerWave && a.wavesCo == b.wavesCo && a.wavesPg == b.wavesPg &&
           a.pgPerWave == b.pgPerWave;
}

// The workgroup shapes the convolution is built for, in the order a probe
// indexes them. Each is compiled for every supported board size.
constexpr ConvTiling kConvTilings[] = {{2, 2, 2, 12}, {1, 4, 1, 0}, {1, 2, 1, 0}, {1, 1, 1, 0}, {1, 8, 1, 0},
                                       {1, 2, 2, 12}, {1, 1, 4, 6}, {1, 1, 4, 2}, {1, 1, 4, 1}, {1, 1, 8, 1}};
constexpr int kConvTilingCount = sizeof kConvTilings / sizeof kConvTilings[0];

// One (board size, workgroup shape) instance of the convolution; defined in
// azh_conv.hpp and instantiated by azh_conv_inst.hip, one object per shape.
template <int N, int COW, int WCO, int WPG, int PPW>
hipError_t launchConvT(const float* x, const float* wp, const float* scale, const float* shift, const float* skip,
                       float* y, int B, int cin, int cout, bool relu, hipStream_t stream);

// y[b][co][p] = relu?( (scale[co] * conv(x)[b][co][p] + shift[co]) (+ skip[b][co][p]) )
// with each multiply and add rounded separately (BatchNorm2d::forwardInfer,
// src/layers.cpp:88-97, then the skip add and reluForward,
// src/network.cpp:264-271). skip may alias y (in-place residual).
// x [B][cin][n*n], y and skip [B][cout][n*n].
hipError_t launchConv3x3(const float* x, const float* wPacked, const float* scale, const float* shift,
                         const float* skip, float* y, int B, int n, int cin, int cout, bool relu, ConvTiling tiling,
                         hipStream_t stream);
bool conv3x3Supported(int boardSize);

// y = relu?(scale * acc + shift (+ skip)), each operation rounded on its own.
__device__ inline float epilogue(float acc, float s, float h, bool addSkip, float skipv, bool relu) {
    float v = __fadd_rn(__fmul_rn(s, acc), h);
    if (addSkip) v = __fadd_rn(v, skipv);
    if (relu) v = v > 0.0f ? v : 0.0f;   // -0 and NaN become +0 (reluForward)
    return v;
}

// The heads (src/network.cpp:274-308), two kernels: the 1x1 convs F -> 2
// (policy) and F -> 1 (value) with BN and ReLU, one position per workgroup,
// into act [B][3][n*n], and, when the network has it, the ownership head's
// 1x1 conv F -> 1 with BN and tanh straight into own [B][n*n]; then the
// policy Linear (2A -> A+1) and the value Linears (A -> V, ReLU, V -> 1) and
// tanh as MFMA GEMMs, 16 positions per workgroup. V at most 256.
struct HeadWeights {
    const float* convW;      // [4][F]: policy rows 0-1, value row 2, ownership row 3
    const float* scale;      // [4] folded BN scale
    const float* shift;      // [4] folded BN shift
    const float* policyWT;   // [pad16(2A)][pad16(A+1)]: policy.fc.w transposed, zero-padded
    const float* policyB;    // [A+1]
    const float* fc1WT;      // [pad16(A)][pad16(V)]: value.fc1.w transposed, zero-padded
    const float* fc1B;       // [V]
    const float* fc2W;       // [V]
    const float* fc2B;       // [1]
};
size_t headPolicyWTFloats(int n);
size_t headFc1WTFloats(int n, int V);
hipError_t launchHeads(const float* trunk, const HeadWeights& w, float* act, float* logits, float* values,
                       float* own, int B, int n, int F, int V, hipStream_t stream);

// priors[b][a] = exp(l - max) / sum over legal a of the same, 0 where
// illegal (Mcts::expand's softmax, src/mcts.cpp:170-183). One wavefront per
// position. legal [B][actions] bytes (nonzero = legal).
hipError_t launchSoftmaxLegal(const float* logits, const uint8_t* legal, float* priors, int B, int actions,
                              hipStream_t stream);

// ---- the steps either side of the pass (azh_positions.hip)

// encodePlanes (src/encode.cpp:14-43) for B positions: stones [B][H][n*n]
// Color bytes (ply k = k moves ago, 0 = now), plies[b] of them present
// (1..H; the rest are zero planes), toMove[b] 1 (Black) or 2 (White),
// sym[b] 0..7 (NULL: identity) -> planes [B][2H+2][n*n].
hipError_t launchEncodePlanes(const uint8_t* stones, const int* plies, const uint8_t* toMove, const uint8_t* sym,
                              float* planes, int B, int n, int H, hipStream_t stream);

// The legal actions of Mcts::expand (src/mcts.cpp:152-169) for B positions:
// board b's stones at stones + b * stride (n*n Color bytes), toMove[b];
// Board::isLegal plus positional superko against seen[seenOffsets[b] ..
// seenOffsets[b+1]). legal [B][n*n+1] bytes, pass always 1. One workgroup
// of 512 threads per position.
hipError_t launchLegalMoves(const uint8_t* stones, size_t stride, const uint8_t* toMove, const uint64_t* seen,
                            const long long* seenOffsets, uint8_t* legal, int B, int n, hipStream_t stream);

// The priors of Mcts::evaluateLeaves + expand (src/mcts.cpp:136-146,
// 170-183): the logits mapped back from symmetry sym[b] (NULL: identity;
// action a reads logit transformAction(sym, a)), into mapped when not NULL,
// then the softmax over the legal actions, into priors. actions = n*n + 1
// when sym is given.
hipError_t launchPriors(const float* logits, const uint8_t* legal, const uint8_t* sym, float* mapped, float* priors,
                        int B, int actions, int n, hipStream_t stream);

// Test hooks: holds the stream for about `nanoseconds` (a bounded wait on the
// wall clock), and fills data[0..n) with value.
hipError_t launchSpin(unsigned long long nanoseconds, hipStream_t stream);
hipError_t launchFill(float* data, size_t n, float value, hipStream_t stream);

} // namespace azh
