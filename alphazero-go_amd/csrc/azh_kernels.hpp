// Kernel interface of the MI355X (gfx950) inference pass: the fused 3x3
// convolution (azh_conv_iface.hpp), the fused heads, the legal-move softmax,
// and the steps either side of the pass (encoding, legal moves, priors).
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

#include "azh_conv_iface.hpp"

namespace azh {

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
// Compute units of the current device (cached; 256 if the query fails).
int deviceCUs();

// The whole residual tower of a 5x5, 9x9 or 13x13 board of up to 64
// channels (as LDS allows) in one launch, one workgroup per board with its activations in LDS
// (azh_small_tower.hip):
// `layers` (even) convolutions on trunk [B][ceil(F/4)][n*n] quads in place,
// layer l's packed weights at w0 + l * layerStride floats and its BN scale
// and shift at scaleOff and shiftOff floats after them. The same bits as
// the per-layer launches. smallTowerLdsBytes: the LDS a workgroup needs (0
// for other boards); launches need at most kSmallTowerMaxLds.
// With a stem, the launch first runs the stem convolution from the
// network's input planes [B][planes][n*n] (its packed weights, BN scale and
// shift) into the trunk, as conv3x3Stem does; without one (nullptr or in ==
// nullptr) it reads the trunk.
constexpr size_t kSmallTowerMaxLds = 64 * 1024;
constexpr int kSmallTowerMaxChunks = 4;   // up to 64 channels: one channel block per wave
struct SmallStem {
    const float* in = nullptr;
    const float* w = nullptr;
    const float* scale = nullptr;
    const float* shift = nullptr;
    int planes = 0;
};
// With heads (logits set), the launch ends with the heads on the board's
// trunk, as launchHeads computes them: logits [B][n*n+1], values [B], and
// with own set the ownership [B][n*n]; the trunk is written back either way.
struct SmallHeads {
    HeadWeights w{};
    float* logits = nullptr;
    float* values = nullptr;
    float* own = nullptr;
    int V = 0;
};
size_t smallTowerLdsBytes(int n, int F, int planes, bool heads, int V);
hipError_t launchSmallTower(float* trunk, const SmallStem* stem, const SmallHeads* heads, const float* w0,
                            size_t layerStride, size_t scaleOff, size_t shiftOff, int layers, int B, int n, int F,
                            hipStream_t stream);
// Workgroups of one convolution launch of shape t over B boards of
// boardSize x boardSize with cout output channels (the launcher's grid).
long convWorkgroups(ConvTiling t, int cout, int B, int boardSize);

// The heads on a trunk of F channels in channel quads (azh_conv_iface.hpp).
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

// The fp32 matrix units' rate with nothing else in the way: `workgroups`
// workgroups of kMfmaChainThreads threads, each wave a dependent chain of
// 4 * chain 16x16x4 MFMAs (2048 flops each); out holds one float per thread.
constexpr int kMfmaChainThreads = 512;
hipError_t launchMfmaChains(float* out, int workgroups, int chain, hipStream_t stream);

} // namespace azh
