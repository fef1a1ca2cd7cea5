// The 3x3 convolution's interface: weight packing, workgroup shapes, the
// launcher and its BN/skip/ReLU epilogue. Kept apart from the other
// kernels' declarations so that a hash of the convolution's sources (this
// file, azh_conv.hpp, azh_conv_inst.hip) changes only with the convolution.
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
// channel sums its inputs in one fixed order (chunk, tap, channel-in-chunk;
// the stem's short last chunk of input planes in its packed (plane, tap)
// order, azh_stem.hpp), so results are bitwise independent of the cut and
// of the batch.
struct ConvTiling {
    int coPerWave;   // MFMA blocks of 16 output channels per wave: 1 or 2
    int wavesCo;     // waves along the output channels (at most 128 channels per workgroup)
    int wavesPg;     // waves along the board's 16-point column groups
    int pgPerWave;   // column groups per wave; 0: all of the board's
    int waves() const { return wavesCo * wavesPg; }
    int coTile() const { return 16 * coPerWave * wavesCo; }
};
// alone: no other pass is in flight on the device (the runner's other slots
// idle), which admits the shapes that are fastest for one pass but slower
// for two side by side.
ConvTiling chooseConvTiling(int cout, int B, int boardSize, bool alone = false);
// The stem's shape in a pass whose tower runs `tower` over B boards in all
// (both halves of a split pass, which run at once).
ConvTiling chooseStemTiling(ConvTiling tower, int cout, int B);
inline constexpr bool operator==(const ConvTiling& a, const ConvTiling& b) {
    return a.coPerWave == b.coPerWave && a.wavesCo == b.wavesCo && a.wavesPg == b.wavesPg &&
           a.pgPerWave == b.pgPerWave;
}

// The workgroup shapes the convolution is built for, in the order a probe
// indexes them. Each is compiled for every supported board size.
constexpr ConvTiling kConvTilings[] = {{2, 2, 2, 12}, {1, 4, 1, 0}, {1, 2, 1, 0}, {1, 1, 1, 0}, {1, 8, 1, 0},
                                       {1, 2, 2, 12}, {1, 1, 4, 6}, {1, 1, 4, 2}, {1, 1, 4, 1}, {1, 1, 8, 1},
                                       {1, 1, 3, 1}, {1, 1, 6, 1}, {1, 1, 6, 2}};
constexpr int kConvTilingCount = sizeof kConvTilings / sizeof kConvTilings[0];

// Trunk activations (every convolution's output, the residual input and the
// tower's input) are stored in channel quads: [B][ceil(C/4)][n*n][4], the
// four channels 4g..4g+3 of a point side by side. A lane then moves four
// channels with one 16-byte access: the LDS staging wants exactly that
// interleave, and an MFMA lane's accumulators are four consecutive channels
// of one point. Channels past C in the last quad are stored as zeros. The
// network's input planes stay [B][P][n*n], as the reference hands them over.
inline int channelQuads(int channels) { return ceilDiv(channels, 4); }
inline size_t quadFloats(int B, int channels, int points) { return (size_t)B * channelQuads(channels) * 4 * points; }

// Reorders between the planar [B][C][A] layout and channel quads (zeros in
// the padding), on the host: for test hooks that take or return planar data.
std::vector<float> toChannelQuads(const float* planar, int B, int C, int A);
void fromChannelQuads(const float* quads, int B, int C, int A, float* planar);

// One (board size, workgroup shape) instance of the convolution; defined in
// azh_conv.hpp and instantiated by azh_conv_inst.hip, one object per shape.
template <int N, int COW, int WCO, int WPG, int PPW>
hipError_t launchConvT(const float* x, const float* wp, const float* scale, const float* shift, const float* skip,
                       float* y, int B, int cin, int cout, bool relu, bool planarInput, hipStream_t stream);

// y[b][co][p] = relu?( (scale[co] * conv(x)[b][co][p] + shift[co]) (+ skip[b][co][p]) )
// with each multiply and add rounded separately (BatchNorm2d::forwardInfer,
// src/layers.cpp:88-97, then the skip add and reluForward,
// src/network.cpp:264-271). skip may alias y (in-place residual).
// y and skip in channel quads. x: planarInput, the network's input planes
// [B][cin][n*n] (the stem); otherwise a trunk activation in channel quads.
hipError_t launchConv3x3(const float* x, const float* wPacked, const float* scale, const float* shift,
                         const float* skip, float* y, int B, int n, int cin, int cout, bool relu, bool planarInput,
                         ConvTiling tiling, hipStream_t stream);
bool conv3x3Supported(int boardSize);

// The stem and the residual tower in one launch, each board resident in one
// workgroup of 8 waves (128 output channels) from its first layer to its
// last: the per-layer launches' arithmetic without their kernel boundaries.
// For networks of 113-128 channels (every wave a block of 16) and stems of
// up to 32 planes, on the board sizes residentTowerSupported names.
struct ResidentTower {
    const float* in;   // the network's input planes [B][P][A]; null: no stem (x holds the tower's input)
    const float *stemW, *stemScale, *stemShift;   // the stem's packed weights and folded BN
    int P;
    float* x;     // the trunk (channel quads), in place
    float* mid;   // the blocks' middle activations
    // Tower layer l (conv1, conv2 of each block in turn): packed weights at
    // w0 + l * stride, its BN scale and shift scaleOff and shiftOff floats
    // after them.
    const float* w0;
    size_t stride, scaleOff, shiftOff;
    int layers, B, F;
};
bool residentTowerSupported(int boardSize, int F, int P);
// workgroups: at most B; each takes every workgroups-th board.
hipError_t launchResidentTower(const ResidentTower& t, int boardSize, int workgroups, hipStream_t stream);
template <int N>
hipError_t launchResidentTowerT(const ResidentTower& t, int workgroups, hipStream_t stream);

// y = relu?(scale * acc + shift (+ skip)), each operation rounded on its own.
__device__ inline float epilogue(float acc, float s, float h, bool addSkip, float skipv, bool relu) {
    float v = __fadd_rn(__fmul_rn(s, acc), h);
    if (addSkip) v = __fadd_rn(v, skipv);
    if (relu) v = v > 0.0f ? v : 0.0f;   // -0 and NaN become +0 (reluForward)
    return v;
}

} // namespace azh
