// The steps either side of the network pass, on the GPU: the positions'
// input planes (encodePlanes), the legal moves with positional superko
// (Board::isLegal + hashAfter, as Mcts::expand builds its edges), and the
// priors (the policy mapped back from the symmetry the network saw, then the
// softmax over the legal moves). All of it integer and byte work except the
// softmax; every output element is written by exactly one thread.
#include "azh_kernels.hpp"

#include <hip/hip_runtime.h>
#include <cmath>

namespace azh {

namespace {

// The padded board of include/azgo/board.hpp:21-24: rows of 21 cells, one
// sentinel column each side of the largest (19 x 19) board; a smaller board
// sits in the top-left corner and every other cell is Off.
constexpr int kStride = 21;
constexpr int kCells = kStride * kStride;
constexpr int kEmpty = 0, kBlack = 1, kWhite = 2, kOff = 3;

// transformPoint (src/symmetry.cpp:6-19): mirror left-right first when
// sym & 4, then sym & 3 clockwise quarter turns.
__device__ inline int transformPoint(int sym, int p, int n) {
    int row = p / n, col = p - (p / n) * n;
    if (sym & 4) col = n - 1 - col;
    for (int t = 0; t < (sym & 3); ++t) {
        const int r = col;
        col = n - 1 - row;
        row = r;
    }
    return row * n + col;
}

// inverseSymmetry (src/symmetry.cpp:25-33): mirrored transforms are their
// own inverse; k turns are undone by 4 - k.
__device__ inline int inverseSymmetry(int sym) { return (sym & 4) ? sym : (4 - sym) & 3; }

// ------------------------------------------------------------------ encodePlanes

// out[b][plane][q] for plane < 2H: ply k = plane / 2 of the history, "own"
// (plane even: the side to move now) or "opponent" stones, present when
// k < plies[b]; planes 2H and 2H + 1: all ones for Black / White to move
// (src/encode.cpp:14-43). encodePlanes scatters point p to
// transformPoint(sym, p); this gathers q from transformPoint(sym^-1, q),
// the same permutation, so each output is written once, coalesced.
__global__ __launch_bounds__(256) void encodePlanesKernel(const uint8_t* __restrict__ stones,
                                                          const int* __restrict__ plies,
                                                          const uint8_t* __restrict__ toMove,
                                                          const uint8_t* __restrict__ sym, float* __restrict__ planes,
                                                          int n, int H) {
    const int b = blockIdx.y;
    const int A = n * n, P = 2 * H + 2;
    const int me = toMove[b], them = me == kBlack ? kWhite : kBlack;
    const int present = plies[b] < H ? plies[b] : H;
    const int inv = inverseSymmetry(sym ? sym[b] : 0);
    const uint8_t* sb = stones + (size_t)b * H * A;
    float* ob = planes + (size_t)b * P * A;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < P * A; i += gridDim.x * blockDim.x) {
        const int plane = i / A, q = i - plane * A;
        float v;
        if (plane < 2 * H) {
            const int k = plane >> 1;
            v = 0.0f;
            if (k < present) {
                const int s = sb[(size_t)k * A + transformPoint(inv, q, n)];
                v = s == ((plane & 1) ? them : me) ? 1.0f : 0.0f;
            }
        } else {
            v = (plane == 2 * H) == (me == kBlack) ? 1.0f : 0.0f;
        }
        ob[i] = v;
    }
}

// ------------------------------------------------------------------ legal moves

// Zobrist key of (padded cell, colour) (src/board.cpp:19-33): the table is
// one splitmix64 stream seeded 0x5EEDB0A4D5EEDB0A, black then white per
// cell, and splitmix64's m-th output is mix(seed + m * gamma) (Steele, Lea &
// Flood, "Fast splittable pseudorandom number generators", 2014), so any
// key is computed directly.
__device__ inline uint64_t zobristKey(int cell, int color) {
    uint64_t z = 0x5EEDB0A4D5EEDB0AULL + (uint64_t)(2 * cell + (color == kWhite ? 1 : 0) + 1) * 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

constexpr int kLegalThreads = 512;   // one thread per padded cell (441), the rest idle

// One workgroup per position, one thread per padded cell, all in LDS:
//  1. groups: every stone's label converges to the smallest cell index of
//     its group (minimum over same-coloured neighbours plus one pointer
//     jump per round; at most one round per stone of the longest path, so
//     the bound of kCells + 1 rounds is never reached);
//  2. liberties: each empty cell adds one to each distinct group beside it
//     (exact counts, as countLiberties with no limit); group and board
//     Zobrist hashes: XOR of the keys of their stones;
//  3. each empty point is legal (Board::isLegal, src/board.cpp:131-150) if a
//     neighbour is empty, or an opponent group beside it has one liberty
//     (which is this point: it is captured), or a friendly group beside it
//     has two or more; the hash after the move (Board::hashAfter,
//     src/board.cpp:176-190) is the board's and the new stone's key XORed,
//     and, when an opponent group beside it has one liberty (hashAfter then
//     plays the move, src/board.cpp:152-174), the hashes of every opponent
//     group beside it left without liberties: those with one liberty, and
//     those with none already (only on boards no game reaches);
//  4. positional superko (src/mcts.cpp:161-166): a move whose hash after is
//     in the position's seen list is not legal. Pass always is.
__global__ __launch_bounds__(kLegalThreads) void legalMovesKernel(const uint8_t* __restrict__ stones, size_t stride,
                                                                  const uint8_t* __restrict__ toMove,
                                                                  const unsigned long long* __restrict__ seen,
                                                                  const long long* __restrict__ seenOffsets,
                                                                  uint8_t* __restrict__ legal, int n) {
    __shared__ int cell[kCells];
    __shared__ int lab[kCells];
    __shared__ int libs[kCells];
    __shared__ unsigned ghash[2 * kCells];
    __shared__ unsigned bhash[2];
    __shared__ int flag[3];
    __shared__ unsigned long long chunk[kLegalThreads];
    const int b = blockIdx.x, t = threadIdx.x, A = n * n;
    const int me = toMove[b], them = me == kBlack ? kWhite : kBlack;
    const int row = t / kStride - 1, col = t - (t / kStride) * kStride - 1;
    const bool isCell = t < kCells;
    const bool onBoard = isCell && row >= 0 && row < n && col >= 0 && col < n;
    const int point = row * n + col;
    const int dirs[4] = {-kStride, -1, 1, kStride};

    int c = kOff;
    if (isCell) {
        c = onBoard ? stones[(size_t)b * stride + point] : kOff;
        cell[t] = c;
        libs[t] = 0;
        ghash[2 * t] = 0;
        ghash[2 * t + 1] = 0;
    }
    const bool stone = c == kBlack || c == kWhite;
    if (isCell) lab[t] = stone ? t : kCells;
    if (t < 2) bhash[t] = 0;
    if (t < 3) flag[t] = 0;
    __syncthreads();

    // 1. Labels. Round r sets flag[r % 3]; the flag of round r + 1 is cleared
    //    during round r, which every thread's read of it (two rounds
    //    earlier) precedes by a barrier.
    for (int r = 0; r <= kCells; ++r) {
        const int f = r % 3;
        if (t == 0) flag[(r + 1) % 3] = 0;
        if (stone) {
            const int mine = lab[t];
            int m = mine;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const int q = t + dirs[d];
                if (cell[q] == c) m = min(m, lab[q]);
            }
            m = min(m, lab[m]);   // m is a stone of this group: its label is valid
            if (m < mine) {
                lab[t] = m;
                flag[f] = 1;
            }
        }
        __syncthreads();
        if (!flag[f]) break;   // the same value for every thread: read after the barrier
    }

    // 2. Liberties and hashes.
    if (onBoard && c == kEmpty) {
        int counted[4], nc = 0;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const int q = t + dirs[d], cq = cell[q];
            if (cq == kBlack || cq == kWhite) {
                const int L = lab[q];
                bool dup = false;
                for (int j = 0; j < nc; ++j) dup |= counted[j] == L;
                if (!dup) {
                    counted[nc++] = L;
                    atomicAdd(&libs[L], 1);
                }
            }
        }
    }
    if (stone) {
        const uint64_t k = zobristKey(t, c);
        atomicXor(&ghash[2 * lab[t]], (unsigned)k);
        atomicXor(&ghash[2 * lab[t] + 1], (unsigned)(k >> 32));
        atomicXor(&bhash[0], (unsigned)k);
        atomicXor(&bhash[1], (unsigned)(k >> 32));
    }
    __syncthreads();

    // 3. Board::isLegal and the hash after the move.
    bool ok = false;
    unsigned long long h = 0;
    if (onBoard && c == kEmpty) {
        int caps[4], ncap = 0;
        bool atari = false;   // an opponent group beside the point has exactly one liberty
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const int q = t + dirs[d], cq = cell[q];
            if (cq == kEmpty) {
                ok = true;
            } else if (cq == them) {
                const int L = lab[q];
                if (libs[L] == 1) ok = atari = true;
                if (libs[L] <= 1) {
                    bool dup = false;
                    for (int j = 0; j < ncap; ++j) dup |= caps[j] == L;
                    if (!dup) caps[ncap++] = L;
                }
            } else if (cq == me) {
                if (libs[lab[q]] >= 2) ok = true;
            }
        }
        if (ok) {
            h = ((unsigned long long)bhash[1] << 32 | bhash[0]) ^ zobristKey(t, me);
            if (atari)
                for (int j = 0; j < ncap; ++j)
                    h ^= (unsigned long long)ghash[2 * caps[j] + 1] << 32 | ghash[2 * caps[j]];
        }
    }

    // 4. Superko against the position's seen hashes, staged through LDS.
    const long long s0 = seenOffsets[b], s1 = seenOffsets[b + 1];
    for (long long base = s0; base < s1; base += kLegalThreads) {
        const int cnt = (int)min((long long)kLegalThreads, s1 - base);
        __syncthreads();
        if (t < cnt) chunk[t] = seen[base + t];
        __syncthreads();
        if (ok)
            for (int i = 0; i < cnt; ++i) ok &= chunk[i] != h;
    }
    uint8_t* lb = legal + (size_t)b * (A + 1);
    if (onBoard) lb[point] = ok ? 1 : 0;
    if (t == 0) lb[A] = 1;
}

// ------------------------------------------------------------------ priors

// One wavefront per position. With sym, the logits come back from the
// transformed board first (Mcts::evaluateLeaves, src/mcts.cpp:136-146:
// action a reads the logit of transformAction(sym, a); pass stays); then
// the softmax over the legal actions (Mcts::expand, src/mcts.cpp:170-183):
// the maximum legal logit subtracted, exp, divided by the sum over legal.
// mapped (optional) receives the mapped-back logits.
__global__ __launch_bounds__(256) void priorsKernel(const float* __restrict__ logits, const uint8_t* __restrict__ legal,
                                                    const uint8_t* __restrict__ sym, float* __restrict__ mapped,
                                                    float* __restrict__ priors, int B, int actions, int n) {
    const int pos = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (pos >= B) return;   // a whole wave leaves together
    const float* l = logits + (size_t)pos * actions;
    const uint8_t* m = legal + (size_t)pos * actions;
    float* o = priors + (size_t)pos * actions;
    const int s = sym ? sym[pos] : 0;
    const int area = actions - 1;
    auto logit = [&](int a) { return l[(s == 0 || a == area) ? a : transformPoint(s, a, n)]; };
    if (mapped)
        for (int a = lane; a < actions; a += 64) mapped[(size_t)pos * actions + a] = logit(a);
    float mx = -INFINITY;
    for (int a = lane; a < actions; a += 64)
        if (m[a]) mx = fmaxf(mx, logit(a));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if (mx == -INFINITY) {   // no legal action: nothing to normalise
        for (int a = lane; a < actions; a += 64) o[a] = 0.0f;
        return;
    }
    float sum = 0.0f;
    for (int a = lane; a < actions; a += 64)
        if (m[a]) sum += expf(logit(a) - mx);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    for (int a = lane; a < actions; a += 64) o[a] = m[a] ? expf(logit(a) - mx) / sum : 0.0f;
}

// The same priors with a lane's actions (a = lane + 64u, u < PER) held in
// registers: every logit and legal byte is loaded once, all of them before
// the first reduction, and each exp is computed once. Same arithmetic in
// the same order as priorsKernel (per-lane partial sums in a ascending,
// then the same butterfly), so the same bits; for actions <= 64 * PER.
template <int PER>
__global__ __launch_bounds__(256) void priorsRegsKernel(const float* __restrict__ logits,
                                                        const uint8_t* __restrict__ legal,
                                                        const uint8_t* __restrict__ sym, float* __restrict__ mapped,
                                                        float* __restrict__ priors, int B, int actions, int n) {
    const int pos = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (pos >= B) return;   // a whole wave leaves together
    const float* l = logits + (size_t)pos * actions;
    const uint8_t* m = legal + (size_t)pos * actions;
    float* o = priors + (size_t)pos * actions;
    const int s = sym ? sym[pos] : 0;
    const int area = actions - 1;
    float v[PER];
    bool ok[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        const int a = lane + 64 * u;
        const int at = a < actions ? a : 0;   // lanes past the actions read action 0, unused
        v[u] = l[(s == 0 || at == area) ? at : transformPoint(s, at, n)];
        ok[u] = a < actions && m[at] != 0;
    }
    if (mapped) {
#pragma unroll
        for (int u = 0; u < PER; ++u)
            if (lane + 64 * u < actions) mapped[(size_t)pos * actions + lane + 64 * u] = v[u];
    }
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < PER; ++u)
        if (ok[u]) mx = fmaxf(mx, v[u]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if (mx == -INFINITY) {   // no legal action: nothing to normalise
#pragma unroll
        for (int u = 0; u < PER; ++u)
            if (lane + 64 * u < actions) o[lane + 64 * u] = 0.0f;
        return;
    }
    float e[PER];
    float sum = 0.0f;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        e[u] = ok[u] ? expf(v[u] - mx) : 0.0f;
        if (ok[u]) sum += e[u];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
#pragma unroll
    for (int u = 0; u < PER; ++u)
        if (lane + 64 * u < actions) o[lane + 64 * u] = ok[u] ? e[u] / sum : 0.0f;
}

} // namespace

hipError_t launchEncodePlanes(const uint8_t* stones, const int* plies, const uint8_t* toMove, const uint8_t* sym,
                              float* planes, int B, int n, int H, hipStream_t stream) {
    if (B < 1) return hipSuccess;
    if (n < 5 || n > 19 || H < 1) return hipErrorInvalidValue;
    const int work = (2 * H + 2) * n * n;
    const dim3 grid(ceilDiv(work, 256), B);
    hipLaunchKernelGGL(encodePlanesKernel, grid, dim3(256), 0, stream, stones, plies, toMove, sym, planes, n, H);
    return hipGetLastError();
}

hipError_t launchLegalMoves(const uint8_t* stones, size_t stride, const uint8_t* toMove, const uint64_t* seen,
                            const long long* seenOffsets, uint8_t* legal, int B, int n, hipStream_t stream) {
    if (B < 1) return hipSuccess;
    if (n < 5 || n > 19 || stride < (size_t)n * n) return hipErrorInvalidValue;
    hipLaunchKernelGGL(legalMovesKernel, dim3(B), dim3(kLegalThreads), 0, stream, stones, stride, toMove,
                       reinterpret_cast<const unsigned long long*>(seen), seenOffsets, legal, n);
    return hipGetLastError();
}

hipError_t launchPriors(const float* logits, const uint8_t* legal, const uint8_t* sym, float* mapped, float* priors,
                        int B, int actions, int n, hipStream_t stream) {
    if (B < 1) return hipSuccess;
    if (sym && actions != n * n + 1) return hipErrorInvalidValue;
    // Up to 384 actions (every board up to 19x19 and its pass) from registers.
    if (actions <= 64 * 6)
        hipLaunchKernelGGL(priorsRegsKernel<6>, dim3(ceilDiv(B, 4)), dim3(256), 0, stream, logits, legal, sym, mapped,
                           priors, B, actions, n);
    else
        hipLaunchKernelGGL(priorsKernel, dim3(ceilDiv(B, 4)), dim3(256), 0, stream, logits, legal, sym, mapped, priors,
                           B, actions, n);
    return hipGetLastError();
}

} // namespace azh
