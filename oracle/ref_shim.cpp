// A C entry layer over the reference's own sources, compiled from the files
// where they lie in the reference tree (oracle/Makefile) into
// oracle/_ref/libazgo_ref.so. TEST INFRASTRUCTURE ONLY: tests use it to pin
// the oracle's restatement bit for bit (weights, encoding, the naive forward
// pass); the product never loads it.
//
// Only the naive backend is available: the reference's BLAS backend
// (src/backend_blas.cpp) needs <cblas.h>, which this image does not have.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "azgo/backend.hpp"
#include "azgo/bn_calibration.hpp"
#include "azgo/checkpoint.hpp"
#include "azgo/encode.hpp"
#include "azgo/game.hpp"
#include "azgo/layers.hpp"
#include "azgo/network.hpp"
#include "azgo/param_layout.hpp"
#include "azgo/rng.hpp"
#include "azgo/symmetry.hpp"

using namespace azgo;

extern "C" {

uint64_t ref_splitmix64(uint64_t* x) { return splitmix64(*x); }
uint64_t ref_derive_seed(uint64_t a, uint64_t b, uint64_t c, uint64_t d) { return deriveSeed(a, b, c, d); }

// n draws of kind (0 next, 1 uniform, 2 normal, 3 below(bound)) from Rng(seed), as doubles.
void ref_rng_draws(uint64_t seed, int kind, int bound, int n, double* out) {
    Rng r(seed);
    for (int i = 0; i < n; ++i) {
        switch (kind) {
        case 0: out[i] = static_cast<double>(r.next()); break;
        case 1: out[i] = r.uniform(); break;
        case 2: out[i] = r.normal(); break;
        default: out[i] = r.below(bound); break;
        }
    }
}
void ref_rng_next_u64(uint64_t seed, int n, uint64_t* out) {
    Rng r(seed);
    for (int i = 0; i < n; ++i) out[i] = r.next();
}

int ref_transform_point(int sym, int p, int n) { return transformPoint(sym, p, n); }

void ref_encode_planes(const uint8_t* stones, int count, int n, int toMove, int H, int sym, float* out) {
    std::vector<const uint8_t*> s;
    for (int k = 0; k < count; ++k) s.push_back(stones + static_cast<size_t>(k) * n * n);
    encodePlanes(s, n, toMove == 1 ? Color::Black : Color::White, H, sym, out);
}

void* ref_network_new(int board, int history, int blocks, int filters, int valueHidden, int ownership,
                      uint64_t seed) {
    NetConfig cfg;
    cfg.boardSize = board;
    cfg.history = history;
    cfg.blocks = blocks;
    cfg.filters = filters;
    cfg.valueHidden = valueHidden;
    cfg.ownership = ownership != 0;
    return new Network(cfg, seed);
}

void ref_network_free(void* net) { delete static_cast<Network*>(net); }

// Every tensor in ParamLayout order (params, then buffers): name, size, offset, arena.
int ref_layout_count(void* net) {
    ParamLayout l = ParamLayout::of(*static_cast<Network*>(net));
    return static_cast<int>(l.params.size() + l.buffers.size());
}
int ref_layout_entry(void* net, int i, char* name, size_t cap, size_t* size, size_t* offset, int* buffer) {
    ParamLayout l = ParamLayout::of(*static_cast<Network*>(net));
    const int np = static_cast<int>(l.params.size());
    const ParamLayout::Entry* e = i < np ? &l.params[i] : (i - np < static_cast<int>(l.buffers.size()) ? &l.buffers[i - np] : nullptr);
    if (!e) return -1;
    std::snprintf(name, cap, "%s", e->name.c_str());
    *size = e->size;
    *offset = e->offset;
    *buffer = i < np ? 0 : 1;
    return 0;
}
void ref_layout_sizes(void* net, size_t* paramFloats, size_t* bufferFloats) {
    ParamLayout l = ParamLayout::of(*static_cast<Network*>(net));
    *paramFloats = l.paramFloats;
    *bufferFloats = l.bufferFloats;
}

// Copies a tensor out of / into the network by name. Returns its size, or -1.
long ref_tensor_get(void* net, const char* name, float* out) {
    Network& n = *static_cast<Network*>(net);
    for (const ParamView& p : n.params())
        if (p.name == name) {
            if (out) std::memcpy(out, p.value, p.size * sizeof(float));
            return static_cast<long>(p.size);
        }
    for (const BufferView& b : n.buffers())
        if (b.name == name) {
            if (out) std::memcpy(out, b.value, b.size * sizeof(float));
            return static_cast<long>(b.size);
        }
    return -1;
}
long ref_tensor_set(void* net, const char* name, const float* in) {
    Network& n = *static_cast<Network*>(net);
    for (const ParamView& p : n.params())
        if (p.name == name) {
            std::memcpy(p.value, in, p.size * sizeof(float));
            return static_cast<long>(p.size);
        }
    for (const BufferView& b : n.buffers())
        if (b.name == name) {
            std::memcpy(b.value, in, b.size * sizeof(float));
            return static_cast<long>(b.size);
        }
    return -1;
}

// Network::infer with the single-threaded naive backend (LocalEvaluator's setup).
void ref_network_infer(void* net, const float* input, int B, float* logits, float* values, float* ownership) {
    Network& n = *static_cast<Network*>(net);
    NaiveBackend be(1);
    Workspace ws(n.config(), B, be);
    n.infer(ws, input, B, logits, values, ownership);
}

// Backend::im2col and Conv2d::forward (k = 3) with the naive backend.
void ref_im2col(const float* in, int C, int B, int n, int k, float* col) {
    NaiveBackend be(1);
    be.im2col(in, C, B, n, k, col);
}
void ref_conv_forward(const float* w, int cin, int cout, int k, const float* x, int B, int n, float* y) {
    NaiveBackend be(1);
    Conv2d conv(cin, cout, k);
    std::memcpy(conv.w.data(), w, conv.w.size() * sizeof(float));
    std::vector<float> col(conv.colSize(B, n) + 1);
    conv.forward(be, x, B, n, col.data(), y);
}
void ref_bn_infer(const float* gamma, const float* beta, const float* mean, const float* var, int C, int M,
                  const float* x, float* y) {
    BatchNorm2d bn(C);
    std::memcpy(bn.gamma.data(), gamma, C * sizeof(float));
    std::memcpy(bn.beta.data(), beta, C * sizeof(float));
    std::memcpy(bn.runMean.data(), mean, C * sizeof(float));
    std::memcpy(bn.runVar.data(), var, C * sizeof(float));
    bn.forwardInfer(x, M, y);
}

// calibrateBatchNorm (src/bn_calibration.cpp:33-45): generation 0's
// running statistics from one training-mode pass over the seeded positions.
void ref_calibrate_bn(void* net, uint64_t seed, int threads) {
    calibrateBatchNorm(*static_cast<Network*>(net), seed, threads);
}

// bnCalibrationPositions (src/bn_calibration.cpp:12-31): count x planes x area floats.
void ref_bn_calibration_positions(int board, int history, uint64_t seed, int count, float* out) {
    const std::vector<float> v = bnCalibrationPositions(board, history, seed, count);
    std::memcpy(out, v.data(), v.size() * sizeof(float));
}

// saveNetwork / loadNetwork (src/checkpoint.cpp:84-128). Errors come back as
// the message the reference throws, in err; the return is nonzero then.
int ref_save_network(void* net, const char* path, char* err, size_t cap) {
    try {
        saveNetwork(*static_cast<Network*>(net), path);
        return 0;
    } catch (const std::exception& e) {
        std::snprintf(err, cap, "%s", e.what());
        return 1;
    }
}
void* ref_load_network(const char* path, char* err, size_t cap) {
    try {
        return new Network(loadNetwork(path));
    } catch (const std::exception& e) {
        std::snprintf(err, cap, "%s", e.what());
        return nullptr;
    }
}

// A random game played by the reference's Game with bnCalibrationPositions'
// move choice (src/bn_calibration.cpp:19-28): each move legal[rng.below(points)]
// over Game::legalActions (ascending, pass last), a pass only when no point
// is legal. Records every position: stones, side to move, Board::hash, and
// the legal set as Mcts::expand builds it at a root (src/mcts.cpp:152-169:
// Board::isLegal and hashAfter not seen in the game). Returns moves played.
int ref_random_game(int n, uint64_t seed, int moves, uint8_t* stones, uint8_t* toMove, uint64_t* hashes,
                    uint8_t* legal) {
    Game game(n, 0.0f, defaultMaxMoves(n));
    Rng rng(seed);
    const int area = n * n;
    for (int ply = 0;; ++ply) {
        const Board& b = game.board();
        b.exportStones(stones + static_cast<size_t>(ply) * area);
        toMove[ply] = static_cast<uint8_t>(b.toMove());
        hashes[ply] = b.hash();
        uint8_t* lg = legal + static_cast<size_t>(ply) * (area + 1);
        for (int a = 0; a < area; ++a) lg[a] = b.isLegal(a) && !game.seen(b.hashAfter(a));
        lg[area] = 1;
        if (ply == moves || game.isTerminal()) return ply;
        const std::vector<int> acts = game.legalActions();
        const int points = static_cast<int>(acts.size()) - 1;
        game.play(points > 0 ? acts[rng.below(points)] : acts.back());
    }
}

// Board::isLegal, hashAfter and play on a position given as stones.
static Board boardOf(const uint8_t* stones, int n, int toMove) {
    Board b(n);
    for (int p = 0; p < n * n; ++p) b.setStone(p, static_cast<Color>(stones[p]));
    b.setToMove(toMove == 1 ? Color::Black : Color::White);
    return b;
}
void ref_board_legal(const uint8_t* stones, int n, int toMove, uint8_t* legal) {
    const Board b = boardOf(stones, n, toMove);
    for (int a = 0; a <= n * n; ++a) legal[a] = b.isLegal(a);
}
void ref_hash_after(const uint8_t* stones, int n, int toMove, uint64_t* out) {
    const Board b = boardOf(stones, n, toMove);
    for (int a = 0; a <= n * n; ++a) out[a] = b.isLegal(a) ? b.hashAfter(a) : 0;
}
uint64_t ref_board_hash(const uint8_t* stones, int n) { return boardOf(stones, n, 1).hash(); }

} // extern "C"
