/*
 * The oracle: a CPU restatement of the reference's inference forward pass.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (the HIP library under
 * alphazero-go_amd/) links, loads or calls this file; only tests/, the smoke
 * check and the bench's CPU-baseline leg use it, to check results against.
 *
 * Every function cites the reference file:line it follows (paths relative to
 * the reference repository). Compiled with -ffp-contract=off, as the
 * reference's exact CPU checks are (CMakeLists.txt:184-186), so every
 * multiply and add rounds separately, as on the reference's x86-64 build.
 *
 * Parity pinning (what each part is checked against in tests/):
 *   rng          splitmix64 known-answer vector (tests/test_rng.cpp:11-18);
 *                bitwise against the reference's own Rng compiled from source
 *                (oracle/_ref), xoshiro256** published algorithm.
 *   weights      bitwise against Network(cfg, seed) compiled from source;
 *                He-normal scale statistics (tests/test_layers.cpp:212-236).
 *   encode       plane cases of tests/test_encode.cpp:46-137; symmetry images
 *                of tests/test_symmetry.cpp:18-39.
 *   im2col/conv  hand examples (tests/test_backend.cpp:121-138,
 *                tests/test_layers.cpp:145-157).
 *   BN           hand values (tests/test_layers.cpp:159-171).
 *   naive pass   bitwise against Network::infer with the naive backend,
 *                compiled from source.
 *   blas pass    within 1e-4 relative of a double gemm per layer
 *                (tests/test_backend.cpp:36-82), and maxErr against the
 *                double pass. OpenBLAS's own summation order is unpinned
 *                beyond that (the reference pins it no further either).
 *   double pass  brute force on tiny inputs; closed-form hand networks.
 *   softmax      sums to 1 over legal moves, zero elsewhere; closed form on
 *                hand logits.
 *   rules        the legal-move positions of tests/test_board.cpp:109-146 and
 *                the ko of tests/test_game.cpp:19-55, restated; whole random
 *                games (every position's stones, hash and legal set) played
 *                move for move identically by the reference's Game compiled
 *                from source (tests/golden/games.npz).
 */
#define _GNU_SOURCE
#include <dlfcn.h>
#include <math.h>
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ rng */

/* src/rng.cpp:19-25 (splitmix64, Steele et al.). */
uint64_t azo_splitmix64(uint64_t* x) {
    uint64_t z = (*x += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

/* src/rng.cpp:27-37: h = splitmix(h ^ v) over (a, b, c, d) from a pi constant. */
uint64_t azo_derive_seed(uint64_t a, uint64_t b, uint64_t c, uint64_t d) {
    const uint64_t v[4] = {a, b, c, d};
    uint64_t h = 0x243F6A8885A308D3ULL;
    for (int i = 0; i < 4; ++i) {
        uint64_t x = h ^ v[i];
        h = azo_splitmix64(&x);
    }
    return h;
}

typedef struct { uint64_t s[4]; } azo_rng;

/* src/rng.cpp:39-44: four splitmix64 outputs seed xoshiro256**. */
void azo_rng_init(azo_rng* r, uint64_t seed) {
    uint64_t x = seed;
    for (int i = 0; i < 4; ++i) r->s[i] = azo_splitmix64(&x);
}

static uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

/* src/rng.cpp:46-57: xoshiro256** (Blackman & Vigna). */
uint64_t azo_rng_next(azo_rng* r) {
    uint64_t* s = r->s;
    const uint64_t result = rotl64(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return result;
}

/* src/rng.cpp:59-62: top 53 bits / 2^53. */
double azo_rng_uniform(azo_rng* r) { return (double)(azo_rng_next(r) >> 11) * 0x1.0p-53; }

/* src/rng.cpp:64-80: Lemire multiply-shift with rejection. */
int azo_rng_below(azo_rng* r, int n) {
    const uint32_t range = (uint32_t)n;
    uint64_t m = (azo_rng_next(r) >> 32) * range;
    uint32_t low = (uint32_t)m;
    if (low < range) {
        const uint32_t threshold = (0u - range) % range;
        while (low < threshold) {
            m = (azo_rng_next(r) >> 32) * range;
            low = (uint32_t)m;
        }
    }
    return (int)(m >> 32);
}

/* src/rng.cpp:82-86: Box-Muller, one value per two uniforms, no caching. */
double azo_rng_normal(azo_rng* r) {
    const double u1 = 1.0 - azo_rng_uniform(r);
    const double u2 = azo_rng_uniform(r);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925286766559 * u2);
}

/* ------------------------------------------------------------------ config and tensor layout */

/* include/azgo/network.hpp:24-36. */
typedef struct {
    int board, history, blocks, filters, value_hidden, ownership;
} azo_cfg;

static int cfg_planes(const azo_cfg* c) { return 2 * c->history + 2; }
static int cfg_area(const azo_cfg* c) { return c->board * c->board; }
static int cfg_actions(const azo_cfg* c) { return c->board * c->board + 1; }

enum { KIND_CONV = 0, KIND_GAMMA, KIND_BETA, KIND_FCW, KIND_FCB, KIND_MEAN, KIND_VAR };

typedef struct {
    char name[48];
    size_t size;
    size_t offset;   /* floats from the start of its arena */
    int buffer;      /* 0: params() arena, 1: buffers() arena */
    int kind;
    int fan_in;      /* He-normal fan-in for conv/fc weights */
    int init_rank;   /* order of the weight in the init sequence, -1 if not random */
} azo_entry;

#define AZO_ALIGN 64 /* include/azgo/param_layout.hpp:19 (kAlignFloats) */
#define AZO_MAX_ENTRIES 1024

static size_t align_up(size_t f) { return (f + AZO_ALIGN - 1) / AZO_ALIGN * AZO_ALIGN; }

/*
 * Network::params() then Network::buffers() (src/network.cpp:113-165), at the
 * offsets ParamLayout::of gives them (src/param_layout.cpp:18-29).
 * init_rank follows the constructor's Rng order (src/network.cpp:96-110):
 * stem conv, each block's conv1 then conv2, policy conv, policy fc, value
 * conv, fc1, fc2, then the ownership conv.
 */
static int build_layout(const azo_cfg* c, azo_entry* e, size_t* param_floats, size_t* buffer_floats) {
    int n = 0, rank = 0;
    size_t pf = 0, bf = 0;
    const int F = c->filters, P = cfg_planes(c), A = cfg_area(c), V = c->value_hidden;
#define ADD(nm, sz, kd, fan, rk)                                                  \
    do {                                                                          \
        snprintf(e[n].name, sizeof e[n].name, "%s", nm);                         \
        e[n].size = (size_t)(sz);                                                 \
        e[n].buffer = 0;                                                          \
        e[n].kind = kd;                                                           \
        e[n].fan_in = fan;                                                        \
        e[n].init_rank = rk;                                                      \
        e[n].offset = pf;                                                         \
        pf = align_up(pf + e[n].size);                                            \
        ++n;                                                                      \
    } while (0)
#define ADDBUF(nm, sz, kd)                                                        \
    do {                                                                          \
        snprintf(e[n].name, sizeof e[n].name, "%s", nm);                         \
        e[n].size = (size_t)(sz);                                                 \
        e[n].buffer = 1;                                                          \
        e[n].kind = kd;                                                           \
        e[n].fan_in = 0;                                                          \
        e[n].init_rank = -1;                                                      \
        e[n].offset = bf;                                                         \
        bf = align_up(bf + e[n].size);                                            \
        ++n;                                                                      \
    } while (0)
    char nm[48];
    ADD("stem.conv.w", (size_t)F * P * 9, KIND_CONV, P * 9, rank++);
    ADD("stem.bn.gamma", F, KIND_GAMMA, 0, -1);
    ADD("stem.bn.beta", F, KIND_BETA, 0, -1);
    for (int i = 0; i < c->blocks; ++i) {
        snprintf(nm, sizeof nm, "block%d.conv1.w", i);
        ADD(nm, (size_t)F * F * 9, KIND_CONV, F * 9, rank++);
        snprintf(nm, sizeof nm, "block%d.bn1.gamma", i);
        ADD(nm, F, KIND_GAMMA, 0, -1);
        snprintf(nm, sizeof nm, "block%d.bn1.beta", i);
        ADD(nm, F, KIND_BETA, 0, -1);
        snprintf(nm, sizeof nm, "block%d.conv2.w", i);
        ADD(nm, (size_t)F * F * 9, KIND_CONV, F * 9, rank++);
        snprintf(nm, sizeof nm, "block%d.bn2.gamma", i);
        ADD(nm, F, KIND_GAMMA, 0, -1);
        snprintf(nm, sizeof nm, "block%d.bn2.beta", i);
        ADD(nm, F, KIND_BETA, 0, -1);
    }
    ADD("policy.conv.w", 2 * F, KIND_CONV, F, rank++);
    ADD("policy.bn.gamma", 2, KIND_GAMMA, 0, -1);
    ADD("policy.bn.beta", 2, KIND_BETA, 0, -1);
    ADD("policy.fc.w", (size_t)2 * A * (A + 1), KIND_FCW, 2 * A, rank++);
    ADD("policy.fc.b", A + 1, KIND_FCB, 0, -1);
    ADD("value.conv.w", F, KIND_CONV, F, rank++);
    ADD("value.bn.gamma", 1, KIND_GAMMA, 0, -1);
    ADD("value.bn.beta", 1, KIND_BETA, 0, -1);
    ADD("value.fc1.w", (size_t)A * V, KIND_FCW, A, rank++);
    ADD("value.fc1.b", V, KIND_FCB, 0, -1);
    ADD("value.fc2.w", V, KIND_FCW, V, rank++);
    ADD("value.fc2.b", 1, KIND_FCB, 0, -1);
    if (c->ownership) {
        ADD("ownership.conv.w", F, KIND_CONV, F, rank++);
        ADD("ownership.bn.gamma", 1, KIND_GAMMA, 0, -1);
        ADD("ownership.bn.beta", 1, KIND_BETA, 0, -1);
    }
    ADDBUF("stem.bn.runMean", F, KIND_MEAN);
    ADDBUF("stem.bn.runVar", F, KIND_VAR);
    for (int i = 0; i < c->blocks; ++i) {
        snprintf(nm, sizeof nm, "block%d.bn1.runMean", i);
        ADDBUF(nm, F, KIND_MEAN);
        snprintf(nm, sizeof nm, "block%d.bn1.runVar", i);
        ADDBUF(nm, F, KIND_VAR);
        snprintf(nm, sizeof nm, "block%d.bn2.runMean", i);
        ADDBUF(nm, F, KIND_MEAN);
        snprintf(nm, sizeof nm, "block%d.bn2.runVar", i);
        ADDBUF(nm, F, KIND_VAR);
    }
    ADDBUF("policy.bn.runMean", 2, KIND_MEAN);
    ADDBUF("policy.bn.runVar", 2, KIND_VAR);
    ADDBUF("value.bn.runMean", 1, KIND_MEAN);
    ADDBUF("value.bn.runVar", 1, KIND_VAR);
    if (c->ownership) {
        ADDBUF("ownership.bn.runMean", 1, KIND_MEAN);
        ADDBUF("ownership.bn.runVar", 1, KIND_VAR);
    }
#undef ADD
#undef ADDBUF
    *param_floats = pf;
    *buffer_floats = bf;
    return n;
}

int azo_tensor_count(const azo_cfg* c) {
    static azo_entry e[AZO_MAX_ENTRIES];
    size_t pf, bf;
    return build_layout(c, e, &pf, &bf);
}

/* One layout entry: name, size, offset, arena (0 params, 1 buffers). */
int azo_tensor_info(const azo_cfg* c, int idx, char* name, size_t cap, size_t* size, size_t* offset,
                    int* buffer) {
    azo_entry e[AZO_MAX_ENTRIES];
    size_t pf, bf;
    const int n = build_layout(c, e, &pf, &bf);
    if (idx < 0 || idx >= n) return -1;
    snprintf(name, cap, "%s", e[idx].name);
    *size = e[idx].size;
    *offset = e[idx].offset;
    *buffer = e[idx].buffer;
    return 0;
}

void azo_arena_sizes(const azo_cfg* c, size_t* param_floats, size_t* buffer_floats) {
    azo_entry e[AZO_MAX_ENTRIES];
    build_layout(c, e, param_floats, buffer_floats);
}

/*
 * Network(cfg, seed) (src/network.cpp:77-111): one Rng(seed), He-normal
 * weights N(0, 2/fanIn) drawn as float(normal() * sqrt(2/fanIn))
 * (src/layers.cpp:14-17), in constructor order; biases 0 (src/layers.cpp:164-167);
 * BN gamma 1, beta 0, runMean 0, runVar 1 (src/layers.cpp:79-83).
 * Arena padding is zero.
 */
void azo_init_network(const azo_cfg* c, uint64_t seed, float* params, float* buffers) {
    azo_entry e[AZO_MAX_ENTRIES];
    size_t pf, bf;
    const int n = build_layout(c, e, &pf, &bf);
    memset(params, 0, pf * sizeof(float));
    memset(buffers, 0, bf * sizeof(float));
    for (int i = 0; i < n; ++i) {
        float* t = (e[i].buffer ? buffers : params) + e[i].offset;
        if (e[i].kind == KIND_GAMMA || e[i].kind == KIND_VAR)
            for (size_t j = 0; j < e[i].size; ++j) t[j] = 1.0f;
    }
    azo_rng rng;
    azo_rng_init(&rng, seed);
    int rank = 0;
    for (;;) {
        int found = -1;
        for (int i = 0; i < n; ++i)
            if (e[i].init_rank == rank) found = i;
        if (found < 0) break;
        const double stddev = sqrt(2.0 / e[found].fan_in);
        float* t = params + e[found].offset;
        for (size_t j = 0; j < e[found].size; ++j) t[j] = (float)(azo_rng_normal(&rng) * stddev);
        ++rank;
    }
}

/*
 * The synthetic batch-norm statistics of the benchmark workloads (not from
 * the reference, which starts at mean 0, var 1): one Rng(deriveSeed(seed,
 * 0xB4)); for each batch norm in buffers() order, every channel's running
 * mean as float(0.1 * normal()), then every channel's running variance as
 * float(0.5 + uniform()), i.e. mean ~ N(0, 0.1^2), var ~ U(0.5, 1.5).
 */
void azo_synthetic_bn(const azo_cfg* c, uint64_t seed, float* buffers) {
    azo_entry e[AZO_MAX_ENTRIES];
    size_t pf, bf;
    const int n = build_layout(c, e, &pf, &bf);
    azo_rng rng;
    azo_rng_init(&rng, azo_derive_seed(seed, 0xB4, 0, 0));
    for (int i = 0; i < n; ++i) {
        if (!e[i].buffer) continue;
        float* t = buffers + e[i].offset;
        for (size_t j = 0; j < e[i].size; ++j)
            t[j] = e[i].kind == KIND_MEAN ? (float)(0.1 * azo_rng_normal(&rng)) : (float)(0.5 + azo_rng_uniform(&rng));
    }
}

/* ------------------------------------------------------------------ boards and encoding */

/* src/symmetry.cpp:6-19: mirror left-right first, then (sym & 3) clockwise turns. */
int azo_transform_point(int sym, int point, int n) {
    int row = point / n, col = point % n;
    if (sym & 4) col = n - 1 - col;
    for (int turn = 0; turn < (sym & 3); ++turn) {
        const int r = col, cc = n - 1 - row;
        row = r;
        col = cc;
    }
    return row * n + col;
}

/*
 * encodePlanes (src/encode.cpp:14-43): stones[k] = n*n Color bytes (0 empty,
 * 1 black, 2 white; include/azgo/board.hpp:24) k plies ago; "own" = to_move
 * in every plane; planes 2k / 2k+1 own / opponent; plane 2H (black to move)
 * or 2H+1 (white to move) all ones; value of point p lands at
 * transformPoint(sym, p). count may be below H: missing plies stay zero.
 */
void azo_encode_planes(const uint8_t* stones, int count, int n, int to_move, int H, int sym, float* out) {
    const int area = n * n;
    memset(out, 0, sizeof(float) * (size_t)(2 * H + 2) * area);
    int dest[19 * 19];
    for (int p = 0; p < area; ++p) dest[p] = azo_transform_point(sym, p, n);
    const uint8_t own = (uint8_t)to_move;
    const uint8_t opp = (uint8_t)(to_move == 1 ? 2 : 1);
    const int available = count < H ? count : H;
    for (int k = 0; k < available; ++k) {
        float* ownPlane = out + (size_t)(2 * k) * area;
        float* oppPlane = ownPlane + area;
        const uint8_t* s = stones + (size_t)k * area;
        for (int p = 0; p < area; ++p) {
            if (s[p] == own) ownPlane[dest[p]] = 1.0f;
            else if (s[p] == opp) oppPlane[dest[p]] = 1.0f;
        }
    }
    float* plane = out + (size_t)(2 * H + (to_move == 1 ? 0 : 1)) * area;
    for (int p = 0; p < area; ++p) plane[p] = 1.0f;
}

/*
 * The synthetic positions of the benchmark workloads: position i of workload
 * `tag` uses its own Rng(deriveSeed(seed, tag, i)); point by point in index
 * order u = uniform() makes it black if u < p_black, white if
 * u < p_black + p_white, else empty; then the side to move is black if
 * below(2) == 0, else white. One board of history (the current one).
 * stones [B][n*n], to_move [B] (1 black, 2 white).
 */
void azo_random_boards(int n, int B, uint64_t seed, uint64_t tag, double p_black, double p_white, uint8_t* stones,
                       uint8_t* to_move) {
    const int area = n * n;
    for (int i = 0; i < B; ++i) {
        azo_rng rng;
        azo_rng_init(&rng, azo_derive_seed(seed, tag, (uint64_t)i, 0));
        for (int p = 0; p < area; ++p) {
            const double u = azo_rng_uniform(&rng);
            stones[(size_t)i * area + p] = u < p_black ? 1 : (u < p_black + p_white ? 2 : 0);
        }
        to_move[i] = azo_rng_below(&rng, 2) == 0 ? 1 : 2;
    }
}

/* Boards -> network input [B][2H+2][n*n] (identity symmetry) and the legal
 * mask [B][n*n+1] used for the softmax: empty points plus pass. */
void azo_encode_batch(int n, int H, int B, const uint8_t* stones, const uint8_t* to_move, float* input,
                      uint8_t* legal) {
    const int area = n * n;
    for (int i = 0; i < B; ++i) {
        azo_encode_planes(stones + (size_t)i * area, 1, n, to_move[i], H, 0,
                          input + (size_t)i * (2 * H + 2) * area);
        if (legal) {
            for (int p = 0; p < area; ++p) legal[(size_t)i * (area + 1) + p] = stones[(size_t)i * area + p] == 0;
            legal[(size_t)i * (area + 1) + area] = 1;
        }
    }
}

/* ------------------------------------------------------------------ rules: legal moves and superko */

/* The padded board of include/azgo/board.hpp:21-24: rows of 21 cells (a
 * sentinel column each side of the largest board), cells Empty 0, Black 1,
 * White 2, Off 3 outside the n x n area. */
#define AZO_STRIDE 21
#define AZO_CELLS (AZO_STRIDE * AZO_STRIDE)
enum { AZO_EMPTY = 0, AZO_BLACK = 1, AZO_WHITE = 2, AZO_OFF = 3 };

static uint64_t zkeys[AZO_CELLS][2];
static pthread_once_t zonce = PTHREAD_ONCE_INIT;

/* src/board.cpp:19-33: one key per (padded cell, colour), black then white
 * for each cell in order, from one splitmix64 stream seeded 0x5EEDB0A4D5EEDB0A. */
static void zinit(void) {
    uint64_t x = 0x5EEDB0A4D5EEDB0AULL;
    for (int c = 0; c < AZO_CELLS; ++c) {
        zkeys[c][0] = azo_splitmix64(&x);
        zkeys[c][1] = azo_splitmix64(&x);
    }
}

uint64_t azo_zobrist_key(int padded, int color) {
    pthread_once(&zonce, zinit);
    return zkeys[padded][color == AZO_BLACK ? 0 : 1];
}

typedef struct {
    int n, to_move;
    uint8_t cell[AZO_CELLS];
    uint64_t hash;
} azo_board;

static int padded(int n, int p) { return (p / n + 1) * AZO_STRIDE + (p % n + 1); }
static int other(int c) { return c == AZO_BLACK ? AZO_WHITE : AZO_BLACK; }
static const int kDirs[4] = {-AZO_STRIDE, -1, 1, AZO_STRIDE};

/* Board(n) + setStone per point (src/board.cpp:44-52, 273-281): the hash is
 * the XOR of the keys of every stone. */
static void board_from(azo_board* b, int n, const uint8_t* stones, int to_move) {
    b->n = n;
    b->to_move = to_move;
    b->hash = 0;
    memset(b->cell, AZO_OFF, sizeof b->cell);
    for (int p = 0; p < n * n; ++p) {
        const int q = padded(n, p);
        b->cell[q] = stones[p];
        if (stones[p] == AZO_BLACK || stones[p] == AZO_WHITE) b->hash ^= azo_zobrist_key(q, stones[p]);
    }
}

/* Board::countLiberties (src/board.cpp:68-94): flood fill over the group at
 * padded cell p; each liberty counted once; stops once `limit` are found. */
static int count_libs(const azo_board* b, int p, int limit) {
    int stack[AZO_CELLS], top = 0, libs = 0;
    uint8_t mark[AZO_CELLS];
    memset(mark, 0, sizeof mark);
    const int color = b->cell[p];
    stack[top++] = p;
    mark[p] = 1;
    while (top > 0) {
        const int q = stack[--top];
        for (int d = 0; d < 4; ++d) {
            const int r = q + kDirs[d];
            if (mark[r]) continue;
            if (b->cell[r] == AZO_EMPTY) {
                mark[r] = 1;
                if (++libs >= limit) return libs;
            } else if (b->cell[r] == color) {
                mark[r] = 1;
                stack[top++] = r;
            }
        }
    }
    return libs;
}

/* Board::removeGroup (src/board.cpp:96-121). */
static int remove_group(azo_board* b, int p) {
    int stack[AZO_CELLS], top = 0, removed = 0;
    const int color = b->cell[p];
    stack[top++] = p;
    b->cell[p] = AZO_EMPTY;
    b->hash ^= azo_zobrist_key(p, color);
    while (top > 0) {
        const int q = stack[--top];
        ++removed;
        for (int d = 0; d < 4; ++d) {
            const int r = q + kDirs[d];
            if (b->cell[r] == color) {
                b->cell[r] = AZO_EMPTY;
                b->hash ^= azo_zobrist_key(r, color);
                stack[top++] = r;
            }
        }
    }
    return removed;
}

/* Board::isLegal (src/board.cpp:131-150): pass always; else an empty point
 * where the new stone gets a liberty from an empty neighbour, from capturing
 * an opponent group whose last liberty it is, or from a friendly group with
 * another liberty. Superko is not checked here. */
static int is_legal(const azo_board* b, int action) {
    const int area = b->n * b->n;
    if (action == area) return 1;
    if (action < 0 || action > area) return 0;
    const int p = padded(b->n, action);
    if (b->cell[p] != AZO_EMPTY) return 0;
    const int me = b->to_move, them = other(me);
    for (int d = 0; d < 4; ++d) {
        const int q = p + kDirs[d];
        const int c = b->cell[q];
        if (c == AZO_EMPTY) return 1;
        if (c == them && count_libs(b, q, 2) == 1) return 1;
        if (c == me && count_libs(b, q, 2) >= 2) return 1;
    }
    return 0;
}

/* Board::play (src/board.cpp:152-174): places the stone, removes opponent
 * groups left without liberties, passes the turn. Returns stones captured. */
static int play(azo_board* b, int action) {
    const int area = b->n * b->n;
    if (action == area) {
        b->to_move = other(b->to_move);
        return 0;
    }
    const int p = padded(b->n, action);
    const int me = b->to_move, them = other(me);
    b->cell[p] = (uint8_t)me;
    b->hash ^= azo_zobrist_key(p, me);
    int captured = 0;
    for (int d = 0; d < 4; ++d) {
        const int q = p + kDirs[d];
        if (b->cell[q] == them && count_libs(b, q, 1) == 0) captured += remove_group(b, q);
    }
    b->to_move = them;
    return captured;
}

/* Board::hashAfter (src/board.cpp:176-190) for a legal action: the move is
 * played on a copy only when an opponent group beside it has exactly one
 * liberty; otherwise the hash gains the new stone's key alone (which
 * differs from play() only where an opponent group beside the point already
 * has no liberty, a position no game reaches). */
static uint64_t hash_after(const azo_board* b, int action) {
    if (action == b->n * b->n) return b->hash;
    const int p = padded(b->n, action), them = other(b->to_move);
    for (int d = 0; d < 4; ++d) {
        const int q = p + kDirs[d];
        if (b->cell[q] == them && count_libs(b, q, 2) == 1) {
            azo_board next = *b;
            play(&next, action);
            return next.hash;
        }
    }
    return b->hash ^ azo_zobrist_key(p, b->to_move);
}

static int seen_has(const uint64_t* seen, int nseen, uint64_t h) {
    for (int i = 0; i < nseen; ++i)
        if (seen[i] == h) return 1;
    return 0;
}

/* The legal set Mcts::expand builds (src/mcts.cpp:152-169), and
 * Game::isLegal for a game that is not over (src/game.cpp:19-29): pass, and
 * every point Board::isLegal allows whose resulting stones are not among
 * `seen` (positional superko). legal[0..n*n] = 1 / 0. */
void azo_legal_moves(const uint8_t* stones, int n, int to_move, const uint64_t* seen, int nseen, uint8_t* legal) {
    azo_board b;
    board_from(&b, n, stones, to_move);
    for (int a = 0; a < n * n; ++a)
        legal[a] = (uint8_t)(is_legal(&b, a) && !seen_has(seen, nseen, hash_after(&b, a)));
    legal[n * n] = 1;
}

/* Board::isLegal alone (no superko) for every action. */
void azo_board_legal(const uint8_t* stones, int n, int to_move, uint8_t* legal) {
    azo_board b;
    board_from(&b, n, stones, to_move);
    for (int a = 0; a <= n * n; ++a) legal[a] = (uint8_t)is_legal(&b, a);
}

uint64_t azo_board_hash(const uint8_t* stones, int n) {
    azo_board b;
    board_from(&b, n, stones, AZO_BLACK);
    return b.hash;
}

/* Board::hashAfter for every action (0 where Board::isLegal refuses it). */
void azo_hash_after(const uint8_t* stones, int n, int to_move, uint64_t* out) {
    azo_board b;
    board_from(&b, n, stones, to_move);
    for (int a = 0; a <= n * n; ++a) out[a] = is_legal(&b, a) ? hash_after(&b, a) : 0;
}

/* Board::play on a copy: the stones after `action` (which must be legal). */
int azo_play(const uint8_t* stones, int n, int to_move, int action, uint8_t* out) {
    azo_board b;
    board_from(&b, n, stones, to_move);
    const int captured = play(&b, action);
    for (int p = 0; p < n * n; ++p) out[p] = b.cell[padded(n, p)];
    return captured;
}

/* A random game as bnCalibrationPositions plays them (src/bn_calibration.cpp:19-28):
 * from the empty board, Black first, each move a uniformly random legal
 * point (Rng::below over Game::legalActions' points, ascending), a pass only
 * when no point is legal; stops after `moves` moves or when the game ends
 * (two passes, or 2 n^2 moves: src/game.cpp:51-53, 69-71). Records every
 * position 0..played: stones [moves+1][n*n], side to move, Zobrist hash and
 * the legal set (Game::isLegal: superko against every earlier position and
 * the current one) [moves+1][n*n+1]. Returns the moves played. */
int azo_random_game(int n, uint64_t seed, int moves, uint8_t* stones, uint8_t* to_move, uint64_t* hashes,
                    uint8_t* legal) {
    const int area = n * n, max_moves = 2 * area;
    azo_rng rng;
    azo_rng_init(&rng, seed);
    azo_board b;
    uint8_t* empty = calloc((size_t)area, 1);
    board_from(&b, n, empty, AZO_BLACK);
    free(empty);
    uint64_t* seen = malloc(sizeof(uint64_t) * (size_t)(moves + 1));
    int nseen = 0, passes = 0, ply = 0;
    int* points = malloc(sizeof(int) * (size_t)area);
    for (;;) {
        for (int p = 0; p < area; ++p) stones[(size_t)ply * area + p] = b.cell[padded(n, p)];
        to_move[ply] = (uint8_t)b.to_move;
        hashes[ply] = b.hash;
        if (!seen_has(seen, nseen, b.hash)) seen[nseen++] = b.hash;
        uint8_t* lg = legal + (size_t)ply * (area + 1);
        int count = 0;
        for (int a = 0; a < area; ++a) {
            lg[a] = (uint8_t)(is_legal(&b, a) && !seen_has(seen, nseen, hash_after(&b, a)));
            if (lg[a]) points[count++] = a;
        }
        lg[area] = 1;
        if (ply == moves || passes >= 2 || ply >= max_moves) break;
        const int action = count > 0 ? points[azo_rng_below(&rng, count)] : area;
        passes = action == area ? passes + 1 : 0;
        play(&b, action);
        ++ply;
    }
    free(points);
    free(seen);
    return ply;
}

/* ------------------------------------------------------------------ cblas */

typedef void (*sgemm_fn)(int, int, int, int, int, int, float, const float*, int, const float*, int, float, float*,
                         int);
static sgemm_fn g_sgemm = NULL;
static char g_blas_desc[512] = "";
static pthread_once_t g_blas_once = PTHREAD_ONCE_INIT;

/*
 * The reference's BlasBackend calls cblas_sgemm from OpenBLAS kept on one
 * thread (src/backend_blas.cpp:30-70) and records openblas_get_config
 * (:74-81). The image has no cblas.h, so the library is resolved at run time:
 * scipy's bundled OpenBLAS (symbols prefixed scipy_), a system OpenBLAS, or
 * MKL. Without any, blas mode reports -2.
 */
static void blas_load(void) {
    static const char* libs[] = {
        "/usr/local/lib/python3.10/dist-packages/scipy.libs/libscipy_openblas-68440149.so",
        "libopenblas.so.0",
        "libopenblas.so",
        "/opt/conda/lib/libmkl_rt.so",
        NULL,
    };
    const char* env = getenv("AZO_CBLAS_LIB");
    for (int i = env ? -1 : 0; i < 0 || libs[i]; ++i) {
        const char* path = i < 0 ? env : libs[i];
        void* h = dlopen(path, RTLD_NOW | RTLD_LOCAL);
        if (!h) continue;
        sgemm_fn f = (sgemm_fn)dlsym(h, "scipy_cblas_sgemm");
        const char* prefix = "scipy_";
        if (!f) {
            f = (sgemm_fn)dlsym(h, "cblas_sgemm");
            prefix = "";
        }
        if (!f) continue;
        char sym[96];
        snprintf(sym, sizeof sym, "%sopenblas_set_num_threads", prefix);
        void (*setThreads)(int) = (void (*)(int))dlsym(h, sym);
        if (setThreads) setThreads(1);
        int (*mklThreads)(int) = (int (*)(int))dlsym(h, "MKL_Set_Num_Threads");
        if (mklThreads) mklThreads(1);
        snprintf(sym, sizeof sym, "%sopenblas_get_config", prefix);
        char* (*config)(void) = (char* (*)(void))dlsym(h, sym);
        snprintf(g_blas_desc, sizeof g_blas_desc, "%s [%s]", config ? config() : "cblas", path);
        g_sgemm = f;
        return;
    }
}

const char* azo_blas_description(void) {
    pthread_once(&g_blas_once, blas_load);
    return g_sgemm ? g_blas_desc : "";
}

/* ------------------------------------------------------------------ layers */

/*
 * Backend::im2col (src/backend.cpp:21-55): in [C][B][n*n] -> col
 * [C*k*k][B*n*n], row (c*k + dy)*k + dx, zero off the board.
 */
void azo_im2col(const float* in, int C, int B, int n, int k, float* col) {
    const int r = k / 2;
    const size_t area = (size_t)n * n, M = (size_t)B * area;
    for (int c = 0; c < C; ++c)
        for (int dy = 0; dy < k; ++dy)
            for (int dx = 0; dx < k; ++dx) {
                float* row = col + (size_t)((c * k + dy) * k + dx) * M;
                const int oy = dy - r, ox = dx - r;
                for (int b = 0; b < B; ++b) {
                    const float* src = in + ((size_t)c * B + b) * area;
                    float* dst = row + (size_t)b * area;
                    for (int y = 0; y < n; ++y)
                        for (int x = 0; x < n; ++x) {
                            const int sy = y + oy, sx = x + ox;
                            dst[y * n + x] = (sy < 0 || sy >= n || sx < 0 || sx >= n) ? 0.0f : src[sy * n + sx];
                        }
                }
            }
}

/*
 * NaiveBackend::gemm with alpha 1, beta 0 (src/backend.cpp:115-185): C
 * zeroed, then every element sums a[i][p] * b[p][j] over p = 0..K-1 in that
 * order, one rounding per multiply and per add. transB reads B stored N x K.
 */
static void naive_gemm(int transB, int M, int N, int K, const float* A, const float* B, float* C) {
    for (size_t i = 0; i < (size_t)M * N; ++i) C[i] = 0.0f;
    if (!transB) {
        for (int i = 0; i < M; ++i) {
            float* c = C + (size_t)i * N;
            const float* a = A + (size_t)i * K;
            for (int p = 0; p < K; ++p) {
                const float s = a[p];
                const float* b = B + (size_t)p * N;
                for (int j = 0; j < N; ++j) c[j] += s * b[j];
            }
        }
    } else {
        for (int i = 0; i < M; ++i)
            for (int j = 0; j < N; ++j) {
                float acc = 0.0f;
                for (int p = 0; p < K; ++p) acc += A[(size_t)i * K + p] * B[(size_t)j * K + p];
                C[(size_t)i * N + j] = acc;
            }
    }
}

/* mode 0: naive; mode 1: cblas_sgemm row-major (src/backend_blas.cpp:50-52). */
static int gemm(int mode, int transB, int M, int N, int K, const float* A, const float* B, float* C) {
    if (mode == 0) {
        naive_gemm(transB, M, N, K, A, B, C);
        return 0;
    }
    pthread_once(&g_blas_once, blas_load);
    if (!g_sgemm) return -2;
    g_sgemm(101 /*RowMajor*/, 111 /*NoTrans*/, transB ? 112 : 111, M, N, K, 1.0f, A, K, B, transB ? K : N, 0.0f, C,
            N);
    return 0;
}

/* BatchNorm2d::forwardInfer (src/layers.cpp:88-97): per channel
 * scale = gamma / sqrt(var + eps), shift = beta - scale * mean, y = scale * x + shift. */
static void bn_infer(const float* gamma, const float* beta, const float* mean, const float* var, int C, size_t M,
                     const float* x, float* y) {
    for (int ch = 0; ch < C; ++ch) {
        const float scale = gamma[ch] / sqrtf(var[ch] + 1e-5f);
        const float shift = beta[ch] - scale * mean[ch];
        const float* xc = x + (size_t)ch * M;
        float* yc = y + (size_t)ch * M;
        for (size_t i = 0; i < M; ++i) yc[i] = scale * xc[i] + shift;
    }
}

/* reluForward (src/layers.cpp:191-195). */
static void relu(float* x, size_t count) {
    for (size_t i = 0; i < count; ++i) x[i] = x[i] > 0.0f ? x[i] : 0.0f;
}

/* Public single-layer entry points, for per-layer parity tests. */
void azo_bn_infer(const float* gamma, const float* beta, const float* mean, const float* var, int C, size_t M,
                  const float* x, float* y) {
    bn_infer(gamma, beta, mean, var, C, M, x, y);
}

/* Conv2d::forward (src/layers.cpp:35-46) for k = 3: im2col, then
 * y [cout][B*n*n] = w [cout][cin*9] . col. col: scratch of cin*9*B*n*n. */
int azo_conv3x3(int mode, const float* w, int cin, int cout, const float* x, int B, int n, float* col, float* y) {
    azo_im2col(x, cin, B, n, 3, col);
    return gemm(mode, 0, cout, B * n * n, cin * 9, w, col, y);
}

int azo_gemm(int mode, int transB, int M, int N, int K, const float* A, const float* B, float* C) {
    return gemm(mode, transB, M, N, K, A, B, C);
}

/* ------------------------------------------------------------------ forward */

static const float* tensor(const azo_entry* e, int n, const float* params, const float* buffers, const char* name) {
    for (int i = 0; i < n; ++i)
        if (strcmp(e[i].name, name) == 0) return (e[i].buffer ? buffers : params) + e[i].offset;
    fprintf(stderr, "azgo oracle: no tensor %s\n", name);
    abort();
}

/*
 * Network::forward in inference mode (src/network.cpp:228-309) and
 * Network::infer's copies (:171-183). input [B][P][A]; logits [B][A+1];
 * values [B]; ownership [B][A] when the config has the head (else ignored).
 * mode 0 = naive backend, 1 = blas. Returns 0, or -2 when blas is not
 * loadable, -1 when out of memory.
 */
static int forward_impl(const azo_cfg* c, const float* params, const float* buffers, const float* input, int B,
                        int mode, int blocks, float* trunk_out, float* logits, float* values, float* ownership);

int azo_forward(const azo_cfg* c, const float* params, const float* buffers, const float* input, int B, int mode,
                float* logits, float* values, float* ownership) {
    return forward_impl(c, params, buffers, input, B, mode, c->blocks, NULL, logits, values, ownership);
}

/*
 * The trunk alone: the stem and the first `blocks` residual blocks of
 * Network::forward (src/network.cpp:241-272), the same arithmetic as
 * azo_forward, returned batch-major as trunk [B][F][A] (the network keeps it
 * channel-major, [F][B][A]).
 */
int azo_trunk(const azo_cfg* c, const float* params, const float* buffers, const float* input, int B, int mode,
              int blocks, float* trunk) {
    if (blocks < 0 || blocks > c->blocks) return -3;
    return forward_impl(c, params, buffers, input, B, mode, blocks, trunk, NULL, NULL, NULL);
}

static int forward_impl(const azo_cfg* c, const float* params, const float* buffers, const float* input, int B,
                        int mode, int blocks, float* trunk_out, float* logits, float* values, float* ownership) {
    azo_entry e[AZO_MAX_ENTRIES];
    size_t pf, bf;
    const int ne = build_layout(c, e, &pf, &bf);
    const int n = c->board, A = cfg_area(c), P = cfg_planes(c), F = c->filters, V = c->value_hidden;
    const int acts = cfg_actions(c);
    const size_t M = (size_t)B * A, trunk = (size_t)F * M;
    const size_t colFloats = (size_t)(P > F ? P : F) * 9 * M;
    float* in = malloc(sizeof(float) * (size_t)P * M);
    float* col = malloc(sizeof(float) * colFloats);
    float* convOut = malloc(sizeof(float) * (F > 2 ? (size_t)F : 2) * M);
    float* x = malloc(sizeof(float) * trunk);
    float* mid = malloc(sizeof(float) * trunk);
    float* out = malloc(sizeof(float) * trunk);
    float* pol = malloc(sizeof(float) * 2 * M);
    float* flat = malloc(sizeof(float) * 2 * M);
    float* val = malloc(sizeof(float) * M);
    float* hid = malloc(sizeof(float) * (size_t)B * V);
    int rc = 0;
    if (!in || !col || !convOut || !x || !mid || !out || !pol || !flat || !val || !hid) {
        rc = -1;
        goto done;
    }
#define T(name) tensor(e, ne, params, buffers, name)
#define NORM(pre, C, src, dst) \
    bn_infer(T(pre ".gamma"), T(pre ".beta"), T(pre ".runMean"), T(pre ".runVar"), C, M, src, dst)
    /* [B][P][A] -> [P][B][A] (src/network.cpp:241-246). */
    for (int p = 0; p < P; ++p)
        for (int b = 0; b < B; ++b)
            memcpy(in + ((size_t)p * B + b) * A, input + ((size_t)b * P + p) * A, sizeof(float) * A);
    /* Stem: conv3x3 -> BN -> ReLU (:254-257). */
    if ((rc = azo_conv3x3(mode, T("stem.conv.w"), P, F, in, B, n, col, convOut))) goto done;
    NORM("stem.bn", F, convOut, x);
    relu(x, trunk);
    /* Blocks: conv -> BN -> ReLU -> conv -> BN -> + input -> ReLU (:259-272). */
    for (int i = 0; i < blocks; ++i) {
        char pre[64], nm[96];
        snprintf(pre, sizeof pre, "block%d", i);
        snprintf(nm, sizeof nm, "%s.conv1.w", pre);
        if ((rc = azo_conv3x3(mode, T(nm), F, F, x, B, n, col, convOut))) goto done;
        {
            char g[96], bt[96], mn[96], vr[96];
            snprintf(g, sizeof g, "%s.bn1.gamma", pre);
            snprintf(bt, sizeof bt, "%s.bn1.beta", pre);
            snprintf(mn, sizeof mn, "%s.bn1.runMean", pre);
            snprintf(vr, sizeof vr, "%s.bn1.runVar", pre);
            bn_infer(T(g), T(bt), T(mn), T(vr), F, M, convOut, mid);
        }
        relu(mid, trunk);
        snprintf(nm, sizeof nm, "%s.conv2.w", pre);
        if ((rc = azo_conv3x3(mode, T(nm), F, F, mid, B, n, col, convOut))) goto done;
        {
            char g[96], bt[96], mn[96], vr[96];
            snprintf(g, sizeof g, "%s.bn2.gamma", pre);
            snprintf(bt, sizeof bt, "%s.bn2.beta", pre);
            snprintf(mn, sizeof mn, "%s.bn2.runMean", pre);
            snprintf(vr, sizeof vr, "%s.bn2.runVar", pre);
            bn_infer(T(g), T(bt), T(mn), T(vr), F, M, convOut, out);
        }
        for (size_t j = 0; j < trunk; ++j) out[j] += x[j];
        relu(out, trunk);
        float* t = x;
        x = out;
        out = t;
    }
    if (trunk_out) {
        for (int ch = 0; ch < F; ++ch)
            for (int b = 0; b < B; ++b)
                memcpy(trunk_out + ((size_t)b * F + ch) * A, x + ((size_t)ch * B + b) * A, sizeof(float) * A);
        goto done;
    }
    /* Policy head: 1x1 conv F -> 2, BN, ReLU, flatten c*A + p, Linear (:274-286). */
    if ((rc = gemm(mode, 0, 2, (int)M, F, T("policy.conv.w"), x, convOut))) goto done;
    NORM("policy.bn", 2, convOut, pol);
    relu(pol, 2 * M);
    for (int b = 0; b < B; ++b)
        for (int ch = 0; ch < 2; ++ch)
            memcpy(flat + (size_t)b * 2 * A + (size_t)ch * A, pol + ((size_t)ch * B + b) * A, sizeof(float) * A);
    /* Linear::forward (src/layers.cpp:169-176): y = x . w^T, then + b per row. */
    if ((rc = gemm(mode, 1, B, acts, 2 * A, flat, T("policy.fc.w"), logits))) goto done;
    {
        const float* bias = T("policy.fc.b");
        for (int s = 0; s < B; ++s)
            for (int o = 0; o < acts; ++o) logits[(size_t)s * acts + o] += bias[o];
    }
    /* Value head: 1x1 conv F -> 1, BN, ReLU, fc1, ReLU, fc2, tanh (:288-296). */
    if ((rc = gemm(mode, 0, 1, (int)M, F, T("value.conv.w"), x, convOut))) goto done;
    NORM("value.bn", 1, convOut, val);
    relu(val, M);
    if ((rc = gemm(mode, 1, B, V, A, val, T("value.fc1.w"), hid))) goto done;
    {
        const float* bias = T("value.fc1.b");
        for (int s = 0; s < B; ++s)
            for (int o = 0; o < V; ++o) hid[(size_t)s * V + o] += bias[o];
    }
    relu(hid, (size_t)B * V);
    if ((rc = gemm(mode, 1, B, 1, V, hid, T("value.fc2.w"), values))) goto done;
    {
        const float b2 = T("value.fc2.b")[0];
        for (int s = 0; s < B; ++s) values[s] = tanhf(values[s] + b2);
    }
    /* Ownership head: 1x1 conv F -> 1, BN, tanh per point (:298-308). */
    if (c->ownership && ownership) {
        if ((rc = gemm(mode, 0, 1, (int)M, F, T("ownership.conv.w"), x, convOut))) goto done;
        NORM("ownership.bn", 1, convOut, ownership);
        for (size_t j = 0; j < M; ++j) ownership[j] = tanhf(ownership[j]);
    }
#undef NORM
#undef T
done:
    free(in);
    free(col);
    free(convOut);
    free(x);
    free(mid);
    free(out);
    free(pol);
    free(flat);
    free(val);
    free(hid);
    return rc;
}

/*
 * The whole network in double precision straight from its definition, the
 * structure of doubleInfer (tests/test_cuda.cpp:659-752): direct 'same'
 * convolutions, BN as (x - mean) * gamma / sqrt(var + eps) + beta, heads as
 * in forward. Outputs rounded to float once at the end.
 */
int azo_forward_double(const azo_cfg* c, const float* params, const float* buffers, const float* input, int B,
                       float* logits, float* values, float* ownership) {
    azo_entry e[AZO_MAX_ENTRIES];
    size_t pf, bf;
    const int ne = build_layout(c, e, &pf, &bf);
    const int n = c->board, A = cfg_area(c), P = cfg_planes(c), F = c->filters, V = c->value_hidden;
    const int acts = cfg_actions(c);
    const size_t M = (size_t)B * A;
    const int maxC = P > F ? P : F;
    double* h = malloc(sizeof(double) * (size_t)maxC * M);
    double* mid = malloc(sizeof(double) * (size_t)F * M);
    double* out = malloc(sizeof(double) * (size_t)F * M);
    double* head = malloc(sizeof(double) * 3 * M);
    double* hid = malloc(sizeof(double) * (size_t)V);
    if (!h || !mid || !out || !head || !hid) {
        free(h);
        free(mid);
        free(out);
        free(head);
        free(hid);
        return -1;
    }
#define T(name) tensor(e, ne, params, buffers, name)
    /* x [cin][B][A] -> y [cout][B][A]. */
#define CONV(xin, cin, cout, k, wname, yout)                                                          \
    do {                                                                                              \
        const float* w_ = T(wname);                                                                   \
        for (int o = 0; o < (cout); ++o)                                                              \
            for (int b = 0; b < B; ++b)                                                               \
                for (int p = 0; p < A; ++p) {                                                         \
                    double sum = 0.0;                                                                 \
                    for (int ci = 0; ci < (cin); ++ci)                                                \
                        for (int dy = 0; dy < (k); ++dy)                                              \
                            for (int dx = 0; dx < (k); ++dx) {                                        \
                                const int yy = p / n + dy - (k) / 2, xx = p % n + dx - (k) / 2;       \
                                if (yy < 0 || yy >= n || xx < 0 || xx >= n) continue;                 \
                                sum += (double)w_[(((size_t)o * (cin) + ci) * (k) + dy) * (k) + dx] * \
                                       (xin)[((size_t)ci * B + b) * A + yy * n + xx];                 \
                            }                                                                         \
                    (yout)[((size_t)o * B + b) * A + p] = sum;                                        \
                }                                                                                     \
    } while (0)
#define NORM(buf, C, pre)                                                                       \
    do {                                                                                        \
        const float *g_ = T(pre ".gamma"), *b_ = T(pre ".beta"), *m_ = T(pre ".runMean"),       \
                    *v_ = T(pre ".runVar");                                                     \
        for (int ch = 0; ch < (C); ++ch) {                                                      \
            const double scale = (double)g_[ch] / sqrt((double)v_[ch] + (double)1e-5f);         \
            for (size_t i = 0; i < M; ++i) {                                                    \
                double* v = &(buf)[(size_t)ch * M + i];                                         \
                *v = (*v - m_[ch]) * scale + b_[ch];                                            \
            }                                                                                   \
        }                                                                                       \
    } while (0)
    {
        double* xin = malloc(sizeof(double) * (size_t)P * M);
        if (!xin) abort();
        for (int b = 0; b < B; ++b)
            for (int p = 0; p < P; ++p)
                for (int a = 0; a < A; ++a) xin[((size_t)p * B + b) * A + a] = input[((size_t)b * P + p) * A + a];
        CONV(xin, P, F, 3, "stem.conv.w", h);
        free(xin);
    }
    NORM(h, F, "stem.bn");
    for (size_t i = 0; i < (size_t)F * M; ++i) h[i] = h[i] > 0 ? h[i] : 0;
    for (int i = 0; i < c->blocks; ++i) {
        char w1[64], w2[64], b1[64], b2[64];
        snprintf(w1, sizeof w1, "block%d.conv1.w", i);
        snprintf(w2, sizeof w2, "block%d.conv2.w", i);
        snprintf(b1, sizeof b1, "block%d.bn1", i);
        snprintf(b2, sizeof b2, "block%d.bn2", i);
        CONV(h, F, F, 3, w1, mid);
        {
            char g[80], bt[80], mn[80], vr[80];
            snprintf(g, sizeof g, "%s.gamma", b1);
            snprintf(bt, sizeof bt, "%s.beta", b1);
            snprintf(mn, sizeof mn, "%s.runMean", b1);
            snprintf(vr, sizeof vr, "%s.runVar", b1);
            const float *g_ = T(g), *b_ = T(bt), *m_ = T(mn), *v_ = T(vr);
            for (int ch = 0; ch < F; ++ch) {
                const double scale = (double)g_[ch] / sqrt((double)v_[ch] + (double)1e-5f);
                for (size_t j = 0; j < M; ++j) {
                    double* v = &mid[(size_t)ch * M + j];
                    *v = (*v - m_[ch]) * scale + b_[ch];
                    *v = *v > 0 ? *v : 0;
                }
            }
        }
        CONV(mid, F, F, 3, w2, out);
        {
            char g[80], bt[80], mn[80], vr[80];
            snprintf(g, sizeof g, "%s.gamma", b2);
            snprintf(bt, sizeof bt, "%s.beta", b2);
            snprintf(mn, sizeof mn, "%s.runMean", b2);
            snprintf(vr, sizeof vr, "%s.runVar", b2);
            const float *g_ = T(g), *b_ = T(bt), *m_ = T(mn), *v_ = T(vr);
            for (int ch = 0; ch < F; ++ch) {
                const double scale = (double)g_[ch] / sqrt((double)v_[ch] + (double)1e-5f);
                for (size_t j = 0; j < M; ++j) {
                    double* v = &out[(size_t)ch * M + j];
                    *v = (*v - m_[ch]) * scale + b_[ch] + h[(size_t)ch * M + j];
                    *v = *v > 0 ? *v : 0;
                }
            }
        }
        double* t = h;
        h = out;
        out = t;
    }
    /* Heads: 1x1 convs (policy rows 0-1, value row 2). */
    CONV(h, F, 2, 1, "policy.conv.w", head);
    NORM(head, 2, "policy.bn");
    for (size_t i = 0; i < 2 * M; ++i) head[i] = head[i] > 0 ? head[i] : 0;
    {
        const float *w = T("policy.fc.w"), *bias = T("policy.fc.b");
        for (int s = 0; s < B; ++s)
            for (int o = 0; o < acts; ++o) {
                double sum = bias[o];
                for (int ch = 0; ch < 2; ++ch)
                    for (int a = 0; a < A; ++a)
                        sum += head[((size_t)ch * B + s) * A + a] * (double)w[(size_t)o * 2 * A + (size_t)ch * A + a];
                logits[(size_t)s * acts + o] = (float)sum;
            }
    }
    double* v1 = head + 2 * M;
    CONV(h, F, 1, 1, "value.conv.w", v1);
    NORM(v1, 1, "value.bn");
    for (size_t i = 0; i < M; ++i) v1[i] = v1[i] > 0 ? v1[i] : 0;
    {
        const float *w1 = T("value.fc1.w"), *b1 = T("value.fc1.b"), *w2 = T("value.fc2.w"), *b2 = T("value.fc2.b");
        for (int s = 0; s < B; ++s) {
            for (int o = 0; o < V; ++o) {
                double sum = b1[o];
                for (int a = 0; a < A; ++a) sum += v1[(size_t)s * A + a] * (double)w1[(size_t)o * A + a];
                hid[o] = sum > 0 ? sum : 0;
            }
            double sum = b2[0];
            for (int o = 0; o < V; ++o) sum += hid[o] * (double)w2[o];
            values[s] = (float)tanh(sum);
        }
    }
    if (c->ownership && ownership) {
        CONV(h, F, 1, 1, "ownership.conv.w", v1);
        NORM(v1, 1, "ownership.bn");
        for (size_t i = 0; i < M; ++i) ownership[i] = (float)tanh(v1[i]);
    }
#undef NORM
#undef CONV
#undef T
    free(h);
    free(mid);
    free(out);
    free(head);
    free(hid);
    return 0;
}

/* ------------------------------------------------------------------ softmax over legal moves */

/*
 * Mcts::expand's priors (src/mcts.cpp:170-183): over the legal actions only,
 * max in float, p = exp(l - max) in float, sum in action order in float,
 * prior = p / sum. Illegal actions get 0 here (search never creates them).
 */
void azo_softmax_legal(const float* logits, const uint8_t* legal, int B, int actions, float* out) {
    for (int b = 0; b < B; ++b) {
        const float* l = logits + (size_t)b * actions;
        const uint8_t* m = legal + (size_t)b * actions;
        float* o = out + (size_t)b * actions;
        float mx = -INFINITY;
        for (int a = 0; a < actions; ++a)
            if (m[a] && l[a] > mx) mx = l[a];
        float sum = 0.0f;
        for (int a = 0; a < actions; ++a) {
            o[a] = m[a] ? expf(l[a] - mx) : 0.0f;
            sum += o[a];
        }
        for (int a = 0; a < actions; ++a) o[a] = m[a] ? o[a] / sum : 0.0f;
    }
}

/* ------------------------------------------------------------------ CPU baseline timing */

typedef struct {
    const azo_cfg* cfg;
    const float *params, *buffers, *input;
    int B, mode, calls;
    double seconds;
    long long positions;
} worker_arg;

static double now_seconds(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec * 1e-9;
}

static void* worker_main(void* p) {
    worker_arg* w = p;
    const int acts = cfg_actions(w->cfg);
    float* logits = malloc(sizeof(float) * (size_t)w->B * acts);
    float* values = malloc(sizeof(float) * (size_t)w->B);
    w->positions = 0;
    for (int i = 0; i < w->calls; ++i) {
        if (azo_forward(w->cfg, w->params, w->buffers, w->input, w->B, w->mode, logits, values, NULL) != 0) break;
        w->positions += w->B;
    }
    free(logits);
    free(values);
    return NULL;
}

/*
 * The reference bench's "cpu (blas)" row (apps/bench.cpp:452-476): `workers`
 * threads, each running the single-threaded forward pass on its own batch of
 * B positions `calls` times, after one warm-up call on the caller's thread
 * when `warm` is set.
 * Returns positions per second, all workers together; *elapsed the seconds.
 */
double azo_time_workers(const azo_cfg* c, const float* params, const float* buffers, const float* input, int B,
                        int mode, int workers, int calls, int warm, double* elapsed) {
    const int acts = cfg_actions(c);
    if (warm) {
        float* logits = malloc(sizeof(float) * (size_t)B * acts);
        float* values = malloc(sizeof(float) * (size_t)B);
        azo_forward(c, params, buffers, input, B, mode, logits, values, NULL);
        free(logits);
        free(values);
    }
    pthread_t* th = calloc((size_t)workers, sizeof(pthread_t));
    worker_arg* args = calloc((size_t)workers, sizeof(worker_arg));
    const double t0 = now_seconds();
    for (int w = 0; w < workers; ++w) {
        args[w] = (worker_arg){c, params, buffers, input, B, mode, calls, 0.0, 0};
        pthread_create(&th[w], NULL, worker_main, &args[w]);
    }
    long long total = 0;
    for (int w = 0; w < workers; ++w) {
        pthread_join(th[w], NULL);
        total += args[w].positions;
    }
    const double dt = now_seconds() - t0;
    if (elapsed) *elapsed = dt;
    free(th);
    free(args);
    return dt > 0 ? (double)total / dt : 0.0;
}

/*
 * The steps either side of the pass on the CPU, as the search does them per
 * leaf (Mcts::evaluateLeaves encodes, src/mcts.cpp:113-134; Mcts::expand
 * builds the legal set with superko, src/mcts.cpp:152-169): `workers`
 * threads, each encoding and finding the legal moves of the B positions
 * (stones [B][n*n], the current board only, H planes of history) in turn,
 * over and over, until `budget` seconds have passed. Position b's superko
 * list is seen[offsets[b] .. offsets[b+1]). Returns positions per second,
 * all workers together; *elapsed the seconds.
 */
typedef struct {
    const uint8_t *stones, *to_move;
    const uint64_t* seen;
    const int* offsets;
    int n, H, B;
    double stop;
    long long positions;
} positions_arg;

static void* positions_main(void* p) {
    positions_arg* w = p;
    const int area = w->n * w->n;
    float* planes = malloc(sizeof(float) * (size_t)(2 * w->H + 2) * area);
    uint8_t* legal = malloc((size_t)area + 1);
    w->positions = 0;
    while (now_seconds() < w->stop) {
        for (int b = 0; b < w->B; ++b) {
            azo_encode_planes(w->stones + (size_t)b * area, 1, w->n, w->to_move[b], w->H, b % 8, planes);
            azo_legal_moves(w->stones + (size_t)b * area, w->n, w->to_move[b], w->seen + w->offsets[b],
                            w->offsets[b + 1] - w->offsets[b], legal);
            ++w->positions;
            if ((b & 15) == 15 && now_seconds() >= w->stop) break;
        }
    }
    free(planes);
    free(legal);
    return NULL;
}

double azo_time_positions_workers(int n, int H, int B, const uint8_t* stones, const uint8_t* to_move,
                                  const uint64_t* seen, const int* offsets, int workers, double budget,
                                  double* elapsed) {
    pthread_t* th = calloc((size_t)workers, sizeof(pthread_t));
    positions_arg* args = calloc((size_t)workers, sizeof(positions_arg));
    const double t0 = now_seconds();
    for (int w = 0; w < workers; ++w) {
        args[w] = (positions_arg){stones, to_move, seen, offsets, n, H, B, t0 + budget, 0};
        pthread_create(&th[w], NULL, positions_main, &args[w]);
    }
    long long total = 0;
    for (int w = 0; w < workers; ++w) {
        pthread_join(th[w], NULL);
        total += args[w].positions;
    }
    const double dt = now_seconds() - t0;
    if (elapsed) *elapsed = dt;
    free(th);
    free(args);
    return dt > 0 ? (double)total / dt : 0.0;
}
