// The seeded benchmark workloads, as the caller of the backend builds them:
// a network's tensors exactly as azgo::Network(cfg, seed) initialises them
// (src/network.cpp:77-111), the synthetic batch-norm statistics of the
// benchmark configurations, and synthetic positions encoded as
// encodePlanes does (src/encode.cpp:14-43). Host C++ only; the benchmark
// and the smoke check feed these arrays to the HIP library through its C ABI.
//
// Conventions (the same as the oracle's, and checked equal to it bit for bit
// by the CPU tests):
//   weights  one Rng(seed) (xoshiro256** seeded by splitmix64,
//            src/rng.cpp:19-86); He-normal float(normal() * sqrt(2/fanIn)),
//            Box-Muller with two uniforms per draw, in the constructor's order:
//            stem conv, block convs (conv1, conv2), policy conv, policy fc,
//            value conv, value fc1, value fc2. Biases 0, gamma 1, beta 0.
//   BN stats Rng(deriveSeed(seed, 0xB4)): per batch norm in buffers() order,
//            every channel's mean float(0.1 * normal()), then every channel's
//            variance float(0.5 + uniform()).
//   boards   position i of workload `tag`: Rng(deriveSeed(seed, tag, i));
//            per point u = uniform(): black if u < pBlack, white if
//            u < pBlack + pWhite, else empty; then black to move if
//            below(2) == 0. The current board only (no history).
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace {

class Xoshiro {
  public:
    static uint64_t splitmix(uint64_t& x) {
        uint64_t z = (x += 0x9E3779B97F4A7C15ULL);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
        return z ^ (z >> 31);
    }
    static uint64_t derive(uint64_t a, uint64_t b, uint64_t c, uint64_t d) {
        uint64_t h = 0x243F6A8885A308D3ULL;
        for (uint64_t v : {a, b, c, d}) {
            uint64_t x = h ^ v;
            h = splitmix(x);
        }
        return h;
    }
    explicit Xoshiro(uint64_t seed) {
        for (uint64_t& w : s_) w = splitmix(seed);
    }
    uint64_t next() {
        const uint64_t out = rotl(s_[1] * 5, 7) * 9;
        const uint64_t t = s_[1] << 17;
        s_[2] ^= s_[0];
        s_[3] ^= s_[1];
        s_[1] ^= s_[2];
        s_[0] ^= s_[3];
        s_[2] ^= t;
        s_[3] = rotl(s_[3], 45);
        return out;
    }
    double uniform() { return static_cast<double>(next() >> 11) * 0x1.0p-53; }
    double normal() {
        const double u1 = 1.0 - uniform();
        const double u2 = uniform();
        return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586476925286766559 * u2);
    }
    int below(int n) {
        const uint32_t range = static_cast<uint32_t>(n);
        uint64_t m = (next() >> 32) * range;
        uint32_t low = static_cast<uint32_t>(m);
        if (low < range) {
            const uint32_t threshold = (0u - range) % range;
            while (low < threshold) {
                m = (next() >> 32) * range;
                low = static_cast<uint32_t>(m);
            }
        }
        return static_cast<int>(m >> 32);
    }

  private:
    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
    uint64_t s_[4];
};

enum class Kind { Weight, One, Zero, Mean, Var };
struct Tensor {
    std::string name;
    size_t size;
    Kind kind;
    int fanIn;   // He-normal fan-in for weights
    int order;   // position in the constructor's draw order, -1 if drawn never
};

// Network::params() then buffers() (src/network.cpp:113-165).
std::vector<Tensor> tensors(int n, int history, int blocks, int F, int V) {
    const int P = 2 * history + 2, A = n * n;
    std::vector<Tensor> t;
    int order = 0;
    auto weight = [&](const std::string& name, size_t size, int fan) { t.push_back({name, size, Kind::Weight, fan, order++}); };
    auto bn = [&](const std::string& p, size_t c) {
        t.push_back({p + ".gamma", c, Kind::One, 0, -1});
        t.push_back({p + ".beta", c, Kind::Zero, 0, -1});
    };
    weight("stem.conv.w", (size_t)F * P * 9, P * 9);
    bn("stem.bn", F);
    for (int i = 0; i < blocks; ++i) {
        const std::string p = "block" + std::to_string(i);
        weight(p + ".conv1.w", (size_t)F * F * 9, F * 9);
        bn(p + ".bn1", F);
        weight(p + ".conv2.w", (size_t)F * F * 9, F * 9);
        bn(p + ".bn2", F);
    }
    weight("policy.conv.w", 2 * (size_t)F, F);
    bn("policy.bn", 2);
    weight("policy.fc.w", (size_t)2 * A * (A + 1), 2 * A);
    t.push_back({"policy.fc.b", (size_t)A + 1, Kind::Zero, 0, -1});
    weight("value.conv.w", F, F);
    bn("value.bn", 1);
    weight("value.fc1.w", (size_t)A * V, A);
    t.push_back({"value.fc1.b", (size_t)V, Kind::Zero, 0, -1});
    weight("value.fc2.w", V, V);
    t.push_back({"value.fc2.b", 1, Kind::Zero, 0, -1});
    auto stats = [&](const std::string& p, size_t c) {
        t.push_back({p + ".runMean", c, Kind::Mean, 0, -1});
        t.push_back({p + ".runVar", c, Kind::Var, 0, -1});
    };
    stats("stem.bn", F);
    for (int i = 0; i < blocks; ++i) {
        const std::string p = "block" + std::to_string(i);
        stats(p + ".bn1", F);
        stats(p + ".bn2", F);
    }
    stats("policy.bn", 2);
    stats("value.bn", 1);
    return t;
}

} // namespace

extern "C" {

// The number of tensors; name/size of tensor i (params() then buffers()).
int azw_tensor_count(int n, int history, int blocks, int F, int V) {
    return static_cast<int>(tensors(n, history, blocks, F, V).size());
}
int azw_tensor_info(int n, int history, int blocks, int F, int V, int i, char* name, size_t cap, size_t* size) {
    const std::vector<Tensor> t = tensors(n, history, blocks, F, V);
    if (i < 0 || i >= static_cast<int>(t.size())) return -1;
    std::snprintf(name, cap, "%s", t[i].name.c_str());
    *size = t[i].size;
    return 0;
}

// Every tensor, concatenated in that order, into out (sum of sizes floats).
void azw_network(int n, int history, int blocks, int F, int V, uint64_t seed, float* out) {
    const std::vector<Tensor> t = tensors(n, history, blocks, F, V);
    std::vector<size_t> offset(t.size());
    size_t off = 0;
    for (size_t i = 0; i < t.size(); ++i) {
        offset[i] = off;
        off += t[i].size;
    }
    for (size_t i = 0; i < t.size(); ++i) {
        float* d = out + offset[i];
        const float v = t[i].kind == Kind::One ? 1.0f : 0.0f;
        for (size_t j = 0; j < t[i].size; ++j) d[j] = v;
    }
    Xoshiro weights(seed);
    for (int k = 0;; ++k) {
        size_t i = 0;
        while (i < t.size() && t[i].order != k) ++i;
        if (i == t.size()) break;
        const double sd = std::sqrt(2.0 / t[i].fanIn);
        for (size_t j = 0; j < t[i].size; ++j) out[offset[i] + j] = static_cast<float>(weights.normal() * sd);
    }
    Xoshiro stats(Xoshiro::derive(seed, 0xB4, 0, 0));
    for (size_t i = 0; i < t.size(); ++i) {
        if (t[i].kind == Kind::Mean)
            for (size_t j = 0; j < t[i].size; ++j) out[offset[i] + j] = static_cast<float>(0.1 * stats.normal());
        else if (t[i].kind == Kind::Var)
            for (size_t j = 0; j < t[i].size; ++j) out[offset[i] + j] = static_cast<float>(0.5 + stats.uniform());
    }
}

// B synthetic positions of workload `tag`: input [B][2H+2][n*n] and the
// legal-move mask [B][n*n+1] (empty points, and pass).
void azw_positions(int n, int history, int B, uint64_t seed, uint64_t tag, double pBlack, double pWhite,
                   float* input, uint8_t* legal) {
    const int A = n * n, P = 2 * history + 2;
    std::vector<uint8_t> stones(A);
    for (int i = 0; i < B; ++i) {
        Xoshiro rng(Xoshiro::derive(seed, tag, static_cast<uint64_t>(i), 0));
        for (int p = 0; p < A; ++p) {
            const double u = rng.uniform();
            stones[p] = u < pBlack ? 1 : (u < pBlack + pWhite ? 2 : 0);
        }
        const uint8_t toMove = rng.below(2) == 0 ? 1 : 2;
        const uint8_t opp = toMove == 1 ? 2 : 1;
        float* x = input + static_cast<size_t>(i) * P * A;
        std::memset(x, 0, sizeof(float) * static_cast<size_t>(P) * A);
        for (int p = 0; p < A; ++p) {
            if (stones[p] == toMove) x[p] = 1.0f;              // plane 0: own stones
            else if (stones[p] == opp) x[A + p] = 1.0f;        // plane 1: opponent's
        }
        float* colour = x + static_cast<size_t>(2 * history + (toMove == 1 ? 0 : 1)) * A;
        for (int p = 0; p < A; ++p) colour[p] = 1.0f;
        if (legal) {
            uint8_t* m = legal + static_cast<size_t>(i) * (A + 1);
            for (int p = 0; p < A; ++p) m[p] = stones[p] == 0;
            m[A] = 1;
        }
    }
}

// The same boards as azw_positions, as bytes: stones [B][n*n] (0 empty,
// 1 black, 2 white) and the side to move [B] (1 or 2).
void azw_stones(int n, int B, uint64_t seed, uint64_t tag, double pBlack, double pWhite, uint8_t* stones,
                uint8_t* toMove) {
    const int A = n * n;
    for (int i = 0; i < B; ++i) {
        Xoshiro rng(Xoshiro::derive(seed, tag, static_cast<uint64_t>(i), 0));
        uint8_t* s = stones + static_cast<size_t>(i) * A;
        for (int p = 0; p < A; ++p) {
            const double u = rng.uniform();
            s[p] = u < pBlack ? 1 : (u < pBlack + pWhite ? 2 : 0);
        }
        toMove[i] = rng.below(2) == 0 ? 1 : 2;
    }
}

} // extern "C"
