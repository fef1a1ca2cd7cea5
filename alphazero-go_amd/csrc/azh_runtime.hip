// The runtime behind include/azgo_hip.h: device context and architecture
// check, the upload contract (named tensors, checked against the network's
// params() and buffers()), weight packing and BN folding, per-slot device
// workspaces with pinned staging and their own stream, the pass as one
// hipGraph per batch size, the completion thread, timing entry points,
// kernel probes, the test hooks, and the .azn checkpoint reader.
//
// Compiled with -ffp-contract=off (host and device), so the host-side BN
// fold rounds exactly as BatchNorm2d::forwardInfer does (src/layers.cpp:91-92).
#include "azgo_hip.h"
#include "azh_kernels.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <mutex>
#include <semaphore.h>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#ifndef AZH_KERNEL_HASH
#define AZH_KERNEL_HASH "unhashed"
#endif
#ifndef AZH_CONV_HASH
#define AZH_CONV_HASH "unhashed"
#endif

namespace {

thread_local std::string gLastError;

struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw Error(AZH_ERR_HIP, std::string("hip: ") + what + ": " + hipGetErrorString(e));
}

template <class Fn>
int guarded(Fn&& fn) {
    try {
        fn();
        return AZH_OK;
    } catch (const Error& e) {
        gLastError = e.what();
        return e.code;
    } catch (const std::bad_alloc&) {
        gLastError = "hip: host memory exhausted";
        return AZH_ERR_MEMORY;
    } catch (const std::exception& e) {
        gLastError = e.what();
        return AZH_ERR_HIP;
    }
}

// The process-wide test hooks behind the azh_set_* / azh_fail_* entry points
// (their meaning is cuda_probe's, include/azgo/cuda.hpp:138-155). Every
// pass any runner reports gets the next report index; an injected failure
// names the index it hits, so it fires once, on exactly one pass, whichever
// runner's reporter gets there.
struct TestHooks {
    std::atomic<uint64_t> hubChaosSeed{0};
    std::atomic<long long> reports{0};         // passes reported so far
    std::atomic<long long> failingReport{-1};  // the report index to fail; -1: none
    std::atomic<size_t> memoryLimit{0};        // 0: the device's own free memory
    std::atomic<int> copyOutDelayUs{0};

    // Called once per reported pass: its report index, and whether the
    // injected failure lands on it.
    bool takeReport() {
        long long index = reports.fetch_add(1);
        return failingReport.compare_exchange_strong(index, -1);
    }
};
TestHooks gHooks;

constexpr int kMaxSlots = 2;   // kInferenceSlots (include/azgo/inference_hub.hpp:56)
// The workgroup shapes a probe may force (include/azgo_hip.h lists them).
const azh::ConvTiling* const kTilings = azh::kConvTilings;
constexpr int kTilingCount = azh::kConvTilingCount;

// ---------------------------------------------------------------- context

struct Context {
    bool ok = false;
    std::string why, name, arch;
    int runtime = 0;

    static Context& get() {
        static Context c;
        return c;
    }

  private:
    Context() {
        int count = 0;
        if (hipGetDeviceCount(&count) != hipSuccess || count < 1) {
            why = "no HIP device";
            return;
        }
        int dev = 0;
        hipDeviceProp_t p;
        if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&p, dev) != hipSuccess) {
            why = "cannot query the HIP device";
            return;
        }
        name = p.name;
        if (name.empty()) {
            char buf[256] = {};
            if (hipDeviceGetName(buf, sizeof buf, dev) == hipSuccess) name = buf;
        }
        if (name.empty()) name = "AMD GPU";
        arch = p.gcnArchName;
        const std::string base = arch.substr(0, arch.find(':'));
        (void)hipRuntimeGetVersion(&runtime);
        if (base != "gfx950") {
            why = "kernels built for gfx950; this GPU is " + base;
            return;
        }
        // A first kernel, so a missing or unloadable code object shows here.
        float* d = nullptr;
        float h[16] = {};
        if (hipMalloc(&d, sizeof h) != hipSuccess) {
            why = "cannot allocate device memory";
            return;
        }
        const bool ran = azh::launchFill(d, 16, 3.0f, nullptr) == hipSuccess &&
                         hipMemcpy(h, d, sizeof h, hipMemcpyDeviceToHost) == hipSuccess && h[0] == 3.0f &&
                         h[15] == 3.0f;
        (void)hipFree(d);
        if (!ran) {
            why = "the first kernel did not run";
            return;
        }
        ok = true;
    }
};

void requireContext() {
    Context& c = Context::get();
    if (!c.ok) throw Error(AZH_ERR_UNAVAILABLE, "hip: no usable GPU (" + c.why + ")");
}

} // namespace

// ---------------------------------------------------------------- the allocation-free pass's scratch

// The device memory azh_infer_noalloc works in (the trunk, the blocks'
// middle activations and the heads' rows; 256 boards of 19x19 at 128
// channels take 91.3 MiB of it): one array per device, there from the
// library's load until the process ends, shared by every such call on that
// device. Host code never hands the name `scratch` to a kernel (on the host
// it is only a stand-in for the symbol): it uses the device address that
// scratchOnCurrentDevice resolved.
constexpr size_t kScratchBytes = size_t(96) << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<float*> gScratchByDevice[kMaxDevices];   // null until resolved
std::mutex gScratchResolve;

// The scratch array's address on the current device, resolved (with that
// device current) the first time, then read without a lock.
float* scratchOnCurrentDevice() {
    int dev = 0;
    check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) throw Error(AZH_ERR_UNAVAILABLE, "hip: device index above 63");
    if (float* p = gScratchByDevice[dev].load(std::memory_order_acquire)) return p;
    std::lock_guard<std::mutex> lock(gScratchResolve);
    if (float* p = gScratchByDevice[dev].load(std::memory_order_acquire)) return p;
    void* p = nullptr;
    check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!p) throw Error(AZH_ERR_HIP, "hip: the scratch array has no device address");
    gScratchByDevice[dev].store(static_cast<float*>(p), std::memory_order_release);
    return static_cast<float*>(p);
}

// ---------------------------------------------------------------- network shape

struct Shape {
    int n, H, P, A, A1, F, V, blocks;
    bool ownership;
    explicit Shape(const azh_netcfg& c)
        : n(c.board), H(c.history), P(2 * c.history + 2), A(c.board * c.board), A1(c.board * c.board + 1),
          F(c.filters), V(c.value_hidden), blocks(c.blocks), ownership(c.ownership != 0) {}
};

void validate(const azh_netcfg* c) {
    if (!c) throw Error(AZH_ERR_ARGUMENT, "hip: no network config");
    if (!azh::conv3x3Supported(c->board))
        throw Error(AZH_ERR_ARGUMENT, "hip: board size " + std::to_string(c->board) + " not supported (5, 9, 13, 19)");
    if (c->history < 1 || c->blocks < 0 || c->filters < 1 || c->value_hidden < 1)
        throw Error(AZH_ERR_ARGUMENT, "hip: invalid network config");
    if (c->value_hidden > 256) throw Error(AZH_ERR_ARGUMENT, "hip: value_hidden above 256 not supported");
}

// Network::params() then Network::buffers() (src/network.cpp:113-165).
struct TensorSpec {
    std::string name;
    size_t size;
};
std::vector<TensorSpec> tensorSpec(const azh_netcfg& c) {
    const Shape s(c);
    const size_t F = s.F;
    std::vector<TensorSpec> t;
    auto bn = [&](const std::string& p, size_t ch) {
        t.push_back({p + ".gamma", ch});
        t.push_back({p + ".beta", ch});
    };
    t.push_back({"stem.conv.w", F * s.P * 9});
    bn("stem.bn", F);
    for (int i = 0; i < s.blocks; ++i) {
        const std::string p = "block" + std::to_string(i);
        t.push_back({p + ".conv1.w", F * F * 9});
        bn(p + ".bn1", F);
        t.push_back({p + ".conv2.w", F * F * 9});
        bn(p + ".bn2", F);
    }
    t.push_back({"policy.conv.w", 2 * F});
    bn("policy.bn", 2);
    t.push_back({"policy.fc.w", (size_t)2 * s.A * s.A1});
    t.push_back({"policy.fc.b", (size_t)s.A1});
    t.push_back({"value.conv.w", F});
    bn("value.bn", 1);
    t.push_back({"value.fc1.w", (size_t)s.A * s.V});
    t.push_back({"value.fc1.b", (size_t)s.V});
    t.push_back({"value.fc2.w", (size_t)s.V});
    t.push_back({"value.fc2.b", 1});
    if (s.ownership) {
        t.push_back({"ownership.conv.w", F});
        bn("ownership.bn", 1);
    }
    auto stats = [&](const std::string& p, size_t ch) {
        t.push_back({p + ".runMean", ch});
        t.push_back({p + ".runVar", ch});
    };
    stats("stem.bn", F);
    for (int i = 0; i < s.blocks; ++i) {
        const std::string p = "block" + std::to_string(i);
        stats(p + ".bn1", F);
        stats(p + ".bn2", F);
    }
    stats("policy.bn", 2);
    stats("value.bn", 1);
    if (s.ownership) stats("ownership.bn", 1);
    return t;
}

// ---------------------------------------------------------------- weights

struct ConvW {
    const float* w;   // packed MFMA fragments
    const float* scale;
    const float* shift;
};

struct DeviceWeights {
    float* arena = nullptr;
    size_t bytes = 0;
    ConvW stem{};
    std::vector<ConvW> conv1, conv2;
    azh::HeadWeights heads{};
    ~DeviceWeights() {
        if (arena) (void)hipFree(arena);
    }
};

size_t alignFloats(size_t f) { return (f + 63) / 64 * 64; }   // 256-byte offsets

size_t weightFloats(const azh_netcfg& c) {
    const Shape s(c);
    size_t f = 0;
    f += alignFloats(azh::packedConv3x3Floats(s.P, s.F)) + 2 * alignFloats(s.F);
    f += (size_t)s.blocks * 2 * (alignFloats(azh::packedConv3x3Floats(s.F, s.F)) + 2 * alignFloats(s.F));
    f += alignFloats(4 * s.F) + 2 * alignFloats(4);
    f += alignFloats(azh::headPolicyWTFloats(s.n)) + alignFloats(s.A1);
    f += alignFloats(azh::headFc1WTFloats(s.n, s.V)) + alignFloats(s.V) + alignFloats(s.V) + alignFloats(1);
    return f;
}

// BatchNorm2d::forwardInfer's fold (src/layers.cpp:91-92), in float with
// each operation rounded on its own.
void foldBn(const float* gamma, const float* beta, const float* mean, const float* var, int C, float* scale,
            float* shift) {
    for (int ch = 0; ch < C; ++ch) {
        scale[ch] = gamma[ch] / std::sqrt(var[ch] + 1e-5f);
        shift[ch] = beta[ch] - scale[ch] * mean[ch];
    }
}

// Checks the tensors against the spec (CudaWeights::upload's contract,
// src/cuda/cuda_network.cu:24-41, 71-106): exactly the network's tensors, each
// once, with its size. Host-only, so it runs before any device work.
std::map<std::string, const float*> checkTensors(const azh_netcfg& c, const azh_tensor* tensors, int count) {
    const std::vector<TensorSpec> spec = tensorSpec(c);
    std::map<std::string, const float*> given;
    if (count < 0 || (count > 0 && !tensors)) throw Error(AZH_ERR_ARGUMENT, "hip: no tensors");
    for (int i = 0; i < count; ++i) {
        const azh_tensor& t = tensors[i];
        if (!t.name) throw Error(AZH_ERR_TENSOR, "hip: a tensor without a name");
        const std::string name = t.name;
        const auto it = std::find_if(spec.begin(), spec.end(), [&](const TensorSpec& x) { return x.name == name; });
        if (it == spec.end())
            throw Error(AZH_ERR_TENSOR, "hip: tensor '" + name + "' is not read by this backend's pass");
        if (t.size != it->size)
            throw Error(AZH_ERR_TENSOR, "hip: tensor '" + name + "' has " + std::to_string(t.size) +
                                            " floats, expected " + std::to_string(it->size));
        if (!t.data) throw Error(AZH_ERR_TENSOR, "hip: tensor '" + name + "' has no data");
        if (!given.emplace(name, t.data).second)
            throw Error(AZH_ERR_TENSOR, "hip: tensor '" + name + "' given twice");
    }
    for (const TensorSpec& x : spec)
        if (!given.count(x.name)) throw Error(AZH_ERR_TENSOR, "hip: tensor '" + x.name + "' missing");
    return given;
}

// ---------------------------------------------------------------- checkpoints (.azn)

// The checkpoint format of saveNetwork / loadNetwork (src/checkpoint.cpp:84-124,
// include/azgo/checkpoint.hpp:12-18), little-endian throughout: u32 magic
// 0x4F475A41 ("AZGO"), u32 version (1; 2 adds the ownership flag), i32 board,
// history, blocks, filters, value_hidden, in version 2 an i32 ownership flag
// (0 or 1), u32 tensor count, then per tensor a u32 name length and the
// name's bytes, a u64 float count and the floats (IEEE-754 bits), params()
// then buffers() order. Failures read as loadNetwork's: the message names
// the file and the problem, and running out of data is "truncated".
constexpr uint32_t kAznMagic = 0x4F475A41;
constexpr uint32_t kAznPlain = 1, kAznOwnership = 2;

struct Truncated {};

class AznReader {
public:
    explicit AznReader(const std::string& path) : path_(path), in_(path, std::ios::binary) {
        if (!in_) throw Error(AZH_ERR_FORMAT, "cannot open checkpoint " + path);
    }
    [[noreturn]] void fail(const std::string& what) const { throw Error(AZH_ERR_FORMAT, path_ + ": " + what); }
    void bytes(void* p, size_t n) {
        in_.read(static_cast<char*>(p), static_cast<std::streamsize>(n));
        if (static_cast<size_t>(in_.gcount()) != n) throw Truncated{};
    }
    uint32_t u32() {
        unsigned char b[4];
        bytes(b, 4);
        return uint32_t(b[0]) | uint32_t(b[1]) << 8 | uint32_t(b[2]) << 16 | uint32_t(b[3]) << 24;
    }
    uint64_t u64() {
        const uint64_t lo = u32();
        return lo | uint64_t(u32()) << 32;
    }
    int32_t i32() { return static_cast<int32_t>(u32()); }
    std::string str(size_t limit) {
        const uint32_t len = u32();
        if (len > limit) fail("tensor name of " + std::to_string(len) + " bytes");
        std::string s(len, '\0');
        if (len) bytes(&s[0], len);
        return s;
    }
    void floats(float* out, size_t n) {
        static_assert(sizeof(float) == 4, "IEEE-754 binary32");
        unsigned char buf[4096];
        while (n > 0) {
            const size_t count = std::min(n, sizeof buf / 4);
            bytes(buf, 4 * count);
            for (size_t i = 0; i < count; ++i) {
                const uint32_t bits = uint32_t(buf[4 * i]) | uint32_t(buf[4 * i + 1]) << 8 |
                                      uint32_t(buf[4 * i + 2]) << 16 | uint32_t(buf[4 * i + 3]) << 24;
                std::memcpy(out + i, &bits, 4);
            }
            out += count;
            n -= count;
        }
    }
    bool atEnd() { return in_.peek() == std::char_traits<char>::eof(); }

    // The header (readHeader, src/checkpoint.cpp:37-60), with the shape
    // ranges the reference's config accepts (kMaxBlocks 40, kMaxFilters 512,
    // include/azgo/config.hpp:20-21).
    azh_netcfg header() {
        if (u32() != kAznMagic) fail("not an AZGO checkpoint");
        const uint32_t version = u32();
        if (version != kAznPlain && version != kAznOwnership) fail("unsupported version " + std::to_string(version));
        azh_netcfg c{};
        c.board = i32();
        c.history = i32();
        c.blocks = i32();
        c.filters = i32();
        c.value_hidden = i32();
        c.ownership = 0;
        if (version == kAznOwnership) {
            const int32_t flag = i32();
            if (flag != 0 && flag != 1) fail("invalid ownership flag in header");
            c.ownership = flag;
        }
        if (c.board < 5 || c.board > 19 || c.history < 1 || c.history > 16 || c.blocks < 0 || c.blocks > 40 ||
            c.filters < 1 || c.filters > 512 || c.value_hidden < 1 || c.value_hidden > 1024)
            fail("invalid network shape in header");
        return c;
    }

    // Every tensor, checked by position, name and size against the network
    // the header describes (loadNetwork, src/checkpoint.cpp:102-124), into
    // one array in file order.
    std::vector<float> tensors(const std::vector<TensorSpec>& spec) {
        size_t total = 0;
        for (const TensorSpec& t : spec) total += t.size;
        const uint32_t count = u32();
        if (count != spec.size())
            fail("has " + std::to_string(count) + " tensors but the network needs " + std::to_string(spec.size()));
        std::vector<float> values(total);
        size_t off = 0;
        for (size_t i = 0; i < spec.size(); ++i) {
            const std::string name = str(4096);
            if (name != spec[i].name)
                fail("tensor " + std::to_string(i) + " is '" + name + "' but expected '" + spec[i].name + "'");
            const uint64_t size = u64();
            if (size != spec[i].size)
                fail("tensor '" + name + "' has " + std::to_string(size) + " values but expected " +
                     std::to_string(spec[i].size));
            floats(values.data() + off, spec[i].size);
            off += spec[i].size;
        }
        if (!atEnd()) fail("unexpected data after the last tensor");
        return values;
    }

    template <class Fn>
    static auto read(const std::string& path, Fn&& fn) {
        AznReader r(path);
        try {
            return fn(r);
        } catch (const Truncated&) {
            r.fail("truncated");
        }
    }

private:
    std::string path_;
    std::ifstream in_;
};

// Packs, folds and uploads checked tensors into one device arena.
void uploadWeights(const azh_netcfg& c, const std::map<std::string, const float*>& given, DeviceWeights& dw) {
    const Shape s(c);
    auto T = [&](const std::string& name) { return given.at(name); };

    std::vector<float> host(weightFloats(c), 0.0f);
    size_t off = 0;
    auto take = [&](size_t floats) {
        const size_t o = off;
        off += alignFloats(floats);
        return o;
    };
    struct ConvOff {
        size_t w, scale, shift;
    };
    auto conv = [&](const std::string& wname, const std::string& bn, int cin) {
        ConvOff o;
        const std::vector<float> packed = azh::packConv3x3(T(wname), cin, s.F);
        o.w = take(packed.size());
        std::copy(packed.begin(), packed.end(), host.begin() + o.w);
        o.scale = take(s.F);
        o.shift = take(s.F);
        foldBn(T(bn + ".gamma"), T(bn + ".beta"), T(bn + ".runMean"), T(bn + ".runVar"), s.F, &host[o.scale],
               &host[o.shift]);
        return o;
    };
    const ConvOff stem = conv("stem.conv.w", "stem.bn", s.P);
    std::vector<ConvOff> c1, c2;
    for (int i = 0; i < s.blocks; ++i) {
        const std::string p = "block" + std::to_string(i);
        c1.push_back(conv(p + ".conv1.w", p + ".bn1", s.F));
        c2.push_back(conv(p + ".conv2.w", p + ".bn2", s.F));
    }
    // The heads' 1x1 rows: policy 0-1, value 2, ownership 3 (zero without the head).
    const size_t hConv = take(4 * s.F), hScale = take(4), hShift = take(4);
    std::copy(T("policy.conv.w"), T("policy.conv.w") + 2 * s.F, host.begin() + hConv);
    std::copy(T("value.conv.w"), T("value.conv.w") + s.F, host.begin() + hConv + 2 * s.F);
    foldBn(T("policy.bn.gamma"), T("policy.bn.beta"), T("policy.bn.runMean"), T("policy.bn.runVar"), 2,
           &host[hScale], &host[hShift]);
    foldBn(T("value.bn.gamma"), T("value.bn.beta"), T("value.bn.runMean"), T("value.bn.runVar"), 1,
           &host[hScale + 2], &host[hShift + 2]);
    if (s.ownership) {
        std::copy(T("ownership.conv.w"), T("ownership.conv.w") + s.F, host.begin() + hConv + 3 * s.F);
        foldBn(T("ownership.bn.gamma"), T("ownership.bn.beta"), T("ownership.bn.runMean"), T("ownership.bn.runVar"),
               1, &host[hScale + 3], &host[hShift + 3]);
    }
    // The head Linears transposed ([in][out]) and zero-padded to whole 16 x 16
    // MFMA blocks.
    const size_t np = azh::headPolicyWTFloats(s.n) / (size_t)((2 * s.A + 15) / 16 * 16);
    const size_t pW = take(azh::headPolicyWTFloats(s.n)), pB = take(s.A1);
    const float* pw = T("policy.fc.w");   // [A+1][2A]
    for (int a = 0; a < s.A1; ++a)
        for (int i = 0; i < 2 * s.A; ++i) host[pW + (size_t)i * np + a] = pw[(size_t)a * 2 * s.A + i];
    std::copy(T("policy.fc.b"), T("policy.fc.b") + s.A1, host.begin() + pB);
    const size_t f1W = take(azh::headFc1WTFloats(s.n, s.V)), f1B = take(s.V), f2W = take(s.V), f2B = take(1);
    const float* w1 = T("value.fc1.w");   // [V][A]
    const size_t vp = (size_t)(s.V + 15) / 16 * 16;
    for (int v = 0; v < s.V; ++v)
        for (int p = 0; p < s.A; ++p) host[f1W + (size_t)p * vp + v] = w1[(size_t)v * s.A + p];
    std::copy(T("value.fc1.b"), T("value.fc1.b") + s.V, host.begin() + f1B);
    std::copy(T("value.fc2.w"), T("value.fc2.w") + s.V, host.begin() + f2W);
    host[f2B] = T("value.fc2.b")[0];

    dw.bytes = host.size() * sizeof(float);
    check(hipMalloc(&dw.arena, dw.bytes), "hipMalloc(weights)");
    check(hipMemcpy(dw.arena, host.data(), dw.bytes, hipMemcpyHostToDevice), "hipMemcpy(weights)");
    const float* base = dw.arena;
    auto mk = [&](const ConvOff& o) { return ConvW{base + o.w, base + o.scale, base + o.shift}; };
    dw.stem = mk(stem);
    for (int i = 0; i < s.blocks; ++i) {
        dw.conv1.push_back(mk(c1[i]));
        dw.conv2.push_back(mk(c2[i]));
    }
    dw.heads = azh::HeadWeights{base + hConv, base + hScale, base + hShift, base + pW, base + pB,
                                base + f1W,   base + f1B,    base + f2W,    base + f2B};
}

// ---------------------------------------------------------------- slots

size_t slotFloats(const Shape& s, int maxBatch) {
    const size_t B = maxBatch;
    return alignFloats(B * s.P * s.A) + 2 * alignFloats(azh::quadFloats(B, s.F, s.A)) + alignFloats(B * 3 * s.A) +
           alignFloats(B * s.A1) + alignFloats(B) + (s.ownership ? alignFloats(B * s.A) : 0);
}

// Floats of scratch an allocation-free pass of B boards takes: the trunk and
// the middle activations in channel quads, then the heads' rows, each
// 256-byte aligned.
size_t noallocScratchFloats(const Shape& sh, int B) {
    return 2 * alignFloats(azh::quadFloats(B, sh.F, sh.A)) + alignFloats((size_t)B * 3 * sh.A);
}

size_t runnerBytes(const azh_netcfg& c, int maxBatch, int slots) {
    return (size_t)slots * slotFloats(Shape(c), maxBatch) * sizeof(float) + weightFloats(c) * sizeof(float);
}

// A batch of positions staged on the device (azh_evaluate_positions).
struct PositionsOnDevice {
    const uint8_t* stones = nullptr;   // [B][H][A]
    const int* plies = nullptr;        // [B]
    const uint8_t* turn = nullptr;     // [B]
    const uint8_t* sym = nullptr;      // [B]
    const long long* offsets = nullptr;   // [B+1]
    const uint64_t* seen = nullptr;
    uint8_t* legal = nullptr;          // [B][A+1]
    float* mapped = nullptr;           // [B][A+1]
    float* priors = nullptr;           // [B][A+1]
};

// A device allocation released on scope exit (the synchronous kernel entry points).
struct DeviceBuffer {
    void* p = nullptr;
    explicit DeviceBuffer(size_t bytes) {
        if (bytes) check(hipMalloc(&p, bytes), "hipMalloc");
    }
    ~DeviceBuffer() {
        if (p) (void)hipFree(p);
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    template <class T>
    T* as() const {
        return static_cast<T*>(p);
    }
};

// A device allocation that grows to the largest size asked of it.
struct GrowingBuffer {
    void* p = nullptr;
    size_t cap = 0;
    void* reserve(size_t bytes) {
        if (bytes > cap) {
            if (p) (void)hipFree(p);
            p = nullptr;
            cap = 0;
            check(hipMalloc(&p, bytes), "hipMalloc");
            cap = bytes;
        }
        return p;
    }
    ~GrowingBuffer() {
        if (p) (void)hipFree(p);
    }
};

// Pinned host memory that grows to the largest size asked of it. Only while
// nothing in flight reads the old block (its slot idle).
struct PinnedBuffer {
    void* p = nullptr;
    size_t cap = 0;
    void* reserve(size_t bytes) {
        if (bytes > cap) {
            if (p) (void)hipHostFree(p);
            p = nullptr;
            cap = 0;
            check(hipHostMalloc(&p, bytes, hipHostMallocDefault), "hipHostMalloc(positions)");
            cap = bytes;
        }
        return p;
    }
    ~PinnedBuffer() {
        if (p) (void)hipHostFree(p);
    }
};

// Where B positions' arrays sit, in bytes from the start of a slot's
// positions block, packed for B (each part 256-byte aligned): the inputs
// [0, inputEnd), then the outputs [mapped, end). Host staging and device
// block share it, so the inputs go up in one copy and the outputs come back
// in one. Every offset grows with B, so the block sized for maxBatch holds
// any B's layout.
struct PositionsLayout {
    size_t stones, plies, turn, sym, offsets, inputEnd, mapped, priors, legal, end;
    PositionsLayout(size_t B, size_t H, size_t A, size_t A1) {
        size_t off = 0;
        auto take = [&](size_t bytes) {
            const size_t o = off;
            off += (bytes + 255) / 256 * 256;
            return o;
        };
        stones = take(B * H * A);
        plies = take(B * sizeof(int));
        turn = take(B);
        sym = take(B);
        offsets = take((B + 1) * sizeof(int64_t));
        inputEnd = off;
        mapped = take(B * A1 * sizeof(float));
        priors = take(B * A1 * sizeof(float));
        legal = take(B * A1);
        end = off;
    }
};

// The inputs a batch of positions brings (azh_positions), checked on the
// host before anything reaches the GPU: every index the kernels form from
// them then stays inside its array.
void checkPositions(const uint8_t* stones, size_t stoneBytes, const int32_t* plies, const uint8_t* toMove,
                    const uint8_t* sym, const int64_t* seenOffsets, const uint64_t* seen, int B, int H) {
    if (!stones || !toMove || !seenOffsets) throw Error(AZH_ERR_ARGUMENT, "hip: positions need stones, to_move and seen_offsets");
    uint8_t top = 0;   // the largest byte: one vectorisable pass, no early exit
    for (size_t i = 0; i < stoneBytes; ++i) top = std::max(top, stones[i]);
    if (top > 2) throw Error(AZH_ERR_ARGUMENT, "hip: a stone byte is not Empty (0), Black (1) or White (2)");
    for (int b = 0; b < B; ++b) {
        if (toMove[b] != 1 && toMove[b] != 2)
            throw Error(AZH_ERR_ARGUMENT, "hip: position " + std::to_string(b) + " has no side to move (1 or 2)");
        if (plies && (plies[b] < 1 || plies[b] > H))
            throw Error(AZH_ERR_ARGUMENT, "hip: position " + std::to_string(b) + " has " + std::to_string(plies[b]) +
                                              " plies of history, outside [1, " + std::to_string(H) + "]");
        if (sym && sym[b] > 7) throw Error(AZH_ERR_ARGUMENT, "hip: symmetry outside [0, 8)");
    }
    if (seenOffsets[0] < 0) throw Error(AZH_ERR_ARGUMENT, "hip: seen_offsets[0] is negative");
    for (int b = 0; b < B; ++b)
        if (seenOffsets[b + 1] < seenOffsets[b]) throw Error(AZH_ERR_ARGUMENT, "hip: seen_offsets decrease");
    if (seenOffsets[B] > 0 && !seen) throw Error(AZH_ERR_ARGUMENT, "hip: seen hashes missing");
}

struct Slot {
    hipStream_t stream = nullptr;
    hipEvent_t event = nullptr;
    // A large pass runs as two half-batch chains, the second on `aux`,
    // forked from and joined back into `stream` (azh_runner::launchPass).
    hipStream_t aux = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    float* dev = nullptr;
    float *dIn = nullptr, *dX = nullptr, *dMid = nullptr, *dAct = nullptr, *dLogits = nullptr, *dValues = nullptr;
    float* dOwn = nullptr;   // [B][A] after tanh, only with the ownership head
    float *hIn = nullptr, *hLogits = nullptr, *hValues = nullptr;
    // Captured passes by key (batch size and tower form), with the last
    // time each was replayed (a count of replays on this slot), so the
    // least recently replayed one goes when the cache is full.
    struct CachedGraph {
        hipGraphExec_t exec;
        unsigned long long lastUse;
    };
    std::map<int, CachedGraph> graphs;
    unsigned long long replays = 0;
    // Set while a pass or a synchronous call holds the slot.
    std::atomic<bool> claimed{false};
    // The positions path (azh_evaluate_positions, azh_begin_positions),
    // allocated on first use: the device block (PositionsLayout at
    // maxBatch) and the concatenated superko hashes (grown as needed), and
    // their pinned host sides: the inputs staged for the copy up, the
    // hashes, and the outputs of the last azh_begin_positions (of posLastB
    // positions; values go to hValues).
    GrowingBuffer posBytes, posSeen;
    PinnedBuffer posIn, posSeenIn, posOut;
    int posLastB = 0;

    Slot(const Shape& s, int maxBatch) {
        const size_t B = maxBatch;
        check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
        // Blocking sync: the completion thread sleeps in the driver until the
        // pass's end wakes it, without spinning a core and without the
        // tens of microseconds a timed sleep overshoots by (on small passes
        // that overshoot was up to 40% of the runner-kept-full rate).
        check(hipEventCreateWithFlags(&event, hipEventDisableTiming | hipEventBlockingSync), "hipEventCreate");
        check(hipStreamCreateWithFlags(&aux, hipStreamNonBlocking), "hipStreamCreate");
        check(hipEventCreateWithFlags(&fork, hipEventDisableTiming), "hipEventCreate");
        check(hipEventCreateWithFlags(&join, hipEventDisableTiming), "hipEventCreate");
        check(hipMalloc(&dev, slotFloats(s, maxBatch) * sizeof(float)), "hipMalloc(workspace)");
        size_t off = 0;
        auto take = [&](size_t f) {
            float* p = dev + off;
            off += alignFloats(f);
            return p;
        };
        dIn = take(B * s.P * s.A);
        dX = take(azh::quadFloats(B, s.F, s.A));     // trunk activations in channel quads
        dMid = take(azh::quadFloats(B, s.F, s.A));
        dAct = take(B * 3 * s.A);
        dLogits = take(B * s.A1);
        dValues = take(B);
        if (s.ownership) dOwn = take(B * s.A);
        check(hipHostMalloc((void**)&hIn, B * s.P * s.A * sizeof(float), hipHostMallocDefault), "hipHostMalloc");
        check(hipHostMalloc((void**)&hLogits, B * s.A1 * sizeof(float), hipHostMallocDefault), "hipHostMalloc");
        check(hipHostMalloc((void**)&hValues, B * sizeof(float), hipHostMallocDefault), "hipHostMalloc");
        std::fill(hIn, hIn + B * s.P * s.A, 0.0f);
    }
    ~Slot() {
        if (stream) (void)hipStreamSynchronize(stream);
        if (aux) (void)hipStreamSynchronize(aux);
        for (auto& g : graphs) (void)hipGraphExecDestroy(g.second.exec);
        if (event) (void)hipEventDestroy(event);
        if (fork) (void)hipEventDestroy(fork);
        if (join) (void)hipEventDestroy(join);
        if (aux) (void)hipStreamDestroy(aux);
        if (stream) (void)hipStreamDestroy(stream);
        if (dev) (void)hipFree(dev);
        if (hIn) (void)hipHostFree(hIn);
        if (hLogits) (void)hipHostFree(hLogits);
        if (hValues) (void)hipHostFree(hValues);
    }
};

// Holds a slot for a synchronous call's scope, so that neither a pass begun
// meanwhile nor another call can use its buffers and streams.
class SlotClaim {
public:
    Slot& slot;
    SlotClaim(Slot& s, int index) : slot(s) {
        bool idle = false;
        if (!s.claimed.compare_exchange_strong(idle, true))
            throw Error(AZH_ERR_STATE, "hip: slot " + std::to_string(index) + " has a pass in flight");
    }
    ~SlotClaim() { slot.claimed.store(false, std::memory_order_release); }
    SlotClaim(const SlotClaim&) = delete;
    SlotClaim& operator=(const SlotClaim&) = delete;
};

// ---------------------------------------------------------------- memory admission

// Device bytes that runners may still take: the device's free memory less a
// 512 MB reserve kept for the HIP runtime and the rest of the process (the
// reserve the reference's CUDA runner keeps, src/cuda/cuda_runner.cu:50), or
// the test hook's stand-in when one is set.
double spendableDeviceBytes() {
    if (const size_t limit = gHooks.memoryLimit.load()) return (double)limit;
    size_t freeBytes = 0, totalBytes = 0;
    check(hipMemGetInfo(&freeBytes, &totalBytes), "hipMemGetInfo");
    constexpr double kReserve = 512.0 * 1024 * 1024;
    return std::max(0.0, (double)freeBytes - kReserve);
}

// Every runner a process holds on the GPU at once, as groups of identical
// runners (GpuHubs, include/azgo/gpu_memory.hpp), admitted or refused as one
// sum. The refusal's wording is the reference's, which its callers and
// users read (src/cuda/cuda_runner.cu:206-223): whole MB, the hub count when
// above one, the largest batch, and "lower inference_batch" last.
void admitRunners(const azh_netcfg& cfg, const azh_hub_group* groups, int count) {
    if (count < 1 || !groups) throw Error(AZH_ERR_ARGUMENT, "checkHipInferenceMemory: no hubs");
    double need = 0.0;
    int hubs = 0, widest = 0;
    for (const azh_hub_group* g = groups; g != groups + count; ++g) {
        if (g->hubs < 1 || g->slots_per_hub < 1 || g->max_batch < 1)
            throw Error(AZH_ERR_ARGUMENT, "checkHipInferenceMemory: bad arguments");
        need += (double)g->hubs * (double)runnerBytes(cfg, g->max_batch, g->slots_per_hub);
        hubs += g->hubs;
        widest = std::max(widest, g->max_batch);
    }
    requireContext();
    const double room = spendableDeviceBytes();
    if (need <= room) return;
    const auto wholeMB = [](double bytes) { return std::to_string((long long)(bytes / 1e6)); };
    std::string refusal = "hip: inference needs " + wholeMB(need) + " MB of GPU memory at inference_batch " +
                          std::to_string(widest);
    if (hubs > 1) refusal += " (" + std::to_string(hubs) + " hubs)";
    refusal += ", more than the " + wholeMB(room) + " MB the GPU has free; lower inference_batch";
    throw Error(AZH_ERR_MEMORY, refusal);
}

template <class Body>
float timeOnStream(hipStream_t stream, int iters, Body body) {
    hipEvent_t a = nullptr, b = nullptr;
    check(hipEventCreate(&a), "hipEventCreate");
    check(hipEventCreate(&b), "hipEventCreate");
    float ms = 0.0f;
    try {
        check(hipEventRecord(a, stream), "hipEventRecord");
        for (int i = 0; i < iters; ++i) body();
        check(hipEventRecord(b, stream), "hipEventRecord");
        check(hipEventSynchronize(b), "hipEventSynchronize");
        check(hipEventElapsedTime(&ms, a, b), "hipEventElapsedTime");
    } catch (...) {
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
        throw;
    }
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return ms;
}

// ---------------------------------------------------------------- the reporter

// Reports a runner's passes: calls each pass's done exactly once, in the
// order the passes were begun, from a thread of its own, once the event the
// pass recorded behind its copy-out has fired (BatchRunner::begin's contract,
// include/azgo/inference_hub.hpp:47-50).
//
// A slot holds at most one pass, so no more than kMaxSlots notices, plus the
// closing one, are ever waiting: they sit in a fixed ring, and a counting
// semaphore hands each to the thread. Closing posts a last notice that the
// thread reaches only after every earlier one, so every pass begun before
// it is reported before the thread ends and the slots may go.
class Reporter {
public:
    struct Notice {
        int slot = -1;                        // -1: the closing notice
        hipEvent_t event = nullptr;           // recorded after the pass's copy-out
        std::atomic<bool>* claim = nullptr;   // the slot's claim, released before done
        azh_done_fn done = nullptr;
        void* user = nullptr;
        std::string error;                    // from enqueueing the pass, if that failed
    };

    Reporter() {
        if (sem_init(&posted_, 0, 0) != 0) throw Error(AZH_ERR_HIP, "hip: cannot create the reporter's semaphore");
    }
    ~Reporter() {
        close();
        sem_destroy(&posted_);
    }
    Reporter(const Reporter&) = delete;
    Reporter& operator=(const Reporter&) = delete;

    void start() { thread_ = std::thread([this] { run(); }); }

    // Hands a begun pass (or the closing notice) to the thread.
    void post(Notice notice) {
        {
            std::lock_guard<std::mutex> lock(writing_);
            if (written_ - taken_.load(std::memory_order_acquire) >= kRing)
                throw Error(AZH_ERR_STATE, "hip: more passes waiting to be reported than the runner has slots");
            ring_[written_ % kRing] = std::move(notice);
            ++written_;
        }
        sem_post(&posted_);
    }

    // Reports every pass posted so far, then ends the thread.
    void close() {
        if (!thread_.joinable()) return;
        post(Notice{});
        thread_.join();
    }

private:
    static constexpr size_t kRing = kMaxSlots + 1;

    // A pass's end: polled for up to kPollUs (a small network's pass ends
    // within it, and the driver's wake-up from a blocking wait costs tens of
    // microseconds), then slept on (the slots' events are blocking-sync).
    static constexpr int kPollUs = 50;
    static hipError_t waitFor(hipEvent_t e) {
        const auto until = std::chrono::steady_clock::now() + std::chrono::microseconds(kPollUs);
        for (;;) {
            const hipError_t q = hipEventQuery(e);
            if (q != hipErrorNotReady) return q;
            if (std::chrono::steady_clock::now() >= until) break;
        }
        return hipEventSynchronize(e);
    }

    void run() {
        for (size_t next = 0;; ++next) {
            while (sem_wait(&posted_) != 0) {   // only a signal interrupts it
            }
            Notice n = std::move(ring_[next % kRing]);
            taken_.store(next + 1, std::memory_order_release);
            if (n.slot < 0) return;
            std::string error = std::move(n.error);
            const hipError_t e = waitFor(n.event);
            if (error.empty() && e != hipSuccess) error = std::string("hip: ") + hipGetErrorString(e);
            if (gHooks.takeReport() && error.empty()) error = "hip: injected failure (a test hook)";
            n.claim->store(false, std::memory_order_release);   // done may begin the slot again
            n.done(n.user, n.slot, error.empty() ? nullptr : error.c_str());
        }
    }

    Notice ring_[kRing];
    std::mutex writing_;      // begin may come from more than one thread
    size_t written_ = 0;      // under writing_
    std::atomic<size_t> taken_{0};
    sem_t posted_;
    std::thread thread_;
};

} // namespace

// ---------------------------------------------------------------- the runner

struct azh_runner {
    azh_netcfg cfg{};
    Shape shape;
    int maxBatch = 0;
    DeviceWeights weights;
    std::vector<std::unique_ptr<Slot>> slots;
    bool graphs = true;
    // The whole pass in one launch on small boards (azh::launchSmallTower):
    // allowed (a test hook turns it off), and the tower convolutions' place
    // in the weight arena (one fixed stride; `tower.ok` once checked).
    bool smallTower = true;
    // The board-resident tower (azh::launchResidentTower): 0 never, 1 for a
    // pass alone on the device whose batch fills its rounds of CUs
    // (useResidentTower), 2 wherever the network allows it (a test hook).
    int residentTower = 1;
    struct TowerLayout {
        bool ok = false;
        const float* w0 = nullptr;
        size_t stride = 0, scaleOff = 0, shiftOff = 0;
    } tower;

    Reporter reporter;
    int device = 0;   // where the weights and slots live

    azh_runner(const azh_netcfg& c, int mb) : cfg(c), shape(c), maxBatch(mb) {}

    // The reporter goes first: closing it reports every pass begun, whose
    // slots (events, pinned outputs) must still be there meanwhile.
    ~azh_runner() {
        reporter.close();
        slots.clear();
    }

    // The residual tower's first `blocksToRun` blocks on a trunk of Bp
    // boards (x in place; mid, the blocks' middle activations), workgroup
    // shape t, on `stream`: each block's second convolution reads the skip
    // at exactly the element it writes. Returns the number of launches.
    int launchTowerOn(float* x, float* mid, int Bp, azh::ConvTiling t, hipStream_t stream, int blocksToRun) {
        const Shape& sh = shape;
        for (int i = 0; i < blocksToRun; ++i) {
            const ConvW& a = weights.conv1[i];
            const ConvW& b = weights.conv2[i];
            check(azh::launchConv3x3(x, a.w, a.scale, a.shift, nullptr, mid, Bp, sh.n, sh.F, sh.F, true, false, t,
                                     stream),
                  "conv3x3 (conv1)");
            check(azh::launchConv3x3(mid, b.w, b.scale, b.shift, x, x, Bp, sh.n, sh.F, sh.F, true, false, t, stream),
                  "conv3x3 (conv2)");
        }
        return 2 * std::max(blocksToRun, 0);
    }

    // The residual tower over slot s's whole batch on one stream, every
    // launch over all B boards (the tower kernel as timed on its own).
    int launchTower(Slot& s, int B, hipStream_t stream, int blocksToRun, bool alone) {
        return launchTowerOn(s.dX, s.dMid, B, azh::chooseConvTiling(shape.F, B, shape.n, alone), stream,
                             blocksToRun);
    }

    // Whether no slot but `except` (null: none) has a pass in flight or a
    // synchronous call running: a pass enqueued now has the device to
    // itself, as far as this runner knows (the workgroup shapes then may
    // take every CU, chooseConvTiling).
    bool othersIdle(const Slot* except) const {
        for (const auto& o : slots)
            if (o.get() != except && o->claimed.load(std::memory_order_acquire)) return false;
        return true;
    }

    // Where a pass over Bp boards reads and writes: the input planes
    // [Bp][P][A], the trunk and the blocks' middle activations (channel
    // quads), the heads' rows [Bp][3][A], and the outputs (own may be null:
    // no ownership).
    struct PassBuffers {
        const float* in;
        float *x, *mid, *act, *logits, *values, *own;
    };
    // Slot s's buffers from board b0 on.
    PassBuffers slotBuffers(Slot& s, int b0) const {
        const Shape& sh = shape;
        const size_t trunk = azh::quadFloats(1, sh.F, sh.A);   // floats per board
        return PassBuffers{s.dIn + (size_t)b0 * sh.P * sh.A,  s.dX + b0 * trunk,
                           s.dMid + b0 * trunk,               s.dAct + (size_t)b0 * 3 * sh.A,
                           s.dLogits + (size_t)b0 * sh.A1,    s.dValues + b0,
                           s.dOwn ? s.dOwn + (size_t)b0 * sh.A : nullptr};
    }

    // A pass over Bp boards on `stream`: the stem, `blocksToRun` residual
    // blocks, then the heads when asked; workgroup shape t (the shape
    // decides only which workgroup computes an output, never how, so a
    // part's bits are the whole batch's).
    void launchPassPart(const PassBuffers& io, int Bp, int Bpass, azh::ConvTiling t, hipStream_t stream,
                        int blocksToRun, bool heads, bool small) {
        const Shape& sh = shape;
        if (small) {
            // The stem, the tower and the heads in one launch.
            const azh::SmallStem stem{io.in, weights.stem.w, weights.stem.scale, weights.stem.shift, sh.P};
            azh::SmallHeads hd;
            if (heads) {
                hd.w = weights.heads;
                hd.logits = io.logits;
                hd.values = io.values;
                hd.own = io.own;
                hd.V = sh.V;
            }
            check(azh::launchSmallTower(io.x, &stem, &hd, tower.w0, tower.stride, tower.scaleOff, tower.shiftOff,
                                        2 * std::max(blocksToRun, 0), Bp, sh.n, sh.F, stream),
                  "small-board pass");
            return;
        }
        check(azh::launchConv3x3(io.in, weights.stem.w, weights.stem.scale, weights.stem.shift, nullptr, io.x, Bp,
                                 sh.n, sh.P, sh.F, true, true, azh::chooseStemTiling(t, sh.F, Bpass), stream),
              "conv3x3 (stem)");
        launchTowerOn(io.x, io.mid, Bp, t, stream, blocksToRun);
        if (heads)
            check(azh::launchHeads(io.x, weights.heads, io.act, io.logits, io.values, io.own, Bp, sh.n, sh.F, sh.V,
                                   stream),
                  "heads");
    }

    // Checks that the tower's convolutions sit in the weight arena at one
    // fixed stride (conv1 and conv2 of each block in turn, each with its BN
    // scale and shift at fixed offsets after its packed weights), as the
    // small-board tower kernel reads them.
    void initTowerLayout() {
        const std::vector<ConvW>& c1 = weights.conv1;
        const std::vector<ConvW>& c2 = weights.conv2;
        tower = TowerLayout{};
        if (c1.empty() || c2.size() != c1.size()) return;
        const float* w0 = c1[0].w;
        if (c2[0].w <= w0 || c1[0].scale < w0 || c1[0].shift < w0) return;
        const size_t stride = (size_t)(c2[0].w - w0), scaleOff = (size_t)(c1[0].scale - w0),
                     shiftOff = (size_t)(c1[0].shift - w0);
        for (size_t i = 0; i < c1.size(); ++i)
            for (int h = 0; h < 2; ++h) {
                const ConvW& c = h == 0 ? c1[i] : c2[i];
                const float* w = w0 + (2 * i + h) * stride;
                if (c.w != w || c.scale != w + scaleOff || c.shift != w + shiftOff) return;
            }
        tower = TowerLayout{true, w0, stride, scaleOff, shiftOff};
    }

    // Whether a pass of B runs as one small-board launch (stem, tower,
    // heads): 5x5 up to 64 channels at any batch (5x5 4x32 per pass: 26.8
    // against 46.2 us as per-layer launches at 8 boards, 29.6 against 60.0
    // at 256); 9x9 up to 32 channels at any batch (6x16: 41.7 against 65.1
    // us at 8 boards; 6x32: 73.7 against 75.8 at 8, 75.5 against 124.2 at
    // 256) and up to 64 past 128 boards (6x48: 168.8 against 210.8 us at
    // 256, 167.5 against 153.9 at 128; 6x64: 214.7 against 235.4 at 256,
    // 212.5 against 186.3 at 128: a board's pass in one workgroup runs at
    // its CU's matrix rate, about 200 us at 64 channels whatever the batch);
    // 13x13 up to 16 channels at any batch (6x16: 59.1 against 70.9 us at
    // 8 boards, 60.3 against 122.2 at 256) and up to 32 past 100 boards
    // (6x32: 132.6 against 150.2 at 128, 131.7 against 105.4 at 64; two
    // 13x13 tiles of 32 channels fill 57.6 of the 64 KB).
    bool useSmallTower(int B) const {
        if (!smallTower || !tower.ok) return false;
        const Shape& sh = shape;
        const size_t lds = azh::smallTowerLdsBytes(sh.n, sh.F, sh.P, true, sh.V);
        if (lds == 0 || lds > azh::kSmallTowerMaxLds) return false;
        if (sh.n == 5) return sh.F <= 64;
        if (sh.n == 9) return sh.F <= 32 || (sh.F <= 64 && B > 128);
        if (sh.n == 13) return sh.F <= 16 || (sh.F <= 32 && B > 100);
        return false;
    }

    // Whether a pass of B runs its stem and tower as one board-resident
    // launch (alone: no other pass in flight, othersIdle). A board's tower
    // takes the same time on its CU whatever the batch (19x19 10x128: 3.90
    // ms per pass up to 256 boards, 7.77 up to 512), so a part-filled round
    // of workgroups idles CUs for all of it, while the per-layer launches
    // shrink with the batch. Per pass against the per-layer launches (256
    // CUs): 256 boards 3.905 against 3.970 ms, 250 3.901 / 3.940, 244
    // 3.886 / 3.912, 240 3.883 / 3.858; 512 7.774 / 7.816, 504 7.770 /
    // 7.710; 768 11.651 / 11.751, 746 11.657 / 11.695, 740 11.661 / 11.612.
    // So taken for one round from 95% of the CUs, and for more rounds only
    // when they are full. Not with another pass in flight: its workgroups
    // hold every CU's registers for a whole tower, so the other pass's
    // kernels (heads included) wait for them (two slots kept full: 63.7k
    // against 64.7k positions/s).
    bool useResidentTower(int B, bool alone) const {
        const Shape& sh = shape;
        if (residentTower == 0 || (!tower.ok && sh.blocks > 0) || B < 1 ||
            !azh::residentTowerSupported(sh.n, sh.F, sh.P))
            return false;
        if (residentTower == 2) return true;
        const long cus = azh::deviceCUs();
        const long rounds = (B + cus - 1) / cus;
        return alone && (rounds == 1 ? 20L * B >= 19L * cus : B == rounds * cus);
    }

    // The stem (when asked) and the tower's first `blocksToRun` blocks over
    // io's Bp boards as one board-resident launch.
    void launchResident(const PassBuffers& io, int Bp, hipStream_t stream, int blocksToRun, bool stem) {
        const Shape& sh = shape;
        azh::ResidentTower t{};
        if (stem) {
            t.in = io.in;
            t.stemW = weights.stem.w;
            t.stemScale = weights.stem.scale;
            t.stemShift = weights.stem.shift;
            t.P = sh.P;
        }
        t.x = io.x;
        t.mid = io.mid;
        t.w0 = tower.w0;
        t.stride = tower.stride;
        t.scaleOff = tower.scaleOff;
        t.shiftOff = tower.shiftOff;
        t.layers = 2 * std::max(blocksToRun, 0);
        t.B = Bp;
        t.F = sh.F;
        const int workgroups = (int)std::min<long>(Bp, azh::deviceCUs());
        check(azh::launchResidentTower(t, sh.n, workgroups, stream), "board-resident tower");
    }

    // Whether a pass of B runs as two half-batch chains on two streams.
    // - Whole-board shapes with more than one round of workgroups (more than
    //   one per CU): two independent halves drift apart, so one half's
    //   partly filled last round, its launches and its epilogue's output
    //   bursts overlap the other half's contraction (19x19 10x128: 197.9 ->
    //   193.1 us per layer of 256 boards, 391.6 -> 382.9 us at 512). Not at
    //   one round (128 boards at 19x19: 104.8 us on one stream, 135 in
    //   halves).
    // - The four-wave shape of 6 column groups past one round, or at up to
    //   7/8 of one: there each half takes its own batch's finer shape, so
    //   the halves together run more workgroups (19x19 10x128, 18 boards:
    //   34.4 -> 26.2 us per layer, 24.4k -> 32.5k positions/s).
    // - The smaller shapes past two rounds (9x9 6x64, 140 boards: 19.6 ->
    //   17.2 us per layer, 517k -> 577k positions/s). Not below: their
    //   layers take 7-46 us, where a second chain's launches and heads cost
    //   what the overlap gains, and with two passes in flight on a runner's
    //   two slots the four chains lose (9x9 6x64, 100 boards: -4% alone,
    //   -18% with two slots; 19x19 20x256, 8 boards: +7% alone, -19% with
    //   two slots).
    bool splitPass(int B, bool alone) const {
        if (B < 2 || useSmallTower(B) || useResidentTower(B, alone)) return false;
        // A layer of under 0.5 GFLOP of matrix work (3 us at the fp32 MFMA
        // peak) is bound by its launch, and a second chain's launches only
        // add to it (5x5 4x32, 300 boards: 0.14 GFLOP per layer, 5.4 ->
        // 10.9 us per layer in halves).
        const double layerFlops = 2.0 * B * shape.A * 16.0 * azh::ceilDiv(shape.F, azh::kCoBlock) * 16.0 *
                                  azh::ceilDiv(shape.F, azh::kChunk) * 9.0;
        if (layerFlops < 0.5e9) return false;
        const azh::ConvTiling t = azh::chooseConvTiling(shape.F, B, shape.n, alone);
        const long workgroups = azh::convWorkgroups(t, shape.F, B, shape.n);
        const long cus = azh::deviceCUs();
        if (t.pgPerWave == 0) return workgroups > cus;
        if (t == azh::ConvTiling{1, 1, 4, 6}) return workgroups > cus || 8 * workgroups <= 7 * cus;
        return workgroups > 2 * cus;
    }

    // The workgroup shape of a part of Bp boards of a pass of B: the batch's
    // whole-board shape for both halves (the halves of a large batch), else
    // the part's own batch's shape unless that is a whole-board one (a
    // 19x19 half of 120 boards at 96 channels would take the one-round
    // shape: 141.7 us per layer in halves, 122.1 with the batch's shape).
    azh::ConvTiling partTiling(int B, int Bp, bool alone) const {
        const azh::ConvTiling t = azh::chooseConvTiling(shape.F, B, shape.n, alone);
        if (t.pgPerWave == 0 || Bp == B) return t;
        // The two halves run side by side: neither is alone.
        const azh::ConvTiling own = azh::chooseConvTiling(shape.F, Bp, shape.n, false);
        return own.pgPerWave == 0 ? t : own;
    }

    // Runs part(b0, Bp, stream) over slot s's batch of B on `stream` (slot
    // s's own or its capture): the whole batch, or when the pass splits, its
    // two halves, the second on s.aux, forked from `stream` and joined back
    // into it.
    template <typename Part>
    void overHalves(Slot& s, int B, hipStream_t stream, bool alone, Part part) {
        if (!splitPass(B, alone)) {
            part(0, B, stream);
            return;
        }
        const int B0 = (B + 1) / 2;
        check(hipEventRecord(s.fork, stream), "hipEventRecord(fork)");
        check(hipStreamWaitEvent(s.aux, s.fork, 0), "hipStreamWaitEvent(fork)");
        part(0, B0, stream);
        part(B0, B - B0, s.aux);
        check(hipEventRecord(s.join, s.aux), "hipEventRecord(join)");
        check(hipStreamWaitEvent(stream, s.join, 0), "hipStreamWaitEvent(join)");
    }

    // The pass's kernels, on `stream`, in halves when the pass splits;
    // alone: no other pass in flight (othersIdle).
    void launchPass(Slot& s, int B, hipStream_t stream, int blocksToRun, bool heads, bool alone) {
        if (useResidentTower(B, alone)) {
            launchPassOn(slotBuffers(s, 0), B, stream, blocksToRun, heads, alone);
            return;
        }
        const bool small = useSmallTower(B);
        overHalves(s, B, stream, alone, [&](int b0, int Bp, hipStream_t st) {
            launchPassPart(slotBuffers(s, b0), Bp, B, partTiling(B, Bp, alone), st, blocksToRun, heads, small);
        });
    }

    // A pass over io's B boards on one stream (no half-batch chains), in
    // the form the runner takes for it otherwise: board-resident, the
    // small-board pass, or per-layer launches.
    void launchPassOn(const PassBuffers& io, int B, hipStream_t stream, int blocksToRun, bool heads, bool alone) {
        if (useResidentTower(B, alone)) {
            launchResident(io, B, stream, blocksToRun, true);
            if (heads)
                check(azh::launchHeads(io.x, weights.heads, io.act, io.logits, io.values, io.own, B, shape.n, shape.F,
                                       shape.V, stream),
                      "heads");
            return;
        }
        launchPassPart(io, B, B, azh::chooseConvTiling(shape.F, B, shape.n, alone), stream, blocksToRun, heads,
                       useSmallTower(B));
    }

    // The tower as the pass runs it, on slot s's staged trunk (the effective
    // time per layer within a pass).
    void launchTowerAsPass(Slot& s, int B, int blocksToRun, bool alone) {
        if (useResidentTower(B, alone)) {
            launchResident(slotBuffers(s, 0), B, s.stream, blocksToRun, false);
            return;
        }
        if (useSmallTower(B)) {
            check(azh::launchSmallTower(s.dX, nullptr, nullptr, tower.w0, tower.stride, tower.scaleOff,
                                        tower.shiftOff, 2 * std::max(blocksToRun, 0), B, shape.n, shape.F,
                                        s.stream),
                  "small-board tower");
            return;
        }
        const size_t trunk = azh::quadFloats(1, shape.F, shape.A);
        overHalves(s, B, s.stream, alone, [&](int b0, int Bp, hipStream_t st) {
            launchTowerOn(s.dX + b0 * trunk, s.dMid + b0 * trunk, Bp, partTiling(B, Bp, alone), st, blocksToRun);
        });
    }

    // The device-resident pass: one captured graph per batch size, replayed.
    // A slot keeps up to kGraphsPerSlot of them (a hub's passes come in up
    // to max_batch sizes); capturing one more first drops the one replayed
    // least recently, after the slot's stream has finished with it.
    static constexpr size_t kGraphsPerSlot = 64;
    void enqueuePass(Slot& s, int B) {
        const bool alone = othersIdle(&s);
        if (!graphs) {
            launchPass(s, B, s.stream, shape.blocks, true, alone);
            return;
        }
        // One graph per batch size, workgroup-shape regime (another pass in
        // flight or not) and tower form (test hooks switch the small-board
        // and the board-resident towers).
        const int key = 8 * B + (useResidentTower(B, alone) ? 4 : 0) + (alone ? 2 : 0) + (useSmallTower(B) ? 1 : 0);
        auto it = s.graphs.find(key);
        if (it == s.graphs.end()) {
            if (s.graphs.size() >= kGraphsPerSlot) {
                auto oldest = std::min_element(s.graphs.begin(), s.graphs.end(), [](const auto& a, const auto& b) {
                    return a.second.lastUse < b.second.lastUse;
                });
                check(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
                check(hipGraphExecDestroy(oldest->second.exec), "hipGraphExecDestroy");
                s.graphs.erase(oldest);
            }
            hipGraph_t g = nullptr;
            check(hipStreamBeginCapture(s.stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
            try {
                launchPass(s, B, s.stream, shape.blocks, true, alone);
            } catch (...) {
                (void)hipStreamEndCapture(s.stream, &g);
                if (g) (void)hipGraphDestroy(g);
                throw;
            }
            check(hipStreamEndCapture(s.stream, &g), "hipStreamEndCapture");
            hipGraphExec_t exec = nullptr;
            const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            check(e, "hipGraphInstantiate");
            it = s.graphs.emplace(key, Slot::CachedGraph{exec, 0}).first;
        }
        it->second.lastUse = ++s.replays;
        check(hipGraphLaunch(it->second.exec, s.stream), "hipGraphLaunch");
    }

    // Checks B positions' host arrays (checkPositions) for this network.
    void checkPositionsFor(const azh_positions& pos, int B) const {
        checkPositions(pos.stones, (size_t)B * shape.H * shape.A, pos.plies, pos.to_move, pos.sym, pos.seen_offsets,
                       pos.seen, B, shape.H);
    }
    // The positions path's device arrays for B positions in slot s, staged
    // from the caller's host arrays, checked beforehand (checkPositionsFor),
    // on the slot's stream: copied into the slot's pinned staging
    // (PositionsLayout for B), then up in one copy, and the superko hashes
    // in a second.
    PositionsOnDevice stagePositions(Slot& s, const azh_positions& pos, int B) {
        const Shape& sh = shape;
        const size_t A = sh.A, A1 = sh.A1, H = sh.H;
        const PositionsLayout L(B, H, A, A1);
        uint8_t* dev = static_cast<uint8_t*>(s.posBytes.reserve(PositionsLayout(maxBatch, H, A, A1).end));
        uint8_t* host = static_cast<uint8_t*>(s.posIn.reserve(PositionsLayout(maxBatch, H, A, A1).inputEnd));
        const size_t nSeen = (size_t)pos.seen_offsets[B];
        uint64_t* seen = static_cast<uint64_t*>(s.posSeen.reserve(std::max<size_t>(nSeen, 1) * sizeof(uint64_t)));
        std::memcpy(host + L.stones, pos.stones, (size_t)B * H * A);
        int* plies = reinterpret_cast<int*>(host + L.plies);
        if (pos.plies)
            std::memcpy(plies, pos.plies, (size_t)B * sizeof(int));
        else
            std::fill(plies, plies + B, sh.H);
        std::memcpy(host + L.turn, pos.to_move, B);
        if (pos.sym)
            std::memcpy(host + L.sym, pos.sym, B);
        else
            std::memset(host + L.sym, 0, B);
        std::memcpy(host + L.offsets, pos.seen_offsets, (size_t)(B + 1) * sizeof(int64_t));
        check(hipMemcpyAsync(dev, host, L.inputEnd, hipMemcpyHostToDevice, s.stream), "hipMemcpyAsync(positions)");
        if (nSeen) {
            uint64_t* seenHost = static_cast<uint64_t*>(s.posSeenIn.reserve(nSeen * sizeof(uint64_t)));
            std::memcpy(seenHost, pos.seen, nSeen * sizeof(uint64_t));
            check(hipMemcpyAsync(seen, seenHost, nSeen * sizeof(uint64_t), hipMemcpyHostToDevice, s.stream),
                  "hipMemcpyAsync(seen)");
        }
        PositionsOnDevice d;
        d.stones = dev + L.stones;
        d.plies = reinterpret_cast<const int*>(dev + L.plies);
        d.turn = dev + L.turn;
        d.sym = dev + L.sym;
        d.offsets = reinterpret_cast<const long long*>(dev + L.offsets);
        d.seen = seen;
        d.legal = dev + L.legal;
        d.mapped = reinterpret_cast<float*>(dev + L.mapped);
        d.priors = reinterpret_cast<float*>(dev + L.priors);
        return d;
    }
    // The positions path on staged positions: encoding, the pass, the
    // legal moves, the mapped logits and the priors, on the slot's stream.
    void positionsChain(Slot& s, const PositionsOnDevice& d, int B) {
        encodeStep(s, d, B);
        enqueuePass(s, B);
        legalStep(s, d, B);
        priorsStep(s, d, B);
    }
    // encodePlanes into the pass's input.
    void encodeStep(Slot& s, const PositionsOnDevice& d, int B) {
        check(azh::launchEncodePlanes(d.stones, d.plies, d.turn, d.sym, s.dIn, B, shape.n, shape.H, s.stream), "encode");
    }
    // The legal moves of each position's current board (ply 0 of its stones).
    void legalStep(Slot& s, const PositionsOnDevice& d, int B) {
        check(azh::launchLegalMoves(d.stones, (size_t)shape.H * shape.A, d.turn, d.seen, d.offsets, d.legal, B,
                                    shape.n, s.stream),
              "legal moves");
    }
    // The pass's logits mapped back from the symmetry, and the priors.
    void priorsStep(Slot& s, const PositionsOnDevice& d, int B) {
        check(azh::launchPriors(s.dLogits, d.legal, d.sym, d.mapped, d.priors, B, shape.A1, shape.n, s.stream),
              "priors");
    }

    void copyIn(Slot& s, int B) {
        check(hipMemcpyAsync(s.dIn, s.hIn, (size_t)B * shape.P * shape.A * sizeof(float), hipMemcpyHostToDevice,
                             s.stream),
              "hipMemcpyAsync(input)");
    }
    // The test hook's hold before a pass's outputs are copied back.
    void copyOutDelay(Slot& s) {
        const int delayUs = gHooks.copyOutDelayUs.load();
        if (delayUs > 0) check(azh::launchSpin(1000ull * delayUs, s.stream), "spin");
    }
    void copyOut(Slot& s, int B) {
        copyOutDelay(s);
        check(hipMemcpyAsync(s.hLogits, s.dLogits, (size_t)B * shape.A1 * sizeof(float), hipMemcpyDeviceToHost,
                             s.stream),
              "hipMemcpyAsync(logits)");
        check(hipMemcpyAsync(s.hValues, s.dValues, (size_t)B * sizeof(float), hipMemcpyDeviceToHost, s.stream),
              "hipMemcpyAsync(values)");
    }

    Slot& slotAt(int slot) {
        if (slot < 0 || slot >= (int)slots.size())
            throw Error(AZH_ERR_ARGUMENT, "hip: slot " + std::to_string(slot) + " outside [0, " +
                                              std::to_string(slots.size()) + ")");
        return *slots[slot];
    }
    void checkBatch(int B) const {
        if (B < 1 || B > maxBatch)
            throw Error(AZH_ERR_ARGUMENT, "hip: batch of " + std::to_string(B) + " positions outside [1, " +
                                              std::to_string(maxBatch) + "]");
    }
    // The slot, held for the caller's scope (a synchronous call), or an
    // error when a pass or another call holds it.
    SlotClaim claimIdle(int slot) { return SlotClaim(slotAt(slot), slot); }
};

// makeCudaRunner's steps (src/cuda/cuda_runner.cu:227-234): checks, memory,
// upload, slots, then the reporter's thread.
void createRunner(const azh_netcfg* cfg, const azh_tensor* tensors, int count, int max_batch, int slots,
                  azh_runner** out) {
    if (!out) throw Error(AZH_ERR_ARGUMENT, "hip: no output handle");
    *out = nullptr;
    validate(cfg);
    if (max_batch < 1) throw Error(AZH_ERR_ARGUMENT, "makeHipRunner: maxBatch must be >= 1");
    if (slots < 1 || slots > kMaxSlots)
        throw Error(AZH_ERR_ARGUMENT, "makeHipRunner: slots must be in [1, " + std::to_string(kMaxSlots) + "]");
    const std::map<std::string, const float*> given = checkTensors(*cfg, tensors, count);
    requireContext();
    const azh_hub_group one{1, slots, max_batch};
    admitRunners(*cfg, &one, 1);
    std::unique_ptr<azh_runner> r(new azh_runner(*cfg, max_batch));
    check(hipGetDevice(&r->device), "hipGetDevice");
    scratchOnCurrentDevice();   // azh_infer_noalloc's scratch, resolved at set-up on the runner's device
    azh::deviceCUs();           // the launch rules' CU count, read once here, not during a caller's capture
    uploadWeights(*cfg, given, r->weights);
    r->initTowerLayout();
    for (int i = 0; i < slots; ++i) r->slots.push_back(std::make_unique<Slot>(r->shape, max_batch));
    r->reporter.start();
    *out = r.release();
}

// ---------------------------------------------------------------- C ABI

namespace {

// Claims an idle slot, runs enqueue(slot) (copies and kernels on its
// stream), records the slot's event and hands the pass to the reporter. From
// the claim on, done is called exactly once, by the reporter, which also
// releases the claim: an error while enqueueing travels through it, as a
// failed pass.
template <class Enqueue>
void beginOnSlot(azh_runner* r, int slot, azh_done_fn done, void* user, Enqueue enqueue) {
    Slot& s = r->slotAt(slot);
    bool idle = false;
    if (!s.claimed.compare_exchange_strong(idle, true))
        throw Error(AZH_ERR_STATE, "hip: slot " + std::to_string(slot) + " has a pass in flight");
    std::string error;
    try {
        enqueue(s);
        check(hipEventRecord(s.event, s.stream), "hipEventRecord");
    } catch (const std::exception& e) {
        error = e.what();
        if (error.empty()) error = "hip: enqueue failed";
        (void)hipEventRecord(s.event, s.stream);
    }
    Reporter::Notice notice;
    notice.slot = slot;
    notice.event = s.event;
    notice.claim = &s.claimed;
    notice.done = done;
    notice.user = user;
    notice.error = std::move(error);
    try {
        r->reporter.post(std::move(notice));
    } catch (...) {
        s.claimed.store(false);   // never handed over: no done will come
        throw;
    }
}

} // namespace

namespace {

// The last azh_begin_positions' outputs in the slot's pinned block (NULL
// before the slot's first).
const uint8_t* positionOutputs(const azh_runner* r, int slot, size_t PositionsLayout::*part) {
    if (!r || slot < 0 || slot >= (int)r->slots.size()) return nullptr;
    const Slot& s = *r->slots[slot];
    if (!s.posOut.p || s.posLastB < 1) return nullptr;
    const Shape& sh = r->shape;
    const PositionsLayout L(s.posLastB, sh.H, sh.A, sh.A1);
    return static_cast<const uint8_t*>(s.posOut.p) + (L.*part - L.mapped);
}

} // namespace

namespace {

// Keeps every slot of r busy through begin(slot, done, user) (one pass in
// flight per slot, each resubmitted as soon as its done comes) until
// `passes` have completed; wall ms from the first begin to the last done.
// A pass that fails stops the resubmission; the passes in flight are drained
// and the error is thrown.
template <class Begin>
float keepFull(azh_runner* r, int passes, Begin begin) {
    const int slots = azh_slots(r);
    for (int i = 0; i < slots; ++i) r->claimIdle(i);   // each idle now (claimed and released)
    // The done handler's state outlives every pass it is handed to: all
    // of them are drained before this function returns.
    struct Done {
        std::mutex m;
        std::condition_variable cv;
        std::vector<int> ready;
        std::string error;
    } st;
    const azh_done_fn done = [](void* user, int slot, const char* error) {
        Done* d = static_cast<Done*>(user);
        std::lock_guard<std::mutex> lock(d->m);
        if (error && *error && d->error.empty()) d->error = error;
        d->ready.push_back(slot);
        d->cv.notify_one();
    };
    int inFlight = 0, begun = 0;
    auto start = [&](int slot) {
        if (begin(slot, done, &st) != AZH_OK) {
            std::lock_guard<std::mutex> lock(st.m);
            if (st.error.empty()) st.error = azh_last_error();
            return;
        }
        ++inFlight;
        ++begun;
    };
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < slots && begun < passes; ++i) start(i);
    while (inFlight > 0) {
        int slot;
        bool failed;
        {
            std::unique_lock<std::mutex> lock(st.m);
            st.cv.wait(lock, [&] { return !st.ready.empty(); });
            slot = st.ready.back();
            st.ready.pop_back();
            failed = !st.error.empty();
        }
        --inFlight;
        if (!failed && begun < passes) start(slot);
    }
    const float ms = (float)std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    if (!st.error.empty()) throw Error(AZH_ERR_HIP, st.error);
    return ms;
}

} // namespace

extern "C" {

int azh_built(void) { return 1; }

int azh_available(char* why, size_t cap) {
    Context& c = Context::get();
    if (!c.ok && why && cap) std::snprintf(why, cap, "%s", c.why.c_str());
    return c.ok ? 1 : 0;
}

int azh_describe(char* out, size_t cap) {
    return guarded([&] {
        Context& c = Context::get();
        std::string d;
        if (!c.ok) {
            d = c.why;
        } else {
            const std::string base = c.arch.substr(0, c.arch.find(':'));
            char rt[32];
            std::snprintf(rt, sizeof rt, "%d.%d.%d", c.runtime / 10000000, (c.runtime / 100000) % 100,
                          c.runtime % 100000);
            d = c.name + " " + base + ", HIP runtime " + rt + ", kernels " + AZH_KERNEL_HASH + " (conv " + AZH_CONV_HASH + ")";
        }
        if (out && cap) std::snprintf(out, cap, "%s", d.c_str());
    });
}

int azh_device_cus(int* cus) {
    return guarded([&] {
        if (!cus) throw Error(AZH_ERR_ARGUMENT, "hip: bad arguments");
        requireContext();
        *cus = azh::deviceCUs();
    });
}

const char* azh_last_error(void) { return gLastError.c_str(); }

int azh_memory_need(const azh_netcfg* cfg, int max_batch, int slots, size_t* bytes) {
    return guarded([&] {
        validate(cfg);
        if (max_batch < 1 || slots < 1 || !bytes) throw Error(AZH_ERR_ARGUMENT, "hip: bad arguments");
        *bytes = runnerBytes(*cfg, max_batch, slots);
    });
}

int azh_check_memory(const azh_netcfg* cfg, int max_batch, int hubs, int slots_per_hub) {
    const azh_hub_group one{hubs, slots_per_hub, max_batch};
    return azh_check_memory_groups(cfg, &one, 1);
}

int azh_check_memory_groups(const azh_netcfg* cfg, const azh_hub_group* groups, int count) {
    return guarded([&] {
        validate(cfg);
        admitRunners(*cfg, groups, count);
    });
}

int azh_create(const azh_netcfg* cfg, const azh_tensor* tensors, int count, int max_batch, int slots,
               azh_runner** out) {
    return guarded([&] { createRunner(cfg, tensors, count, max_batch, slots, out); });
}

int azh_tensor_count(const azh_netcfg* cfg, int* count) {
    return guarded([&] {
        validate(cfg);
        if (!count) throw Error(AZH_ERR_ARGUMENT, "hip: bad arguments");
        *count = (int)tensorSpec(*cfg).size();
    });
}

int azh_tensor_info(const azh_netcfg* cfg, int i, char* name, size_t cap, size_t* size) {
    return guarded([&] {
        validate(cfg);
        const std::vector<TensorSpec> spec = tensorSpec(*cfg);
        if (i < 0 || i >= (int)spec.size()) throw Error(AZH_ERR_ARGUMENT, "hip: tensor index out of range");
        if (name && cap) std::snprintf(name, cap, "%s", spec[i].name.c_str());
        if (size) *size = spec[i].size;
    });
}

int azh_checkpoint_config(const char* path, azh_netcfg* cfg) {
    return guarded([&] {
        if (!path || !cfg) throw Error(AZH_ERR_ARGUMENT, "hip: bad arguments");
        *cfg = AznReader::read(path, [](AznReader& r) { return r.header(); });
    });
}

int azh_checkpoint_read(const char* path, azh_netcfg* cfg, float* values, size_t cap, size_t* floats) {
    return guarded([&] {
        if (!path || !cfg || !floats) throw Error(AZH_ERR_ARGUMENT, "hip: bad arguments");
        AznReader::read(path, [&](AznReader& r) {
            const azh_netcfg c = r.header();
            const std::vector<TensorSpec> spec = tensorSpec(c);
            size_t total = 0;
            for (const TensorSpec& t : spec) total += t.size;
            *cfg = c;
            *floats = total;
            if (!values) return 0;
            if (cap < total)
                throw Error(AZH_ERR_ARGUMENT, "hip: checkpoint needs " + std::to_string(total) + " floats, got " +
                                                  std::to_string(cap));
            const std::vector<float> v = r.tensors(spec);
            std::memcpy(values, v.data(), total * sizeof(float));
            return 0;
        });
    });
}

int azh_create_from_checkpoint(const char* path, int max_batch, int slots, azh_runner** out) {
    return guarded([&] {
        if (!path || !out) throw Error(AZH_ERR_ARGUMENT, "hip: bad arguments");
        *out = nullptr;
        azh_netcfg c{};
        std::vector<TensorSpec> spec;
        const std::vector<float> values = AznReader::read(path, [&](AznReader& r) {
            c = r.header();
            spec = tensorSpec(c);
            return r.tensors(spec);
        });
        std::vector<azh_tensor> tensors;
        size_t off = 0;
        for (const TensorSpec& t : spec) {
            tensors.push_back({t.name.c_str(), values.data() + off, t.size});
            off += t.size;
        }
        createRunner(&c, tensors.data(), (int)tensors.size(), max_batch, slots, out);
    });
}

void azh_destroy(azh_runner* r) { delete r; }

int azh_slots(const azh_runner* r) { return r ? (int)r->slots.size() : 0; }
int azh_max_batch(const azh_runner* r) { return r ? r->maxBatch : 0; }

float* azh_slot_input(azh_runner* r, int slot) {
    return r && slot >= 0 && slot < (int)r->slots.size() ? r->slots[slot]->hIn : nullptr;
}
const float* azh_slot_logits(const azh_runner* r, int slot) {
    return r && slot >= 0 && slot < (int)r->slots.size() ? r->slots[slot]->hLogits : nullptr;
}
const float* azh_slot_values(const azh_runner* r, int slot) {
    return r && slot >= 0 && slot < (int)r->slots.size() ? r->slots[slot]->hValues : nullptr;
}

const float* azh_slot_position_logits(const azh_runner* r, int slot) {
    return reinterpret_cast<const float*>(positionOutputs(r, slot, &PositionsLayout::mapped));
}

const float* azh_slot_priors(const azh_runner* r, int slot) {
    return reinterpret_cast<const float*>(positionOutputs(r, slot, &PositionsLayout::priors));
}

const uint8_t* azh_slot_legal(const azh_runner* r, int slot) {
    return positionOutputs(r, slot, &PositionsLayout::legal);
}

int azh_begin(azh_runner* r, int slot, int B, azh_done_fn done, void* user) {
    return guarded([&] {
        if (!r || !done) throw Error(AZH_ERR_ARGUMENT, "hip: begin needs a runner and a done callback");
        r->checkBatch(B);
        beginOnSlot(r, slot, done, user, [&](Slot& s) {
            r->copyIn(s, B);
            r->enqueuePass(s, B);
            r->copyOut(s, B);
        });
    });
}

int azh_begin_positions(azh_runner* r, int slot, int B, const azh_positions* pos, azh_done_fn done, void* user) {
    return guarded([&] {
        if (!r || !pos || !done)
            throw Error(AZH_ERR_ARGUMENT, "hip: begin_positions needs a runner, positions and a done callback");
        r->checkBatch(B);
        const Shape& sh = r->shape;
        // Checked here, so that bad positions fail the call, before the claim.
        r->checkPositionsFor(*pos, B);
        beginOnSlot(r, slot, done, user, [&](Slot& s) {
            const PositionsOnDevice d = r->stagePositions(s, *pos, B);
            r->positionsChain(s, d, B);
            const PositionsLayout L(B, sh.H, sh.A, sh.A1);
            const PositionsLayout M(r->maxBatch, sh.H, sh.A, sh.A1);
            void* out = s.posOut.reserve(M.end - M.mapped);
            s.posLastB = B;
            r->copyOutDelay(s);
            check(hipMemcpyAsync(out, d.mapped, L.end - L.mapped, hipMemcpyDeviceToHost, s.stream),
                  "hipMemcpyAsync(position outputs)");
            check(hipMemcpyAsync(s.hValues, s.dValues, (size_t)B * sizeof(float), hipMemcpyDeviceToHost, s.stream),
                  "hipMemcpyAsync(values)");
        });
    });
}

int azh_infer(azh_runner* r, const float* input, int B, float* logits, float* values, float* ownership) {
    return guarded([&] {
        if (!r || !input || !logits || !values) throw Error(AZH_ERR_ARGUMENT, "hip: infer needs its arrays");
        if (ownership && !r->shape.ownership) throw Error(AZH_ERR_ARGUMENT, "hip: the network has no ownership head");
        r->checkBatch(B);
        const SlotClaim held = r->claimIdle(0);
        Slot& s = held.slot;
        std::memcpy(s.hIn, input, (size_t)B * r->shape.P * r->shape.A * sizeof(float));
        r->copyIn(s, B);
        r->enqueuePass(s, B);
        r->copyOut(s, B);
        if (ownership)
            check(hipMemcpyAsync(ownership, s.dOwn, (size_t)B * r->shape.A * sizeof(float), hipMemcpyDeviceToHost,
                                 s.stream),
                  "hipMemcpyAsync(ownership)");
        check(hipStreamSynchronize(s.stream), "GPU inference failed");
        std::memcpy(logits, s.hLogits, (size_t)B * r->shape.A1 * sizeof(float));
        std::memcpy(values, s.hValues, (size_t)B * sizeof(float));
    });
}

int azh_infer_noalloc(azh_runner* r, const float* input, int B, float* logits, float* values, float* ownership,
                      void* stream) {
    return guarded([&] {
        if (!r || !input || !logits || !values)
            throw Error(AZH_ERR_ARGUMENT, "hip: infer_noalloc needs a runner and device input, logits and values");
        if (ownership && !r->shape.ownership) throw Error(AZH_ERR_ARGUMENT, "hip: the network has no ownership head");
        if (B < 1) throw Error(AZH_ERR_ARGUMENT, "hip: batch of " + std::to_string(B) + " positions");
        const Shape& sh = r->shape;
        const size_t need = noallocScratchFloats(sh, B) * sizeof(float);
        if (need > kScratchBytes) {
            int most = (int)(kScratchBytes / (need / B));
            while (most > 0 && noallocScratchFloats(sh, most) * sizeof(float) > kScratchBytes) --most;
            throw Error(AZH_ERR_ARGUMENT, "hip: a pass of " + std::to_string(B) + " positions needs " +
                                              std::to_string(need) + " bytes of scratch; azh_infer_noalloc holds " +
                                              std::to_string(kScratchBytes) + " (at most " + std::to_string(most) +
                                              " positions of this network per call)");
        }
        int dev = 0;
        check(hipGetDevice(&dev), "hipGetDevice");
        if (dev != r->device)
            throw Error(AZH_ERR_STATE, "hip: the runner lives on device " + std::to_string(r->device) + ", device " +
                                           std::to_string(dev) + " is current");
        float* x = scratchOnCurrentDevice();
        float* mid = x + alignFloats(azh::quadFloats(B, sh.F, sh.A));
        float* act = mid + alignFloats(azh::quadFloats(B, sh.F, sh.A));
        // Alone when none of the runner's slots has a pass in flight.
        r->launchPassOn(azh_runner::PassBuffers{input, x, mid, act, logits, values, ownership}, B,
                        static_cast<hipStream_t>(stream), sh.blocks, true, r->othersIdle(nullptr));
    });
}

int azh_softmax_legal(const float* logits, const uint8_t* legal, int B, int actions, float* priors) {
    return guarded([&] {
        if (B < 0 || actions < 1 || (B > 0 && (!logits || !legal || !priors)))
            throw Error(AZH_ERR_ARGUMENT, "hip: softmax needs its arrays");
        if (B == 0) return;
        requireContext();
        const size_t n = (size_t)B * actions;
        float *dl = nullptr, *dp = nullptr;
        uint8_t* dm = nullptr;
        struct Free {
            void* p[3];
            ~Free() {
                for (void* x : p)
                    if (x) (void)hipFree(x);
            }
        } guard{{nullptr, nullptr, nullptr}};
        check(hipMalloc(&dl, n * sizeof(float)), "hipMalloc");
        guard.p[0] = dl;
        check(hipMalloc(&dp, n * sizeof(float)), "hipMalloc");
        guard.p[1] = dp;
        check(hipMalloc(&dm, n), "hipMalloc");
        guard.p[2] = dm;
        check(hipMemcpy(dl, logits, n * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
        check(hipMemcpy(dm, legal, n, hipMemcpyHostToDevice), "hipMemcpy");
        check(azh::launchSoftmaxLegal(dl, dm, dp, B, actions, nullptr), "softmax");
        check(hipMemcpy(priors, dp, n * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy");
    });
}

int azh_encode_planes(const uint8_t* stones, const int32_t* plies, const uint8_t* to_move, const uint8_t* sym, int B,
                      int n, int H, float* planes) {
    return guarded([&] {
        if (B < 0 || n < 5 || n > 19 || H < 1 || H > 16 || (B > 0 && !planes))
            throw Error(AZH_ERR_ARGUMENT, "hip: encode needs n in [5, 19], H in [1, 16] and its arrays");
        if (B == 0) return;
        if (!stones || !to_move) throw Error(AZH_ERR_ARGUMENT, "hip: encode needs stones and to_move");
        const int64_t zero[2] = {0, 0};
        const size_t A = (size_t)n * n, stoneBytes = (size_t)B * H * A;
        for (int b = 0; b < B; ++b)   // seen lists do not apply: check the rest one position at a time
            checkPositions(stones + b * H * A, H * A, plies ? plies + b : nullptr, to_move ? to_move + b : nullptr,
                           sym ? sym + b : nullptr, zero, nullptr, 1, H);
        requireContext();
        const size_t P = 2 * (size_t)H + 2;
        DeviceBuffer dS(stoneBytes), dPl((size_t)B * sizeof(int)), dT(B), dSym(sym ? B : 0),
            dOut((size_t)B * P * A * sizeof(float));
        std::vector<int> pl(B, H);
        if (plies) std::copy(plies, plies + B, pl.begin());
        check(hipMemcpy(dS.p, stones, stoneBytes, hipMemcpyHostToDevice), "hipMemcpy");
        check(hipMemcpy(dPl.p, pl.data(), (size_t)B * sizeof(int), hipMemcpyHostToDevice), "hipMemcpy");
        check(hipMemcpy(dT.p, to_move, B, hipMemcpyHostToDevice), "hipMemcpy");
        if (sym) check(hipMemcpy(dSym.p, sym, B, hipMemcpyHostToDevice), "hipMemcpy");
        check(azh::launchEncodePlanes(dS.as<uint8_t>(), dPl.as<int>(), dT.as<uint8_t>(), sym ? dSym.as<uint8_t>() : nullptr,
                                      dOut.as<float>(), B, n, H, nullptr),
              "encode");
        check(hipMemcpy(planes, dOut.p, (size_t)B * P * A * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy");
    });
}

int azh_legal_moves(const uint8_t* stones, int n, const uint8_t* to_move, const uint64_t* seen,
                    const int64_t* seen_offsets, int B, uint8_t* legal) {
    return guarded([&] {
        if (B < 0 || n < 5 || n > 19 || (B > 0 && !legal))
            throw Error(AZH_ERR_ARGUMENT, "hip: legal moves need n in [5, 19] and their arrays");
        if (B == 0) return;
        const size_t A = (size_t)n * n;
        checkPositions(stones, (size_t)B * A, nullptr, to_move, nullptr, seen_offsets, seen, B, 1);
        requireContext();
        const size_t nSeen = (size_t)seen_offsets[B];
        DeviceBuffer dS((size_t)B * A), dT(B), dSeen(nSeen * sizeof(uint64_t)), dOff((size_t)(B + 1) * sizeof(int64_t)),
            dL((size_t)B * (A + 1));
        check(hipMemcpy(dS.p, stones, (size_t)B * A, hipMemcpyHostToDevice), "hipMemcpy");
        check(hipMemcpy(dT.p, to_move, B, hipMemcpyHostToDevice), "hipMemcpy");
        if (nSeen) check(hipMemcpy(dSeen.p, seen, nSeen * sizeof(uint64_t), hipMemcpyHostToDevice), "hipMemcpy");
        check(hipMemcpy(dOff.p, seen_offsets, (size_t)(B + 1) * sizeof(int64_t), hipMemcpyHostToDevice), "hipMemcpy");
        check(azh::launchLegalMoves(dS.as<uint8_t>(), A, dT.as<uint8_t>(), dSeen.as<uint64_t>(), dOff.as<long long>(),
                                    dL.as<uint8_t>(), B, n, nullptr),
              "legal moves");
        check(hipMemcpy(legal, dL.p, (size_t)B * (A + 1), hipMemcpyDeviceToHost), "hipMemcpy");
    });
}

int azh_evaluate_positions(azh_runner* r, const azh_positions* pos, int B, float* logits, float* priors,
                           uint8_t* legal, float* values) {
    return guarded([&] {
        if (!r || !pos || !priors || !legal || !values)
            throw Error(AZH_ERR_ARGUMENT, "hip: evaluate_positions needs its arrays");
        r->checkBatch(B);
        r->checkPositionsFor(*pos, B);
        const SlotClaim held = r->claimIdle(0);
        Slot& s = held.slot;
        const PositionsOnDevice d = r->stagePositions(s, *pos, B);
        r->positionsChain(s, d, B);
        const size_t A1 = r->shape.A1;
        auto down = [&](void* dst, const void* src, size_t bytes) {
            check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s.stream), "hipMemcpyAsync(outputs)");
        };
        down(priors, d.priors, (size_t)B * A1 * sizeof(float));
        down(legal, d.legal, (size_t)B * A1);
        down(values, s.dValues, (size_t)B * sizeof(float));
        if (logits) down(logits, d.mapped, (size_t)B * A1 * sizeof(float));
        check(hipStreamSynchronize(s.stream), "GPU inference failed");
    });
}

int azh_time_positions(azh_runner* r, const azh_positions* pos, int B, int iters, float* ms) {
    return guarded([&] {
        if (!r || !pos || !ms || iters < 1) throw Error(AZH_ERR_ARGUMENT, "hip: bad arguments");
        r->checkBatch(B);
        r->checkPositionsFor(*pos, B);
        const SlotClaim held = r->claimIdle(0);
        Slot& s = held.slot;
        const PositionsOnDevice d = r->stagePositions(s, *pos, B);
        // One untimed run of everything (the pass's graph for B is captured here).
        r->positionsChain(s, d, B);
        hipEvent_t e0 = nullptr, e1 = nullptr;
        check(hipEventCreate(&e0), "hipEventCreate");
        check(hipEventCreate(&e1), "hipEventCreate");
        struct Events {
            hipEvent_t a, b;
            ~Events() {
                (void)hipEventDestroy(a);
                (void)hipEventDestroy(b);
            }
        } guard{e0, e1};
        for (int step = 0; step < 4; ++step) {
            check(hipEventRecord(e0, s.stream), "hipEventRecord");
            for (int i = 0; i < iters; ++i) {
                if (step == 0 || step == 3) r->encodeStep(s, d, B);
                if (step == 3) r->enqueuePass(s, B);
                if (step == 1 || step == 3) r->legalStep(s, d, B);
                if (step == 2 || step == 3) r->priorsStep(s, d, B);
            }
            check(hipEventRecord(e1, s.stream), "hipEventRecord");
            check(hipEventSynchronize(e1), "hipEventSynchronize");
            check(hipEventElapsedTime(&ms[step], e0, e1), "hipEventElapsedTime");
        }
    });
}

int azh_set_graphs(azh_runner* r, int enabled) {
    return guarded([&] {
        if (!r) throw Error(AZH_ERR_ARGUMENT, "hip: no runner");
        r->graphs = enabled != 0;
    });
}

int azh_set_small_tower(azh_runner* r, int enabled) {
    return guarded([&] {
        if (!r) throw Error(AZH_ERR_ARGUMENT, "hip: no runner");
        r->smallTower = enabled != 0;
    });
}

int azh_set_resident_tower(azh_runner* r, int mode) {
    return guarded([&] {
        if (!r) throw Error(AZH_ERR_ARGUMENT, "hip: no runner");
        if (mode < 0 || mode > 2) throw Error(AZH_ERR_ARGUMENT, "hip: resident tower mode must be 0, 1 or 2");
        r->residentTower = mode;
    });
}

int azh_stage(azh_runner* r, int slot, int B) {
    return guarded([&] {
        if (!r) throw Error(AZH_ERR_ARGUMENT, "hip: no runner");
        r->checkBatch(B);
        const SlotClaim held = r->claimIdle(slot);
        Slot& s = held.slot;
        r->copyIn(s, B);
        check(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
    });
}

int azh_enqueue(azh_runner* r, int slot, int B) {
    return guarded([&] {
        if (!r) throw Error(AZH_ERR_ARGUMENT, "hip: no runner");
        r->checkBatch(B);
        const SlotClaim held = r->claimIdle(slot);
        r->enqueuePass(held.slot, B);
    });
}

int azh_synchronize(azh_runner* r, int slot) {
    return guarded([&] {
        if (!r) throw Error(AZH_ERR_ARGUMENT, "hip: no runner");
        check(hipStreamSynchronize(r->slotAt(slot).stream), "hipStreamSynchronize");
    });
}

int azh_fetch(azh_runner* r, int slot, int B) {
    return guarded([&] {
        if (!r) throw Error(AZH_ERR_ARGUMENT, "hip: no runner");
        r->checkBatch(B);
        const SlotClaim held = r->claimIdle(slot);
        Slot& s = held.slot;
        check(hipMemcpyAsync(s.hLogits, s.dLogits, (size_t)B * r->shape.A1 * sizeof(float),
                             hipMemcpyDeviceToHost, s.stream),
              "hipMemcpyAsync");
        check(hipMemcpyAsync(s.hValues, s.dValues, (size_t)B * sizeof(float), hipMemcpyDeviceToHost, s.stream),
              "hipMemcpyAsync");
        check(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
    });
}


int azh_time_passes(azh_runner* r, int slot, int B, int iters, float* ms) {
    return guarded([&] {
        if (!r || !ms || iters < 1) throw Error(AZH_ERR_ARGUMENT, "hip: bad timing arguments");
        r->checkBatch(B);
        const SlotClaim held = r->claimIdle(slot);
        Slot& s = held.slot;
        *ms = timeOnStream(s.stream, iters, [&] { r->enqueuePass(s, B); });
    });
}

int azh_time_tower_convs(azh_runner* r, int slot, int B, int iters, float* ms, int* launches, int* layers) {
    return guarded([&] {
        if (!r || !ms || !launches || !layers || iters < 1) throw Error(AZH_ERR_ARGUMENT, "hip: bad timing arguments");
        if (r->shape.blocks < 1) throw Error(AZH_ERR_ARGUMENT, "hip: the network has no residual block");
        r->checkBatch(B);
        const SlotClaim held = r->claimIdle(slot);
        Slot& s = held.slot;
        // The tower as the pass runs it: every block's two convolutions in
        // order, each reading the previous one's output.
        int per = 0;
        const bool alone = r->othersIdle(&s);
        *ms = timeOnStream(s.stream, iters, [&] { per = r->launchTower(s, B, s.stream, r->shape.blocks, alone); });
        *launches = iters * per;
        *layers = iters * 2 * r->shape.blocks;
    });
}

int azh_time_tower_layers(azh_runner* r, int slot, int B, int iters, float* ms, int* layers) {
    return guarded([&] {
        if (!r || !ms || !layers || iters < 1) throw Error(AZH_ERR_ARGUMENT, "hip: bad timing arguments");
        if (r->shape.blocks < 1) throw Error(AZH_ERR_ARGUMENT, "hip: the network has no residual block");
        r->checkBatch(B);
        const SlotClaim held = r->claimIdle(slot);
        Slot& s = held.slot;
        const bool alone = r->othersIdle(&s);
        *ms = timeOnStream(s.stream, iters, [&] { r->launchTowerAsPass(s, B, r->shape.blocks, alone); });
        *layers = iters * 2 * r->shape.blocks;
    });
}

int azh_time_resident_tower(azh_runner* r, int slot, int B, int iters, int stem, float* ms) {
    return guarded([&] {
        if (!r || !ms || iters < 1) throw Error(AZH_ERR_ARGUMENT, "hip: bad timing arguments");
        const Shape& sh = r->shape;
        if (!azh::residentTowerSupported(sh.n, sh.F, sh.P) || (!r->tower.ok && sh.blocks > 0))
            throw Error(AZH_ERR_ARGUMENT, "hip: the board-resident tower does not take this network");
        r->checkBatch(B);
        const SlotClaim held = r->claimIdle(slot);
        Slot& s = held.slot;
        *ms = timeOnStream(s.stream, iters,
                           [&] { r->launchResident(r->slotBuffers(s, 0), B, s.stream, sh.blocks, stem != 0); });
    });
}

int azh_pass_form(azh_runner* r, int B, int alone, int* form) {
    return guarded([&] {
        if (!r || !form) throw Error(AZH_ERR_ARGUMENT, "hip: no runner or no output");
        r->checkBatch(B);
        *form = (r->useSmallTower(B) ? 1 : 0) | (r->useResidentTower(B, alone != 0) ? 2 : 0) |
                (r->splitPass(B, alone != 0) ? 4 : 0);
    });
}

int azh_time_round_trips(azh_runner* r, int slot, int B, int iters, float* ms) {
    return guarded([&] {
        if (!r || !ms || iters < 1) throw Error(AZH_ERR_ARGUMENT, "hip: bad timing arguments");
        r->checkBatch(B);
        const SlotClaim held = r->claimIdle(slot);
        Slot& s = held.slot;
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < iters; ++i) {
            r->copyIn(s, B);
            r->enqueuePass(s, B);
            r->copyOut(s, B);
            check(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
        }
        *ms = (float)std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    });
}

int azh_time_pipelined(azh_runner* r, int B, int passes, float* ms) {
    return guarded([&] {
        if (!r || !ms || passes < 1) throw Error(AZH_ERR_ARGUMENT, "hip: bad timing arguments");
        r->checkBatch(B);
        *ms = keepFull(r, passes,
                       [&](int slot, azh_done_fn done, void* user) { return azh_begin(r, slot, B, done, user); });
    });
}

int azh_time_pipelined_positions(azh_runner* r, const azh_positions* pos, int B, int passes, float* ms) {
    return guarded([&] {
        if (!r || !pos || !ms || passes < 1) throw Error(AZH_ERR_ARGUMENT, "hip: bad timing arguments");
        r->checkBatch(B);
        *ms = keepFull(r, passes, [&](int slot, azh_done_fn done, void* user) {
            return azh_begin_positions(r, slot, B, pos, done, user);
        });
    });
}

int azh_probe_conv3x3(const float* x, const float* w, const float* scale, const float* shift, const float* skip,
                      int relu, int B, int n, int cin, int cout, int tiling, float* y) {
    return guarded([&] {
        if (!x || !w || !scale || !shift || !y || B < 1 || cin < 1 || cout < 1)
            throw Error(AZH_ERR_ARGUMENT, "hip: bad conv probe arguments");
        if (!azh::conv3x3Supported(n)) throw Error(AZH_ERR_ARGUMENT, "hip: board size not supported");
        if (tiling < -1 || tiling >= kTilingCount) throw Error(AZH_ERR_ARGUMENT, "hip: tiling index out of range");
        requireContext();
        const size_t A = (size_t)n * n;
        const std::vector<float> packed = azh::packConv3x3(w, cin, cout);
        // The pass's two input layouts: a channel count that fills whole
        // 16-channel chunks is tried as a trunk activation (channel quads,
        // the tower kernel), any other as input planes (the stem kernel).
        // Outputs and residuals are channel quads; the probe's own arrays
        // are planar, converted here. Tiling -1: the shape a pass of B alone
        // on the device gives that kernel.
        const bool planarIn = cin % azh::kChunk != 0;
        const azh::ConvTiling pass = azh::chooseConvTiling(cout, B, n, true);
        const azh::ConvTiling t = tiling >= 0 ? kTilings[tiling]
                                  : planarIn  ? azh::chooseStemTiling(pass, cout, B)
                                              : pass;
        const std::vector<float> xq = planarIn ? std::vector<float>() : azh::toChannelQuads(x, B, cin, (int)A);
        const std::vector<float> kq = skip ? azh::toChannelQuads(skip, B, cout, (int)A) : std::vector<float>();
        const size_t fx = planarIn ? B * cin * A : xq.size(), fy = azh::quadFloats(B, cout, (int)A);
        std::vector<float*> bufs;
        auto dev = [&](size_t floats) {
            float* p = nullptr;
            check(hipMalloc(&p, std::max<size_t>(floats, 1) * sizeof(float)), "hipMalloc");
            bufs.push_back(p);
            return p;
        };
        struct Free {
            std::vector<float*>& b;
            ~Free() {
                for (float* p : b) (void)hipFree(p);
            }
        } guard{bufs};
        float* dx = dev(fx);
        float* dw = dev(packed.size());
        float* ds = dev(cout);
        float* dh = dev(cout);
        float* dy = dev(fy);
        float* dk = skip ? dev(fy) : nullptr;
        check(hipMemcpy(dx, planarIn ? x : xq.data(), fx * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
        check(hipMemcpy(dw, packed.data(), packed.size() * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
        check(hipMemcpy(ds, scale, cout * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
        check(hipMemcpy(dh, shift, cout * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
        if (dk) check(hipMemcpy(dk, kq.data(), fy * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
        check(azh::launchConv3x3(dx, dw, ds, dh, dk, dy, B, n, cin, cout, relu != 0, planarIn, t, nullptr),
              "conv3x3");
        std::vector<float> yq(fy);
        check(hipMemcpy(yq.data(), dy, fy * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy");
        azh::fromChannelQuads(yq.data(), B, cout, (int)A, y);
    });
}

int azh_time_conv3x3(int B, int n, int cin, int cout, int tiling, int iters, float* ms) {
    return guarded([&] {
        if (!ms || B < 1 || cin < 1 || cout < 1 || iters < 1)
            throw Error(AZH_ERR_ARGUMENT, "hip: bad conv timing arguments");
        if (!azh::conv3x3Supported(n)) throw Error(AZH_ERR_ARGUMENT, "hip: board size not supported");
        if (tiling < -1 || tiling >= kTilingCount) throw Error(AZH_ERR_ARGUMENT, "hip: tiling index out of range");
        const bool planarIn = cin % azh::kChunk != 0;   // as azh_probe_conv3x3 chooses
        // Tiling -1: the shape a pass of B alone on the device gives that
        // kernel.
        const azh::ConvTiling pass = azh::chooseConvTiling(cout, B, n, true);
        const azh::ConvTiling t = tiling >= 0 ? kTilings[tiling]
                                  : planarIn  ? azh::chooseStemTiling(pass, cout, B)
                                              : pass;
        requireContext();
        const size_t A = (size_t)n * n;
        std::vector<float> w((size_t)cout * cin * 9);
        uint32_t st = 12345;
        for (float& v : w) {
            st = st * 1664525u + 1013904223u;
            v = ((st >> 8) * (1.0f / 16777216.0f) - 0.5f) * 0.05f;
        }
        const std::vector<float> packed = azh::packConv3x3(w.data(), cin, cout);
        std::vector<float*> bufs;
        struct Free {
            std::vector<float*>& b;
            ~Free() {
                for (float* p : b) (void)hipFree(p);
            }
        } guard{bufs};
        auto dev = [&](size_t floats) {
            float* p = nullptr;
            check(hipMalloc(&p, std::max<size_t>(floats, 1) * sizeof(float)), "hipMalloc");
            bufs.push_back(p);
            return p;
        };
        const size_t fx = planarIn ? B * cin * A : azh::quadFloats(B, cin, (int)A);
        float* dx = dev(fx);
        float* dw = dev(packed.size());
        float* ds = dev(cout);
        float* dh = dev(cout);
        float* dy = dev(azh::quadFloats(B, cout, (int)A));
        check(azh::launchFill(dx, fx, 0.5f, nullptr), "fill");
        check(azh::launchFill(ds, cout, 1.0f, nullptr), "fill");
        check(azh::launchFill(dh, cout, 0.0f, nullptr), "fill");
        check(hipMemcpy(dw, packed.data(), packed.size() * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
        check(azh::launchConv3x3(dx, dw, ds, dh, nullptr, dy, B, n, cin, cout, true, planarIn, t, nullptr),
              "conv3x3");
        // A tower layer adds its input (here its own output); the stem adds
        // nothing, as in the pass.
        float* skip = planarIn ? nullptr : dy;
        *ms = timeOnStream(nullptr, iters, [&] {
            check(azh::launchConv3x3(dx, dw, ds, dh, skip, dy, B, n, cin, cout, true, planarIn, t, nullptr),
                  "conv3x3");
        });
    });
}

int azh_probe_heads(azh_runner* r, const float* trunk, int B, float* logits, float* values, float* ownership) {
    return guarded([&] {
        if (!r || !trunk || !logits || !values) throw Error(AZH_ERR_ARGUMENT, "hip: bad heads probe arguments");
        if (ownership && !r->shape.ownership) throw Error(AZH_ERR_ARGUMENT, "hip: the network has no ownership head");
        r->checkBatch(B);
        const SlotClaim held = r->claimIdle(0);
        Slot& s = held.slot;
        const Shape& sh = r->shape;
        const std::vector<float> tq = azh::toChannelQuads(trunk, B, sh.F, sh.A);
        check(hipMemcpyAsync(s.dX, tq.data(), tq.size() * sizeof(float), hipMemcpyHostToDevice, s.stream),
              "hipMemcpyAsync");
        check(azh::launchHeads(s.dX, r->weights.heads, s.dAct, s.dLogits, s.dValues, s.dOwn, B, sh.n, sh.F, sh.V,
                               s.stream),
              "heads");
        check(hipMemcpyAsync(logits, s.dLogits, (size_t)B * sh.A1 * sizeof(float), hipMemcpyDeviceToHost, s.stream),
              "hipMemcpyAsync");
        if (ownership)
            check(hipMemcpyAsync(ownership, s.dOwn, (size_t)B * sh.A * sizeof(float), hipMemcpyDeviceToHost, s.stream),
                  "hipMemcpyAsync");
        check(hipMemcpyAsync(values, s.dValues, (size_t)B * sizeof(float), hipMemcpyDeviceToHost, s.stream),
              "hipMemcpyAsync");
        check(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
    });
}

int azh_probe_trunk(azh_runner* r, const float* input, int B, int blocks, float* trunk) {
    return guarded([&] {
        if (!r || !input || !trunk) throw Error(AZH_ERR_ARGUMENT, "hip: bad trunk probe arguments");
        if (blocks < 0 || blocks > r->shape.blocks) throw Error(AZH_ERR_ARGUMENT, "hip: blocks outside the network");
        r->checkBatch(B);
        const SlotClaim held = r->claimIdle(0);
        Slot& s = held.slot;
        const Shape& sh = r->shape;
        check(hipMemcpyAsync(s.dIn, input, (size_t)B * sh.P * sh.A * sizeof(float), hipMemcpyHostToDevice, s.stream),
              "hipMemcpyAsync");
        r->launchPass(s, B, s.stream, blocks, false, r->othersIdle(&s));
        std::vector<float> tq(azh::quadFloats(B, sh.F, sh.A));
        check(hipMemcpyAsync(tq.data(), s.dX, tq.size() * sizeof(float), hipMemcpyDeviceToHost, s.stream),
              "hipMemcpyAsync");
        check(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
        azh::fromChannelQuads(tq.data(), B, sh.F, sh.A, trunk);
    });
}

int azh_probe_fill(float* data, size_t n, float value, size_t tail) {
    return guarded([&] {
        if (!data) throw Error(AZH_ERR_ARGUMENT, "hip: no data");
        requireContext();
        float* d = nullptr;
        const size_t total = n + tail;
        check(hipMalloc(&d, std::max<size_t>(total, 1) * sizeof(float)), "hipMalloc");
        hipError_t e = hipMemcpy(d, data, total * sizeof(float), hipMemcpyHostToDevice);
        if (e == hipSuccess) e = azh::launchFill(d, n, value, nullptr);
        if (e == hipSuccess) e = hipMemcpy(data, d, total * sizeof(float), hipMemcpyDeviceToHost);
        (void)hipFree(d);
        check(e, "fill");
    });
}

int azh_probe_mfma(int chain, int iters, float* ms, double* flops) {
    return guarded([&] {
        if (!ms || !flops || iters < 1 || chain < 1) throw Error(AZH_ERR_ARGUMENT, "hip: bad MFMA probe arguments");
        requireContext();
        const int workgroups = azh::deviceCUs();
        float* out = nullptr;
        check(hipMalloc(&out, (size_t)workgroups * azh::kMfmaChainThreads * sizeof(float)), "hipMalloc");
        hipStream_t st = nullptr;
        hipError_t e = hipStreamCreateWithFlags(&st, hipStreamNonBlocking);
        float t = 0.0f;
        if (e == hipSuccess) {
            try {
                auto launch = [&] { check(azh::launchMfmaChains(out, workgroups, chain, st), "MFMA chains"); };
                launch();   // untimed: loads the kernel
                t = timeOnStream(st, iters, launch);
            } catch (const Error& err) {
                e = hipErrorUnknown;
                gLastError = err.what();
            }
        }
        if (st) (void)hipStreamDestroy(st);
        (void)hipFree(out);
        check(e, "MFMA probe");
        *ms = t;
        *flops = (double)workgroups * (azh::kMfmaChainThreads / 64) * 4.0 * chain * 2048.0;
    });
}

int azh_probe_copy(size_t bytes, int iters, float* ms) {
    return guarded([&] {
        if (!ms || iters < 1 || bytes == 0) throw Error(AZH_ERR_ARGUMENT, "hip: bad copy probe arguments");
        requireContext();
        void *a = nullptr, *b = nullptr;
        check(hipMalloc(&a, bytes), "hipMalloc");
        hipError_t e = hipMalloc(&b, bytes);
        if (e != hipSuccess) {
            (void)hipFree(a);
            check(e, "hipMalloc");
        }
        hipStream_t st = nullptr;
        e = hipStreamCreateWithFlags(&st, hipStreamNonBlocking);
        if (e == hipSuccess) e = hipMemsetAsync(a, 0, bytes, st);
        float t = 0.0f;
        if (e == hipSuccess) {
            try {
                t = timeOnStream(st, iters,
                                 [&] { check(hipMemcpyAsync(b, a, bytes, hipMemcpyDeviceToDevice, st), "copy"); });
            } catch (const Error& err) {
                e = hipErrorUnknown;
                gLastError = err.what();
            }
        }
        if (st) (void)hipStreamDestroy(st);
        (void)hipFree(a);
        (void)hipFree(b);
        check(e, "copy probe");
        *ms = t;
    });
}

void azh_set_hub_chaos_seed(uint64_t seed) { gHooks.hubChaosSeed.store(seed); }
uint64_t azh_hub_chaos_seed(void) { return gHooks.hubChaosSeed.load(); }
// The pass reported after n more have been reported fails (once); n <= 0
// turns the injection off.
void azh_fail_passes_after(int n) { gHooks.failingReport.store(n > 0 ? gHooks.reports.load() + n : -1); }
void azh_set_memory_limit(size_t bytes) { gHooks.memoryLimit.store(bytes); }
long long azh_passes_completed(void) { return gHooks.reports.load(); }
void azh_set_copy_out_delay(int microseconds) { gHooks.copyOutDelayUs.store(std::max(microseconds, 0)); }

} // extern "C"
