// HipBatchRunner: the gfx950 network behind the reference's BatchRunner
// interface (include/azgo/inference_hub.hpp:41-53), as CudaBatchRunner is
// (src/cuda/cuda_runner.cu:53-194). All GPU work, the slots' pinned staging
// and the completion thread live in libazgo_hip.so; this file adapts the C
// ABI (include/azgo_hip.h) to the reference's C++ types and exceptions.
#include "hip.hpp"

#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

#include "azgo/inference_hub.hpp"
#include "azgo_hip.h"

namespace azgo {

namespace {

// An ABI status as the exception the reference's CUDA backend throws for the
// same failure.
void check(int rc) {
    if (rc == AZH_OK) return;
    const std::string msg = azh_last_error();
    switch (rc) {
    case AZH_ERR_ARGUMENT: throw std::invalid_argument(msg);
    case AZH_ERR_TENSOR: throw std::logic_error(msg);
    default: throw std::runtime_error(msg);
    }
}

azh_netcfg toC(const NetConfig& c) {
    return azh_netcfg{c.boardSize, c.history, c.blocks, c.filters, c.valueHidden, c.ownership ? 1 : 0};
}

// Every tensor of net, params() then buffers(), as named views. The views'
// names point into `params` and `buffers`, which must outlive the call that
// reads them.
std::vector<azh_tensor> tensorViews(const std::vector<ParamView>& params, const std::vector<BufferView>& buffers) {
    std::vector<azh_tensor> out;
    out.reserve(params.size() + buffers.size());
    for (const ParamView& p : params) out.push_back(azh_tensor{p.name.c_str(), p.value, p.size});
    for (const BufferView& b : buffers) out.push_back(azh_tensor{b.name.c_str(), b.value, b.size});
    return out;
}

azh_runner* createRunner(const Network& network, int maxBatch, int slots) {
    // params() hands out views; nothing is written (as ParamLayout::of).
    Network& net = const_cast<Network&>(network);
    const std::vector<ParamView> params = net.params();
    const std::vector<BufferView> buffers = net.buffers();
    const std::vector<azh_tensor> views = tensorViews(params, buffers);
    const azh_netcfg cfg = toC(net.config());
    azh_runner* r = nullptr;
    check(azh_create(&cfg, views.data(), static_cast<int>(views.size()), maxBatch, slots, &r));
    return r;
}

class HipBatchRunner : public BatchRunner {
public:
    HipBatchRunner(const Network& net, int maxBatch, int slots) : runner_(createRunner(net, maxBatch, slots)) {}

    // azh_destroy waits for every pass in flight (and its done) first.
    ~HipBatchRunner() override { azh_destroy(runner_); }

    int slots() const override { return azh_slots(runner_); }
    int maxBatch() const override { return azh_max_batch(runner_); }
    float* input(int slot) override { return azh_slot_input(runner_, slot); }
    const float* logits(int slot) const override { return azh_slot_logits(runner_, slot); }
    const float* values(int slot) const override { return azh_slot_values(runner_, slot); }

    // Each pass carries its own callback: a heap copy handed to the library
    // as the pass's `user`, which the library's reporter passes back exactly
    // once (completed runs it and frees it). A begin the library refuses
    // (batch out of range, busy slot) throws and calls nothing, and leaves
    // any pass already in flight on the slot, and its callback, untouched:
    // the hub fails the new batch (src/inference_hub.cpp:237-246).
    void begin(int slot, int B, std::function<void(int slot, std::string error)> done) override {
        auto* fn = new std::function<void(int, std::string)>(std::move(done));
        const int rc = azh_begin(runner_, slot, B, &HipBatchRunner::completed, fn);
        if (rc != AZH_OK) {
            delete fn;
            check(rc);
        }
    }

private:
    static void completed(void* user, int slot, const char* error) {
        std::unique_ptr<std::function<void(int, std::string)>> fn(
            static_cast<std::function<void(int, std::string)>*>(user));
        (*fn)(slot, error ? std::string(error) : std::string());
    }

    azh_runner* runner_;
};

} // namespace

bool hipBuilt() { return azh_built() == 1; }

bool hipAvailable(std::string* why) {
    char buf[512] = {};
    const bool ok = azh_available(buf, sizeof buf) == 1;
    if (!ok && why) *why = buf;
    return ok;
}

std::string hipDescription() {
    char buf[512] = {};
    if (azh_describe(buf, sizeof buf) != AZH_OK) return azh_last_error();
    return buf;
}

std::unique_ptr<BatchRunner> makeHipRunner(const Network& net, int maxBatch, int slots) {
    if (maxBatch < 1) throw std::invalid_argument("makeHipRunner: maxBatch must be >= 1");
    if (slots < 1 || slots > kInferenceSlots)
        throw std::invalid_argument("makeHipRunner: slots must be in [1, " + std::to_string(kInferenceSlots) + "]");
    return std::make_unique<HipBatchRunner>(net, maxBatch, slots);
}

void checkHipInferenceMemory(const NetConfig& cfg, int inferenceBatch, int hubs, int slotsPerHub) {
    const azh_netcfg c = toC(cfg);
    check(azh_check_memory(&c, inferenceBatch, hubs, slotsPerHub));
}

void checkHipInferenceMemory(const NetConfig& cfg, const std::vector<GpuHubs>& groups) {
    const azh_netcfg c = toC(cfg);
    std::vector<azh_hub_group> g;
    g.reserve(groups.size());
    for (const GpuHubs& h : groups) g.push_back(azh_hub_group{h.hubs, h.slotsPerHub, h.inferenceBatch});
    check(azh_check_memory_groups(&c, g.data(), static_cast<int>(g.size())));
}

struct HipInference::Impl {
    azh_runner* runner = nullptr;
    ~Impl() {
        if (runner) azh_destroy(runner);
    }
};

HipInference::HipInference(const Network& net, int maxBatch) : impl_(new Impl) {
    impl_->runner = createRunner(net, maxBatch, 1);
}

HipInference::~HipInference() = default;

void HipInference::infer(const float* input, int B, float* logits, float* values, float* ownership) {
    const int rc = azh_infer(impl_->runner, input, B, logits, values, ownership);
    if (rc == AZH_ERR_ARGUMENT) throw std::invalid_argument(azh_last_error());
    if (rc != AZH_OK) throw std::runtime_error(std::string("GPU inference failed: ") + azh_last_error());
}

namespace hip_probe {

std::string deviceName() {
    const std::string d = hipDescription();
    const size_t gfx = d.find(" gfx");
    return gfx == std::string::npos ? d : d.substr(0, gfx);
}

void fill(float* data, size_t n, float value, size_t tail) { check(azh_probe_fill(data, n, value, tail)); }
void setHubChaosSeed(uint64_t seed) { azh_set_hub_chaos_seed(seed); }
uint64_t hubChaosSeed() { return azh_hub_chaos_seed(); }
void failPassesAfter(int n) { azh_fail_passes_after(n); }
void setMemoryLimit(size_t bytes) { azh_set_memory_limit(bytes); }
long long passesCompleted() { return azh_passes_completed(); }
void setCopyOutDelay(int microseconds) { azh_set_copy_out_delay(microseconds); }

} // namespace hip_probe

} // namespace azgo
