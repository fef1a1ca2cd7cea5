// The MI355X (gfx950) HIP backend as the reference's C++ sees it: the
// counterpart of include/azgo/cuda.hpp, declared in namespace azgo so that a
// `hip` branch in WorkerEvaluators (src/inference_hub.cpp:255-295) and the
// backend checks (src/backend.cpp:297-320) call it exactly as they call the
// CUDA backend. Plain C++17; every call goes through the C ABI of
// libazgo_hip.so (include/azgo_hip.h).
#pragma once
#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>
#include "azgo/gpu_memory.hpp"
#include "azgo/network.hpp"

namespace azgo {

class BatchRunner;   // azgo/inference_hub.hpp

// cudaBuilt (include/azgo/cuda.hpp:29-30): true in a build that links
// libazgo_hip.so.
bool hipBuilt();

// cudaAvailable (include/azgo/cuda.hpp:32-39): a gfx950 device is present and
// a first kernel ran; else false and *why says what is missing.
bool hipAvailable(std::string* why = nullptr);

// cudaDescription (include/azgo/cuda.hpp:41-49): "<GPU> gfx950, HIP runtime
// x.y.z, kernels <hash>", or hipAvailable's reason.
std::string hipDescription();

// makeCudaRunner (include/azgo/cuda.hpp:53-58): net's weights uploaded once,
// `slots` (1..kInferenceSlots) passes of up to maxBatch positions in flight,
// each on its own stream. Throws std::runtime_error ("hip: inference needs N MB
// ...; lower inference_batch") when the slots would not fit, std::logic_error
// naming a tensor the backend does not read, std::invalid_argument for bad
// arguments or a network shape the backend does not run.
std::unique_ptr<BatchRunner> makeHipRunner(const Network& net, int maxBatch, int slots = 2);

// checkCudaInferenceMemory (include/azgo/cuda.hpp:60-66).
void checkHipInferenceMemory(const NetConfig& cfg, int inferenceBatch, int hubs, int slotsPerHub = 2);
void checkHipInferenceMemory(const NetConfig& cfg, const std::vector<GpuHubs>& groups);

// CudaInference (include/azgo/cuda.hpp:68-84): the whole pass synchronously.
// Errors throw std::runtime_error("GPU inference failed: ...").
class HipInference {
public:
    HipInference(const Network& net, int maxBatch);
    ~HipInference();
    HipInference(const HipInference&) = delete;
    HipInference& operator=(const HipInference&) = delete;
    // Network::infer's arguments; ownership needs a network with the head
    // (std::invalid_argument otherwise, as CudaInference).
    void infer(const float* input, int B, float* logits, float* values, float* ownership = nullptr);
private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

// cuda_probe (include/azgo/cuda.hpp:91-157): test hooks with the same meaning.
namespace hip_probe {
std::string deviceName();
void fill(float* data, size_t n, float value, size_t tail = 0);
using InferNet = HipInference;
void setHubChaosSeed(uint64_t seed);
uint64_t hubChaosSeed();
void failPassesAfter(int n);
void setMemoryLimit(size_t bytes);
long long passesCompleted();
void setCopyOutDelay(int microseconds);
} // namespace hip_probe

} // namespace azgo
