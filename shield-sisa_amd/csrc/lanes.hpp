// The GPU side of the batched API: a sched::Device whose lanes are the engine's per-batch buffer sets, fed over a
// copy stream and run on a compute stream of one HIP device.
#pragma once
#include "engine.hpp"
#include "sched.hpp"

#include <memory>

namespace shv {

class HipLanes final : public sched::Device {
public:
    // Builds the engine (weights uploaded and repacked on `device`), pinned staging for every lane and the
    // device token pool of `token_slots` blocks (zeroed).
    HipLanes(const HostModel& hm, Precision p, const EngineConfig& cfg, int token_slots, int device);
    ~HipLanes() override;

    int lanes() const override { return int(lane_.size()); }
    bool host_pinned(const void* p, size_t bytes) override;
    void start(const sched::Batch& b) override;
    const float* land(const sched::Batch& b, double* device_ms) override;
    void scrub(const sched::Batch& b) noexcept override;

    Engine& engine() { return *eng_; }
    hipStream_t compute_stream() const { return compute_; }
    int device() const { return device_; }
    size_t device_bytes() const;

private:
    struct Staging {                       // pinned host memory of one lane
        uint8_t* frames = nullptr;         // [max_frames][172800]: frames not already in pinned memory
        float* blocks = nullptr;           // [max_host_tokens][6144]: host token blocks of the windows
        const float** table = nullptr;     // [max_windows * 20]: device address of every window entry's tokens
        int32_t* store = nullptr;          // [max_frames]
        float* tokens = nullptr;           // [max_frames][6144]: tokens bound for non-pinned caller buffers
        float* logits = nullptr;           // [max_windows]
        hipEvent_t uploaded = nullptr, t0 = nullptr, t1 = nullptr;
    };
    std::unique_ptr<Engine> eng_;
    std::vector<Staging> lane_;
    hipStream_t copy_ = nullptr, compute_ = nullptr;
    float* pool_ = nullptr;                // [token_slots][6144] on the device
    size_t pool_bytes_ = 0;
    int device_ = 0;
    void release() noexcept;
};

}  // namespace shv
