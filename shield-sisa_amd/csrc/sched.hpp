// Host side of the batched API (include/shv_hip.h): job records, request validation, the batch planner, and two
// threads per model -- a launcher that plans batches and starts them on free lanes, and a completer that lands
// them in start order, writes the callers' outputs and finalises the jobs.  No HIP in this file or in sched.cpp:
// the GPU side is a Device (lanes.cpp), and a CPU stub device runs this same code under the thread and address
// sanitizers (tests/native/sched_check.cpp).
//
// Contract (engine/include/shv_cuda.h:28-59, 116-147): FIFO execution, consecutive jobs coalesced into one batch
// up to the frame / window / host-block limits; a job storing into a token slot that an earlier job of the batch
// read or stored starts a new batch; NaN logits (and tokens) for every job of a failed batch and NaN for each
// non-finite logit; callbacks after the outputs are final; job_free waits for the callback's return; closing a
// model completes every queued job first; jobs outlive their model.
#pragma once
#include "../../include/shv_hip.h"

#include <chrono>
#include <condition_variable>
#include <cstddef>
#include <cstdint>
#include <deque>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace shv {
namespace sched {

using Clock = std::chrono::steady_clock;

constexpr size_t kFrameBytes = SHV_HIP_FRAME_BYTES;
constexpr size_t kTokenFloats = SHV_HIP_TOKEN_FLOATS;
constexpr int kWindowFrames = SHV_HIP_WINDOW_FRAMES;

// Where one window entry (window * 20 + frame position) takes its 16 x 384 tokens from.
struct TokenRef {
    enum Kind : int32_t { kFrame = 0, kSlot = 1, kHost = 2 };
    int32_t kind;
    int32_t index;   // kFrame: frame of the job (of the batch, once planned); kSlot: pool slot; kHost: host block
};

// A run of frames of one job, placed at batch frame `at`.
struct FrameSpan {
    const uint8_t* src;
    int at, count;
    bool pinned;
};
// Frames [at, at + count) of the batch whose tokens go back to the caller at dst.
struct TokenSpan {
    float* dst;
    int at, count;
    bool pinned;
};

// One coalesced GPU batch as the device sees it.
struct Batch {
    int lane = 0;
    int frames = 0, windows = 0;
    std::vector<FrameSpan> frame_spans;
    std::vector<int32_t> store_to;           // per batch frame: pool slot or -1; empty if no frame stores
    std::vector<TokenRef> refs;              // windows * 20, frame indices relative to the batch
    std::vector<const float*> host_blocks;   // indexed by kHost refs
    std::vector<TokenSpan> token_spans;
};

// What the scheduler needs from the hardware.  Calls for one lane never overlap; start() and land() of different
// lanes may run on different threads at the same time.
class Device {
public:
    virtual ~Device() = default;
    virtual int lanes() const = 0;
    // true if [p, p + bytes) is page-locked host memory the device reads or writes directly
    virtual bool host_pinned(const void* p, size_t bytes) = 0;
    // Queue the batch's copies and kernels on its lane.  Throws if something could not be queued.
    virtual void start(const Batch& b) = 0;
    // Wait for the lane's batch; write its staged token spans; return its b.windows logits (valid until the lane
    // is started again) and the device time in ms.  Throws on a device error.
    virtual const float* land(const Batch& b, double* device_ms) = 0;
    // After a failed start() or land(): return once nothing queued for b can still run.  Never throws.
    virtual void scrub(const Batch& b) noexcept = 0;
};

struct Limits {
    int frames = 640;         // frames per batch
    int windows = 512;        // windows per batch
    int host_blocks = 2048;   // host token blocks per batch
    int token_slots = 0;      // device token pool size
    int delay_us = 0;         // idle launcher: wait this long for a fuller batch
};

// thread-local error text of the C API
void set_error(const std::string& e);
void clear_error();
const char* last_error();

}  // namespace sched
}  // namespace shv

// The opaque job handle of the C API.
struct shv_hip_job {
    // the request, validated and resolved at submit
    const uint8_t* frames = nullptr;
    size_t n_frames = 0;
    bool frames_pinned = false;
    float* tokens_out = nullptr;
    bool tokens_pinned = false;
    std::vector<int32_t> store_to;                 // empty, or one slot (or -1) per frame
    size_t n_windows = 0;
    std::vector<shv::sched::TokenRef> refs;        // n_windows * 20
    std::vector<const float*> host_blocks;
    float* logits_out = nullptr;
    shv_hip_callback callback = nullptr;
    void* user = nullptr;
    shv::sched::Clock::time_point t_submit{};
    // the outcome, written once by the completer under mu
    mutable std::mutex mu;
    mutable std::condition_variable cv;
    int status = 0;          // 0 pending, 1 done, -1 failed
    bool settled = false;    // status final and the callback (if any) has returned: job_free may delete
    std::string error;
    struct Timing {
        double queue_ms = 0.0, run_ms = 0.0, device_ms = 0.0;   // submit -> batch start -> outputs final; GPU time
        int batch_frames = 0, batch_windows = 0;                  // size of the batch that carried the job
    } timing;
};

namespace shv {
namespace sched {

class Frontend {
public:
    Frontend(Device& dev, const Limits& lim);
    ~Frontend();
    Frontend(const Frontend&) = delete;
    Frontend& operator=(const Frontend&) = delete;

    const Limits& limits() const { return lim_; }
    // Validate, copy the index arrays, queue.  nullptr + last_error on invalid input or a closing model.
    shv_hip_job* submit(const shv_hip_request* r);
    // Complete every queued job, then stop both threads.  Idempotent; not concurrent with submit.
    void close();

    // synchronous wrappers: split into jobs of at most one batch each, wait; NaN outputs and -1 on failure
    int encode_frames(const uint8_t* rgb, size_t n, float* tokens);
    int classify(const float* tokens, size_t b, float* logits);
    int predict(const uint8_t* clips, size_t b, float* logits);

    // job queries do not touch the frontend: jobs outlive it
    static int job_status(const shv_hip_job* j);
    static int job_wait(shv_hip_job* j);
    static const char* job_error(const shv_hip_job* j);
    static int job_timing(const shv_hip_job* j, double* queue_ms, double* run_ms, double* device_ms,
                          int* batch_frames, int* batch_windows);
    static void job_free(shv_hip_job* j);

private:
    struct Member {
        shv_hip_job* job;
        int frame_at, window_at;
    };
    struct Flight {
        Batch batch;
        std::vector<Member> members;
        bool failed = false;
        std::string error;
        Clock::time_point t_start;
    };

    void launcher_main();
    void completer_main();
    bool lane_idle_locked() const { return int(free_lanes_.size()) == lanes_ && flights_.empty(); }
    bool queue_fills_batch_locked() const;
    void pick_locked(std::vector<shv_hip_job*>& picked);
    Flight* assemble(int lane, std::vector<shv_hip_job*>& picked) const;
    void deliver(Flight& f, const float* logits) const;
    static void finalize(shv_hip_job* j, bool ok, const std::string& err, double device_ms, int bf, int bw,
                         Clock::time_point t_start);
    template <class Fill, class Poison> int run_pieces(size_t total, size_t per, Fill&& fill, Poison&& poison);

    Device& dev_;
    const Limits lim_;
    const int lanes_;

    std::mutex mu_;
    std::condition_variable launcher_cv_;   // queue grew, a lane came free, or closing
    std::condition_variable completer_cv_;  // a flight started, or the launcher ended
    std::deque<shv_hip_job*> queue_;
    std::vector<int> free_lanes_;
    std::deque<Flight*> flights_;           // started, not yet landed, in start order
    bool closing_ = false;
    bool launcher_done_ = false;
    // planner: slot_mark_[s] == mark_ <=> slot s was read or stored by a job already in the batch being planned
    std::vector<uint32_t> slot_mark_;
    uint32_t mark_ = 0;

    std::thread launcher_, completer_;
};

}  // namespace sched
}  // namespace shv
