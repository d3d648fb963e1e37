// HipLanes: see lanes.hpp.  Per batch, on the copy stream: frames (pinned callers' memory DMA'd in place, the rest
// gathered into the lane's pinned staging and sent as one copy per run), the window entry table, host token blocks
// and the store table; an event hands the lane to the compute stream, which encodes, stores tokens into the pool,
// classifies and copies the logits and requested tokens back.  Two lanes let one batch's uploads run while the
// previous batch computes.
#include "lanes.hpp"

#include "kernels.hpp"

#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>

namespace shv {

namespace {
constexpr size_t FB = sched::kFrameBytes;
constexpr size_t TF = sched::kTokenFloats;

template <class U> U* pinned(size_t count) {
    void* p = nullptr;
    SHV_HIP_CHECK(hipHostMalloc(&p, std::max<size_t>(count * sizeof(U), 64), hipHostMallocDefault));
    return static_cast<U*>(p);
}
}  // namespace

HipLanes::HipLanes(const HostModel& hm, Precision p, const EngineConfig& cfg, int token_slots, int device)
    : device_(device) {
    SHV_HIP_CHECK(hipSetDevice(device_));
    try {
        SHV_HIP_CHECK(hipStreamCreateWithFlags(&copy_, hipStreamNonBlocking));
        SHV_HIP_CHECK(hipStreamCreateWithFlags(&compute_, hipStreamNonBlocking));
        eng_ = make_engine(hm, p, cfg);
        const size_t frames = size_t(cfg.max_frames), windows = size_t(cfg.max_windows);
        const size_t blocks = std::max<size_t>(size_t(cfg.max_host_tokens), 1);
        lane_.resize(size_t(cfg.slots));
        for (Staging& L : lane_) {
            L.frames = pinned<uint8_t>(frames * FB);
            L.blocks = pinned<float>(blocks * TF);
            L.table = pinned<const float*>(windows * sched::kWindowFrames);
            L.store = pinned<int32_t>(2 * frames);
            L.tokens = pinned<float>(frames * TF);
            L.logits = pinned<float>(windows);
            SHV_HIP_CHECK(hipEventCreateWithFlags(&L.uploaded, hipEventDisableTiming));
            SHV_HIP_CHECK(hipEventCreate(&L.t0));
            SHV_HIP_CHECK(hipEventCreate(&L.t1));
        }
        if (token_slots > 0) {
            pool_bytes_ = size_t(token_slots) * TF * sizeof(float);
            SHV_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&pool_), pool_bytes_));
            SHV_HIP_CHECK(hipMemset(pool_, 0, pool_bytes_));
        }
        SHV_HIP_CHECK(hipDeviceSynchronize());
    } catch (...) {
        release();
        throw;
    }
}

HipLanes::~HipLanes() { release(); }

void HipLanes::release() noexcept {
    if (compute_) (void)hipStreamSynchronize(compute_);
    if (copy_) (void)hipStreamSynchronize(copy_);
    for (Staging& L : lane_) {
        for (void* p : {static_cast<void*>(L.frames), static_cast<void*>(L.blocks), static_cast<void*>(L.table),
                        static_cast<void*>(L.store), static_cast<void*>(L.tokens), static_cast<void*>(L.logits)})
            if (p) (void)hipHostFree(p);
        for (hipEvent_t e : {L.uploaded, L.t0, L.t1})
            if (e) (void)hipEventDestroy(e);
    }
    lane_.clear();
    if (pool_) (void)hipFree(pool_);
    pool_ = nullptr;
    eng_.reset();
    if (compute_) (void)hipStreamDestroy(compute_);
    if (copy_) (void)hipStreamDestroy(copy_);
    compute_ = copy_ = nullptr;
}

size_t HipLanes::device_bytes() const { return eng_->device_bytes() + pool_bytes_; }

bool HipLanes::host_pinned(const void* p, size_t bytes) {
    if (!p || !bytes) return false;
    const uint8_t* first = static_cast<const uint8_t*>(p);
    for (const uint8_t* q : {first, first + bytes - 1}) {
        hipPointerAttribute_t a{};
        if (hipPointerGetAttributes(&a, q) != hipSuccess) {
            (void)hipGetLastError();   // pageable memory: not an error for the caller
            return false;
        }
        if (a.type != hipMemoryTypeHost) return false;
    }
    return true;
}

void HipLanes::start(const sched::Batch& b) {
    if (const char* f = std::getenv("SHV_HIP_TEST_FAIL_BATCH"))
        if (*f && std::strcmp(f, "0") != 0) throw std::runtime_error("injected batch failure (SHV_HIP_TEST_FAIL_BATCH)");
    SHV_HIP_CHECK(hipSetDevice(device_));
    Staging& L = lane_.at(size_t(b.lane));
    const Engine::Slot& d = eng_->slot(b.lane);

    // frames: pinned spans in place, pageable spans gathered into staging and sent per contiguous run
    int run_at = 0, run_len = 0;
    const auto send_run = [&] {
        if (run_len)
            SHV_HIP_CHECK(hipMemcpyAsync(d.d_frames + size_t(run_at) * FB, L.frames + size_t(run_at) * FB,
                                         size_t(run_len) * FB, hipMemcpyHostToDevice, copy_));
        run_len = 0;
    };
    for (const sched::FrameSpan& sp : b.frame_spans) {
        if (sp.pinned) {
            send_run();
            SHV_HIP_CHECK(hipMemcpyAsync(d.d_frames + size_t(sp.at) * FB, sp.src, size_t(sp.count) * FB,
                                         hipMemcpyHostToDevice, copy_));
            continue;
        }
        std::memcpy(L.frames + size_t(sp.at) * FB, sp.src, size_t(sp.count) * FB);
        if (!run_len) run_at = sp.at;
        run_len += sp.count;
    }
    send_run();

    // window entries -> device addresses of their token blocks
    const float* const base[3] = {d.d_tokens, pool_, d.d_tok_stage};
    for (size_t e = 0; e < b.refs.size(); ++e) {
        const sched::TokenRef& r = b.refs[e];
        if (r.kind == sched::TokenRef::kSlot && !pool_) throw std::runtime_error("window reads a slot without a pool");
        L.table[e] = base[r.kind] + size_t(r.index) * TF;
    }
    for (size_t h = 0; h < b.host_blocks.size(); ++h)
        std::memcpy(L.blocks + h * TF, b.host_blocks[h], TF * sizeof(float));
    if (!b.refs.empty())
        SHV_HIP_CHECK(hipMemcpyAsync(d.d_tokptr, L.table, b.refs.size() * sizeof(float*), hipMemcpyHostToDevice,
                                     copy_));
    if (!b.host_blocks.empty())
        SHV_HIP_CHECK(hipMemcpyAsync(d.d_tok_stage, L.blocks, b.host_blocks.size() * TF * sizeof(float),
                                     hipMemcpyHostToDevice, copy_));
    // token-slot stores as (batch frame, slot) pairs of the frames that store
    int n_store = 0;
    if (!b.store_to.empty()) {
        if (!pool_) throw std::runtime_error("batch stores tokens without a pool");
        for (int f = 0; f < int(b.store_to.size()); ++f)
            if (b.store_to[size_t(f)] >= 0) {
                L.store[2 * n_store] = f;
                L.store[2 * n_store + 1] = b.store_to[size_t(f)];
                ++n_store;
            }
        if (n_store)
            SHV_HIP_CHECK(hipMemcpyAsync(d.d_store, L.store, size_t(n_store) * 2 * sizeof(int32_t),
                                         hipMemcpyHostToDevice, copy_));
    }
    SHV_HIP_CHECK(hipEventRecord(L.uploaded, copy_));

    // compute
    SHV_HIP_CHECK(hipStreamWaitEvent(compute_, L.uploaded, 0));
    SHV_HIP_CHECK(hipEventRecord(L.t0, compute_));
    // a batch whose window w reads exactly its frames [20 w, 20 w + 20) runs as one branched forward
    bool aligned = b.windows > 0 && b.frames == b.windows * kFrames && b.refs.size() == size_t(b.frames);
    for (size_t e = 0; aligned && e < b.refs.size(); ++e)
        aligned = b.refs[e].kind == sched::TokenRef::kFrame && b.refs[e].index == int32_t(e);
    const bool fused = aligned && eng_->forward_slot(b.lane, b.windows, compute_);
    if (b.frames && !fused) eng_->encode_slot(b.lane, b.frames, compute_);
    if (n_store) {
        launch_slot_store(d.d_tokens, d.d_store, n_store, pool_, compute_);
        SHV_HIP_CHECK(hipGetLastError());
    }
    if (b.windows) {
        if (!fused) eng_->classify_slot(b.lane, b.windows, compute_);
        SHV_HIP_CHECK(hipMemcpyAsync(L.logits, d.d_logits, size_t(b.windows) * sizeof(float), hipMemcpyDeviceToHost,
                                     compute_));
    }
    for (const sched::TokenSpan& sp : b.token_spans) {
        float* dst = sp.pinned ? sp.dst : L.tokens + size_t(sp.at) * TF;
        SHV_HIP_CHECK(hipMemcpyAsync(dst, d.d_tokens + size_t(sp.at) * TF, size_t(sp.count) * TF * sizeof(float),
                                     hipMemcpyDeviceToHost, compute_));
    }
    SHV_HIP_CHECK(hipEventRecord(L.t1, compute_));
}

const float* HipLanes::land(const sched::Batch& b, double* device_ms) {
    Staging& L = lane_.at(size_t(b.lane));
    SHV_HIP_CHECK(hipSetDevice(device_));
    const hipError_t e = hipEventSynchronize(L.t1);
    if (e != hipSuccess) throw std::runtime_error(std::string("HIP error: ") + hipGetErrorString(e));
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, L.t0, L.t1) != hipSuccess) {
        (void)hipGetLastError();
        ms = 0.0f;
    }
    *device_ms = ms;
    for (const sched::TokenSpan& sp : b.token_spans)
        if (!sp.pinned)
            std::memcpy(sp.dst, L.tokens + size_t(sp.at) * TF, size_t(sp.count) * TF * sizeof(float));
    return L.logits;
}

void HipLanes::scrub(const sched::Batch&) noexcept {
    (void)hipSetDevice(device_);
    (void)hipStreamSynchronize(copy_);
    (void)hipStreamSynchronize(compute_);
    (void)hipGetLastError();
}

}  // namespace shv
