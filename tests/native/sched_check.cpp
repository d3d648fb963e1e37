// CPU check of the batched API's host side (shield-sisa_amd/csrc/sched.cpp) on a stub device, built and run under
// the thread sanitizer and under the address + undefined-behaviour sanitizers by tests/test_scheduler.py.
//
// The stub behaves like one in-order GPU stream: start() queues a batch for a device thread that "encodes" each
// frame (token t[0] = the frame's 32-bit id, t[1..] a fixed pattern), stores tokens into a host-side slot pool,
// and "classifies" each window: logit = sum over positions p of (p + 1) * t_p[0].  Pinned caller buffers are read
// and written by the device thread (DMA); pageable ones through the lane's staging, as the HIP device does.
// Every scenario checks outputs against the same function evaluated directly from the request.
#include "../../shield-sisa_amd/csrc/sched.hpp"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <random>
#include <string>
#include <thread>
#include <vector>

using namespace shv::sched;

namespace {

std::atomic<int> g_failures{0};   // CHECKs also run on the launcher thread (StubDevice::start)
#define CHECK(cond)                                                                                 \
    do {                                                                                            \
        if (!(cond)) {                                                                              \
            std::fprintf(stderr, "CHECK failed %s:%d: %s\n", __FILE__, __LINE__, #cond);            \
            ++g_failures;                                                                           \
        }                                                                                           \
    } while (0)

constexpr int32_t kInfId = -1;          // a frame whose token makes its windows' logits infinite
constexpr int32_t kFailStartId = -2;    // start() refuses a batch holding such a frame
constexpr int32_t kFailLandId = -3;     // land() reports a device error for such a batch

// ------------------------------------------------------------------------------------------ frames and tokens
struct Frames {   // n frames of 172800 bytes, frame i tagged with id[i] in its first 4 bytes
    std::vector<uint8_t> bytes;
    explicit Frames(const std::vector<int32_t>& ids) : bytes(ids.size() * kFrameBytes, 0) {
        for (size_t i = 0; i < ids.size(); ++i) std::memcpy(&bytes[i * kFrameBytes], &ids[i], 4);
    }
    const uint8_t* data() const { return bytes.data(); }
};
int32_t id_of(const uint8_t* frame) {
    int32_t id;
    std::memcpy(&id, frame, 4);
    return id;
}
void token_of(int32_t id, float* t) {
    t[0] = float(id);
    for (size_t i = 1; i < kTokenFloats; ++i) t[i] = float(int(i % 97) - 48) * 0.25f;
}
float logit_of(const std::vector<int32_t>& ids20) {   // the stub's classifier on the 20 token ids of a window
    float acc = 0.0f;
    for (int p = 0; p < kWindowFrames; ++p) {
        if (ids20[size_t(p)] == kInfId) return INFINITY;
        acc += float(p + 1) * float(ids20[size_t(p)]);
    }
    return acc;
}

// ------------------------------------------------------------------------------------------ the stub device
class StubDevice final : public Device {
public:
    struct Record {
        int frames, windows, host_blocks;
        bool stores;
        std::vector<int32_t> frame_ids;
    };

    StubDevice(const Limits& lim, int lanes, int exec_us)
        : lim_(lim), exec_us_(exec_us), lanes_(size_t(lanes)), pool_(size_t(std::max(lim.token_slots, 0)) * 4, 0) {
        for (Lane& L : lanes_) {
            L.logits.assign(size_t(lim.windows), 0.0f);
            L.tokens.assign(size_t(lim.frames) * kTokenFloats, 0.0f);
        }
        worker_ = std::thread([this] { run(); });
    }
    ~StubDevice() override {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        worker_.join();
    }

    void mark_pinned(const void* p, size_t bytes) {
        std::lock_guard<std::mutex> lk(mu_);
        pinned_.emplace_back(static_cast<const uint8_t*>(p), bytes);
    }
    std::vector<Record> records() {
        std::lock_guard<std::mutex> lk(mu_);
        return records_;
    }
    void set_exec_us(int us) { exec_us_.store(us); }
    int32_t pool_id(int slot) {
        std::lock_guard<std::mutex> lk(mu_);
        return pool_[size_t(slot) * 4];
    }

    int lanes() const override { return int(lanes_.size()); }
    bool host_pinned(const void* p, size_t bytes) override {
        std::lock_guard<std::mutex> lk(mu_);
        const uint8_t* a = static_cast<const uint8_t*>(p);
        for (const auto& r : pinned_)
            if (a >= r.first && a + bytes <= r.first + r.second) return true;
        return false;
    }
    void start(const Batch& b) override {
        validate(b);
        std::vector<int32_t> ids;
        for (const FrameSpan& sp : b.frame_spans)
            for (int i = 0; i < sp.count; ++i) ids.push_back(id_of(sp.src + size_t(i) * kFrameBytes));
        if (std::find(ids.begin(), ids.end(), kFailStartId) != ids.end())
            throw std::runtime_error("stub: batch refused at start");
        std::lock_guard<std::mutex> lk(mu_);
        Lane& L = lanes_.at(size_t(b.lane));
        if (L.busy) throw std::runtime_error("stub: lane started twice without landing");   // scheduler bug
        L.busy = true;
        L.done = false;
        L.fail = std::find(ids.begin(), ids.end(), kFailLandId) != ids.end();
        records_.push_back(Record{b.frames, b.windows, int(b.host_blocks.size()), !b.store_to.empty(), ids});
        queue_.push_back(b);
        cv_.notify_all();
    }
    const float* land(const Batch& b, double* device_ms) override {
        std::unique_lock<std::mutex> lk(mu_);
        Lane& L = lanes_.at(size_t(b.lane));
        cv_.wait(lk, [&] { return L.done; });
        L.busy = false;
        if (L.fail) throw std::runtime_error("stub: device error while running the batch");
        for (const TokenSpan& sp : b.token_spans)
            if (!sp.pinned)
                std::memcpy(sp.dst, &L.tokens[size_t(sp.at) * kTokenFloats], size_t(sp.count) * kTokenFloats * 4);
        *device_ms = 0.5;
        return L.logits.data();
    }
    void scrub(const Batch& b) noexcept override {
        std::unique_lock<std::mutex> lk(mu_);
        Lane& L = lanes_.at(size_t(b.lane));
        // a refused start queued nothing; otherwise wait until the device thread is through with the batch
        bool queued = false;
        for (const Batch& q : queue_) queued = queued || q.lane == b.lane;
        if (queued || (L.busy && !L.done)) cv_.wait(lk, [&] { return L.done; });
        L.busy = false;
    }

private:
    struct Lane {
        std::vector<float> logits, tokens;
        bool busy = false, done = false, fail = false;
    };

    void validate(const Batch& b) {
        CHECK(b.frames <= lim_.frames && b.windows <= lim_.windows && int(b.host_blocks.size()) <= lim_.host_blocks);
        CHECK(b.frames > 0 || b.windows > 0);
        CHECK(b.refs.size() == size_t(b.windows) * kWindowFrames);
        int next = 0;
        for (const FrameSpan& sp : b.frame_spans) {
            CHECK(sp.at == next && sp.count > 0);
            next += sp.count;
        }
        CHECK(next == b.frames);
        CHECK(b.store_to.empty() || b.store_to.size() == size_t(b.frames));
        for (int32_t s : b.store_to) CHECK(s >= -1 && s < lim_.token_slots);
        for (const TokenRef& r : b.refs) {
            if (r.kind == TokenRef::kFrame) CHECK(r.index >= 0 && r.index < b.frames);
            else if (r.kind == TokenRef::kSlot) CHECK(r.index >= 0 && r.index < lim_.token_slots);
            else CHECK(r.kind == TokenRef::kHost && r.index >= 0 && size_t(r.index) < b.host_blocks.size());
        }
        // the hazard rule: no slot is stored by a frame after an earlier job of the batch read or stored it.  The
        // stub sees only the batch, so it checks the weaker form that follows from it: no slot stored twice.
        std::vector<int32_t> st;
        for (int32_t s : b.store_to)
            if (s >= 0) st.push_back(s);
        std::sort(st.begin(), st.end());
        CHECK(std::adjacent_find(st.begin(), st.end()) == st.end());
    }

    void run() {
        for (;;) {
            Batch b;
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return stop_ || !queue_.empty(); });
                if (queue_.empty()) return;
                b = queue_.front();
            }
            if (exec_us_ > 0) std::this_thread::sleep_for(std::chrono::microseconds(exec_us_.load()));
            execute(b);
            std::lock_guard<std::mutex> lk(mu_);
            queue_.pop_front();
            lanes_.at(size_t(b.lane)).done = true;
            cv_.notify_all();
        }
    }

    // one batch, in stream order: encode, store, classify, copy out
    void execute(const Batch& b) {
        std::vector<int32_t> ids;
        for (const FrameSpan& sp : b.frame_spans)
            for (int i = 0; i < sp.count; ++i) ids.push_back(id_of(sp.src + size_t(i) * kFrameBytes));
        std::lock_guard<std::mutex> lk(mu_);   // the pool and lane buffers belong to the "device"
        Lane& L = lanes_.at(size_t(b.lane));
        for (size_t f = 0; f < b.store_to.size(); ++f)
            if (b.store_to[f] >= 0) pool_[size_t(b.store_to[f]) * 4] = ids[f];
        for (int w = 0; w < b.windows; ++w) {
            std::vector<int32_t> win(kWindowFrames);
            for (int p = 0; p < kWindowFrames; ++p) {
                const TokenRef& r = b.refs[size_t(w) * kWindowFrames + size_t(p)];
                if (r.kind == TokenRef::kFrame) win[size_t(p)] = ids[size_t(r.index)];
                else if (r.kind == TokenRef::kSlot) win[size_t(p)] = pool_[size_t(r.index) * 4];
                else win[size_t(p)] = int32_t(b.host_blocks[size_t(r.index)][0]);
            }
            L.logits[size_t(w)] = logit_of(win);
        }
        for (const TokenSpan& sp : b.token_spans)
            for (int i = 0; i < sp.count; ++i) {
                float* dst = sp.pinned ? sp.dst + size_t(i) * kTokenFloats : &L.tokens[size_t(sp.at + i) * kTokenFloats];
                token_of(ids[size_t(sp.at + i)], dst);
            }
    }

    const Limits lim_;
    std::atomic<int> exec_us_;
    std::mutex mu_;
    std::condition_variable cv_;
    std::vector<Lane> lanes_;
    std::deque<Batch> queue_;
    std::vector<int32_t> pool_;     // 4 ints per slot; [0] = the id of the stored frame
    std::vector<std::pair<const uint8_t*, size_t>> pinned_;
    std::vector<Record> records_;
    bool stop_ = false;
    std::thread worker_;
};

Limits limits(int frames, int windows, int host_blocks, int slots, int delay_us = 0) {
    Limits l;
    l.frames = frames;
    l.windows = windows;
    l.host_blocks = host_blocks;
    l.token_slots = slots;
    l.delay_us = delay_us;
    return l;
}

std::vector<int32_t> iota_ids(int n, int32_t first) {
    std::vector<int32_t> v(static_cast<size_t>(n));
    for (int i = 0; i < n; ++i) v[size_t(i)] = first + i;
    return v;
}

// A request plus the storage its pointers refer to; `expect` holds the logits it must produce.
struct Req {
    std::vector<int32_t> frame_ids;
    std::unique_ptr<Frames> frames;
    std::vector<int32_t> store, wframes, wslots;
    std::vector<std::vector<float>> host_tok;
    std::vector<const float*> wtok;
    std::vector<float> logits, tokens;
    std::vector<float> expect;
    shv_hip_request r{};

    void build() {
        r = shv_hip_request{};
        if (!frame_ids.empty()) {
            frames.reset(new Frames(frame_ids));
            r.frames = frames->data();
            r.n_frames = frame_ids.size();
            tokens.assign(frame_ids.size() * kTokenFloats, -7.0f);
            r.tokens_out = tokens.data();
        }
        if (!store.empty()) r.store_slots = store.data();
        const size_t nw = wframes.size() / kWindowFrames;
        r.n_windows = nw;
        if (nw) {
            logits.assign(nw, -7.0f);
            r.logits_out = logits.data();
            r.window_frames = wframes.data();
            r.window_slots = wslots.data();
            r.window_tokens = wtok.data();
        }
    }
    // a window over frames [f0, f0 + 20) of this request
    void window_own(int f0) {
        for (int p = 0; p < kWindowFrames; ++p) entry(f0 + p, -1, nullptr);
    }
    // a window over device token slots
    void window_slots(const std::vector<int32_t>& slots20) {
        for (int p = 0; p < kWindowFrames; ++p) entry(-1, slots20[size_t(p)], nullptr);
    }
    // a window over host token blocks carrying the given ids
    void window_host(const std::vector<int32_t>& ids20) {
        for (int p = 0; p < kWindowFrames; ++p) {
            host_tok.emplace_back(kTokenFloats);
            token_of(ids20[size_t(p)], host_tok.back().data());
            entry(-1, -1, host_tok.back().data());
        }
    }
    // a window with no token source at all (invalid)
    void window_empty() {
        for (int p = 0; p < kWindowFrames; ++p) entry(-1, -1, nullptr);
    }
    void entry(int32_t f, int32_t s, const float* t) {
        wframes.push_back(f);
        wslots.push_back(s);
        wtok.push_back(t);
    }
};

bool same_float(float a, float b) { return (std::isnan(a) && std::isnan(b)) || a == b; }

void check_tokens(const Req& q) {
    std::vector<float> t(kTokenFloats);
    for (size_t f = 0; f < q.frame_ids.size(); ++f) {
        token_of(q.frame_ids[f], t.data());
        CHECK(std::memcmp(t.data(), &q.tokens[f * kTokenFloats], kTokenFloats * 4) == 0);
    }
}

// ------------------------------------------------------------------------------------------ scenarios
void sync_wrappers() {
    const Limits lim = limits(40, 2, 40, 0);
    StubDevice dev(lim, 2, 200);
    Frontend fe(dev, lim);
    // predict: 5 clips in jobs of min(2, 40 / 20) = 2 clips
    const int clips = 5;
    std::vector<int32_t> ids = iota_ids(clips * 20, 1000);
    Frames fr(ids);
    std::vector<float> lg(clips, -1.0f);
    CHECK(fe.predict(fr.data(), clips, lg.data()) == 0);
    for (int c = 0; c < clips; ++c)
        CHECK(lg[size_t(c)] == logit_of(std::vector<int32_t>(ids.begin() + c * 20, ids.begin() + c * 20 + 20)));
    // encode_frames: 45 frames in jobs of 40
    std::vector<float> tok(45 * kTokenFloats);
    std::vector<int32_t> eids = iota_ids(45, 5000);
    Frames ef(eids);
    CHECK(fe.encode_frames(ef.data(), 45, tok.data()) == 0);
    std::vector<float> t(kTokenFloats);
    for (int f = 0; f < 45; ++f) {
        token_of(eids[size_t(f)], t.data());
        CHECK(std::memcmp(t.data(), &tok[size_t(f) * kTokenFloats], kTokenFloats * 4) == 0);
    }
    // classify host tokens: 3 windows in jobs of min(2, 40 / 20) = 2
    std::vector<float> host(3 * 20 * kTokenFloats);
    for (int e = 0; e < 60; ++e) token_of(7000 + e, &host[size_t(e) * kTokenFloats]);
    std::vector<float> cl(3);
    CHECK(fe.classify(host.data(), 3, cl.data()) == 0);
    for (int w = 0; w < 3; ++w) CHECK(cl[size_t(w)] == logit_of(iota_ids(20, 7000 + 20 * w)));
    // classify with too few host blocks for a window
    {
        const Limits small = limits(40, 2, 10, 0);
        StubDevice d2(small, 2, 0);
        Frontend f2(d2, small);
        CHECK(f2.classify(host.data(), 1, cl.data()) == -1);
        CHECK(std::string(last_error()).find("max_host_tokens is below") != std::string::npos);
    }
    // predict with fewer than 20 frames per batch
    {
        const Limits small = limits(19, 2, 40, 0);
        StubDevice d2(small, 2, 0);
        Frontend f2(d2, small);
        CHECK(f2.predict(fr.data(), 1, lg.data()) == -1);
        CHECK(std::string(last_error()).find("max_frames is below") != std::string::npos);
    }
}

void coalescing_and_limits() {
    const Limits lim = limits(64, 4, 60, 0);
    StubDevice dev(lim, 2, 100000);   // 100 ms per batch: later submits queue up behind two busy lanes
    Frontend fe(dev, lim);
    std::vector<std::unique_ptr<Req>> reqs;
    std::vector<shv_hip_job*> jobs;
    for (int i = 0; i < 14; ++i) {
        std::unique_ptr<Req> q(new Req());
        q->frame_ids = iota_ids(20, 100 * (i + 1));
        q->window_own(0);
        if (i % 3 == 1) q->window_host(iota_ids(20, 50000 + i));
        q->build();
        reqs.push_back(std::move(q));
    }
    for (auto& q : reqs) {
        jobs.push_back(fe.submit(&q->r));
        CHECK(jobs.back() != nullptr);
    }
    int max_bf = 0, max_bw = 0;
    for (size_t i = 0; i < jobs.size(); ++i) {
        CHECK(Frontend::job_wait(jobs[i]) == 0);
        double qm, rm, gm;
        int bf, bw;
        CHECK(Frontend::job_timing(jobs[i], &qm, &rm, &gm, &bf, &bw) == 0);
        CHECK(bf <= lim.frames && bw <= lim.windows && qm >= 0.0 && rm >= 0.0 && gm == 0.5);
        max_bf = std::max(max_bf, bf);
        max_bw = std::max(max_bw, bw);
        const Req& q = *reqs[i];
        CHECK(q.logits[0] == logit_of(q.frame_ids));
        if (q.logits.size() > 1) CHECK(q.logits[1] == logit_of(iota_ids(20, 50000 + int(i))));
        check_tokens(q);
        Frontend::job_free(jobs[i]);
    }
    CHECK(max_bf > 20);   // some jobs were coalesced
    // FIFO: frames reach the device in submission order
    std::vector<int32_t> seen;
    for (const auto& r : dev.records()) seen.insert(seen.end(), r.frame_ids.begin(), r.frame_ids.end());
    std::vector<int32_t> want;
    for (const auto& q : reqs) want.insert(want.end(), q->frame_ids.begin(), q->frame_ids.end());
    CHECK(seen == want);
}

void slot_hazard() {
    const Limits lim = limits(64, 8, 64, 16);
    StubDevice dev(lim, 2, 30000);
    Frontend fe(dev, lim);
    // occupy both lanes so that the jobs below are planned together from the queue: 61-frame busy jobs fit a
    // 64-frame batch neither with each other nor with a and b, and every request is built before the first submit
    // (building under the sanitizers can take longer than a busy batch runs)
    Req b0, b1;
    b0.frame_ids = iota_ids(61, 1000);
    b0.build();
    b1.frame_ids = iota_ids(61, 2000);
    b1.build();
    const std::vector<int32_t> s4 = {0, 1, 2, 3};
    std::vector<int32_t> read20;
    for (int p = 0; p < 20; ++p) read20.push_back(p % 4);
    Req a, b, c, d, e;
    a.frame_ids = {100, 101, 102, 103};     // stores 100..103 into slots 0..3
    a.store = s4;
    a.build();
    b.window_slots(read20);                 // reads slots 0..3 after a's store
    b.build();
    c.frame_ids = {200, 201, 202, 203};     // stores into slots b read: must start a new batch
    c.store = s4;
    c.build();
    d.window_slots(read20);                 // must see c's tokens
    d.build();
    e.frame_ids = {300};                    // stores into an unrelated slot: may join d's batch
    e.store = {9};
    e.window_slots(std::vector<int32_t>(20, 9));
    e.build();
    shv_hip_job* j0 = fe.submit(&b0.r);
    shv_hip_job* j1 = fe.submit(&b1.r);
    shv_hip_job* ja = fe.submit(&a.r);
    shv_hip_job* jb = fe.submit(&b.r);
    shv_hip_job* jc = fe.submit(&c.r);
    shv_hip_job* jd = fe.submit(&d.r);
    shv_hip_job* je = fe.submit(&e.r);
    for (shv_hip_job* j : {j0, j1, ja, jb, jc, jd, je}) CHECK(j && Frontend::job_wait(j) == 0);
    std::vector<int32_t> wa, wc;
    for (int p = 0; p < 20; ++p) {
        wa.push_back(100 + p % 4);
        wc.push_back(200 + p % 4);
    }
    CHECK(b.logits[0] == logit_of(wa));
    CHECK(d.logits[0] == logit_of(wc));
    CHECK(e.logits[0] == logit_of(std::vector<int32_t>(20, 300)));
    int bfa, bwa, bfc, bwc;
    Frontend::job_timing(ja, nullptr, nullptr, nullptr, &bfa, &bwa);
    Frontend::job_timing(jc, nullptr, nullptr, nullptr, &bfc, &bwc);
    CHECK(bfa == 4 && bwa == 1);   // a and b together, c not
    CHECK(bfc >= 4 && bwc >= 1);
    CHECK(dev.pool_id(0) == 200 && dev.pool_id(9) == 300);
    for (shv_hip_job* j : {j0, j1, ja, jb, jc, jd, je}) Frontend::job_free(j);
}

void close_completes_queued_jobs() {
    std::atomic<int> calls{0};
    std::vector<std::unique_ptr<Req>> reqs;
    std::vector<shv_hip_job*> jobs;
    {
        const Limits lim = limits(8, 2, 40, 0);
        StubDevice dev(lim, 2, 3000);
        {
            Frontend fe(dev, lim);
            for (int i = 0; i < 30; ++i) {
                std::unique_ptr<Req> q(new Req());
                q->frame_ids = iota_ids(1 + i % 8, 1000 * i);
                q->build();
                q->r.callback = [](shv_hip_job*, int status, void* u) {
                    if (status == 1) static_cast<std::atomic<int>*>(u)->fetch_add(1);
                };
                q->r.user = &calls;
                jobs.push_back(fe.submit(&q->r));
                CHECK(jobs.back() != nullptr);
                reqs.push_back(std::move(q));
            }
            fe.close();    // what shv_hip_free does: every queued job completes first
            Req late;
            late.frame_ids = {1};
            late.build();
            CHECK(fe.submit(&late.r) == nullptr);
            CHECK(std::string(last_error()).find("stopping") != std::string::npos);
        }
    }
    // the model is gone; the jobs are still valid and final
    CHECK(calls.load() == 30);
    for (size_t i = 0; i < jobs.size(); ++i) {
        CHECK(Frontend::job_status(jobs[i]) == 1);
        CHECK(Frontend::job_wait(jobs[i]) == 0);
        CHECK(std::string(Frontend::job_error(jobs[i])).empty());
        check_tokens(*reqs[i]);
        Frontend::job_free(jobs[i]);
    }
}

void non_finite_becomes_nan() {
    const Limits lim = limits(64, 4, 40, 0);
    StubDevice dev(lim, 2, 0);
    Frontend fe(dev, lim);
    Req q;
    q.frame_ids = iota_ids(40, 10);
    q.frame_ids[25] = kInfId;      // window 1 holds it
    q.window_own(0);
    q.window_own(20);
    q.build();
    shv_hip_job* j = fe.submit(&q.r);
    CHECK(j && Frontend::job_wait(j) == 0 && Frontend::job_status(j) == 1);
    CHECK(q.logits[0] == logit_of(iota_ids(20, 10)));
    CHECK(std::isnan(q.logits[1]));
    Frontend::job_free(j);
}

void failed_batches(int32_t poison, const char* what) {
    const Limits lim = limits(64, 4, 40, 0);
    StubDevice dev(lim, 2, 20000);
    Frontend fe(dev, lim);
    // two busy jobs of 50 frames each: neither fits a 64-frame batch with the other or with x, so they hold both
    // lanes alone however the launcher interleaves with the submits
    Req busy0, busy1;
    busy0.frame_ids = iota_ids(50, 100);
    busy0.build();
    busy1.frame_ids = iota_ids(50, 200);
    busy1.build();
    // x and y are planned into one batch behind the two busy lanes; x poisons it.  Both are built before the busy
    // jobs start (building a request under the sanitizers can take longer than a busy batch runs)
    std::atomic<int> failed_cb{0};
    Req x, y, z;
    x.frame_ids = iota_ids(20, 10);
    x.frame_ids[3] = poison;
    x.window_own(0);
    x.build();
    x.r.callback = [](shv_hip_job* job, int status, void* u) {
        if (status == -1 && Frontend::job_status(job) == -1) static_cast<std::atomic<int>*>(u)->fetch_add(1);
    };
    x.r.user = &failed_cb;
    y.frame_ids = iota_ids(20, 40);
    y.window_own(0);
    y.build();
    shv_hip_job* jb0 = fe.submit(&busy0.r);
    shv_hip_job* jb1 = fe.submit(&busy1.r);
    shv_hip_job* jx = fe.submit(&x.r);
    shv_hip_job* jy = fe.submit(&y.r);
    CHECK(Frontend::job_wait(jx) == -1);
    CHECK(std::string(last_error()).find(what) != std::string::npos);
    CHECK(Frontend::job_wait(jy) == -1);
    CHECK(std::string(Frontend::job_error(jy)).find(what) != std::string::npos);
    CHECK(std::isnan(x.logits[0]) && std::isnan(y.logits[0]));
    CHECK(std::isnan(x.tokens[0]) && std::isnan(y.tokens[kTokenFloats * 20 - 1]));
    // the model keeps working
    z.frame_ids = iota_ids(20, 70);
    z.window_own(0);
    z.build();
    shv_hip_job* jz = fe.submit(&z.r);
    CHECK(Frontend::job_wait(jz) == 0 && z.logits[0] == logit_of(iota_ids(20, 70)));
    for (shv_hip_job* j : {jb0, jb1, jx, jy, jz}) Frontend::job_free(j);
    CHECK(failed_cb.load() == 1);
}

struct CbState {
    std::atomic<bool> returned{false};
    std::atomic<int> seen_status{0};
    std::atomic<int> own_status{0};
    Frontend* fe = nullptr;
    Req* follow = nullptr;
    std::atomic<shv_hip_job*> follow_job{nullptr};
};

void callback_and_free_order() {
    const Limits lim = limits(64, 4, 40, 0);
    StubDevice dev(lim, 2, 1000);
    Frontend fe(dev, lim);
    CbState st;
    st.fe = &fe;
    Req follow;
    follow.frame_ids = iota_ids(20, 900);
    follow.window_own(0);
    follow.build();
    st.follow = &follow;
    Req q;
    q.frame_ids = iota_ids(20, 10);
    q.window_own(0);
    q.build();
    q.r.callback = [](shv_hip_job* job, int status, void* u) {
        CbState* s = static_cast<CbState*>(u);
        s->seen_status = status;
        s->own_status = Frontend::job_status(job);             // final before the callback runs
        s->follow_job = s->fe->submit(&s->follow->r);          // callbacks may submit
        std::this_thread::sleep_for(std::chrono::milliseconds(60));
        s->returned = true;
    };
    q.r.user = &st;
    shv_hip_job* j = fe.submit(&q.r);
    CHECK(Frontend::job_wait(j) == 0);          // returns once the status is final, possibly before the callback ends
    CHECK(q.logits[0] == logit_of(iota_ids(20, 10)));
    Frontend::job_free(j);                       // must wait for the callback's return
    CHECK(st.returned.load());
    CHECK(st.seen_status.load() == 1 && st.own_status.load() == 1);
    shv_hip_job* fj = st.follow_job.load();
    CHECK(fj != nullptr);
    CHECK(Frontend::job_wait(fj) == 0 && follow.logits[0] == logit_of(iota_ids(20, 900)));
    Frontend::job_free(fj);
}

void pending_timing_and_pinned_paths() {
    const Limits lim = limits(64, 4, 40, 0);
    StubDevice dev(lim, 2, 30000);
    Frontend fe(dev, lim);
    Req p, u;
    p.frame_ids = iota_ids(20, 10);
    p.window_own(0);
    p.build();
    dev.mark_pinned(p.frames->data(), p.frames->bytes.size());
    dev.mark_pinned(p.tokens.data(), p.tokens.size() * 4);
    u.frame_ids = iota_ids(20, 10);
    u.window_own(0);
    u.build();
    shv_hip_job* jp = fe.submit(&p.r);
    CHECK(jp->frames_pinned && jp->tokens_pinned);
    shv_hip_job* ju = fe.submit(&u.r);
    CHECK(!ju->frames_pinned && !ju->tokens_pinned);
    double qm;
    CHECK(Frontend::job_timing(jp, &qm, nullptr, nullptr, nullptr, nullptr) == 1);   // still pending
    CHECK(Frontend::job_wait(jp) == 0 && Frontend::job_wait(ju) == 0);
    CHECK(p.logits[0] == u.logits[0] && p.tokens == u.tokens);
    check_tokens(p);
    Frontend::job_free(jp);
    Frontend::job_free(ju);
}

void delay_gathers_jobs() {
    const Limits lim = limits(64, 4, 40, 0, 300000);   // idle launcher waits up to 300 ms for a fuller batch
    StubDevice dev(lim, 2, 0);
    Frontend fe(dev, lim);
    Req a, b;
    a.frame_ids = iota_ids(20, 10);
    a.window_own(0);
    a.build();
    b.frame_ids = iota_ids(20, 40);
    b.window_own(0);
    b.build();
    shv_hip_job* ja = fe.submit(&a.r);
    std::this_thread::sleep_for(std::chrono::milliseconds(20));
    shv_hip_job* jb = fe.submit(&b.r);
    CHECK(Frontend::job_wait(ja) == 0 && Frontend::job_wait(jb) == 0);
    int bw = 0;
    Frontend::job_timing(ja, nullptr, nullptr, nullptr, nullptr, &bw);
    CHECK(bw == 2);
    // a batch that is already full does not wait
    Req c, d;
    c.frame_ids = iota_ids(64, 100);
    c.build();
    const auto t0 = Clock::now();
    shv_hip_job* jc = fe.submit(&c.r);
    CHECK(Frontend::job_wait(jc) == 0);
    CHECK((std::chrono::duration<double, std::milli>(Clock::now() - t0).count() < 250.0));
    for (shv_hip_job* j : {ja, jb, jc}) Frontend::job_free(j);
}

void validation() {
    const Limits lim = limits(40, 2, 30, 4);
    StubDevice dev(lim, 2, 0);
    Frontend fe(dev, lim);
    const auto rejects = [&](Req& q, const char* msg) {
        q.build();
        shv_hip_job* j = fe.submit(&q.r);
        CHECK(j == nullptr);
        if (j) Frontend::job_free(j);
        const bool ok = std::string(last_error()).find(msg) != std::string::npos;
        if (!ok) std::fprintf(stderr, "  expected '%s', got '%s'\n", msg, last_error());
        CHECK(ok);
    };
    CHECK(fe.submit(nullptr) == nullptr);
    { Req q; rejects(q, "empty request"); }
    { Req q; q.frame_ids = iota_ids(41, 0); rejects(q, "more frames than max_frames"); }
    { Req q; q.frame_ids = {1, 2}; q.store = {0, 4}; rejects(q, "store slot out of range"); }
    { Req q; q.frame_ids = {1, 2}; q.store = {1, 1}; rejects(q, "duplicate store slot"); }
    { Req q; q.frame_ids = {1, 2}; q.window_own(0); rejects(q, "window frame index out of range"); }
    { Req q; q.window_slots(std::vector<int32_t>(20, 4)); rejects(q, "window slot out of range"); }
    {
        Req q;
        q.window_empty();
        rejects(q, "no token source");
    }
    {
        Req q;
        q.window_host(iota_ids(20, 0));
        q.window_host(iota_ids(20, 0));
        rejects(q, "more host token blocks");
    }
    {
        Req q;
        for (int w = 0; w < 3; ++w) q.window_slots(std::vector<int32_t>(20, 0));
        rejects(q, "more windows than max_windows");
    }
    {
        Req q;
        q.frame_ids = {1};
        q.build();
        q.r.frames = nullptr;
        shv_hip_job* j = fe.submit(&q.r);
        CHECK(j == nullptr && std::string(last_error()).find("null frames") != std::string::npos);
    }
    {
        const Limits nos = limits(40, 2, 30, 0);
        StubDevice d2(nos, 2, 0);
        Frontend f2(d2, nos);
        Req q;
        q.frame_ids = {1};
        q.store = {0};
        q.build();
        CHECK(f2.submit(&q.r) == nullptr);
        CHECK(std::string(last_error()).find("token_slots > 0") != std::string::npos);
    }
    // an accepted request clears the error
    Req ok;
    ok.frame_ids = {5};
    ok.build();
    shv_hip_job* j = fe.submit(&ok.r);
    CHECK(j != nullptr && std::string(last_error()).empty());
    Frontend::job_wait(j);
    Frontend::job_free(j);
}

// Many threads, random requests, per-thread slot ranges with store-then-read windows.
void concurrent_stress(int threads, int jobs_per_thread) {
    const Limits lim = limits(48, 6, 80, 4 * threads, 100);
    StubDevice dev(lim, 2, 300);
    Frontend fe(dev, lim);
    std::atomic<int> bad{0};
    std::vector<std::thread> ts;
    for (int t = 0; t < threads; ++t)
        ts.emplace_back([&, t] {
            std::mt19937 rng(1234u + unsigned(t));
            const std::vector<int32_t> mine = {4 * t, 4 * t + 1, 4 * t + 2, 4 * t + 3};
            std::deque<std::pair<std::unique_ptr<Req>, shv_hip_job*>> open;
            for (int i = 0; i < jobs_per_thread; ++i) {
                std::unique_ptr<Req> q(new Req());
                const int32_t base = 1000000 * (t + 1) + 1000 * i;
                const int kind = int(rng() % 4);
                std::vector<int32_t> want;
                if (kind == 0) {                    // own frames + window over them
                    q->frame_ids = iota_ids(20, base);
                    q->window_own(0);
                    want = q->frame_ids;
                } else if (kind == 1) {             // store into my slots, window reads them in the same job
                    q->frame_ids = iota_ids(4, base);
                    q->store = mine;
                    std::vector<int32_t> r20;
                    for (int p = 0; p < 20; ++p) {
                        r20.push_back(mine[size_t(p % 4)]);
                        want.push_back(base + p % 4);
                    }
                    q->window_slots(r20);
                } else if (kind == 2) {             // host tokens
                    want = iota_ids(20, base);
                    q->window_host(want);
                } else {                            // frames only, random count
                    q->frame_ids = iota_ids(1 + int(rng() % 12), base);
                }
                q->build();
                shv_hip_job* j = fe.submit(&q->r);
                if (!j) { ++bad; continue; }
                q->expect.clear();
                if (!want.empty()) q->expect.push_back(logit_of(want));
                open.emplace_back(std::move(q), j);
                while (open.size() > 6 || (i == jobs_per_thread - 1 && !open.empty())) {
                    auto& fr = open.front();
                    if (Frontend::job_wait(fr.second) != 0) ++bad;
                    const Req& r = *fr.first;
                    if (!r.expect.empty() && !same_float(r.logits[0], r.expect[0])) ++bad;
                    std::vector<float> tk(kTokenFloats);
                    for (size_t f = 0; f < r.frame_ids.size(); ++f) {
                        token_of(r.frame_ids[f], tk.data());
                        if (std::memcmp(tk.data(), &r.tokens[f * kTokenFloats], kTokenFloats * 4) != 0) ++bad;
                    }
                    Frontend::job_free(fr.second);
                    open.pop_front();
                }
            }
        });
    for (auto& th : ts) th.join();
    CHECK(bad.load() == 0);
    for (const auto& r : dev.records())
        CHECK(r.frames <= lim.frames && r.windows <= lim.windows && r.host_blocks <= lim.host_blocks);
}

}  // namespace

int main(int argc, char** argv) {
    const int scale = argc > 1 ? std::atoi(argv[1]) : 1;
    const std::vector<std::pair<const char*, std::function<void()>>> scenarios = {
        {"sync_wrappers", sync_wrappers},
        {"coalescing_and_limits", coalescing_and_limits},
        {"slot_hazard", slot_hazard},
        {"close_completes_queued_jobs", close_completes_queued_jobs},
        {"non_finite_becomes_nan", non_finite_becomes_nan},
        {"failed_start", [] { failed_batches(kFailStartId, "refused at start"); }},
        {"failed_land", [] { failed_batches(kFailLandId, "device error"); }},
        {"callback_and_free_order", callback_and_free_order},
        {"pending_timing_and_pinned_paths", pending_timing_and_pinned_paths},
        {"delay_gathers_jobs", delay_gathers_jobs},
        {"validation", validation},
        {"concurrent_stress", [scale] { concurrent_stress(8, 40 * scale); }},
    };
    for (const auto& s : scenarios) {
        const int before = g_failures.load();
        s.second();
        std::printf("%-34s %s\n", s.first, g_failures.load() == before ? "ok" : "FAILED");
        std::fflush(stdout);
    }
    const int nf = g_failures.load();
    std::printf("%s: %d failed checks\n", nf ? "FAIL" : "PASS", nf);
    return nf ? 1 : 0;
}
