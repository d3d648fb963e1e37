// Batched API host side: see sched.hpp.  Plain C++17 and the C header; no HIP.
#include "sched.hpp"

#include <algorithm>
#include <cmath>
#include <limits>
#include <memory>
#include <stdexcept>
#include <utility>

namespace shv {
namespace sched {

namespace {
thread_local std::string t_error;
constexpr float kNaN = std::numeric_limits<float>::quiet_NaN();

// Turns a request into a job record; throws std::runtime_error with the message the caller sees.
std::unique_ptr<shv_hip_job> resolve(const shv_hip_request& r, const Limits& lim, Device& dev) {
    if (r.n_frames == 0 && r.n_windows == 0) throw std::runtime_error("empty request (no frames, no windows)");
    if (r.n_frames > size_t(lim.frames)) throw std::runtime_error("request has more frames than max_frames");
    if (r.n_windows > size_t(lim.windows)) throw std::runtime_error("request has more windows than max_windows");
    if (r.n_frames && !r.frames) throw std::runtime_error("null frames for n_frames > 0");
    if (r.n_windows && !r.logits_out) throw std::runtime_error("null logits_out for n_windows > 0");

    std::unique_ptr<shv_hip_job> j(new shv_hip_job());
    j->frames = r.n_frames ? r.frames : nullptr;
    j->n_frames = r.n_frames;
    j->tokens_out = r.n_frames ? r.tokens_out : nullptr;
    j->n_windows = r.n_windows;
    j->logits_out = r.logits_out;
    j->callback = r.callback;
    j->user = r.user;

    if (r.store_slots && r.n_frames) {
        if (lim.token_slots <= 0) throw std::runtime_error("store_slots needs options.token_slots > 0");
        j->store_to.assign(r.store_slots, r.store_slots + r.n_frames);
        std::vector<int32_t> used;
        for (int32_t s : j->store_to) {
            if (s < -1 || s >= lim.token_slots) throw std::runtime_error("store slot out of range");
            if (s >= 0) used.push_back(s);
        }
        std::sort(used.begin(), used.end());
        if (std::adjacent_find(used.begin(), used.end()) != used.end())
            throw std::runtime_error("duplicate store slot in one request");
        if (used.empty()) j->store_to.clear();
    }

    const size_t entries = r.n_windows * size_t(kWindowFrames);
    j->refs.resize(entries);
    for (size_t e = 0; e < entries; ++e) {
        const int32_t f = r.window_frames ? r.window_frames[e] : -1;
        const int32_t s = (f < 0 && r.window_slots) ? r.window_slots[e] : -1;
        TokenRef& ref = j->refs[e];
        if (f >= 0) {
            if (size_t(f) >= r.n_frames) throw std::runtime_error("window frame index out of range");
            ref = TokenRef{TokenRef::kFrame, f};
        } else if (s >= 0) {
            if (s >= lim.token_slots) throw std::runtime_error("window slot out of range");
            ref = TokenRef{TokenRef::kSlot, s};
        } else {
            const float* p = r.window_tokens ? r.window_tokens[e] : nullptr;
            if (!p) throw std::runtime_error("window entry has no token source (frame, slot or host tokens)");
            ref = TokenRef{TokenRef::kHost, int32_t(j->host_blocks.size())};
            j->host_blocks.push_back(p);
        }
    }
    if (j->host_blocks.size() > size_t(lim.host_blocks))
        throw std::runtime_error("request has more host token blocks than max_host_tokens");

    j->frames_pinned = j->n_frames && dev.host_pinned(j->frames, j->n_frames * kFrameBytes);
    j->tokens_pinned = j->tokens_out && dev.host_pinned(j->tokens_out, j->n_frames * kTokenFloats * sizeof(float));
    return j;
}
}  // namespace

void set_error(const std::string& e) { t_error = e; }
void clear_error() { t_error.clear(); }
const char* last_error() { return t_error.c_str(); }

Frontend::Frontend(Device& dev, const Limits& lim) : dev_(dev), lim_(lim), lanes_(dev.lanes()) {
    if (lanes_ < 1) throw std::runtime_error("device has no lanes");
    if (lim_.frames < 1 || lim_.windows < 1 || lim_.host_blocks < 0 || lim_.token_slots < 0 || lim_.delay_us < 0)
        throw std::runtime_error("invalid options");
    for (int l = lanes_ - 1; l >= 0; --l) free_lanes_.push_back(l);
    slot_mark_.assign(size_t(lim_.token_slots), 0u);
    launcher_ = std::thread([this] { launcher_main(); });
    completer_ = std::thread([this] { completer_main(); });
}

Frontend::~Frontend() { close(); }

void Frontend::close() {
    {
        std::lock_guard<std::mutex> lk(mu_);
        closing_ = true;
    }
    launcher_cv_.notify_all();
    if (launcher_.joinable()) launcher_.join();
    if (completer_.joinable()) completer_.join();
}

shv_hip_job* Frontend::submit(const shv_hip_request* r) {
    try {
        if (!r) throw std::runtime_error("null argument");
        std::unique_ptr<shv_hip_job> j = resolve(*r, lim_, dev_);
        j->t_submit = Clock::now();
        {
            std::lock_guard<std::mutex> lk(mu_);
            if (closing_) throw std::runtime_error("model is stopping");
            queue_.push_back(j.get());
        }
        launcher_cv_.notify_all();
        clear_error();
        return j.release();
    } catch (const std::exception& e) {
        set_error(e.what());
        return nullptr;
    }
}

// ------------------------------------------------------------------------------------------------- launcher
bool Frontend::queue_fills_batch_locked() const {
    size_t f = 0, w = 0, h = 0;
    for (const shv_hip_job* j : queue_) {
        f += j->n_frames;
        w += j->n_windows;
        h += j->host_blocks.size();
        if (f >= size_t(lim_.frames) || w >= size_t(lim_.windows) || h >= size_t(lim_.host_blocks)) return true;
    }
    return false;
}

void Frontend::pick_locked(std::vector<shv_hip_job*>& picked) {
    if (!slot_mark_.empty() && ++mark_ == 0) {   // generation wrapped: forget every old mark
        std::fill(slot_mark_.begin(), slot_mark_.end(), 0u);
        mark_ = 1;
    }
    size_t f = 0, w = 0, h = 0;
    while (!queue_.empty()) {
        shv_hip_job* j = queue_.front();
        if (!picked.empty()) {
            if (f + j->n_frames > size_t(lim_.frames) || w + j->n_windows > size_t(lim_.windows) ||
                h + j->host_blocks.size() > size_t(lim_.host_blocks))
                break;
            bool hazard = false;
            for (int32_t s : j->store_to)
                if (s >= 0 && slot_mark_[size_t(s)] == mark_) { hazard = true; break; }
            if (hazard) break;
        }
        queue_.pop_front();
        picked.push_back(j);
        f += j->n_frames;
        w += j->n_windows;
        h += j->host_blocks.size();
        for (int32_t s : j->store_to)
            if (s >= 0) slot_mark_[size_t(s)] = mark_;
        for (const TokenRef& r : j->refs)
            if (r.kind == TokenRef::kSlot) slot_mark_[size_t(r.index)] = mark_;
    }
}

Frontend::Flight* Frontend::assemble(int lane, std::vector<shv_hip_job*>& picked) const {
    std::unique_ptr<Flight> fl(new Flight());
    Batch& b = fl->batch;
    b.lane = lane;
    bool stores = false;
    for (shv_hip_job* j : picked) {
        fl->members.push_back(Member{j, b.frames, b.windows});
        b.frames += int(j->n_frames);
        b.windows += int(j->n_windows);
        stores = stores || !j->store_to.empty();
    }
    if (stores) b.store_to.assign(size_t(b.frames), -1);
    b.refs.reserve(size_t(b.windows) * kWindowFrames);
    for (const Member& m : fl->members) {
        const shv_hip_job* j = m.job;
        if (j->n_frames) {
            b.frame_spans.push_back(FrameSpan{j->frames, m.frame_at, int(j->n_frames), j->frames_pinned});
            if (!j->store_to.empty())
                std::copy(j->store_to.begin(), j->store_to.end(), b.store_to.begin() + m.frame_at);
            if (j->tokens_out)
                b.token_spans.push_back(TokenSpan{j->tokens_out, m.frame_at, int(j->n_frames), j->tokens_pinned});
        }
        const int32_t host0 = int32_t(b.host_blocks.size());
        for (TokenRef r : j->refs) {
            if (r.kind == TokenRef::kFrame) r.index += m.frame_at;
            else if (r.kind == TokenRef::kHost) r.index += host0;
            b.refs.push_back(r);
        }
        b.host_blocks.insert(b.host_blocks.end(), j->host_blocks.begin(), j->host_blocks.end());
    }
    return fl.release();
}

void Frontend::launcher_main() {
    std::unique_lock<std::mutex> lk(mu_);
    for (;;) {
        launcher_cv_.wait(lk, [&] { return closing_ || !queue_.empty(); });
        if (queue_.empty()) break;   // closing, and every queued job has been started
        launcher_cv_.wait(lk, [&] { return !free_lanes_.empty(); });
        if (lim_.delay_us > 0 && lane_idle_locked() && !closing_) {
            // nothing in flight: give later submits a moment to join this batch.  The deadline is on the system
            // clock: libstdc++ waits on it with pthread_cond_timedwait, which every thread sanitizer understands
            // (a steady-clock deadline goes through pthread_cond_clockwait, which GCC 11's does not intercept).
            const auto until = std::chrono::system_clock::now() + std::chrono::microseconds(lim_.delay_us);
            launcher_cv_.wait_until(lk, until, [&] { return closing_ || queue_fills_batch_locked(); });
        }
        const int lane = free_lanes_.back();
        free_lanes_.pop_back();
        std::vector<shv_hip_job*> picked;
        pick_locked(picked);
        lk.unlock();

        Flight* fl = assemble(lane, picked);
        fl->t_start = Clock::now();
        try {
            dev_.start(fl->batch);
        } catch (const std::exception& e) {
            fl->failed = true;
            fl->error = e.what();
        }
        lk.lock();
        flights_.push_back(fl);
        completer_cv_.notify_one();
    }
    launcher_done_ = true;
    completer_cv_.notify_one();
}

// ------------------------------------------------------------------------------------------------- completer
void Frontend::deliver(Flight& f, const float* logits) const {
    for (const Member& m : f.members) {
        shv_hip_job* j = m.job;
        if (f.failed) {
            std::fill(j->logits_out, j->logits_out + j->n_windows, kNaN);
            if (j->tokens_out) std::fill(j->tokens_out, j->tokens_out + j->n_frames * kTokenFloats, kNaN);
            continue;
        }
        for (size_t w = 0; w < j->n_windows; ++w) {
            const float v = logits[size_t(m.window_at) + w];
            j->logits_out[w] = std::isfinite(v) ? v : kNaN;   // a non-finite logit means "unavailable"
        }
    }
}

void Frontend::finalize(shv_hip_job* j, bool ok, const std::string& err, double device_ms, int bf, int bw,
                        Clock::time_point t_start) {
    shv_hip_callback cb;
    void* user;
    const auto ms = [](Clock::time_point a, Clock::time_point b) {
        return std::chrono::duration<double, std::milli>(b - a).count();
    };
    const Clock::time_point now = Clock::now();
    {
        std::lock_guard<std::mutex> lk(j->mu);
        j->status = ok ? 1 : -1;
        j->error = ok ? std::string() : err;
        j->timing.queue_ms = ms(j->t_submit, t_start);
        j->timing.run_ms = ms(t_start, now);
        j->timing.device_ms = device_ms;
        j->timing.batch_frames = bf;
        j->timing.batch_windows = bw;
        cb = j->callback;
        user = j->user;
        if (!cb) j->settled = true;
        j->cv.notify_all();   // while holding j->mu: once settled is seen, job_free may delete the job
    }
    if (!cb) return;
    cb(j, ok ? 1 : -1, user);
    std::lock_guard<std::mutex> lk(j->mu);
    j->settled = true;
    j->cv.notify_all();
}

void Frontend::completer_main() {
    for (;;) {
        Flight* fl;
        {
            std::unique_lock<std::mutex> lk(mu_);
            completer_cv_.wait(lk, [&] { return !flights_.empty() || launcher_done_; });
            if (flights_.empty()) return;
            fl = flights_.front();
            flights_.pop_front();
        }
        const float* logits = nullptr;
        double device_ms = 0.0;
        if (!fl->failed) {
            try {
                logits = dev_.land(fl->batch, &device_ms);
            } catch (const std::exception& e) {
                fl->failed = true;
                fl->error = e.what();
            }
        }
        if (fl->failed) dev_.scrub(fl->batch);
        deliver(*fl, logits);
        {
            std::lock_guard<std::mutex> lk(mu_);   // the lane's buffers are no longer needed
            free_lanes_.push_back(fl->batch.lane);
        }
        launcher_cv_.notify_all();
        for (const Member& m : fl->members)
            finalize(m.job, !fl->failed, fl->error, device_ms, fl->batch.frames, fl->batch.windows, fl->t_start);
        delete fl;
    }
}

// ------------------------------------------------------------------------------------------------- jobs
namespace {
// Looks at a job under its lock; with `until_final`, first waits for the completer to finalise it.
template <class Read> auto read_job(const shv_hip_job& j, bool until_final, Read&& read) {
    std::unique_lock<std::mutex> lk(j.mu);
    if (until_final) j.cv.wait(lk, [&] { return j.status != 0; });
    return read(j);
}
}  // namespace

int Frontend::job_status(const shv_hip_job* j) {
    return j ? read_job(*j, false, [](const shv_hip_job& x) { return x.status; }) : -1;
}

int Frontend::job_wait(shv_hip_job* j) {
    if (!j) {
        set_error("job_wait: the job handle is NULL");
        return -1;
    }
    std::string why;
    const int status = read_job(*j, true, [&](const shv_hip_job& x) {
        why = x.error;
        return x.status;
    });
    if (status < 0) {
        set_error(why);
        return -1;
    }
    return 0;
}

const char* Frontend::job_error(const shv_hip_job* j) {
    // the text lives in the job, which is final once it is non-empty, so the pointer stays valid until job_free
    return j ? read_job(*j, false, [](const shv_hip_job& x) { return x.error.c_str(); }) : "job handle is NULL";
}

int Frontend::job_timing(const shv_hip_job* j, double* queue_ms, double* run_ms, double* device_ms, int* bf,
                         int* bw) {
    if (!j) return -1;
    shv_hip_job::Timing t;
    const bool final = read_job(*j, false, [&](const shv_hip_job& x) {
        t = x.timing;
        return x.status != 0;
    });
    if (!final) return 1;
    const std::pair<double*, double> d[] = {{queue_ms, t.queue_ms}, {run_ms, t.run_ms}, {device_ms, t.device_ms}};
    for (const auto& f : d)
        if (f.first) *f.first = f.second;
    if (bf) *bf = t.batch_frames;
    if (bw) *bw = t.batch_windows;
    return 0;
}

void Frontend::job_free(shv_hip_job* j) {
    if (!j) return;
    {
        std::unique_lock<std::mutex> lk(j->mu);
        j->cv.wait(lk, [&] { return j->settled; });
    }
    delete j;
}

// ------------------------------------------------------------------------------------------------- sync calls
// A synchronous call as requests of at most `per` of its `total` units.  Every piece is submitted before the first
// is waited for, so the pieces pipeline over the lanes.  fill(at, count, request) describes a piece.  A failed job
// writes NaN into its own outputs; the pieces left unsubmitted after a refused submit get poison(at, count).  Each
// job is freed here; the result is 0, or -1 with the first failure in piece order (a refused submit comes last).
template <class Fill, class Poison>
int Frontend::run_pieces(size_t total, size_t per, Fill&& fill, Poison&& poison) {
    std::vector<shv_hip_job*> submitted;
    std::string refused;
    size_t at = 0;
    while (at < total) {
        const size_t count = std::min(per, total - at);
        shv_hip_request r{};
        fill(at, count, r);
        shv_hip_job* j = submit(&r);
        if (!j) {
            refused = last_error();
            poison(at, total - at);
            break;
        }
        submitted.push_back(j);
        at += count;
    }
    bool failed = at < total;
    std::string first;
    for (shv_hip_job* j : submitted) {
        if (job_wait(j) != 0 && !failed) {
            failed = true;
            first = job_error(j);
        }
        job_free(j);
    }
    if (!failed) {
        clear_error();
        return 0;
    }
    set_error(first.empty() ? refused : first);
    return -1;
}

int Frontend::encode_frames(const uint8_t* rgb, size_t n, float* tokens) {
    if (n && (!rgb || !tokens)) {
        set_error("encode_frames: frames and tokens must be non-NULL");
        return -1;
    }
    return run_pieces(
        n, size_t(lim_.frames),
        [&](size_t at, size_t count, shv_hip_request& r) {
            r.frames = rgb + at * kFrameBytes;
            r.n_frames = count;
            r.tokens_out = tokens + at * kTokenFloats;
        },
        [&](size_t at, size_t count) { std::fill_n(tokens + at * kTokenFloats, count * kTokenFloats, kNaN); });
}

int Frontend::classify(const float* tokens, size_t b, float* logits) {
    if (b && (!tokens || !logits)) {
        set_error("classify: tokens and logits must be non-NULL");
        return -1;
    }
    const size_t windows_per_batch = size_t(lim_.host_blocks / kWindowFrames);
    if (b && windows_per_batch == 0) {
        set_error("classify: options.max_host_tokens is below the 20 token blocks of one window");
        return -1;
    }
    std::vector<const float*> blocks;   // one piece's entry table; submit copies it
    return run_pieces(
        b, std::min(size_t(lim_.windows), windows_per_batch),
        [&](size_t at, size_t count, shv_hip_request& r) {
            blocks.resize(count * kWindowFrames);
            const float* first = tokens + at * kWindowFrames * kTokenFloats;
            for (size_t e = 0; e < blocks.size(); ++e) blocks[e] = first + e * kTokenFloats;
            r.n_windows = count;
            r.window_tokens = blocks.data();
            r.logits_out = logits + at;
        },
        [&](size_t at, size_t count) { std::fill_n(logits + at, count, kNaN); });
}

int Frontend::predict(const uint8_t* clips, size_t b, float* logits) {
    if (b && (!clips || !logits)) {
        set_error("predict: clips and logits must be non-NULL");
        return -1;
    }
    const size_t clips_per_batch = std::min(size_t(lim_.windows), size_t(lim_.frames / kWindowFrames));
    if (b && clips_per_batch == 0) {
        set_error("predict: options.max_frames is below the 20 frames of one clip");
        return -1;
    }
    // window w reads frames 20 w .. 20 w + 19 of its own piece
    std::vector<int32_t> frame_of(clips_per_batch * kWindowFrames);
    for (size_t e = 0; e < frame_of.size(); ++e) frame_of[e] = int32_t(e);
    return run_pieces(
        b, clips_per_batch,
        [&](size_t at, size_t count, shv_hip_request& r) {
            r.frames = clips + at * kWindowFrames * kFrameBytes;
            r.n_frames = count * kWindowFrames;
            r.n_windows = count;
            r.window_frames = frame_of.data();
            r.logits_out = logits + at;
        },
        [&](size_t at, size_t count) { std::fill_n(logits + at, count, kNaN); });
}

}  // namespace sched
}  // namespace shv
