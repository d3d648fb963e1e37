// SHIELD-V HIP engine: C API (include/shv_hip.h), scheduler worker, certificates.
//
// Contract: engine/include/shv_cuda.h:28-59 and the reference scheduler's observable behaviour
// (engine/cuda/api.cu:177-383): FIFO jobs coalesced into GPU batches up to the limits, a job that stores into a
// device slot read or stored earlier in the batch starts a new batch, two I/O slots pipelined over a copy
// stream and a compute stream, NaN logits for failed batches and non-finite results, callbacks on the worker
// thread after outputs are final, job_free waits for the callback's return.
#include "../../include/shv_hip.h"

#include "engine.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <fstream>
#include <limits>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <thread>
#include <unordered_set>
#include <vector>

#ifndef SHV_HIP_REVISION
#define SHV_HIP_REVISION "hip-unversioned"
#endif

namespace {
using Clock = std::chrono::steady_clock;
thread_local std::string g_err;
constexpr float kNaN = std::numeric_limits<float>::quiet_NaN();
constexpr size_t FB = SHV_HIP_FRAME_BYTES, TF = SHV_HIP_TOKEN_FLOATS;

bool is_pinned(const void* p, size_t bytes) {
    if (!p || !bytes) return false;
    auto host_side = [](const void* q) {
        hipPointerAttribute_t a{};
        if (hipPointerGetAttributes(&a, q) != hipSuccess) {
            (void)hipGetLastError();
            return false;
        }
        return a.type == hipMemoryTypeHost;
    };
    return host_side(p) && host_side(static_cast<const uint8_t*>(p) + bytes - 1);
}
}  // namespace

struct shv_hip_job {
    const uint8_t* frames = nullptr;
    size_t n_frames = 0;
    float* tokens_out = nullptr;
    std::vector<int32_t> store_slots;
    size_t n_windows = 0;
    std::vector<int32_t> wframes, wslots;
    std::vector<const float*> wtokens;
    float* logits_out = nullptr;
    shv_hip_callback cb = nullptr;
    void* user = nullptr;
    bool frames_pinned = false, tokens_out_pinned = false;
    int host_tokens = 0;
    int frame_off = 0, window_off = 0;   // position inside its batch
    mutable std::mutex m;
    std::condition_variable cv;
    int state = 0;          // 0 pending, 1 done, -1 failed
    bool released = false;  // the callback has returned
    std::string error;
    Clock::time_point t_submit, t_start, t_done;
    float gpu_ms = 0.0f;
    int batch_frames = 0, batch_windows = 0;
};

namespace {

struct HostSlot {
    uint8_t* frames = nullptr;       // pinned staging [max_frames][FB]
    float* tok_stage = nullptr;      // pinned [max_host_tokens][TF]
    const float** tokptr = nullptr;  // pinned [max_windows * 20]
    int32_t* store = nullptr;        // pinned [max_frames]
    float* tokens_out = nullptr;     // pinned [max_frames][TF]
    float* logits = nullptr;         // pinned [max_windows]
    hipEvent_t h2d = nullptr, start = nullptr, end = nullptr;
};

struct Batch {
    int slot = 0;
    std::vector<shv_hip_job*> jobs;
    int F = 0, B = 0;
    bool failed = false;
    std::string error;
    Clock::time_point t_start;
};

class Core {
public:
    std::unique_ptr<shv::Engine> eng;
    std::string mode, fingerprint;
    double threshold = 0.0;
    int device = 0;
    shv_hip_options opt{};
    hipStream_t s_comp = nullptr, s_copy = nullptr;
    std::vector<HostSlot> hs;
    float* d_pool = nullptr;
    size_t device_bytes = 0;

    std::mutex mu;
    std::condition_variable cv;
    std::deque<shv_hip_job*> q;
    bool stopping = false;
    std::thread worker;

    ~Core() {
        for (HostSlot& h : hs) {
            if (h.frames) (void)hipHostFree(h.frames);
            if (h.tok_stage) (void)hipHostFree(h.tok_stage);
            if (h.tokptr) (void)hipHostFree(h.tokptr);
            if (h.store) (void)hipHostFree(h.store);
            if (h.tokens_out) (void)hipHostFree(h.tokens_out);
            if (h.logits) (void)hipHostFree(h.logits);
            if (h.h2d) (void)hipEventDestroy(h.h2d);
            if (h.start) (void)hipEventDestroy(h.start);
            if (h.end) (void)hipEventDestroy(h.end);
        }
        if (d_pool) (void)hipFree(d_pool);
        eng.reset();
        if (s_comp) (void)hipStreamDestroy(s_comp);
        if (s_copy) (void)hipStreamDestroy(s_copy);
    }

    void init(const shv::HostModel& hm, shv::Precision p) {
        SHV_HIP_CHECK(hipSetDevice(device));
        SHV_HIP_CHECK(hipStreamCreateWithFlags(&s_comp, hipStreamNonBlocking));
        SHV_HIP_CHECK(hipStreamCreateWithFlags(&s_copy, hipStreamNonBlocking));
        shv::EngineConfig ec;
        ec.max_frames = opt.max_frames;
        ec.max_windows = opt.max_windows;
        ec.max_host_tokens = opt.max_host_tokens;
        ec.use_graphs = opt.use_graphs != 0;
        ec.slots = 2;
        eng = shv::make_engine(hm, p, ec);
        const size_t Fm = size_t(opt.max_frames), Bm = size_t(opt.max_windows);
        const size_t Hm = std::max<size_t>(size_t(opt.max_host_tokens), 1);
        hs.resize(size_t(ec.slots));
        for (HostSlot& h : hs) {
            SHV_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&h.frames), Fm * FB, hipHostMallocDefault));
            SHV_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&h.tok_stage), Hm * TF * 4, hipHostMallocDefault));
            SHV_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&h.tokptr), Bm * 20 * sizeof(float*), hipHostMallocDefault));
            SHV_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&h.store), Fm * 4, hipHostMallocDefault));
            SHV_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&h.tokens_out), Fm * TF * 4, hipHostMallocDefault));
            SHV_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&h.logits), Bm * 4, hipHostMallocDefault));
            SHV_HIP_CHECK(hipEventCreateWithFlags(&h.h2d, hipEventDisableTiming));
            SHV_HIP_CHECK(hipEventCreate(&h.start));
            SHV_HIP_CHECK(hipEventCreate(&h.end));
        }
        if (opt.token_slots > 0) {
            SHV_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&d_pool), size_t(opt.token_slots) * TF * 4));
            SHV_HIP_CHECK(hipMemset(d_pool, 0, size_t(opt.token_slots) * TF * 4));
        }
        device_bytes = eng->device_bytes() + size_t(std::max(opt.token_slots, 0)) * TF * 4;
        SHV_HIP_CHECK(hipDeviceSynchronize());
        worker = std::thread([this] { run(); });
    }

    void stop() {
        {
            std::lock_guard<std::mutex> lk(mu);
            stopping = true;
        }
        cv.notify_all();
        if (worker.joinable()) worker.join();
    }

    // ---------------------------------------------------------------- completion
    static void complete(shv_hip_job* j, bool ok, const std::string& err, float gpu_ms, int bf, int bw) {
        if (!ok) {
            for (size_t i = 0; i < j->n_windows; ++i) j->logits_out[i] = kNaN;
            if (j->tokens_out) std::fill(j->tokens_out, j->tokens_out + j->n_frames * TF, kNaN);
        }
        shv_hip_callback cb;
        void* user;
        {
            std::lock_guard<std::mutex> lk(j->m);
            j->state = ok ? 1 : -1;
            j->error = ok ? std::string() : err;
            j->t_done = Clock::now();
            j->gpu_ms = gpu_ms;
            j->batch_frames = bf;
            j->batch_windows = bw;
            cb = j->cb;
            user = j->user;
            j->cv.notify_all();  // under j->m: job_free deletes the job once `released` is seen under j->m
        }
        if (cb) cb(j, ok ? 1 : -1, user);
        {
            std::lock_guard<std::mutex> lk(j->m);
            j->released = true;
            j->cv.notify_all();  // last access to *j by the worker
        }
    }

    // ---------------------------------------------------------------- batching (caller holds mu)
    void take(std::vector<shv_hip_job*>& out) {
        int F = 0, B = 0, Hn = 0;
        std::unordered_set<int32_t> read, stored;
        while (!q.empty()) {
            shv_hip_job* j = q.front();
            if (!out.empty()) {
                if (F + int(j->n_frames) > opt.max_frames || B + int(j->n_windows) > opt.max_windows ||
                    Hn + j->host_tokens > opt.max_host_tokens)
                    break;
                bool hazard = false;
                for (int32_t s : j->store_slots)
                    if (s >= 0 && (read.count(s) || stored.count(s))) { hazard = true; break; }
                if (hazard) break;
            }
            q.pop_front();
            out.push_back(j);
            F += int(j->n_frames);
            B += int(j->n_windows);
            Hn += j->host_tokens;
            for (int32_t s : j->store_slots)
                if (s >= 0) stored.insert(s);
            for (size_t e = 0; e < j->wslots.size(); ++e)
                if ((j->wframes.empty() || j->wframes[e] < 0) && j->wslots[e] >= 0) read.insert(j->wslots[e]);
        }
    }

    Batch launch(int slot, const std::vector<shv_hip_job*>& jobs) {
        Batch b;
        b.slot = slot;
        b.jobs = jobs;
        b.t_start = Clock::now();
        HostSlot& h = hs[size_t(slot)];
        const shv::Engine::Slot& d = eng->slot(slot);
        try {
            if (const char* f = std::getenv("SHV_HIP_TEST_FAIL_BATCH"))
                if (*f && std::strcmp(f, "0") != 0) throw std::runtime_error("injected batch failure (SHV_HIP_TEST_FAIL_BATCH)");
            int F = 0, B = 0, Hn = 0;
            bool any_store = false;
            int run0 = -1, run1 = -1;  // staged frames [run0, run1) not yet copied
            auto flush = [&] {
                if (run0 >= 0 && run1 > run0)
                    SHV_HIP_CHECK(hipMemcpyAsync(d.d_frames + size_t(run0) * FB, h.frames + size_t(run0) * FB,
                                                 size_t(run1 - run0) * FB, hipMemcpyHostToDevice, s_copy));
                run0 = run1 = -1;
            };
            for (shv_hip_job* j : jobs) {
                j->t_start = b.t_start;
                j->frame_off = F;
                j->window_off = B;
                if (j->n_frames) {
                    if (j->frames_pinned) {
                        flush();
                        SHV_HIP_CHECK(hipMemcpyAsync(d.d_frames + size_t(F) * FB, j->frames, j->n_frames * FB,
                                                     hipMemcpyHostToDevice, s_copy));
                    } else {
                        std::memcpy(h.frames + size_t(F) * FB, j->frames, j->n_frames * FB);
                        if (run0 < 0) run0 = F;
                        run1 = F + int(j->n_frames);
                    }
                    for (size_t f = 0; f < j->n_frames; ++f) {
                        const int32_t s = j->store_slots.empty() ? -1 : j->store_slots[f];
                        h.store[F + int(f)] = s;
                        any_store |= s >= 0;
                    }
                }
                F += int(j->n_frames);
                B += int(j->n_windows);
            }
            flush();
            for (shv_hip_job* j : jobs) {
                for (size_t e = 0; e < j->n_windows * 20; ++e) {
                    const int32_t wf = j->wframes.empty() ? -1 : j->wframes[e];
                    const int32_t ws = j->wslots.empty() ? -1 : j->wslots[e];
                    const float* p;
                    if (wf >= 0) p = d.d_tokens + size_t(j->frame_off + wf) * TF;
                    else if (ws >= 0) p = d_pool + size_t(ws) * TF;
                    else {
                        std::memcpy(h.tok_stage + size_t(Hn) * TF, j->wtokens[e], TF * 4);
                        p = d.d_tok_stage + size_t(Hn) * TF;
                        ++Hn;
                    }
                    h.tokptr[size_t(j->window_off) * 20 + e] = p;
                }
            }
            if (B) SHV_HIP_CHECK(hipMemcpyAsync(d.d_tokptr, h.tokptr, size_t(B) * 20 * sizeof(float*), hipMemcpyHostToDevice, s_copy));
            if (Hn) SHV_HIP_CHECK(hipMemcpyAsync(d.d_tok_stage, h.tok_stage, size_t(Hn) * TF * 4, hipMemcpyHostToDevice, s_copy));
            if (any_store) SHV_HIP_CHECK(hipMemcpyAsync(d.d_store, h.store, size_t(F) * 4, hipMemcpyHostToDevice, s_copy));
            SHV_HIP_CHECK(hipEventRecord(h.h2d, s_copy));
            SHV_HIP_CHECK(hipStreamWaitEvent(s_comp, h.h2d, 0));
            SHV_HIP_CHECK(hipEventRecord(h.start, s_comp));
            if (F) eng->encode_slot(slot, F, s_comp);
            if (any_store) {
                shv::launch_store_tokens(d.d_tokens, d.d_store, d_pool, F, s_comp);
                SHV_HIP_CHECK(hipGetLastError());
            }
            if (B) eng->classify_slot(slot, B, s_comp);
            if (B) SHV_HIP_CHECK(hipMemcpyAsync(h.logits, d.d_logits, size_t(B) * 4, hipMemcpyDeviceToHost, s_comp));
            for (shv_hip_job* j : jobs) {
                if (!j->tokens_out || !j->n_frames) continue;
                float* dst = j->tokens_out_pinned ? j->tokens_out : h.tokens_out + size_t(j->frame_off) * TF;
                SHV_HIP_CHECK(hipMemcpyAsync(dst, d.d_tokens + size_t(j->frame_off) * TF, j->n_frames * TF * 4,
                                             hipMemcpyDeviceToHost, s_comp));
            }
            SHV_HIP_CHECK(hipEventRecord(h.end, s_comp));
            b.F = F;
            b.B = B;
        } catch (const std::exception& e) {
            b.failed = true;
            b.error = e.what();
        }
        return b;
    }

    void finish(Batch& b) {
        HostSlot& h = hs[size_t(b.slot)];
        float gpu_ms = 0.0f;
        if (!b.failed) {
            const hipError_t e = hipEventSynchronize(h.end);
            if (e != hipSuccess) {
                b.failed = true;
                b.error = std::string("HIP error: ") + hipGetErrorString(e);
            } else if (hipEventElapsedTime(&gpu_ms, h.start, h.end) != hipSuccess) {
                (void)hipGetLastError();
                gpu_ms = 0.0f;
            }
        } else {
            (void)hipStreamSynchronize(s_comp);
            (void)hipStreamSynchronize(s_copy);
        }
        for (shv_hip_job* j : b.jobs) {
            if (!b.failed) {
                for (size_t i = 0; i < j->n_windows; ++i) {
                    const float v = h.logits[size_t(j->window_off) + i];
                    j->logits_out[i] = std::isfinite(v) ? v : kNaN;  // non-finite = unavailable
                }
                if (j->tokens_out && !j->tokens_out_pinned && j->n_frames)
                    std::memcpy(j->tokens_out, h.tokens_out + size_t(j->frame_off) * TF, j->n_frames * TF * 4);
            }
            complete(j, !b.failed, b.error, gpu_ms, b.F, b.B);
        }
    }

    void run() {
        if (hipSetDevice(device) != hipSuccess) (void)hipGetLastError();
        std::deque<Batch> inflight;
        int next_slot = 0;
        const int nslots = int(hs.size());
        for (;;) {
            std::vector<shv_hip_job*> jobs;
            {
                std::unique_lock<std::mutex> lk(mu);
                if (inflight.empty()) cv.wait(lk, [&] { return stopping || !q.empty(); });
                if (q.empty() && inflight.empty() && stopping) break;
                if (!q.empty() && int(inflight.size()) < nslots) {
                    if (opt.max_delay_us > 0 && inflight.empty()) {
                        const auto deadline = Clock::now() + std::chrono::microseconds(opt.max_delay_us);
                        cv.wait_until(lk, deadline, [&] {
                            if (stopping) return true;
                            size_t F = 0, B = 0;
                            for (auto* j : q) { F += j->n_frames; B += j->n_windows; }
                            return F >= size_t(opt.max_frames) || B >= size_t(opt.max_windows);
                        });
                    }
                    take(jobs);
                }
            }
            if (!jobs.empty()) {
                inflight.push_back(launch(next_slot, jobs));
                next_slot = (next_slot + 1) % nslots;
                if (int(inflight.size()) < nslots) {
                    std::lock_guard<std::mutex> lk(mu);
                    if (!q.empty()) continue;  // queue a second batch before waiting on the first
                }
            }
            if (!inflight.empty()) {
                finish(inflight.front());
                inflight.pop_front();
            }
        }
    }
};

// "<weights>.hip.cert": first line SHIELDV_HIP_CERT_V2, then per passing mode
//   "<weights sha256> <mode> <revision> PASS <cert json> <cert json sha256> threshold=<%.17g>"
// The certified threshold must equal the loaded one exactly (engine/cuda/api.cu:423-461 states the rule).
std::string check_certificate(const std::string& weights, const std::string& sha, const std::string& mode, double thr) {
    const std::string path = weights + ".hip.cert";
    std::ifstream in(path);
    if (!in) return "mode " + mode + " needs a quality certificate: " + path + " not found";
    std::string line;
    if (!std::getline(in, line)) return "empty certificate file " + path;
    while (!line.empty() && (line.back() == '\r' || line.back() == ' ')) line.pop_back();
    if (line != "SHIELDV_HIP_CERT_V2") return "invalid certificate file " + path + " (expected SHIELDV_HIP_CERT_V2)";
    bool thr_mismatch = false;
    double cert_thr = std::nan("");
    while (std::getline(in, line)) {
        std::istringstream ls(line);
        std::string h, m, rev, verdict, tok;
        if (!(ls >> h >> m >> rev >> verdict)) continue;
        if (!(h == sha && m == mode && rev == SHV_HIP_REVISION && verdict == "PASS")) continue;
        double t = std::nan("");
        while (ls >> tok)
            if (tok.rfind("threshold=", 0) == 0) {
                const char* b = tok.c_str() + 10;
                char* e = nullptr;
                const double v = std::strtod(b, &e);
                if (e != b && *e == 0) t = v;
            }
        if (std::isfinite(t) && t == thr) return "";
        thr_mismatch = true;
        cert_thr = t;
    }
    if (thr_mismatch) {
        char b[160];
        std::snprintf(b, sizeof b, "certified threshold %.17g, loaded threshold %.17g", cert_thr, thr);
        return "mode " + mode + " certificate in " + path + " does not cover the threshold in " + weights + ".json (" +
               b + ")";
    }
    return "mode " + mode + " has no passing certificate for weights " + sha + " at compute revision " +
           SHV_HIP_REVISION + " in " + path;
}

template <class F> int guarded(F&& f) {
    try {
        return f();
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

}  // namespace

struct shv_hip_model {
    std::unique_ptr<Core> core;
};
struct shv_hip_gemm {
    std::unique_ptr<shv::PwGemm> g;
};

extern "C" {

void shv_hip_default_options(shv_hip_options* o) {
    if (!o) return;
    o->max_frames = 640;
    o->max_windows = 512;
    o->max_host_tokens = 2048;
    o->token_slots = 0;
    o->use_graphs = 1;
    o->max_delay_us = 0;
}

shv_hip_model* shv_hip_load_ex(const char* weights, const char* mode, int device, const shv_hip_options* opt) {
    try {
        if (!weights) throw std::runtime_error("null weights path");
        std::unique_ptr<Core> core(new Core());
        core->mode = mode ? mode : "fp32";
        shv::Precision p;
        if (!shv::parse_precision(core->mode, &p))
            throw std::runtime_error("unknown mode '" + core->mode + "' (fp32, bf16, fp16)");
        shv_hip_default_options(&core->opt);
        if (opt) core->opt = *opt;
        const shv_hip_options& o = core->opt;
        if (o.max_frames < 1 || o.max_frames > 4096 || o.max_windows < 1 || o.max_windows > 4096 ||
            o.max_host_tokens < 0 || o.max_host_tokens > (1 << 20) || o.token_slots < 0 || o.max_delay_us < 0)
            throw std::runtime_error("invalid options");
        core->device = device;
        const shv::HostModel hm = shv::load_host_model(weights);
        core->fingerprint = hm.sha256;
        core->threshold = hm.threshold;
#ifndef SHV_HIP_EXPERIMENTAL
        if (p != shv::Precision::FP32) {
            const std::string err = check_certificate(weights, core->fingerprint, core->mode, core->threshold);
            if (!err.empty()) throw std::runtime_error(err);
        }
#endif
        core->init(hm, p);
        shv_hip_model* m = new shv_hip_model();
        m->core = std::move(core);
        g_err.clear();
        return m;
    } catch (const std::exception& e) {
        g_err = e.what();
        return nullptr;
    }
}

shv_hip_model* shv_hip_load(const char* weights, const char* mode, int device) {
    return shv_hip_load_ex(weights, mode, device, nullptr);
}

void shv_hip_free(shv_hip_model* m) {
    if (!m) return;
    m->core->stop();
    delete m;
}

const char* shv_hip_last_error(void) { return g_err.c_str(); }
const char* shv_hip_mode(const shv_hip_model* m) { return m ? m->core->mode.c_str() : ""; }
const char* shv_hip_fingerprint(const shv_hip_model* m) { return m ? m->core->fingerprint.c_str() : ""; }
double shv_hip_threshold(const shv_hip_model* m) { return m ? m->core->threshold : std::nan(""); }
const char* shv_hip_compute_revision(void) { return SHV_HIP_REVISION; }
int shv_hip_limits(const shv_hip_model* m, int* mf, int* mw, int* mh, int* ts) {
    if (!m) { g_err = "null model"; return -1; }
    if (mf) *mf = m->core->opt.max_frames;
    if (mw) *mw = m->core->opt.max_windows;
    if (mh) *mh = m->core->opt.max_host_tokens;
    if (ts) *ts = m->core->opt.token_slots;
    return 0;
}
size_t shv_hip_weight_bytes(const shv_hip_model* m) { return m ? m->core->eng->weight_bytes() : 0; }
size_t shv_hip_device_bytes(const shv_hip_model* m) { return m ? m->core->device_bytes : 0; }

shv_hip_job* shv_hip_submit(shv_hip_model* m, const shv_hip_request* r) {
    try {
        if (!m || !r) throw std::runtime_error("null argument");
        Core& c = *m->core;
        const shv_hip_options& o = c.opt;
        if (r->n_frames > size_t(o.max_frames)) throw std::runtime_error("request has more frames than max_frames");
        if (r->n_windows > size_t(o.max_windows)) throw std::runtime_error("request has more windows than max_windows");
        if (r->n_frames && !r->frames) throw std::runtime_error("null frames");
        if (r->n_windows && !r->logits_out) throw std::runtime_error("null logits_out");
        if (!r->n_frames && !r->n_windows) throw std::runtime_error("empty request");
        std::unique_ptr<shv_hip_job> j(new shv_hip_job());
        j->frames = r->frames;
        j->n_frames = r->n_frames;
        j->tokens_out = r->tokens_out;
        j->n_windows = r->n_windows;
        j->logits_out = r->logits_out;
        j->cb = r->callback;
        j->user = r->user;
        if (r->store_slots && r->n_frames) {
            if (!c.d_pool) throw std::runtime_error("store_slots needs options.token_slots > 0");
            j->store_slots.assign(r->store_slots, r->store_slots + r->n_frames);
            std::unordered_set<int32_t> seen;
            for (int32_t s : j->store_slots) {
                if (s < -1 || s >= o.token_slots) throw std::runtime_error("store slot out of range");
                if (s >= 0 && !seen.insert(s).second) throw std::runtime_error("duplicate store slot in one request");
            }
        }
        const size_t E = r->n_windows * 20;
        if (E) {
            if (r->window_frames) j->wframes.assign(r->window_frames, r->window_frames + E);
            if (r->window_slots) j->wslots.assign(r->window_slots, r->window_slots + E);
            if (r->window_tokens) j->wtokens.assign(r->window_tokens, r->window_tokens + E);
            for (size_t e = 0; e < E; ++e) {
                const int32_t wf = j->wframes.empty() ? -1 : j->wframes[e];
                const int32_t ws = j->wslots.empty() ? -1 : j->wslots[e];
                if (wf >= 0) {
                    if (size_t(wf) >= r->n_frames) throw std::runtime_error("window frame index out of range");
                } else if (ws >= 0) {
                    if (!c.d_pool || ws >= o.token_slots) throw std::runtime_error("window slot out of range");
                } else {
                    if (j->wtokens.empty() || !j->wtokens[e]) throw std::runtime_error("window entry has no token source");
                    ++j->host_tokens;
                }
            }
            if (j->host_tokens > o.max_host_tokens)
                throw std::runtime_error("request has more host token blocks than max_host_tokens");
        }
        j->frames_pinned = is_pinned(r->frames, r->n_frames * FB);
        j->tokens_out_pinned = r->tokens_out && is_pinned(r->tokens_out, r->n_frames * TF * 4);
        j->t_submit = Clock::now();
        shv_hip_job* raw = j.release();
        {
            std::lock_guard<std::mutex> lk(c.mu);
            if (c.stopping) {
                delete raw;
                throw std::runtime_error("model is stopping");
            }
            c.q.push_back(raw);
        }
        c.cv.notify_all();
        g_err.clear();
        return raw;
    } catch (const std::exception& e) {
        g_err = e.what();
        return nullptr;
    }
}

int shv_hip_job_status(const shv_hip_job* j) {
    if (!j) return -1;
    std::lock_guard<std::mutex> lk(j->m);
    return j->state;
}
int shv_hip_job_wait(shv_hip_job* j) {
    if (!j) { g_err = "null job"; return -1; }
    std::unique_lock<std::mutex> lk(j->m);
    j->cv.wait(lk, [&] { return j->state != 0; });
    if (j->state < 0) { g_err = j->error; return -1; }
    return 0;
}
const char* shv_hip_job_error(const shv_hip_job* j) {
    if (!j) return "null job";
    std::lock_guard<std::mutex> lk(j->m);
    return j->error.c_str();
}
int shv_hip_job_timing(const shv_hip_job* j, double* queue_ms, double* run_ms, double* gpu_ms, int* bf, int* bw) {
    if (!j) return -1;
    std::lock_guard<std::mutex> lk(j->m);
    if (j->state == 0) return 1;
    auto ms = [](Clock::duration d) { return std::chrono::duration<double, std::milli>(d).count(); };
    if (queue_ms) *queue_ms = ms(j->t_start - j->t_submit);
    if (run_ms) *run_ms = ms(j->t_done - j->t_start);
    if (gpu_ms) *gpu_ms = j->gpu_ms;
    if (bf) *bf = j->batch_frames;
    if (bw) *bw = j->batch_windows;
    return 0;
}
void shv_hip_job_free(shv_hip_job* j) {
    if (!j) return;
    {
        std::unique_lock<std::mutex> lk(j->m);
        j->cv.wait(lk, [&] { return j->released; });
    }
    delete j;
}

void* shv_hip_host_alloc(size_t bytes) {
    void* p = nullptr;
    if (hipHostMalloc(&p, bytes, hipHostMallocPortable) != hipSuccess) {
        (void)hipGetLastError();
        g_err = "hipHostMalloc failed";
        return nullptr;
    }
    return p;
}
void shv_hip_host_free(void* p) {
    if (p) (void)hipHostFree(p);
}

// ---------------------------------------------------------------- synchronous wrappers (api.cu:664-729 semantics)
static int wait_all(std::vector<shv_hip_job*>& jobs) {
    int rc = 0;
    std::string err;
    for (auto* j : jobs) {
        if (shv_hip_job_wait(j) != 0) {
            rc = -1;
            if (err.empty()) err = shv_hip_job_error(j);
        }
        shv_hip_job_free(j);
    }
    if (rc) g_err = err;
    return rc;
}

int shv_hip_encode_frames(shv_hip_model* m, const uint8_t* rgb, size_t n, float* tokens) {
    return guarded([&] {
        if (!m || (n && (!rgb || !tokens))) throw std::runtime_error("null argument");
        const size_t step = size_t(m->core->opt.max_frames);
        std::vector<shv_hip_job*> jobs;
        for (size_t off = 0; off < n; off += step) {
            shv_hip_request r{};
            r.frames = rgb + off * FB;
            r.n_frames = std::min(step, n - off);
            r.tokens_out = tokens + off * TF;
            shv_hip_job* j = shv_hip_submit(m, &r);
            if (!j) {
                const std::string e = g_err;
                wait_all(jobs);
                std::fill(tokens, tokens + n * TF, kNaN);
                throw std::runtime_error(e);
            }
            jobs.push_back(j);
        }
        return wait_all(jobs);
    });
}

int shv_hip_classify(shv_hip_model* m, const float* tokens, size_t b, float* logits) {
    return guarded([&] {
        if (!m || (b && (!tokens || !logits))) throw std::runtime_error("null argument");
        const shv_hip_options& o = m->core->opt;
        if (b && o.max_host_tokens < 20) throw std::runtime_error("classify needs max_host_tokens >= 20");
        const size_t step = size_t(std::max(1, std::min(o.max_windows, o.max_host_tokens / 20)));
        std::vector<shv_hip_job*> jobs;
        std::vector<std::vector<const float*>> ptrs;
        for (size_t off = 0; off < b; off += step) {
            const size_t w = std::min(step, b - off);
            ptrs.emplace_back(w * 20);
            for (size_t e = 0; e < w * 20; ++e) ptrs.back()[e] = tokens + (off * 20 + e) * TF;
            shv_hip_request r{};
            r.n_windows = w;
            r.window_tokens = ptrs.back().data();
            r.logits_out = logits + off;
            shv_hip_job* j = shv_hip_submit(m, &r);
            if (!j) {
                const std::string e = g_err;
                wait_all(jobs);
                std::fill(logits, logits + b, kNaN);
                throw std::runtime_error(e);
            }
            jobs.push_back(j);
        }
        return wait_all(jobs);
    });
}

int shv_hip_predict(shv_hip_model* m, const uint8_t* clips, size_t b, float* logits) {
    return guarded([&] {
        if (!m || (b && (!clips || !logits))) throw std::runtime_error("null argument");
        const shv_hip_options& o = m->core->opt;
        const size_t step = size_t(std::min(o.max_windows, o.max_frames / 20));
        if (b && step < 1) throw std::runtime_error("predict needs max_frames >= 20");
        std::vector<int32_t> idx(std::max<size_t>(step, 1) * 20);
        for (size_t e = 0; e < idx.size(); ++e) idx[e] = int32_t(e);
        std::vector<shv_hip_job*> jobs;
        for (size_t off = 0; off < b; off += step) {
            const size_t w = std::min(step, b - off);
            shv_hip_request r{};
            r.frames = clips + off * 20 * FB;
            r.n_frames = w * 20;
            r.n_windows = w;
            r.window_frames = idx.data();
            r.logits_out = logits + off;
            shv_hip_job* j = shv_hip_submit(m, &r);
            if (!j) {
                const std::string e = g_err;
                wait_all(jobs);
                std::fill(logits, logits + b, kNaN);
                throw std::runtime_error(e);
            }
            jobs.push_back(j);
        }
        return wait_all(jobs);
    });
}

// ---------------------------------------------------------------- engine-level entry points
int shv_hip_forward_device(shv_hip_model* m, const uint8_t* d_frames, int n_clips, float* d_logits, void* stream) {
    return guarded([&] {
        if (!m || !d_frames || !d_logits || n_clips < 1) throw std::runtime_error("invalid argument");
        hipStream_t s = stream ? static_cast<hipStream_t>(stream) : m->core->s_comp;
        m->core->eng->forward_direct(d_frames, n_clips, d_logits, s);
        return 0;
    });
}
int shv_hip_encode_device(shv_hip_model* m, const uint8_t* d_frames, int n_frames, float* d_tokens, void* stream) {
    return guarded([&] {
        if (!m || !d_frames || !d_tokens || n_frames < 1) throw std::runtime_error("invalid argument");
        hipStream_t s = stream ? static_cast<hipStream_t>(stream) : m->core->s_comp;
        m->core->eng->encode_direct(d_frames, n_frames, d_tokens, s);
        return 0;
    });
}
int shv_hip_profile_enable(shv_hip_model* m, int on) {
    return guarded([&] {
        if (!m) throw std::runtime_error("null model");
        m->core->eng->profile_enable(on != 0);
        return 0;
    });
}
int shv_hip_profile_read(shv_hip_model* m, const char* name, double* total_ms, long long* launches, double* bytes) {
    return guarded([&] {
        if (!m || !name) throw std::runtime_error("null argument");
        shv::ProfStat st;
        if (!m->core->eng->profile_read(name, &st)) return -1;
        if (total_ms) *total_ms = st.ms;
        if (launches) *launches = st.launches;
        if (bytes) *bytes = st.bytes;
        return 0;
    });
}
int shv_hip_set_dump_dir(shv_hip_model* m, const char* dir) {
    return guarded([&] {
        if (!m) throw std::runtime_error("null model");
        m->core->eng->set_dump_dir(dir ? dir : "");
        return 0;
    });
}


// Pointwise-conv GEMM microbench (bench/gpu_gemm_bench.cu).  The reference's activation codes (common.cuh:69):
// 0 none, 1 ReLU, 2 hardswish, 3 SiLU, 4 hardsigmoid.
shv_hip_gemm* shv_hip_gemm_create(const char* mode, int n, int k, const float* d_w, void* stream) {
    try {
        shv::Precision p;
        if (!mode || !shv::parse_precision(mode, &p)) throw std::runtime_error("unknown mode (fp32, bf16, fp16)");
        if (n < 1 || k < 1 || !d_w) throw std::runtime_error("invalid argument");
        if (p != shv::Precision::FP32 && k % 8) throw std::runtime_error("the matrix-core tiers need K % 8 == 0");
        std::unique_ptr<shv_hip_gemm> g(new shv_hip_gemm());
        g->g.reset(new shv::PwGemm(p, n, k, d_w, static_cast<hipStream_t>(stream)));
        return g.release();
    } catch (const std::exception& e) {
        g_err = e.what();
        return nullptr;
    }
}
int shv_hip_gemm_run(shv_hip_gemm* g, const float* d_a, long long m, const float* d_bias, int act, float* d_c,
                     int variant, void* stream) {
    return guarded([&] {
        if (!g || !d_a || !d_c || m < 1) throw std::runtime_error("invalid argument");
        g->g->run(d_a, m, d_bias, act, d_c, variant, static_cast<hipStream_t>(stream));
        return 0;
    });
}
void shv_hip_gemm_free(shv_hip_gemm* g) { delete g; }

// Face crops on the GPU (shv_prep.h:181-186 on device frames).
int shv_hip_native_crops_rgb(const shv_hip_rgb_image* frames, const shv_hip_rect* rects, int n, uint8_t* d_out,
                             void* stream) {
    return guarded([&] {
        if (n < 0 || (n > 0 && (!frames || !rects || !d_out))) throw std::runtime_error("invalid argument");
        std::vector<shv::CropJob> jobs(static_cast<size_t>(n));
        for (int i = 0; i < n; ++i) {
            const shv_hip_rgb_image& f = frames[i];
            const shv_hip_rect& r = rects[i];
            jobs[size_t(i)] = shv::CropJob{f.data, f.width, f.height, (long long)f.stride, r.x, r.y, r.w, r.h};
        }
        shv::native_crops(jobs.data(), n, d_out, false, static_cast<hipStream_t>(stream));
        return 0;
    });
}
int shv_hip_native_crops_i420(const shv_hip_i420_image* frames, const shv_hip_rect* rects, int n, uint8_t* d_out,
                              void* stream) {
    return guarded([&] {
        if (n < 0 || (n > 0 && (!frames || !rects || !d_out))) throw std::runtime_error("invalid argument");
        std::vector<shv::CropJob> jobs(static_cast<size_t>(n));
        for (int i = 0; i < n; ++i) {
            const shv_hip_i420_image& f = frames[i];
            const shv_hip_rect& r = rects[i];
            jobs[size_t(i)] = shv::CropJob{f.y, f.width, f.height, (long long)f.y_stride, r.x, r.y, r.w, r.h,
                                           f.u, f.v, (long long)f.u_stride, (long long)f.v_stride};
        }
        shv::native_crops(jobs.data(), n, d_out, true, static_cast<hipStream_t>(stream));
        return 0;
    });
}

// Gated delta rule microbench / parity entry (config 3's scan on its own).
int shv_hip_delta_rule(const char* mode, const float* d_q, const float* d_k, const float* d_v, const float* d_decay,
                       const float* d_beta, int n_windows, float* d_o, int variant, void* stream) {
    return guarded([&] {
        shv::Precision p;
        if (!mode || !shv::parse_precision(mode, &p)) throw std::runtime_error("unknown mode (fp32, bf16, fp16)");
        shv::run_delta_rule(p, d_q, d_k, d_v, d_decay, d_beta, n_windows, d_o, variant,
                            static_cast<hipStream_t>(stream));
        return 0;
    });
}

}  // extern "C"
