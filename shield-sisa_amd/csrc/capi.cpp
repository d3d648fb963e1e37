// The C ABI of libshield_v_hip.so (include/shv_hip.h).  Model = HipLanes (engine + lanes on one device) under a
// sched::Frontend (queue, planner, launcher and completer threads).  Every entry point turns exceptions into
// -1 / NULL plus the thread-local error string.
#include "../../include/shv_hip.h"

#include "audio.hpp"
#include "cert.hpp"
#include "kernels.hpp"
#include "lanes.hpp"
#include "sched.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <limits>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#ifndef SHV_HIP_REVISION
#define SHV_HIP_REVISION "hip-unversioned"
#endif

struct shv_hip_model {
    std::string mode, fingerprint;
    double threshold = 0.0;
    shv_hip_options opt{};
    std::unique_ptr<shv::HipLanes> lanes;          // destroyed after the frontend has drained
    std::unique_ptr<shv::sched::Frontend> front;
    ~shv_hip_model() {
        front.reset();
        lanes.reset();
    }
};

struct shv_hip_gemm {
    std::unique_ptr<shv::PwGemm> g;
};

struct shv_hip_audio {
    std::string mode, fingerprint;
    int device = 0;
    std::mutex mu;                              // one call at a time drives the engine
    std::unique_ptr<shv::AudioEngine> eng;
};

namespace {
using shv::sched::Frontend;

template <class F> int guarded(F&& f) {
    try {
        return f();
    } catch (const std::exception& e) {
        shv::sched::set_error(e.what());
        return -1;
    }
}

shv::Precision mode_or_throw(const char* mode) {
    shv::Precision p;
    if (!mode || !shv::parse_precision(mode, &p)) throw std::runtime_error("unknown mode (fp32, bf16, fp16)");
    return p;
}

bool options_valid(const shv_hip_options& o) {
    return o.max_frames >= 1 && o.max_frames <= 4096 && o.max_windows >= 1 && o.max_windows <= 4096 &&
           o.max_host_tokens >= 0 && o.max_host_tokens <= (1 << 20) && o.token_slots >= 0 &&
           o.token_slots <= (1 << 22) && o.max_delay_us >= 0;
}

// Makes `dev` current for a scope, restoring the caller's device after.
class DeviceScope {
public:
    explicit DeviceScope(int dev) {
        SHV_HIP_CHECK(hipGetDevice(&prev_));
        if (dev != prev_) SHV_HIP_CHECK(hipSetDevice(dev));
        switched_ = dev != prev_;
    }
    ~DeviceScope() {
        if (switched_) (void)hipSetDevice(prev_);
    }

private:
    int prev_ = 0;
    bool switched_ = false;
};

hipStream_t stream_or(shv_hip_model* m, void* s) {
    return s ? static_cast<hipStream_t>(s) : m->lanes->compute_stream();
}
}  // namespace

extern "C" {

void shv_hip_default_options(shv_hip_options* o) {
    if (o) *o = shv_hip_options{640, 512, 2048, 0, 1, 0};
}

shv_hip_model* shv_hip_load_ex(const char* weights, const char* mode, int device, const shv_hip_options* opt) {
    try {
        if (!weights) throw std::runtime_error("null weights path");
        std::unique_ptr<shv_hip_model> m(new shv_hip_model());
        m->mode = mode ? mode : "fp32";
        shv::Precision p;
        if (!shv::parse_precision(m->mode, &p)) throw std::runtime_error("unknown mode '" + m->mode + "' (fp32, bf16, fp16)");
        shv_hip_default_options(&m->opt);
        if (opt) m->opt = *opt;
        if (!options_valid(m->opt)) throw std::runtime_error("invalid options");
        const shv::HostModel hm = shv::load_host_model(weights);
        m->fingerprint = hm.sha256;
        m->threshold = hm.threshold;
#ifndef SHV_HIP_EXPERIMENTAL
        if (p != shv::Precision::FP32) {
            const std::string why = shv::certificate_problem(weights, hm.sha256, m->mode, hm.threshold, SHV_HIP_REVISION);
            if (!why.empty()) throw std::runtime_error(why);
        }
#endif
        shv::EngineConfig ec;
        ec.max_frames = m->opt.max_frames;
        ec.max_windows = m->opt.max_windows;
        ec.max_host_tokens = m->opt.max_host_tokens;
        ec.use_graphs = m->opt.use_graphs != 0;
        ec.slots = 2;
        m->lanes.reset(new shv::HipLanes(hm, p, ec, m->opt.token_slots, device));
        shv::sched::Limits lim;
        lim.frames = m->opt.max_frames;
        lim.windows = m->opt.max_windows;
        lim.host_blocks = m->opt.max_host_tokens;
        lim.token_slots = m->opt.token_slots;
        lim.delay_us = m->opt.max_delay_us;
        m->front.reset(new Frontend(*m->lanes, lim));
        shv::sched::clear_error();
        return m.release();
    } catch (const std::exception& e) {
        shv::sched::set_error(e.what());
        return nullptr;
    }
}

shv_hip_model* shv_hip_load(const char* weights, const char* mode, int device) {
    return shv_hip_load_ex(weights, mode, device, nullptr);
}

void shv_hip_free(shv_hip_model* m) { delete m; }

const char* shv_hip_last_error(void) { return shv::sched::last_error(); }
const char* shv_hip_mode(const shv_hip_model* m) { return m ? m->mode.c_str() : ""; }
const char* shv_hip_fingerprint(const shv_hip_model* m) { return m ? m->fingerprint.c_str() : ""; }
double shv_hip_threshold(const shv_hip_model* m) { return m ? m->threshold : std::nan(""); }
const char* shv_hip_compute_revision(void) { return SHV_HIP_REVISION; }

int shv_hip_limits(const shv_hip_model* m, int* max_frames, int* max_windows, int* max_host_tokens, int* token_slots) {
    if (!m) {
        shv::sched::set_error("null model");
        return -1;
    }
    if (max_frames) *max_frames = m->opt.max_frames;
    if (max_windows) *max_windows = m->opt.max_windows;
    if (max_host_tokens) *max_host_tokens = m->opt.max_host_tokens;
    if (token_slots) *token_slots = m->opt.token_slots;
    return 0;
}
size_t shv_hip_weight_bytes(const shv_hip_model* m) { return m ? m->lanes->engine().weight_bytes() : 0; }
size_t shv_hip_device_bytes(const shv_hip_model* m) { return m ? m->lanes->device_bytes() : 0; }

int shv_hip_encode_frames(shv_hip_model* m, const uint8_t* rgb, size_t n, float* tokens) {
    if (!m) { shv::sched::set_error("null argument"); return -1; }
    return m->front->encode_frames(rgb, n, tokens);
}
int shv_hip_classify(shv_hip_model* m, const float* tokens, size_t b, float* logits) {
    if (!m) { shv::sched::set_error("null argument"); return -1; }
    return m->front->classify(tokens, b, logits);
}
int shv_hip_predict(shv_hip_model* m, const uint8_t* clips, size_t b, float* logits) {
    if (!m) { shv::sched::set_error("null argument"); return -1; }
    return m->front->predict(clips, b, logits);
}

shv_hip_job* shv_hip_submit(shv_hip_model* m, const shv_hip_request* r) {
    if (!m) {
        shv::sched::set_error("null argument");
        return nullptr;
    }
    return m->front->submit(r);
}
int shv_hip_job_status(const shv_hip_job* j) { return Frontend::job_status(j); }
int shv_hip_job_wait(shv_hip_job* j) { return Frontend::job_wait(j); }
const char* shv_hip_job_error(const shv_hip_job* j) { return Frontend::job_error(j); }
int shv_hip_job_timing(const shv_hip_job* j, double* queue_ms, double* run_ms, double* gpu_ms, int* batch_frames,
                       int* batch_windows) {
    return Frontend::job_timing(j, queue_ms, run_ms, gpu_ms, batch_frames, batch_windows);
}
void shv_hip_job_free(shv_hip_job* j) { Frontend::job_free(j); }

void* shv_hip_host_alloc(size_t bytes) {
    void* p = nullptr;
    if (hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocPortable) != hipSuccess) {
        (void)hipGetLastError();
        shv::sched::set_error("hipHostMalloc failed");
        return nullptr;
    }
    return p;
}
void shv_hip_host_free(void* p) {
    if (p) (void)hipHostFree(p);
}

// ------------------------------------------------------------------------------------------ engine-level tools
int shv_hip_forward_device(shv_hip_model* m, const uint8_t* d_frames, int n_clips, float* d_logits, void* stream) {
    return guarded([&] {
        if (!m || !d_frames || !d_logits || n_clips < 1) throw std::runtime_error("invalid argument");
        m->lanes->engine().forward_direct(d_frames, n_clips, d_logits, stream_or(m, stream));
        return 0;
    });
}
int shv_hip_classify_device(shv_hip_model* m, const float* d_tokens, int n_windows, float* d_logits, void* stream) {
    return guarded([&] {
        if (!m || !d_tokens || !d_logits || n_windows < 1) throw std::runtime_error("invalid argument");
        m->lanes->engine().classify_direct(d_tokens, n_windows, d_logits, stream_or(m, stream));
        return 0;
    });
}
int shv_hip_encode_device(shv_hip_model* m, const uint8_t* d_frames, int n_frames, float* d_tokens, void* stream) {
    return guarded([&] {
        if (!m || !d_frames || !d_tokens || n_frames < 1) throw std::runtime_error("invalid argument");
        m->lanes->engine().encode_direct(d_frames, n_frames, d_tokens, stream_or(m, stream));
        return 0;
    });
}
int shv_hip_profile_enable(shv_hip_model* m, int on) {
    return guarded([&] {
        if (!m) throw std::runtime_error("null model");
        m->lanes->engine().profile_enable(on != 0);
        return 0;
    });
}
int shv_hip_profile_read(shv_hip_model* m, const char* name, double* total_ms, long long* launches, double* bytes,
                         double* flops) {
    return guarded([&] {
        if (!m || !name) throw std::runtime_error("null argument");
        shv::ProfStat st;
        if (!m->lanes->engine().profile_read(name, &st)) return -1;
        if (total_ms) *total_ms = st.ms;
        if (launches) *launches = st.launches;
        if (bytes) *bytes = st.bytes;
        if (flops) *flops = st.flops;
        return 0;
    });
}
long long shv_hip_profile_list(shv_hip_model* m, char* buf, size_t cap) {
    try {
        if (!m) throw std::runtime_error("null model");
        std::string all;
        for (const std::string& f : m->lanes->engine().profile_families()) all += f + "\n";
        if (buf && cap) {
            const size_t n = std::min(cap - 1, all.size());
            std::memcpy(buf, all.data(), n);
            buf[n] = '\0';
        }
        return (long long)all.size();
    } catch (const std::exception& e) {
        shv::sched::set_error(e.what());
        return -1;
    }
}
int shv_hip_set_dump_dir(shv_hip_model* m, const char* dir) {
    return guarded([&] {
        if (!m) throw std::runtime_error("null model");
        m->lanes->engine().set_dump_dir(dir ? dir : "");
        return 0;
    });
}

shv_hip_gemm* shv_hip_gemm_create(const char* mode, int n, int k, const float* d_w, void* stream) {
    try {
        const shv::Precision p = mode_or_throw(mode);
        if (n < 1 || k < 1 || !d_w) throw std::runtime_error("invalid argument");
        if (p != shv::Precision::FP32 && k % 8) throw std::runtime_error("the matrix-core tiers need K % 8 == 0");
        std::unique_ptr<shv_hip_gemm> g(new shv_hip_gemm());
        g->g.reset(new shv::PwGemm(p, n, k, d_w, static_cast<hipStream_t>(stream)));
        return g.release();
    } catch (const std::exception& e) {
        shv::sched::set_error(e.what());
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

int shv_hip_native_crops_rgb(const shv_hip_rgb_image* frames, const shv_hip_rect* rects, int n, uint8_t* d_out,
                             void* stream) {
    return guarded([&] {
        if (n < 0 || (n > 0 && (!frames || !rects || !d_out))) throw std::runtime_error("invalid argument");
        std::vector<shv::CropJob> jobs(static_cast<size_t>(n));
        for (int i = 0; i < n; ++i)
            jobs[size_t(i)] = shv::CropJob{frames[i].data, frames[i].width, frames[i].height,
                                           (long long)frames[i].stride, rects[i].x, rects[i].y, rects[i].w,
                                           rects[i].h};
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
            jobs[size_t(i)] = shv::CropJob{f.y, f.width, f.height, (long long)f.y_stride, rects[i].x, rects[i].y,
                                           rects[i].w, rects[i].h, f.u, f.v, (long long)f.u_stride,
                                           (long long)f.v_stride};
        }
        shv::native_crops(jobs.data(), n, d_out, true, static_cast<hipStream_t>(stream));
        return 0;
    });
}

int shv_hip_delta_rule(const char* mode, const float* d_q, const float* d_k, const float* d_v, const float* d_decay,
                       const float* d_beta, int n_windows, float* d_o, int variant, void* stream) {
    return guarded([&] {
        shv::run_delta_rule(mode_or_throw(mode), d_q, d_k, d_v, d_decay, d_beta, n_windows, d_o, variant,
                            static_cast<hipStream_t>(stream));
        return 0;
    });
}

int shv_hip_delta_rule_noalloc(const char* mode, const float* d_q, const float* d_k, const float* d_v,
                               const float* d_decay, const float* d_beta, int n_windows, float* d_o, int variant,
                               void* stream) {
    return guarded([&] {
        shv::run_delta_rule_noalloc(mode_or_throw(mode), d_q, d_k, d_v, d_decay, d_beta, n_windows, d_o, variant,
                                    static_cast<hipStream_t>(stream));
        return 0;
    });
}

// ------------------------------------------------------------------------------------------ SHIELD-A sequence
shv_hip_audio* shv_hip_audio_load(const char* weights, const char* mode, int device, int max_windows) {
    try {
        if (!weights) throw std::runtime_error("null weights path");
        if (max_windows < 1 || max_windows > 4096) throw std::runtime_error("max_windows must be in [1, 4096]");
        std::unique_ptr<shv_hip_audio> a(new shv_hip_audio());
        a->mode = mode ? mode : "fp32";
        shv::Precision p;
        if (!shv::parse_precision(a->mode, &p))
            throw std::runtime_error("unknown mode '" + a->mode + "' (fp32, bf16, fp16)");
#ifndef SHV_HIP_EXPERIMENTAL
        if (p != shv::Precision::FP32)
            throw std::runtime_error("audio mode " + a->mode + " is for offline evaluation (experimental library)");
#endif
        const shv::AudioHost ah = shv::load_audio_host(weights);
        a->fingerprint = ah.sha256;
        int count = 0;
        SHV_HIP_CHECK(hipGetDeviceCount(&count));
        if (device < 0 || device >= count) throw std::runtime_error("device out of range");
        a->device = device;
        DeviceScope ds(device);
        a->eng = shv::make_audio_engine(ah, p, max_windows, true);
        shv::sched::clear_error();
        return a.release();
    } catch (const std::exception& e) {
        shv::sched::set_error(e.what());
        return nullptr;
    }
}

void shv_hip_audio_free(shv_hip_audio* a) {
    if (!a) return;
    try {
        DeviceScope ds(a->device);
        a->eng.reset();
    } catch (const std::exception&) {
        a->eng.reset();
    }
    delete a;
}

const char* shv_hip_audio_mode(const shv_hip_audio* a) { return a ? a->mode.c_str() : nullptr; }
const char* shv_hip_audio_fingerprint(const shv_hip_audio* a) { return a ? a->fingerprint.c_str() : nullptr; }
size_t shv_hip_audio_device_bytes(const shv_hip_audio* a) { return a ? a->eng->device_bytes() : 0; }

int shv_hip_audio_sequence(shv_hip_audio* a, const float* tokens, size_t n, size_t stride, float* logits) {
    return guarded([&] {
        if (!a || !tokens || !logits) throw std::runtime_error("null argument");
        if (n == 0) throw std::runtime_error("empty request");
        if (stride < size_t(shv::kAudioWindowFloats)) throw std::runtime_error("window stride below 48000 floats");
        std::lock_guard<std::mutex> lk(a->mu);
        DeviceScope ds(a->device);
        a->eng->run_host(tokens, (long long)stride, (long long)n, logits);
        return 0;
    });
}

int shv_hip_audio_sequence_device(shv_hip_audio* a, const float* d_tokens, int n, size_t stride, float* d_logits,
                                  void* stream) {
    return guarded([&] {
        if (!a || !d_tokens || !d_logits) throw std::runtime_error("null argument");
        if (n < 1 || n > a->eng->max_windows()) throw std::runtime_error("window count out of range");
        if (stride < size_t(shv::kAudioWindowFloats)) throw std::runtime_error("window stride below 48000 floats");
        std::lock_guard<std::mutex> lk(a->mu);
        DeviceScope ds(a->device);
        a->eng->run_device(d_tokens, (long long)stride, n, d_logits, static_cast<hipStream_t>(stream));
        return 0;
    });
}

int shv_hip_audio_has_frontend(const shv_hip_audio* a) { return a && a->eng && a->eng->has_frontend() ? 1 : 0; }

int shv_hip_audio_predict(shv_hip_audio* a, const float* pcm, size_t n, size_t stride_samples, float* logits) {
    if (logits)
        for (size_t i = 0; i < n; ++i) logits[i] = std::numeric_limits<float>::quiet_NaN();
    return guarded([&] {
        if (!a || !pcm || !logits) throw std::runtime_error("null argument");
        if (n == 0 || n > 1000000) throw std::runtime_error("window count out of range");
        if (stride_samples < size_t(shv::kAudioWindowSamples)) throw std::runtime_error("window stride below 160000 samples");
        std::lock_guard<std::mutex> lk(a->mu);
        DeviceScope ds(a->device);
        a->eng->predict_host(pcm, (long long)stride_samples, (long long)n, logits);
        return 0;
    });
}

int shv_hip_audio_predict_device(shv_hip_audio* a, const float* d_pcm, int n, size_t stride_samples,
                                 float* d_logits, void* stream) {
    return guarded([&] {
        if (!a || !d_pcm || !d_logits) throw std::runtime_error("null argument");
        if (n < 1 || n > a->eng->max_windows()) throw std::runtime_error("window count out of range");
        if (stride_samples < size_t(shv::kAudioWindowSamples)) throw std::runtime_error("window stride below 160000 samples");
        std::lock_guard<std::mutex> lk(a->mu);
        DeviceScope ds(a->device);
        a->eng->predict_device(d_pcm, (long long)stride_samples, n, d_logits, static_cast<hipStream_t>(stream));
        return 0;
    });
}

int shv_hip_audio_frontend(shv_hip_audio* a, const float* pcm, size_t n, size_t stride_samples, float* tokens) {
    return guarded([&] {
        if (!a || !pcm || !tokens) throw std::runtime_error("null argument");
        if (n == 0 || n > 1000000) throw std::runtime_error("window count out of range");
        if (stride_samples < size_t(shv::kAudioWindowSamples)) throw std::runtime_error("window stride below 160000 samples");
        std::lock_guard<std::mutex> lk(a->mu);
        DeviceScope ds(a->device);
        a->eng->frontend_host(pcm, (long long)stride_samples, (long long)n, tokens);
        return 0;
    });
}

int shv_hip_audio_profile_enable(shv_hip_audio* a, int on) {
    return guarded([&] {
        if (!a) throw std::runtime_error("null handle");
        std::lock_guard<std::mutex> lk(a->mu);
        DeviceScope ds(a->device);
        a->eng->profile_enable(on != 0);
        return 0;
    });
}

int shv_hip_audio_profile_read(shv_hip_audio* a, const char* name, double* total_ms, long long* launches,
                               double* bytes, double* flops) {
    return guarded([&] {
        if (!a || !name) throw std::runtime_error("null argument");
        std::lock_guard<std::mutex> lk(a->mu);
        DeviceScope ds(a->device);
        shv::ProfStat st;
        if (!a->eng->profile_read(name, &st)) return -1;
        if (total_ms) *total_ms = st.ms;
        if (launches) *launches = st.launches;
        if (bytes) *bytes = st.bytes;
        if (flops) *flops = st.flops;
        return 0;
    });
}

long long shv_hip_audio_profile_list(shv_hip_audio* a, char* buf, size_t cap) {
    try {
        if (!a) throw std::runtime_error("null handle");
        std::string all;
        {
            std::lock_guard<std::mutex> lk(a->mu);
            for (const std::string& f : a->eng->profile_families()) all += f + "\n";
        }
        if (buf && cap) {
            const size_t n = std::min(cap - 1, all.size());
            std::memcpy(buf, all.data(), n);
            buf[n] = '\0';
        }
        return (long long)all.size();
    } catch (const std::exception& e) {
        shv::sched::set_error(e.what());
        return -1;
    }
}

int shv_hip_audio_set_dump_dir(shv_hip_audio* a, const char* dir) {
    return guarded([&] {
        if (!a) throw std::runtime_error("null handle");
        std::lock_guard<std::mutex> lk(a->mu);
        a->eng->set_dump_dir(dir ? dir : "");
        return 0;
    });
}

}  // extern "C"
