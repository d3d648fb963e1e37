// SHIELD-A sequence engine on the GPU.  The stages are SeqStack's, run with the audio model's window length (126),
// its arithmetic where it differs from SHIELD-V's (L2 norm without the q scale, gated norm o * 0.125 with eps 1e-5,
// GDN-B residual h + 0.70710678 * branch, GELU head: engine/audio/sequence.cpp:119-124, 160-171, 226, 318-330) and
// its tensor names; the token assembly is a plain copy plus the readout row (sequence.cpp:322-323).
#include "audio.hpp"

#include "kernels.hpp"
#include "stack.hpp"

#include <map>
#include <tuple>

namespace shv {
namespace {

template <typename G> class AudioEngineT final : public AudioEngine {
public:
    AudioEngineT(const AudioHost& ah, Precision p, int max_windows, bool use_graphs) : use_graphs_(use_graphs) {
        if (max_windows < 1 || max_windows > 65536) throw std::runtime_error("audio: max_windows must be in [1, 65536]");
        prec_ = p;
        max_windows_ = max_windows;
        SHV_HIP_CHECK(hipStreamCreateWithFlags(&setup_, hipStreamNonBlocking));
        try {
            Uploader upl(wmem_, setup_);
            // SHIELD-A: 126-token windows, audio arithmetic, GDN-B residual R + 0.70710678 v; the reference's dump
            // names (sequence.cpp:324-345)
            static constexpr SeqSpec kAudio{kTAudio, true, 3, {"tokens", "gdn_a", "gdn_b", "sisa_last", "logit"}};
            seq_.reset(new SeqStack<G>(kAudio, ah.gdn, ah.sisa, ah.final_norm_w, ah.head0, ah.head2_w, ah.head2_b,
                                       max_windows, upl, amem_));
            readout_ = upl.up(ah.readout);
            upl.finish();
            d_tokens_ = amem_.make<float>(size_t(max_windows) * kAudioWindowFloats);
            d_logits_ = amem_.make<float>(size_t(max_windows));
            // padding windows of a host batch read these before any upload reaches them
            SHV_HIP_CHECK(hipMemset(d_tokens_, 0, size_t(max_windows) * kAudioWindowFloats * 4));
            SHV_HIP_CHECK(hipStreamCreateWithFlags(&work_, hipStreamNonBlocking));
            SHV_HIP_CHECK(hipStreamCreateWithFlags(&capture_, hipStreamNonBlocking));
            SHV_HIP_CHECK(hipEventCreateWithFlags(&last_done_, hipEventDisableTiming));
            SHV_HIP_CHECK(hipEventRecord(last_done_, work_));
        } catch (...) {
            (void)hipStreamSynchronize(setup_);
            (void)hipStreamDestroy(setup_);
            if (last_done_) (void)hipEventDestroy(last_done_);
            if (work_) (void)hipStreamDestroy(work_);
            if (capture_) (void)hipStreamDestroy(capture_);
            throw;
        }
        SHV_HIP_CHECK(hipStreamDestroy(setup_));
        setup_ = nullptr;
        weight_bytes_ = wmem_.bytes();
        device_bytes_ = wmem_.bytes() + amem_.bytes();
    }
    ~AudioEngineT() override {
        if (last_done_) (void)hipEventSynchronize(last_done_);
        for (auto& kv : graphs_) (void)hipGraphExecDestroy(kv.second);
        if (last_done_) (void)hipEventDestroy(last_done_);
        if (work_) (void)hipStreamSynchronize(work_);
        if (work_) (void)hipStreamDestroy(work_);
        if (capture_) (void)hipStreamDestroy(capture_);
    }

    // Every call of one handle uses the same activation buffers, so each call's device work starts after the
    // previous call's has ended, whatever streams the two were issued on: a call waits on last_done_ on its stream
    // and records last_done_ there at its end.  A NULL stream is the handle's own.
    void run_device(const float* d_tokens, long long ldw, int n, float* d_logits, hipStream_t s) override {
        if (n <= 0) return;
        if (n > max_windows_) throw std::runtime_error("audio: more windows than max_windows");
        if (!d_tokens || !d_logits) throw std::runtime_error("audio: null buffer");
        const hipStream_t q = s ? s : work_;
        SHV_HIP_CHECK(hipStreamWaitEvent(q, last_done_, 0));
        forward(d_tokens, ldw, n, d_logits, q);
        SHV_HIP_CHECK(hipEventRecord(last_done_, q));
    }

    void run_host(const float* tokens, long long ldw, long long n, float* logits) override {
        if (n <= 0) return;
        if (!tokens || !logits) throw std::runtime_error("audio: null buffer");
        if (ldw < kAudioWindowFloats) throw std::runtime_error("audio: window stride below 48000 floats");
        SHV_HIP_CHECK(hipStreamWaitEvent(work_, last_done_, 0));
        for (long long w0 = 0; w0 < n; w0 += max_windows_) {
            const int b = int(std::min<long long>(max_windows_, n - w0));
            if (ldw == kAudioWindowFloats) {
                SHV_HIP_CHECK(hipMemcpyAsync(d_tokens_, tokens + w0 * ldw, size_t(b) * kAudioWindowFloats * 4,
                                             hipMemcpyHostToDevice, work_));
            } else {
                SHV_HIP_CHECK(hipMemcpy2DAsync(d_tokens_, size_t(kAudioWindowFloats) * 4, tokens + w0 * ldw,
                                               size_t(ldw) * 4, size_t(kAudioWindowFloats) * 4, size_t(b),
                                               hipMemcpyHostToDevice, work_));
            }
            // graphs are keyed by the window count: host batches run padded to a multiple of 8 windows (the padding
            // windows compute on stale tokens and are not copied back)
            const int bp = use_graphs_ ? std::min(max_windows_, (b + 7) / 8 * 8) : b;
            forward(d_tokens_, kAudioWindowFloats, bp, d_logits_, work_);
            SHV_HIP_CHECK(hipMemcpyAsync(logits + w0, d_logits_, size_t(b) * 4, hipMemcpyDeviceToHost, work_));
            SHV_HIP_CHECK(hipEventRecord(last_done_, work_));
            SHV_HIP_CHECK(hipStreamSynchronize(work_));
        }
    }

private:
    struct Key {
        const void* in;
        long long ldw;
        const void* out;
        int n;
        bool operator<(const Key& o) const { return std::tie(in, ldw, out, n) < std::tie(o.in, o.ldw, o.out, o.n); }
    };
    bool use_graphs_;
    hipStream_t setup_ = nullptr, work_ = nullptr;
    // graphs are captured on this private stream, then launched on the caller's
    hipStream_t capture_ = nullptr;
    hipEvent_t last_done_ = nullptr;   // the end of the latest call's device work
    DevMem wmem_, amem_;
    std::unique_ptr<SeqStack<G>> seq_;
    const float* readout_ = nullptr;
    float *d_tokens_ = nullptr, *d_logits_ = nullptr;
    std::map<Key, hipGraphExec_t> graphs_;

    void forward(const float* d_tokens, long long ldw, int n, float* d_logits, hipStream_t q) {
        run_graph(Key{d_tokens, ldw, d_logits, n}, q, [&](hipStream_t r) {
            WindowInput in;
            in.tokens = d_tokens;
            in.ldw = ldw;
            in.readout = readout_;
            seq_->run(in, n, d_logits, r, *this, dump_dir_);
        });
    }

    template <class F> void run_graph(const Key& key, hipStream_t s, F&& body) {
        auto it = graphs_.find(key);
        // eager when dumping or profiling, and past 64 cached graphs (callers cycling through many device buffers)
        if (!use_graphs_ || !dump_dir_.empty() || profiling() || (it == graphs_.end() && graphs_.size() >= 64)) {
            body(s);
            return;
        }
        if (it == graphs_.end()) {
            hipGraph_t g = nullptr;
            SHV_HIP_CHECK(hipStreamBeginCapture(capture_, hipStreamCaptureModeThreadLocal));
            try {
                body(capture_);
            } catch (...) {
                (void)hipStreamEndCapture(capture_, &g);
                if (g) (void)hipGraphDestroy(g);
                throw;
            }
            SHV_HIP_CHECK(hipStreamEndCapture(capture_, &g));
            hipGraphExec_t ex = nullptr;
            const hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            SHV_HIP_CHECK(e);
            it = graphs_.emplace(key, ex).first;
        }
        SHV_HIP_CHECK(hipGraphLaunch(it->second, s));
    }
};

}  // namespace

std::unique_ptr<AudioEngine> make_audio_engine(const AudioHost& ah, Precision p, int max_windows, bool use_graphs) {
    switch (p) {
    case Precision::FP32: return std::unique_ptr<AudioEngine>(new AudioEngineT<float>(ah, p, max_windows, use_graphs));
    case Precision::BF16: return std::unique_ptr<AudioEngine>(new AudioEngineT<bf16>(ah, p, max_windows, use_graphs));
    case Precision::FP16: return std::unique_ptr<AudioEngine>(new AudioEngineT<f16>(ah, p, max_windows, use_graphs));
    }
    throw std::runtime_error("audio: unknown precision");
}

}  // namespace shv
