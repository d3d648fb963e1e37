// SHIELD-A engine on the GPU.  The sequence stages are SeqStack's, run with the audio model's window length (126),
// its arithmetic where it differs from SHIELD-V's (L2 norm without the q scale, gated norm o * 0.125 with eps 1e-5,
// GDN-B residual h + 0.70710678 * branch, GELU head: engine/audio/sequence.cpp:119-124, 160-171, 226, 318-330) and
// its tensor names; the token assembly is a plain copy plus the readout row (sequence.cpp:322-323).
// The frontend (engine/audio/frontend.cpp:170-280) runs over chunks of kFrontChunk windows: log-mel (afront.hip),
// the stem, eight blocks of pw1 (GEMM, BatchNorm folded, SiLU) -> depthwise (BatchNorm, SiLU) -> pw2 (GEMM,
// BatchNorm folded, + the block input where the shape is kept), the frequency-attention pooling and the token
// projection (GEMM) into the sequence stages' token buffer.  The reference computes the tokens in five time slabs
// with 40-frame halos (frontend.cpp:233-244); with a 77-frame receptive field and slab starts on multiples of the
// time stride 8, that is the whole window's result, which is what this computes in one pass.
#include "audio.hpp"

#include "dev_common.hpp"
#include "kernels.hpp"
#include "stack.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <map>
#include <tuple>
#include <vector>

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
            if (ah.front.present) upload_front(ah.front, upl);
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

    void predict_device(const float* d_pcm, long long stride, int n, float* d_logits, hipStream_t s) override {
        need_frontend();
        if (n <= 0) return;
        if (n > max_windows_) throw std::runtime_error("audio: more windows than max_windows");
        if (!d_pcm || !d_logits) throw std::runtime_error("audio: null buffer");
        if (stride < kAudioWindowSamples) throw std::runtime_error("audio: window stride below 160000 samples");
        const hipStream_t q = s ? s : work_;
        SHV_HIP_CHECK(hipStreamWaitEvent(q, last_done_, 0));
        run_graph(Key{1, d_pcm, stride, d_logits, n}, q, [&](hipStream_t r) {
            frontend(d_pcm, stride, n, d_tokens_, r);
            sequence(d_tokens_, kAudioWindowFloats, n, d_logits, r);
        });
        SHV_HIP_CHECK(hipEventRecord(last_done_, q));
    }

    void predict_host(const float* pcm, long long stride, long long n, float* logits) override {
        host_pcm_pass(pcm, stride, n, [&](long long w0, int b) {
            sequence(d_tokens_, kAudioWindowFloats, b, d_logits_, work_);
            SHV_HIP_CHECK(hipMemcpyAsync(logits + w0, d_logits_, size_t(b) * 4, hipMemcpyDeviceToHost, work_));
        });
    }

    void frontend_host(const float* pcm, long long stride, long long n, float* tokens) override {
        host_pcm_pass(pcm, stride, n, [&](long long w0, int b) {
            SHV_HIP_CHECK(hipMemcpyAsync(tokens + w0 * kAudioWindowFloats, d_tokens_,
                                         size_t(b) * kAudioWindowFloats * 4, hipMemcpyDeviceToHost, work_));
        });
    }

private:
    struct Key {
        int kind;   // 0 tokens -> logits, 1 PCM -> logits
        const void* in;
        long long ldw;
        const void* out;
        int n;
        bool operator<(const Key& o) const {
            return std::tie(kind, in, ldw, out, n) < std::tie(o.kind, o.in, o.ldw, o.out, o.n);
        }
    };
    // the frontend runs over chunks of this many windows (its activations: about 49 MB per window)
    static constexpr int kFrontChunk = 16;
    struct FrontBlock {
        int ci, hid, co, sf, st, T, F, To, Fo;
        bool residual;
        DevW pw1, pw2;
        const float *b1 = nullptr, *b2 = nullptr, *dw_w = nullptr, *dw_scale = nullptr, *dw_shift = nullptr;
    };
    AudioMelTables mel_tables_;
    const float *stem_w_ = nullptr, *stem_scale_ = nullptr, *stem_shift_ = nullptr, *fa_w_ = nullptr;
    float fa_b_ = 0.0f;
    FrontBlock fblk_[8];
    DevW proj_w_;
    int front_chunk_ = 0;
    // frontend activations for front_chunk_ windows: PCM staging (host calls), log-mel, block input / output
    // ping-pong, pw1 output, depthwise output, pooled attention output
    float *d_pcm_ = nullptr, *d_mel_ = nullptr, *d_x_[2] = {nullptr, nullptr}, *d_e_ = nullptr, *d_dwo_ = nullptr,
          *d_pool_ = nullptr;

    void need_frontend() const {
        if (!has_frontend_)
            throw std::runtime_error("audio: the weight file carries no frontend tensors (frontend.*, cnn.*): "
                                     "PCM input needs the whole model");
    }

    const int* up_int(const std::vector<int>& v) {
        int* d = wmem_.make<int>(v.size());
        SHV_HIP_CHECK(hipMemcpy(d, v.data(), v.size() * sizeof(int), hipMemcpyHostToDevice));
        return d;
    }

    void upload_front(const AudioFrontHost& F, Uploader& upl) {
        mel_tables_.window = upl.up(F.window);
        mel_tables_.wr = upl.up(F.wr);
        mel_tables_.wi = upl.up(F.wi);
        mel_tables_.fb_off = up_int(F.fb_off);
        mel_tables_.fb_k = up_int(F.fb_k);
        mel_tables_.fb_w = upl.up(F.fb_w);
        mel_tables_.mean = upl.up(F.mean);
        mel_tables_.stdv = upl.up(F.stdv);
        stem_w_ = upl.up(F.stem_w);
        stem_scale_ = upl.up(F.stem_scale);
        stem_shift_ = upl.up(F.stem_shift);
        int T = kAudioMelFrames, Fq = kAudioMelBins;
        size_t xmax = size_t(T) * Fq * 32, emax = 0, dmax = 0;
        for (int i = 0; i < 8; ++i) {
            const AudioBlockHost& h = F.blocks[i];
            FrontBlock& b = fblk_[i];
            b.ci = h.ci; b.hid = h.hid; b.co = h.co; b.sf = h.sf; b.st = h.st; b.residual = h.residual;
            b.T = T; b.F = Fq;
            b.To = (T + h.st - 1) / h.st;
            b.Fo = (Fq + h.sf - 1) / h.sf;
            // the 1x1 layers in the tier's GEMM arithmetic (fp16: weights stored pre-scaled by a power of two)
            b.pw1 = upl.repack<G>(h.pw1.w, h.hid, h.ci, 0, false, true);
            b.b1 = upl.up(h.pw1.b);
            b.pw2 = upl.repack<G>(h.pw2.w, h.co, h.hid, 0, false, true);
            b.b2 = upl.up(h.pw2.b);
            b.dw_w = upl.up(h.dw_w);
            b.dw_scale = upl.up(h.dw_scale);
            b.dw_shift = upl.up(h.dw_shift);
            emax = std::max(emax, size_t(T) * Fq * h.hid);
            dmax = std::max(dmax, size_t(b.To) * b.Fo * h.hid);
            xmax = std::max(xmax, size_t(b.To) * b.Fo * h.co);
            T = b.To;
            Fq = b.Fo;
        }
        if (T != kAudioTokensPerWindow || Fq != kAudioCnnFreq || fblk_[7].co != kAudioCnnCh)
            throw std::runtime_error("audio: unexpected frontend CNN output shape");
        fa_w_ = upl.up(F.fa_w);
        fa_b_ = F.fa_b;
        proj_w_ = upl.repack<G>(F.proj.w, kD, kAudioCnnCh, 0, false, true);
        front_chunk_ = std::min(max_windows_, kFrontChunk);
        const size_t c = size_t(front_chunk_);
        d_pcm_ = amem_.make<float>(c * kAudioWindowSamples);
        d_mel_ = amem_.make<float>(c * kAudioMelFrames * kAudioMelBins);
        d_x_[0] = amem_.make<float>(c * xmax);
        d_x_[1] = amem_.make<float>(c * xmax);
        d_e_ = amem_.make<float>(c * emax);
        d_dwo_ = amem_.make<float>(c * dmax);
        d_pool_ = amem_.make<float>(c * kAudioTokensPerWindow * kAudioCnnCh);
        has_frontend_ = true;
    }

    void gemm(const char* role, const GemmArgs& p, const DevW& w, hipStream_t s) {
        GemmRunner<G>{*this, nullptr, 0, false}.gemm(role, p, w, s);
    }

    // PCM windows [n] (window w at pcm + w * stride) -> tokens [n][125][384] at `tokens`, in chunks of front_chunk_
    void frontend(const float* pcm, long long stride, int n, float* tokens, hipStream_t s) {
        for (int w0 = 0; w0 < n; w0 += front_chunk_) {
            const int b = std::min(front_chunk_, n - w0);
            timed("audio_mel", double(b) * (kAudioWindowSamples + kAudioMelFrames * kAudioMelBins) * 4, s,
                  [&] { launch_audio_mel(pcm + w0 * stride, stride, b, mel_tables_, d_mel_, s); });
            check_launch();
            if (w0 == 0 && !dump_dir_.empty()) dump_mel(s);
            timed("audio_stem", double(b) * kAudioMelFrames * kAudioMelBins * (1 + 32) * 4, s,
                  [&] { launch_audio_stem(d_mel_, stem_w_, stem_scale_, stem_shift_, d_x_[0], b, s); });
            check_launch();
            int cur = 0;
            for (int i = 0; i < 8; ++i) {
                const FrontBlock& k = fblk_[i];
                const long long rows_in = (long long)b * k.T * k.F, rows_out = (long long)b * k.To * k.Fo;
                GemmArgs p1;
                p1.M = int(rows_in); p1.N = k.hid; p1.K = k.ci;
                p1.A = d_x_[cur]; p1.lda = k.ci; p1.ldw = k.ci;
                p1.bias = k.b1; p1.act = ACT_SILU;
                p1.C = d_e_; p1.ldc = k.hid;
                gemm("audio_pw1", p1, k.pw1, s);
                timed("audio_dw", double(rows_in + rows_out) * k.hid * 4, s, [&] {
                    launch_audio_dw(d_e_, d_dwo_, k.dw_w, k.dw_scale, k.dw_shift, b, k.T, k.F, k.hid, k.st, k.sf, s);
                });
                check_launch();
                GemmArgs p2;
                p2.M = int(rows_out); p2.N = k.co; p2.K = k.hid;
                p2.A = d_dwo_; p2.lda = k.hid; p2.ldw = k.hid;
                p2.bias = k.b2;
                p2.C = d_x_[1 - cur]; p2.ldc = k.co;
                if (k.residual) { p2.R = d_x_[cur]; p2.ldr = k.co; p2.res = 1; }
                gemm("audio_pw2", p2, k.pw2, s);
                cur = 1 - cur;
            }
            timed("audio_freq_pool", double(b) * kAudioTokensPerWindow * (kAudioCnnFreq + 1) * kAudioCnnCh * 4, s,
                  [&] { launch_audio_freq_pool(d_x_[cur], fa_w_, fa_b_, d_pool_, b, s); });
            check_launch();
            GemmArgs pp;
            pp.M = b * kAudioTokensPerWindow; pp.N = kD; pp.K = kAudioCnnCh;
            pp.A = d_pool_; pp.lda = kAudioCnnCh; pp.ldw = kAudioCnnCh;
            pp.C = tokens + (long long)w0 * kAudioWindowFloats; pp.ldc = kD;
            gemm("audio_proj", pp, proj_w_, s);
            if (w0 == 0) dump_f32(dump_dir_, "cnn", tokens, size_t(kAudioWindowFloats), s);
        }
    }

    // window 0's log-mel as the reference dumps it (frontend.cpp:272-274): [80][997]
    void dump_mel(hipStream_t s) {
        std::vector<float> m(size_t(kAudioMelFrames) * kAudioMelBins), t(m.size());
        SHV_HIP_CHECK(hipMemcpyAsync(m.data(), d_mel_, m.size() * 4, hipMemcpyDeviceToHost, s));
        SHV_HIP_CHECK(hipStreamSynchronize(s));
        for (int f = 0; f < kAudioMelFrames; ++f)
            for (int b = 0; b < kAudioMelBins; ++b) t[size_t(b) * kAudioMelFrames + f] = m[size_t(f) * kAudioMelBins + b];
        const std::string path = dump_dir_ + "/mel.f32";
        std::FILE* fp = std::fopen(path.c_str(), "wb");
        if (!fp) throw std::runtime_error("dump: cannot open " + path);
        const size_t put = std::fwrite(t.data(), 4, t.size(), fp);
        if (std::fclose(fp) != 0 || put != t.size()) throw std::runtime_error("dump: short write to " + path);
    }

    // Host PCM in batches of max_windows: each batch's windows through the frontend (uploaded chunk by chunk) into
    // the token buffer, then `tail(w0, b)` on work_; returns when all of it is done.  Rejects PCM that is not finite
    // or outside [-1, 1], as the reference does (engine/audio/api.cpp:25-29), before any work.
    template <class Tail> void host_pcm_pass(const float* pcm, long long stride, long long n, Tail&& tail) {
        need_frontend();
        if (n <= 0) return;
        if (!pcm) throw std::runtime_error("audio: null buffer");
        if (stride < kAudioWindowSamples) throw std::runtime_error("audio: window stride below 160000 samples");
        for (long long w = 0; w < n; ++w)
            for (long long i = 0; i < kAudioWindowSamples; ++i) {
                const float v = pcm[w * stride + i];
                if (!std::isfinite(v) || std::fabs(v) > 1.0f)
                    throw std::runtime_error("audio must be finite float32 in [-1,1]");
            }
        SHV_HIP_CHECK(hipStreamWaitEvent(work_, last_done_, 0));
        for (long long w0 = 0; w0 < n; w0 += max_windows_) {
            const int b = int(std::min<long long>(max_windows_, n - w0));
            for (int c0 = 0; c0 < b; c0 += front_chunk_) {
                const int cb = std::min(front_chunk_, b - c0);
                SHV_HIP_CHECK(hipMemcpy2DAsync(d_pcm_, size_t(kAudioWindowSamples) * 4, pcm + (w0 + c0) * stride,
                                               size_t(stride) * 4, size_t(kAudioWindowSamples) * 4, size_t(cb),
                                               hipMemcpyHostToDevice, work_));
                frontend(d_pcm_, kAudioWindowSamples, cb, d_tokens_ + (long long)c0 * kAudioWindowFloats, work_);
            }
            tail(w0, b);
            SHV_HIP_CHECK(hipEventRecord(last_done_, work_));
            SHV_HIP_CHECK(hipStreamSynchronize(work_));
        }
    }
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
        run_graph(Key{0, d_tokens, ldw, d_logits, n}, q,
                  [&](hipStream_t r) { sequence(d_tokens, ldw, n, d_logits, r); });
    }
    void sequence(const float* d_tokens, long long ldw, int n, float* d_logits, hipStream_t r) {
        WindowInput in;
        in.tokens = d_tokens;
        in.ldw = ldw;
        in.readout = readout_;
        seq_->run(in, n, d_logits, r, *this, dump_dir_);
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
