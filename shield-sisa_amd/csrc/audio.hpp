// SHIELD-A engine: the audio model on the GPU, batched over windows.  The frontend (engine/audio/frontend.cpp:
// 10 s of PCM -> log-mel -> CNN -> 125 tokens of 384) when the weight file carries its tensors, and the sequence
// stages (engine/audio/sequence.cpp:319-348: 125 tokens + the readout -> GDN-A -> GDN-B twice -> SISA last row ->
// head -> one logit per window) on the same kernels as SHIELD-V's sequence.  One thread drives an AudioEngine at a
// time.
#pragma once
#include "engine.hpp"

#include <memory>
#include <string>

namespace shv {

constexpr int kAudioTokens = kTAudio - 1;                              // 125 tokens per window
constexpr long long kAudioWindowFloats = (long long)kAudioTokens * kD;   // 48000

class AudioEngine : public Profiler {
public:
    virtual ~AudioEngine() = default;
    Precision precision() const { return prec_; }
    int max_windows() const { return max_windows_; }
    size_t weight_bytes() const { return weight_bytes_; }
    size_t device_bytes() const { return device_bytes_; }
    void set_dump_dir(const std::string& d) { dump_dir_ = d; }
    // n windows of device tokens (window w at d_tokens + w * ldw, ldw >= 48000 and a multiple of 4 floats, 16-byte
    // aligned) -> d_logits[n], issued on s (n <= max_windows)
    virtual void run_device(const float* d_tokens, long long ldw, int n, float* d_logits, hipStream_t s) = 0;
    // the same from host memory to host memory through the engine's own buffers, in batches of max_windows;
    // returns when the logits are written
    virtual void run_host(const float* tokens, long long ldw, long long n, float* logits) = 0;

    // The whole model from PCM (only with the frontend's tensors: has_frontend()).  Window w's 160,000 samples at
    // pcm + w * stride (stride >= 160,000 samples).  Device: d_pcm and d_logits in device memory, n <= max_windows,
    // issued on s.  Host: returns when the logits are written.
    bool has_frontend() const { return has_frontend_; }
    virtual void predict_device(const float* d_pcm, long long stride, int n, float* d_logits, hipStream_t s) = 0;
    virtual void predict_host(const float* pcm, long long stride, long long n, float* logits) = 0;
    // the frontend alone: host PCM -> host tokens [n][125][384]
    virtual void frontend_host(const float* pcm, long long stride, long long n, float* tokens) = 0;

protected:
    bool has_frontend_ = false;
    Precision prec_ = Precision::FP32;
    int max_windows_ = 0;
    size_t weight_bytes_ = 0, device_bytes_ = 0;
    std::string dump_dir_;
};

// Throws std::runtime_error (HIP errors included).
std::unique_ptr<AudioEngine> make_audio_engine(const AudioHost& ah, Precision p, int max_windows, bool use_graphs);

}  // namespace shv
