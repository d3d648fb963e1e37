// SHIELD-V HIP engine core: device weights (repacked on the GPU), activation buffers, the encode / classify
// forward passes and their HIP graphs.  One thread drives an Engine (the API worker, or a benchmark).
#pragma once
#include "host_model.hpp"

#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#define SHV_HIP_CHECK(expr)                                                                                 \
    do {                                                                                                    \
        const hipError_t err__ = (expr);                                                                    \
        if (err__ != hipSuccess)                                                                            \
            throw std::runtime_error(std::string("HIP error ") + hipGetErrorString(err__) + " at " +        \
                                     __FILE__ + ":" + std::to_string(__LINE__) + ": " #expr);               \
    } while (0)

namespace shv {

// The exact tier's arithmetic in the sequence stages.  The CNN always performs the reference CPU engine's operation
// order (its tokens are bitwise the reference's).  By default the all-row sequence GEMMs run on the fp32 matrix cores
// and the delta rule splits each value column's keys over lane groups (fp32 values and operations, in an order of
// this engine's own); SHV_HIP_F32_CPU_ORDER=1 at load keeps the reference's order there too (VALU GEMMs in K blocks
// of 64, the 64-key fma chains), so that every stage output is the reference's: the check that pins the sequence
// stage code to the reference.
inline bool f32_cpu_order_requested() {
    const char* e = std::getenv("SHV_HIP_F32_CPU_ORDER");
    return e && *e && std::strcmp(e, "0") != 0;
}

enum class Precision { FP32 = 0, BF16 = 1, FP16 = 2 };
const char* precision_name(Precision p);
bool parse_precision(const std::string& s, Precision* p);

struct EngineConfig {
    int max_frames = 640;       // frames per encode launch
    int max_windows = 512;      // windows per classify launch
    int max_host_tokens = 2048; // host token blocks staged per batch
    bool use_graphs = true;     // one HIP graph per (kind, buffers, bucket)
    int slots = 2;              // input/output buffer sets for the scheduler's pipelining
};

// Per-family kernel timing (HIP events on the launching stream), algorithmic bytes and FLOPs.  A family is one
// kernel at the shapes the forward gives it: GEMM families are named "<role>:<kernel template>".
struct ProfStat {
    double ms = 0.0, bytes = 0.0, flops = 0.0;
    long long launches = 0;
};

// Event timing of kernel families.  Used by one thread at a time (the engine's driver).
class Profiler {
public:
    Profiler() = default;
    Profiler(const Profiler&) = delete;
    Profiler& operator=(const Profiler&) = delete;
    ~Profiler();
    void profile_enable(bool on);
    bool profiling() const { return prof_on_; }
    // flushes pending events; false if the family is unknown
    bool profile_read(const std::string& family, ProfStat* out);
    // every family seen since profiling was enabled, in first-launch order
    std::vector<std::string> profile_families() const { return fam_names_; }
    // launch() issues one kernel family on s; timed between two events when profiling is on
    template <class F>
    void timed(const std::string& family, double bytes, hipStream_t s, F&& launch, double flops = 0.0) {
        if (!prof_on_) { launch(); return; }
        Pending p{family_id(family), bytes, flops, take_event(), take_event()};
        SHV_HIP_CHECK(hipEventRecord(p.e0, s));
        launch();
        SHV_HIP_CHECK(hipEventRecord(p.e1, s));
        pending_.push_back(p);
    }

private:
    struct Pending {
        int family;
        double bytes, flops;
        hipEvent_t e0, e1;
    };
    bool prof_on_ = false;
    std::vector<std::string> fam_names_;
    std::vector<ProfStat> fam_stats_;
    std::vector<Pending> pending_;
    std::vector<hipEvent_t> event_pool_;
    int family_id(const std::string& name);
    hipEvent_t take_event();
    void prof_flush();
};

class Engine : public Profiler {
public:
    struct Slot {
        uint8_t* d_frames = nullptr;      // [max_frames][172800]
        float* d_tokens = nullptr;        // [max_frames][6144]
        float* d_tok_stage = nullptr;     // [max(max_host_tokens,1)][6144]
        const float** d_tokptr = nullptr; // [max_windows * 20]
        float* d_logits = nullptr;        // [max_windows]
        int32_t* d_store = nullptr;       // [max_frames][2]: (batch frame, pool slot) of each storing frame
    };
    virtual ~Engine() = default;

    Precision precision() const { return prec_; }
    const EngineConfig& config() const { return cfg_; }
    const Slot& slot(int i) const { return slots_.at(size_t(i)); }
    // Slot path (scheduler): frames of slot -> its tokens; windows through its pointer table -> its logits.
    // F / B are padded to a bucket when graphs are on (padding rows are computed and ignored).
    virtual void encode_slot(int slot, int F, hipStream_t s) = 0;
    virtual void classify_slot(int slot, int B, hipStream_t s) = 0;
    // Both for a batch whose window w reads exactly frames [20 w, 20 w + 20) of the slot (its table filled so): the
    // branches then run their windows' sequence stages right after their encode.  false (nothing queued) if the
    // bucket's frames do not fit the slot.
    virtual bool forward_slot(int slot, int n, hipStream_t s) = 0;
    // Direct path on caller device buffers (no padding): frames [F] -> tokens [F][6144]
    virtual void encode_direct(const uint8_t* d_frames, int F, float* d_tokens, hipStream_t s) = 0;
    // clips [n][20] frames -> logits [n], through the engine's own token buffer
    virtual void forward_direct(const uint8_t* d_frames, int n, float* d_logits, hipStream_t s) = 0;
    // windows [n][20][16][384] of tokens in device memory -> logits [n] (the sequence stages alone)
    virtual void classify_direct(const float* d_tokens, int n, float* d_logits, hipStream_t s) = 0;

    size_t weight_bytes() const { return weight_bytes_; }
    size_t device_bytes() const { return device_bytes_; }
    int frame_bucket(int F) const;
    int window_bucket(int B) const;

    void set_dump_dir(const std::string& d) { dump_dir_ = d; }

protected:
    Precision prec_ = Precision::FP32;
    EngineConfig cfg_;
    std::vector<Slot> slots_;
    size_t weight_bytes_ = 0, device_bytes_ = 0;
    std::string dump_dir_;
};

std::unique_ptr<Engine> make_engine(const HostModel& hm, Precision p, const EngineConfig& cfg);

// Pointwise-conv GEMM tool (the reference's bench/gpu_gemm_bench.cu:27-116): C[M][N] = act(A[M][K] . W[N][K]^T + bias)
// in the tier's arithmetic, W repacked once on the device into the tier's operand parts; A, bias and C are the
// caller's device buffers.  act takes the reference's codes (engine/cuda/common.cuh:69): 0 none, 1 ReLU, 2 hardswish,
// 3 SiLU, 4 hardsigmoid.
// Gated delta rule of one tier on caller device buffers (rows = n_windows * 321; Q, K [rows][384], V, O [rows][768],
// decay, beta [rows][8]).  variant 0: the tier's own kernel (fp32: token by token in the reference's order; fp16 /
// bf16: the chunked scan), 1: token by token, 2: chunked (fp16 / bf16 only).  Allocates its work buffer per call.
void run_delta_rule(Precision p, const float* Q, const float* K, const float* V, const float* dec, const float* beta,
                    int n_windows, float* O, int variant, hipStream_t s);
// The same without any allocation and without synchronising: the chunked scan works in a static device array for
// at most kDeltaNoAllocWindows windows (one per GPU, held until the process ends; looked up on the first call on
// each device).  Calls that overlap on one GPU race on that array.
constexpr int kDeltaNoAllocWindows = 16;
void run_delta_rule_noalloc(Precision p, const float* Q, const float* K, const float* V, const float* dec,
                            const float* beta, int n_windows, float* O, int variant, hipStream_t s);
// The kernel a delta-rule call runs: the chunked scan (matrix cores: split operands in the half tiers, fp32 operands
// in the exact tier), token by token with each value column's keys split over lane groups in one canonical order
// (every tier), or token by token in the reference CPU engine's order (fp32).  variant 0 = the tier's own (the
// chunked scan; fp32 under SHV_HIP_F32_CPU_ORDER: the reference order), 1 = token by token (fp32: the reference
// order; half tiers: key split), 2 = chunked, 3 = key split.  Validates the arguments.
enum class DeltaKernel { Chunked, KeySplit, Reference };
inline DeltaKernel delta_rule_kernel(Precision p, const float* Q, const float* K, const float* V, const float* dec,
                                     const float* beta, int n_windows, const float* O, int variant) {
    if (!Q || !K || !V || !dec || !beta || !O || n_windows < 1 || n_windows > 65536)
        throw std::runtime_error("delta rule: null buffer or bad window count");
    if (variant < 0 || variant > 3) throw std::runtime_error("delta rule: unknown variant");
    if (variant == 3) return DeltaKernel::KeySplit;
    if (variant == 2) return DeltaKernel::Chunked;
    if (p == Precision::FP32) {
        if (variant == 1) return DeltaKernel::Reference;
        return f32_cpu_order_requested() ? DeltaKernel::Reference : DeltaKernel::Chunked;
    }
    return variant == 1 ? DeltaKernel::KeySplit : DeltaKernel::Chunked;
}

class PwGemm {
public:
    PwGemm(Precision p, int N, int K, const float* d_w, hipStream_t s);
    ~PwGemm();
    PwGemm(const PwGemm&) = delete;
    PwGemm& operator=(const PwGemm&) = delete;
    // variant: kernel choice (0 = the engine's own: for fp32 the CNN's, the reference CPU order); see
    // gemm_f32_variant / gemm_mfma_variant; fp32 4 = the fp32 matrix cores (gemm_f32_mfma, the sequence stages'
    // kernel)
    void run(const float* A, long long M, const float* bias, int act, float* C, int variant, hipStream_t s) const;
    Precision precision() const { return prec_; }

private:
    Precision prec_;
    int N_ = 0, K_ = 0;
    void* w_ = nullptr;
    long long wstride_ = 0;
    float wscale_ = 1.0f;   // fp16: the inverse of the power of two the weight parts are stored at
};

}  // namespace shv
