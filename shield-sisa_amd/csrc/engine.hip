// SHIELD-V HIP engine core.  Orchestration of the forward (the reference's engine/cuda/engine.cu:338-470 and the
// CPU engine's isa_impl.hpp:793-851, 1071-1141 define the function), device memory, GPU weight repacking, HIP
// graphs, per-family event timing and debug dumps.
#include "engine.hpp"

#include "dev_common.hpp"
#include "kernels.hpp"
#include "stack.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <tuple>
#include <type_traits>

namespace shv {

namespace {
struct ModeName {
    Precision p;
    const char* name;
};
constexpr ModeName kModes[] = {{Precision::FP32, "fp32"}, {Precision::BF16, "bf16"}, {Precision::FP16, "fp16"}};

// Batch sizes run padded to a bucket so that one HIP graph serves every size in it: n rounded up to a multiple of
// a power of two about n / 8 (at most 12.5% padding, eight buckets per octave), never above the configured maximum.
int bucket_for(int n, int max_n) {
    if (n > max_n) throw std::runtime_error("batch larger than the configured maximum");
    int top = 1;
    while (top * 2 <= n) top *= 2;
    const int quantum = std::max(1, top / 8);
    return std::min(max_n, (n + quantum - 1) / quantum * quantum);
}
}  // namespace

const char* precision_name(Precision p) {
    for (const ModeName& m : kModes)
        if (m.p == p) return m.name;
    return "?";
}
bool parse_precision(const std::string& s, Precision* p) {
    for (const ModeName& m : kModes)
        if (s == m.name) {
            *p = m.p;
            return true;
        }
    return false;
}

int Engine::frame_bucket(int F) const { return cfg_.use_graphs ? bucket_for(F, cfg_.max_frames) : F; }
int Engine::window_bucket(int B) const { return cfg_.use_graphs ? bucket_for(B, cfg_.max_windows) : B; }

// ------------------------------------------------------------------------------------------------ profiling
int Profiler::family_id(const std::string& name) {
    for (size_t i = 0; i < fam_names_.size(); ++i)
        if (fam_names_[i] == name) return int(i);
    fam_names_.push_back(name);
    fam_stats_.push_back(ProfStat{});
    return int(fam_names_.size() - 1);
}
hipEvent_t Profiler::take_event() {
    if (!event_pool_.empty()) {
        hipEvent_t e = event_pool_.back();
        event_pool_.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    SHV_HIP_CHECK(hipEventCreate(&e));
    return e;
}
void Profiler::prof_flush() {
    for (const Pending& p : pending_) {
        SHV_HIP_CHECK(hipEventSynchronize(p.e1));
        float ms = 0.0f;
        SHV_HIP_CHECK(hipEventElapsedTime(&ms, p.e0, p.e1));
        ProfStat& st = fam_stats_[size_t(p.family)];
        st.ms += ms;
        st.bytes += p.bytes;
        st.flops += p.flops;
        st.launches += 1;
        event_pool_.push_back(p.e0);
        event_pool_.push_back(p.e1);
    }
    pending_.clear();
}
Profiler::~Profiler() {
    for (const Pending& p : pending_) { (void)hipEventDestroy(p.e0); (void)hipEventDestroy(p.e1); }
    for (hipEvent_t e : event_pool_) (void)hipEventDestroy(e);
}
void Profiler::profile_enable(bool on) {
    prof_flush();
    for (ProfStat& s : fam_stats_) s = ProfStat{};
    prof_on_ = on;
}
bool Profiler::profile_read(const std::string& family, ProfStat* out) {
    prof_flush();
    for (size_t i = 0; i < fam_names_.size(); ++i)
        if (fam_names_[i] == family) {
            *out = fam_stats_[i];
            return true;
        }
    return false;
}

namespace {

struct GraphKey {
    int kind;
    const void* in;
    const void* out;
    int n;
    bool operator<(const GraphKey& o) const {
        return std::tie(kind, in, out, n) < std::tie(o.kind, o.in, o.out, o.n);
    }
};


template <typename G>
class EngineT final : public Engine {
    static constexpr bool kF32 = std::is_same<G, float>::value;
    static constexpr int TS = 4;   // activations are fp32 in HBM in every mode

public:
    EngineT(const HostModel& hm, Precision p, const EngineConfig& cfg) {
        prec_ = p;
        cfg_ = cfg;
        if (cfg_.max_frames < 1 || cfg_.max_windows < 1 || cfg_.slots < 1 || cfg_.slots > 4 ||
            cfg_.max_host_tokens < 0)
            throw std::runtime_error("invalid engine configuration");
        // half tiers run the fused inverted-residual kernels unless SHV_HIP_NO_FUSE is set (layer-by-layer A/B)
        const char* nf = std::getenv("SHV_HIP_NO_FUSE");
        fused_ = !kF32 && !(nf && *nf && std::strcmp(nf, "0") != 0);
        // the exact tier's CNN keeps the reference CPU order in every case: with the seeded random-init weights
        // the encoder amplifies a reordered fp32 sum ~30x into the logit (fp32 matrix-core 1x1 convs moved logits
        // by 8.1e-4, twice the exact tier's 4e-4 bar); the sequence stages take the engine's own order (SeqStack)
        cpu_order_ = kF32;
        SHV_HIP_CHECK(hipStreamCreateWithFlags(&setup_, hipStreamNonBlocking));
        try {
            Uploader upl(wmem_, setup_);
            upl_ = &upl;
            upload_weights(hm);
            alloc_buffers(hm);
            upl.finish();
            upl_ = nullptr;
        } catch (...) {
            upl_ = nullptr;
            (void)hipStreamDestroy(setup_);
            throw;
        }
        SHV_HIP_CHECK(hipStreamSynchronize(setup_));
        SHV_HIP_CHECK(hipStreamDestroy(setup_));
        setup_ = nullptr;
        SHV_HIP_CHECK(hipStreamCreateWithFlags(&capture_, hipStreamNonBlocking));
        SHV_HIP_CHECK(hipEventCreateWithFlags(&fork_, hipEventDisableTiming));
        for (int b = 0; b < kBranches; ++b) {
            SHV_HIP_CHECK(hipStreamCreateWithFlags(&bstream_[b], hipStreamNonBlocking));
            SHV_HIP_CHECK(hipEventCreateWithFlags(&join_[b], hipEventDisableTiming));
        }
        weight_bytes_ = wmem_.bytes();
        device_bytes_ = wmem_.bytes() + amem_.bytes();
    }
    ~EngineT() override {
        for (auto& kv : graphs_) (void)hipGraphExecDestroy(kv.second);
        if (capture_) (void)hipStreamDestroy(capture_);
        for (int b = 0; b < kBranches; ++b) {
            if (bstream_[b]) (void)hipStreamDestroy(bstream_[b]);
            if (join_[b]) (void)hipEventDestroy(join_[b]);
        }
        if (fork_) (void)hipEventDestroy(fork_);
    }

    void encode_slot(int slot, int F, hipStream_t s) override {
        if (F <= 0) return;
        if (F > cfg_.max_frames) throw std::runtime_error("encode: too many frames");
        const Slot& sl = slots_.at(size_t(slot));
        const int Fb = frame_bucket(F);
        run_graph(GraphKey{0, sl.d_frames, sl.d_tokens, Fb}, s,
                  [&](hipStream_t q) { encode_branched(sl.d_frames, Fb, sl.d_tokens, q); });
    }
    void classify_slot(int slot, int B, hipStream_t s) override {
        if (B <= 0) return;
        if (B > cfg_.max_windows) throw std::runtime_error("classify: too many windows");
        const Slot& sl = slots_.at(size_t(slot));
        const int Bb = window_bucket(B);
        run_graph(GraphKey{1, sl.d_tokptr, sl.d_logits, Bb}, s, [&](hipStream_t q) {
            ws_on_ = true;   // one pass on q
            run_classify(sl.d_tokptr, Bb, sl.d_logits, q, 0);
        });
    }
    void encode_direct(const uint8_t* d_frames, int F, float* d_tokens, hipStream_t s) override {
        if (F <= 0) return;
        if (F > cfg_.max_frames) throw std::runtime_error("encode: too many frames");
        run_graph(GraphKey{2, d_frames, d_tokens, F}, s,
                  [&](hipStream_t q) { encode_branched(d_frames, F, d_tokens, q); });
    }
    bool forward_slot(int slot, int n, hipStream_t s) override {
        if (n <= 0) return false;
        const int nb = window_bucket(n);
        if (nb > cfg_.max_windows || nb * kFrames > cfg_.max_frames) return false;
        const Slot& sl = slots_.at(size_t(slot));
        run_graph(GraphKey{4, sl.d_frames, sl.d_logits, nb}, s, [&](hipStream_t q) {
            forward_branched(sl.d_frames, sl.d_tokens, sl.d_tokptr, nb, sl.d_logits, q);
        });
        return true;
    }
    void forward_direct(const uint8_t* d_frames, int n, float* d_logits, hipStream_t s) override {
        if (n <= 0) return;
        if (n > cfg_.max_windows || n * kFrames > cfg_.max_frames) throw std::runtime_error("forward: too many clips");
        run_graph(GraphKey{3, d_frames, d_logits, n}, s,
                  [&](hipStream_t q) { forward_branched(d_frames, tok_direct_, tokptr_direct_, n, d_logits, q); });
    }
    void classify_direct(const float* d_tokens, int n, float* d_logits, hipStream_t s) override {
        if (n <= 0) return;
        if (n > cfg_.max_windows) throw std::runtime_error("classify: too many windows");
        run_graph(GraphKey{5, d_tokens, d_logits, n}, s, [&](hipStream_t q) {
            ws_on_ = true;   // one pass on q
            WindowInput in;
            in.tokens = d_tokens;
            in.ldw = (long long)kFrames * kTokenFloats;
            in.pos = pos_;
            in.readout = readout_;
            seq_->run(in, n, d_logits, q, *this, dump_dir_, 0, cur_ws(), ws_floats_);
        });
    }

private:
    hipStream_t setup_ = nullptr;
    // Graphs are captured on this private stream, never on a work stream: another thread may be waiting on an event
    // of the work stream (the scheduler lands one lane while it starts the other), and that wait must not meet a
    // stream in capture mode.
    hipStream_t capture_ = nullptr;
    DevMem wmem_, amem_;
    Uploader* upl_ = nullptr;   // alive while the constructor uploads the weights

    // ---------------------------------------------------------------- weights
    struct Blk {
        BlockCfg cfg{};
        int H = 0, W = 0, Ho = 0, Wo = 0, csq = 0;
        bool has_expand = false, residual = false;
        DevW exp_w;
        const float* exp_b = nullptr;
        const float *dw_w = nullptr, *dw_b = nullptr;
        const float *se1_w = nullptr, *se1_b = nullptr, *se2_w = nullptr, *se2_b = nullptr;
        DevW se1_h, se2_h;   // half tiers: the SE fc weights pre-split for the matrix-core GEMM
        DevW proj_w;
        const float* proj_b = nullptr;
        // fused-kernel operands (half tiers): padded, pre-split weights
        IrShape shp{};
        int tiles_x = 0, ntiles = 0;
        char fam[32] = {};   // profiling family: one per fused-kernel instantiation, "ir_<cin>x<cexp>x<cout>"
        DevW fexp_w, fproj_w;
        const float *fexp_b = nullptr, *fdw_w = nullptr, *fdw_b = nullptr, *fproj_b = nullptr;
    };
    const float *lut_ = nullptr, *stem_w_ = nullptr, *stem_b_ = nullptr;
    Blk blk_[15];
    DevW last_w_;
    const float* last_b_ = nullptr;
    DevW proj_w_;
    const float *pos_ = nullptr, *readout_ = nullptr;
    std::unique_ptr<SeqStack<G>> seq_;   // GDN-A, GDN-B x2, SISA last row, head

    const float* up(const float* src, size_t n) { return upl_->up(src, n); }
    const float* up(const std::vector<float>& v) { return upl_->up(v); }
    // CNN weights: the fp16 tier stores them pre-scaled (a power of two per tensor, undone on the GEMM sums)
    template <typename U> DevW repack(const std::vector<float>& src, int N, int K, int perm) {
        return upl_->repack<U>(src, N, K, perm, false, true);
    }
    template <typename U> DevW repack_pad(const std::vector<float>& src, int N, int K, int Np, int Kp) {
        return upl_->repack_pad<U>(src, N, K, Np, Kp, true);
    }
    const float* up_pad(const std::vector<float>& v, int rows, int n, int np) { return upl_->up_pad(v, rows, n, np); }

    void upload_fused(int i, const BlockHost& b, Blk& d) {
        if constexpr (kF32) {
            (void)i; (void)b; (void)d;
            throw std::runtime_error("fused blocks exist for the half tiers only");
        } else {
        const IrShape sh = ir_shape(i, std::is_same<G, bf16>::value);
        const BlockCfg& c = b.cfg;
        if (sh.cin != c.cin || sh.cexp != c.cexp || sh.cout != c.cout || sh.k != c.k || sh.stride != c.stride ||
            sh.se != c.se || sh.hs != c.hs)
            throw std::runtime_error("fused block table disagrees with the architecture at block " + std::to_string(i));
        d.shp = sh;
        std::snprintf(d.fam, sizeof d.fam, "ir_%dx%dx%d", c.cin, c.cexp, c.cout);
        d.tiles_x = (b.Wo + sh.tw - 1) / sh.tw;
        d.ntiles = d.tiles_x * ((b.Ho + sh.th - 1) / sh.th);
        if (b.has_expand) {
            d.fexp_w = repack_pad<G>(b.expand.w, c.cexp, c.cin, sh.cexpp, sh.cinp);
            d.fexp_b = up_pad(b.expand.b, 1, c.cexp, sh.cexpp);
        }
        d.fdw_w = up_pad(b.dw_w, c.k * c.k, c.cexp, sh.cexpp);
        d.fdw_b = up_pad(b.dw_b, 1, c.cexp, sh.cexpp);
        if (!c.se) {
            d.fproj_w = repack_pad<G>(b.project.w, c.cout, c.cexp, sh.coutp, sh.cexpp);
            d.fproj_b = up_pad(b.project.b, 1, c.cout, sh.coutp);
        }
        }
    }

    void upload_weights(const HostModel& hm) {
        lut_ = up(&hm.lut[0][0], 768);
        stem_w_ = up(hm.stem_w);
        stem_b_ = up(hm.stem_b);
        for (int i = 0; i < 15; ++i) {
            const BlockHost& b = hm.blocks[i];
            Blk& d = blk_[i];
            d.cfg = b.cfg;
            d.H = b.H; d.W = b.W; d.Ho = b.Ho; d.Wo = b.Wo; d.csq = b.csq;
            d.has_expand = b.has_expand;
            d.residual = b.residual;
            if (b.has_expand) {
                d.exp_w = repack<G>(b.expand.w, b.expand.N, b.expand.K, 0);
                d.exp_b = up(b.expand.b);
            }
            d.dw_w = up(b.dw_w);
            d.dw_b = up(b.dw_b);
            if (b.cfg.se) {
                d.se1_w = up(b.se1.w); d.se1_b = up(b.se1.b);
                d.se2_w = up(b.se2.w); d.se2_b = up(b.se2.b);
                if constexpr (!kF32) {
                    d.se1_h = repack<G>(b.se1.w, b.se1.N, b.se1.K, 0);
                    d.se2_h = repack<G>(b.se2.w, b.se2.N, b.se2.K, 0);
                }
            }
            d.proj_w = repack<G>(b.project.w, b.project.N, b.project.K, 0);
            d.proj_b = up(b.project.b);
            if (fused_) upload_fused(i, b, d);
        }
        last_w_ = repack<G>(hm.last.w, hm.last.N, hm.last.K, 0);
        last_b_ = up(hm.last.b);
        proj_w_ = repack<G>(hm.proj.w, hm.proj.N, hm.proj.K, 0);
        pos_ = up(hm.pos);
        readout_ = up(hm.readout);
        // the sequence stages: SHIELD-V arithmetic, 321-token windows, GDN-B residual R + v / sqrt(2)
        static constexpr SeqSpec kVideo{kT, false, 2, {"h0", "after_gdn_a", "after_gdn_b", "after_sisa_last", "logit"}};
        seq_.reset(new SeqStack<G>(kVideo, hm.gdn, hm.sisa, hm.final_norm_w, hm.head0, hm.head2_w, hm.head2_b,
                                   cfg_.max_windows, *upl_, amem_));
    }

    // ---------------------------------------------------------------- activations
    // The CNN's activation buffers.  A pass over frames [f0, f0 + F) uses them from frame f0 on (strides of the
    // largest per-frame size of each buffer), so disjoint frame ranges -- the branches of a forward -- can run at
    // once on their own streams.
    struct Acts {
        float *X, *XB, *E, *D, *PO, *se_part, *se_pool, *se_hid, *se_scale;
    };
    Acts acts_{};
    size_t xe_ = 0, ee_ = 0, de_ = 0, pe_ = 0;   // per-frame floats of X / XB, E, D, se_part
    Acts acts_at(int f0) const {
        const size_t f = size_t(f0);
        Acts a;
        a.X = acts_.X + f * xe_;
        a.XB = acts_.XB ? acts_.XB + f * xe_ : nullptr;
        a.E = acts_.E + f * ee_;
        a.D = acts_.D + f * de_;
        a.PO = acts_.PO + f * 16 * kCnnOut;
        a.se_part = acts_.se_part ? acts_.se_part + f * pe_ : nullptr;
        a.se_pool = acts_.se_pool + f * kCnnOut;
        a.se_hid = acts_.se_hid + f * 256;
        a.se_scale = acts_.se_scale + f * kCnnOut;
        return a;
    }
    bool fused_ = false;
    bool cpu_order_ = false;   // the CNN GEMMs in the reference CPU engine's operation order (fp32 tier)
    // Every encode (encode_direct, the scheduler's encode_slot) runs its frames as up to kBranches independent
    // branches on their own streams (forked from and joined to the caller's stream, inside one graph): while one
    // branch's latency-bound kernels and launch tails run, another's fill the device (measured 21.2 -> 20.2 ms per
    // 128 clips).  forward_direct also runs the sequence stages inside the branches (forward_branched).  Frames and
    // windows are independent rows, so the results are bitwise those of one pass.  Branches of at least 16 clips:
    // the scheduler's 32-clip batches (the reference's default options) then run as two (128 clips end to end from
    // pinned memory 4,977 -> 5,286 clips/s); 8 branches of 16 clips at batch 128 measured 20.7 vs 18.4 ms.
    static constexpr int kBranches = 4, kBranchClips = 16;
    // Exact tier: the workspace of the small-M GEMMs' K-block sums (gemm_f32 with ws).  One per engine, so only a
    // pass that runs alone on its stream hands it out: ws_on_ is set by each pass before it queues its kernels
    // (false for branched passes, whose branches run at once).  32 MB covers every small-M GEMM of one clip.
    static constexpr long long kWsFloats = 8ll << 20;
    float* ws_ = nullptr;
    long long ws_floats_ = 0;
    bool ws_on_ = false;
    float* cur_ws() const { return ws_on_ ? ws_ : nullptr; }
    hipStream_t bstream_[kBranches] = {};
    hipEvent_t fork_ = nullptr, join_[kBranches] = {};
    float* tok_direct_ = nullptr;
    const float** tokptr_direct_ = nullptr;

    void alloc_buffers(const HostModel& hm) {
        const size_t Fm = size_t(cfg_.max_frames), Bm = size_t(cfg_.max_windows);
        size_t xe = size_t(90) * 160 * 16, ee = size_t(60) * kCnnOut, de = 0;
        for (int i = 0; i < 15; ++i) {
            const BlockHost& b = hm.blocks[i];
            xe = std::max(xe, size_t(b.Ho) * b.Wo * b.cfg.cout);
            if (b.has_expand) ee = std::max(ee, size_t(b.H) * b.W * b.cfg.cexp);
            de = std::max(de, size_t(b.Ho) * b.Wo * b.cfg.cexp);
        }
        xe_ = xe;
        ee_ = ee;
        de_ = de;
        acts_.X = amem_.make<float>(Fm * xe);
        if (fused_) {
            acts_.XB = amem_.make<float>(Fm * xe);
            size_t pe = 0;
            for (int i = 0; i < 15; ++i)
                if (blk_[i].cfg.se) pe = std::max(pe, size_t(blk_[i].ntiles) * blk_[i].shp.cexpp);
            pe_ = pe;
            acts_.se_part = amem_.make<float>(Fm * pe);
        }
        acts_.E = amem_.make<float>(Fm * ee);
        acts_.D = amem_.make<float>(Fm * de);
        acts_.PO = amem_.make<float>(Fm * 16 * kCnnOut);
        acts_.se_pool = amem_.make<float>(Fm * kCnnOut);
        acts_.se_hid = amem_.make<float>(Fm * 256);
        acts_.se_scale = amem_.make<float>(Fm * kCnnOut);
        if constexpr (kF32) {
            ws_floats_ = kWsFloats;
            ws_ = amem_.make<float>(size_t(ws_floats_));
        }
        // direct path: the engine's own token buffer and the window -> frame table of a plain predict
        const size_t Fd = std::min(Fm, Bm * kFrames);
        tok_direct_ = amem_.make<float>(Fd * kTokenFloats);
        tokptr_direct_ = amem_.make<const float*>(Bm * kFrames);
        {
            std::vector<const float*> t(Bm * kFrames);
            for (size_t e = 0; e < t.size(); ++e) t[e] = tok_direct_ + (e % Fd) * kTokenFloats;
            SHV_HIP_CHECK(hipMemcpy(tokptr_direct_, t.data(), t.size() * sizeof(float*), hipMemcpyHostToDevice));
        }
        slots_.resize(size_t(cfg_.slots));
        for (Slot& sl : slots_) {
            sl.d_frames = amem_.make<uint8_t>(Fm * kFrameBytes);
            sl.d_tokens = amem_.make<float>(Fm * kTokenFloats);
            sl.d_tok_stage = amem_.make<float>(std::max<size_t>(size_t(cfg_.max_host_tokens), 1) * kTokenFloats);
            sl.d_tokptr = amem_.make<const float*>(Bm * kFrames);
            sl.d_logits = amem_.make<float>(Bm);
            sl.d_store = amem_.make<int32_t>(2 * Fm);
            // every table entry starts valid: padding windows of a bucket read it
            std::vector<const float*> init(Bm * kFrames, sl.d_tokens);
            SHV_HIP_CHECK(hipMemcpy(sl.d_tokptr, init.data(), init.size() * sizeof(float*), hipMemcpyHostToDevice));
            SHV_HIP_CHECK(hipMemset(sl.d_frames, 0, Fm * kFrameBytes));
        }
    }

    // ---------------------------------------------------------------- graphs
    std::map<GraphKey, hipGraphExec_t> graphs_;
    // body(q) issues the pass on stream q: directly on s, or into a graph captured on capture_ and launched on s
    template <class F> void run_graph(const GraphKey& key, hipStream_t s, F&& body) {
        if (!cfg_.use_graphs || !dump_dir_.empty() || profiling()) {
            body(s);
            return;
        }
        auto it = graphs_.find(key);
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

    // ---------------------------------------------------------------- debug dumps (frame 0 / window 0)
    template <typename U> void dump(const char* name, const U* dev, size_t n, hipStream_t s) {
        dump_f32(dump_dir_, name, dev, n, s);
    }

    // GEMM in this engine's flavour, and the exact fp32 VALU kernel for the fp32-only layers
    void gemm(const char* role, const GemmArgs& p, const DevW& w, hipStream_t s) {
        GemmRunner<G>{*this, cur_ws(), ws_floats_, cpu_order_}.gemm(role, p, w, s);
    }
    void gemm32(const char* role, const GemmArgs& p, hipStream_t s) {
        GemmRunner<G>{*this, cur_ws(), ws_floats_, cpu_order_}.gemm32(role, p, s);
    }

    // ---------------------------------------------------------------- CNN
    // F frames as up to kBranches branches of at least kBranchClips clips' frames on the branch streams, forked from
    // and joined to q (one branch when dumping: the dumps show frame 0); one after another on q while profiling, so
    // each kernel is timed alone at the shapes the forward gives it
    // n clips end to end as up to kBranches branches of whole clips (at least kBranchClips each).  Each group of
    // kSeqGroup branches runs its clips' sequence stages on its last branch's stream once the group has encoded, so
    // those stages overlap the other branches' encoders instead of waiting for all of them (windows are independent
    // rows and every kernel choice by batch is bitwise neutral: the logits are those of one pass).  Measured per
    // 128 clips, alternating on one box: per branch 18.48-18.60 ms, per pair 18.67-18.87, after all four 18.92 --
    // the 32-window sequence GEMMs are slower per row than 64-window ones, but the last group's stages, which run
    // with nothing beside them, take half as long.
    static constexpr int kSeqGroup = 1;
    // frames [n * 20] -> tokens [n * 20][6144] -> logits [n], window w reading its frames' tokens through
    // tokptr[w * 20 ..]
    void forward_branched(const uint8_t* frames, float* tokens, const float* const* tokptr, int n, float* logits,
                          hipStream_t q) {
        const int nb = dump_dir_.empty() ? std::max(1, std::min(kBranches, n / kBranchClips)) : 1;
        const bool fork = nb > 1 && !profiling();
        ws_on_ = nb == 1;
        const int sg = std::min(nb, kSeqGroup);
        const auto clip = [&](int b) { return int((long long)n * b / nb); };
        if (fork) SHV_HIP_CHECK(hipEventRecord(fork_, q));
        for (int b = 0; b < nb; ++b) {
            const int c0 = clip(b), c1 = clip(b + 1);
            hipStream_t bs = q;
            if (fork) {
                bs = bstream_[b];
                SHV_HIP_CHECK(hipStreamWaitEvent(bs, fork_, 0));
            }
            const int f0 = c0 * kFrames;
            run_encode(frames + size_t(f0) * kFrameBytes, (c1 - c0) * kFrames, tokens + size_t(f0) * kTokenFloats, bs,
                       acts_at(f0));
            if ((b + 1) % sg == 0 || b == nb - 1) {
                const int g0 = b - b % sg;
                if (fork)
                    for (int bb = g0; bb < b; ++bb) SHV_HIP_CHECK(hipStreamWaitEvent(bs, join_[bb], 0));
                const int w0 = clip(g0);
                run_classify(tokptr + size_t(w0) * kFrames, c1 - w0, logits + w0, bs, w0);
            }
            if (fork) SHV_HIP_CHECK(hipEventRecord(join_[b], bs));
        }
        if (fork)
            for (int b = 0; b < nb; ++b) SHV_HIP_CHECK(hipStreamWaitEvent(q, join_[b], 0));
    }
    void encode_branched(const uint8_t* frames, int F, float* tokens, hipStream_t q) {
        const int nb = dump_dir_.empty() ? std::max(1, std::min(kBranches, F / (kBranchClips * kFrames))) : 1;
        const bool fork = nb > 1 && !profiling();
        ws_on_ = nb == 1;
        if (fork) SHV_HIP_CHECK(hipEventRecord(fork_, q));
        for (int b = 0; b < nb; ++b) {
            const int f0 = int((long long)F * b / nb), f1 = int((long long)F * (b + 1) / nb);
            hipStream_t bs = q;
            if (fork) {
                bs = bstream_[b];
                SHV_HIP_CHECK(hipStreamWaitEvent(bs, fork_, 0));
            }
            run_encode(frames + size_t(f0) * kFrameBytes, f1 - f0, tokens + size_t(f0) * kTokenFloats, bs,
                       acts_at(f0));
            if (fork) SHV_HIP_CHECK(hipEventRecord(join_[b], bs));
        }
        if (fork)
            for (int b = 0; b < nb; ++b) SHV_HIP_CHECK(hipStreamWaitEvent(q, join_[b], 0));
    }

    void run_encode(const uint8_t* frames, int F, float* tokens, hipStream_t s, const Acts& a) {
        if constexpr (!kF32) {
            if (fused_) {
                run_encode_fused(frames, F, tokens, s, a);
                return;
            }
        }
        run_encode_layers(frames, F, tokens, s, a);
    }

    // last 1x1 160 -> 960 + hardswish, 4x4 pool, projection 960 -> 384 (fp32 tokens)
    void run_tail(const float* x, int F, float* tokens, hipStream_t s, const Acts& a) {
        if constexpr (!kF32) {
            if (dump_dir_.empty()) {   // fused last 1x1 + pool (the 60x960 map is dumped only by the unfused path)
                timed("tail_pool", double(F) * (60.0 * 160 + 16.0 * kCnnOut) * TS, s, [&] {
                    launch_tail_pool<G>(x, last_w_.w, last_w_.stride, last_w_.scale, last_b_, a.PO, F, s);
                });
                check_launch();
                GemmArgs p;
                p.M = F * 16; p.N = kD; p.K = kCnnOut;
                p.A = a.PO; p.lda = kCnnOut; p.ldw = kCnnOut;
                p.C = tokens; p.ldc = kD;
                gemm("gemm_pw", p, proj_w_, s);
                return;
            }
        }
        {
            GemmArgs p;
            p.M = F * 60; p.N = kCnnOut; p.K = 160;
            p.A = x; p.lda = 160; p.ldw = 160;
            p.bias = last_b_; p.act = ACT_HS;
            p.C = a.E; p.ldc = kCnnOut;
            gemm("gemm_pw", p, last_w_, s);
        }
        dump("cnn16", a.E, size_t(60) * kCnnOut, s);
        timed("pool", double(F) * (60.0 + 16.0) * kCnnOut * TS, s, [&] { launch_pool<float>(a.E, a.PO, F, s); });
        check_launch();
        {
            GemmArgs p;
            p.M = F * 16; p.N = kD; p.K = kCnnOut;
            p.A = a.PO; p.lda = kCnnOut; p.ldw = kCnnOut;
            p.C = tokens; p.ldc = kD;
            gemm("gemm_pw", p, proj_w_, s);
        }
        dump("tokens", tokens, kTokenFloats, s);
    }

    void se_fc(const Blk& b, int F, hipStream_t s, const Acts& a) {
        GemmArgs p1;
        p1.M = F; p1.N = b.csq; p1.K = b.cfg.cexp;
        p1.A = a.se_pool; p1.lda = b.cfg.cexp; p1.W = b.se1_w; p1.ldw = b.cfg.cexp;
        p1.bias = b.se1_b; p1.act = ACT_RELU;
        p1.C = a.se_hid; p1.ldc = b.csq;
        GemmArgs p2;
        p2.M = F; p2.N = b.cfg.cexp; p2.K = b.csq;
        p2.A = a.se_hid; p2.lda = b.csq; p2.W = b.se2_w; p2.ldw = b.csq;
        p2.bias = b.se2_b; p2.act = ACT_HSIG;
        p2.C = a.se_scale; p2.ldc = b.cfg.cexp;
        if constexpr (kF32) {   // exact reference order
            gemm32("gemm_f32_small", p1, s);
            gemm32("gemm_f32_small", p2, s);
        } else {                // split-operand matrix cores, like every other 1x1 layer of the half tiers
            gemm("gemm_se_fc", p1, b.se1_h, s);
            gemm("gemm_se_fc", p2, b.se2_h, s);
        }
    }

    // half tiers: one fused kernel per block (SE blocks: fused expand + depthwise, SE, project GEMM)
    void run_encode_fused(const uint8_t* frames, int F, float* tokens, hipStream_t s, const Acts& ctx) {
        // the stem runs inside block 1's strip kernel unless its output is to be dumped (or SHV_HIP_NO_STEM_FUSE)
        const bool stem_fused = strip_kernels_enabled() && dump_dir_.empty() && !std::getenv("SHV_HIP_NO_STEM_FUSE");
        if (!stem_fused) {
            timed("stem", double(F) * (kFrameBytes + 90.0 * 160 * 16 * TS), s,
                  [&] { launch_stem<float>(frames, ctx.X, lut_, stem_w_, stem_b_, F, s); });
            check_launch();
            dump("cnn00", ctx.X, size_t(90) * 160 * 16, s);
        }
        float* cur = ctx.X;
        float* nxt = ctx.XB;
        for (int i = 0; i < 15; ++i) {
            const Blk& b = blk_[i];
            const BlockCfg& c = b.cfg;
            const long long HWi = (long long)b.H * b.W, HWo = (long long)b.Ho * b.Wo;
            // multiply-adds of the fused kernel: expand, depthwise, and (non-SE blocks) project
            const double mac = double(F) * ((b.has_expand ? double(HWi) * c.cin * c.cexp : 0.0) +
                                            double(HWo) * c.cexp * c.k * c.k +
                                            (c.se ? 0.0 : double(HWo) * c.cexp * c.cout));
            IrArgs a;
            a.X = cur;
            a.H = b.H; a.W = b.W; a.Ho = b.Ho; a.Wo = b.Wo;
            a.tiles_x = b.tiles_x; a.ntiles = b.ntiles; a.frames = F;
            a.wexp = b.fexp_w.w; a.wexp_stride = b.fexp_w.stride; a.bexp = b.fexp_b; a.sexp = b.fexp_w.scale;
            a.wdw = b.fdw_w; a.bdw = b.fdw_b;
            if (!c.se) {
                a.wproj = b.fproj_w.w; a.wproj_stride = b.fproj_w.stride; a.bproj = b.fproj_b;
                a.sproj = b.fproj_w.scale;
                a.Y = nxt;
                if (i == 0 && stem_fused) {
                    a.X = nullptr;
                    a.img = frames; a.lut = lut_; a.stem_w = stem_w_; a.stem_b = stem_b_;
                    timed("stem_ir_16x16x16", double(F) * (kFrameBytes + HWo * c.cout * TS), s,
                          [&] { launch_stem_block1<G>(a, F, s); }, 2.0 * (mac + double(F) * 90 * 160 * 16 * 27));
                } else {
                    timed(b.fam, double(F) * (HWi * c.cin + HWo * c.cout) * TS, s,
                          [&] { launch_ir_block<G>(i, a, F, s); }, 2.0 * mac);
                }
                check_launch();
            } else {
                a.D = ctx.D; a.part = ctx.se_part;
                timed(b.fam, double(F) * (HWi * c.cin + HWo * c.cexp + double(b.ntiles) * b.shp.cexpp) * TS, s,
                      [&] { launch_ir_block<G>(i, a, F, s); }, 2.0 * mac);
                check_launch();
                timed("se_reduce", double(F) * (double(b.ntiles) * b.shp.cexpp + c.cexp) * TS, s, [&] {
                    launch_se_reduce(ctx.se_part, b.ntiles, b.shp.cexpp, c.cexp, int(HWo), ctx.se_pool, F, s);
                });
                check_launch();
                se_fc(b, F, s, ctx);
                GemmArgs p;
                p.M = int(F * HWo); p.N = c.cout; p.K = c.cexp;
                p.A = ctx.D; p.lda = c.cexp; p.ldw = c.cexp;
                p.bias = b.proj_b;
                p.C = nxt; p.ldc = c.cout;
                p.scale = ctx.se_scale; p.scale_rows = int(HWo); p.ld_scale = c.cexp;
                if (b.residual) { p.R = cur; p.ldr = c.cout; p.res = 1; }
                gemm("gemm_pw", p, b.proj_w, s);
            }
            std::swap(cur, nxt);
            if (!dump_dir_.empty()) {
                char name[8];
                std::snprintf(name, sizeof name, "cnn%02d", i + 1);
                dump(name, cur, size_t(HWo) * c.cout, s);
            }
        }
        run_tail(cur, F, tokens, s, ctx);
    }

    // exact tier (and SHV_HIP_NO_FUSE): layer by layer
    void run_encode_layers(const uint8_t* frames, int F, float* tokens, hipStream_t s, const Acts& a) {
        timed("stem", double(F) * (kFrameBytes + 90.0 * 160 * 16 * TS), s,
              [&] { launch_stem<float>(frames, a.X, lut_, stem_w_, stem_b_, F, s); });
        check_launch();
        dump("cnn00", a.X, size_t(90) * 160 * 16, s);
        for (int i = 0; i < 15; ++i) {
            const Blk& b = blk_[i];
            const long long HWi = (long long)b.H * b.W, HWo = (long long)b.Ho * b.Wo;
            const int act = b.cfg.hs ? ACT_HS : ACT_RELU;
            const float* dwin = a.X;
            if (b.has_expand) {
                GemmArgs p;
                p.M = int(F * HWi); p.N = b.cfg.cexp; p.K = b.cfg.cin;
                p.A = a.X; p.lda = b.cfg.cin; p.ldw = b.cfg.cin;
                p.bias = b.exp_b; p.act = act;
                p.C = a.E; p.ldc = b.cfg.cexp;
                gemm("gemm_pw", p, b.exp_w, s);
                dwin = a.E;
            }
            timed("dw", double(F) * (HWi + HWo) * b.cfg.cexp * TS, s, [&] {
                launch_dw<float>(dwin, a.D, b.dw_w, b.dw_b, F, b.H, b.W, b.cfg.cexp, b.cfg.k, b.cfg.stride, b.Ho, b.Wo, act, s);
            });
            check_launch();
            if (b.cfg.se) {
                timed("se_pool", double(F) * HWo * b.cfg.cexp * TS, s,
                      [&] { launch_se_pool<float>(a.D, a.se_pool, F, b.Ho, b.Wo, b.cfg.cexp, s); });
                check_launch();
                se_fc(b, F, s, a);
            }
            GemmArgs p;
            p.M = int(F * HWo); p.N = b.cfg.cout; p.K = b.cfg.cexp;
            p.A = a.D; p.lda = b.cfg.cexp; p.ldw = b.cfg.cexp;
            p.bias = b.proj_b;
            p.C = a.X; p.ldc = b.cfg.cout;
            if (b.cfg.se) { p.scale = a.se_scale; p.scale_rows = int(HWo); p.ld_scale = b.cfg.cexp; }
            if (b.residual) { p.R = a.X; p.ldr = b.cfg.cout; p.res = 1; }
            gemm("gemm_pw", p, b.proj_w, s);
            if (!dump_dir_.empty()) {
                char name[8];
                std::snprintf(name, sizeof name, "cnn%02d", i + 1);
                dump(name, a.X, size_t(HWo) * b.cfg.cout, s);
            }
        }
        run_tail(a.X, F, tokens, s, a);
    }

    // ---------------------------------------------------------------- sequence
    // windows [w0, w0 + B) of the sequence buffers
    void run_classify(const float* const* tokptr, int B, float* logits, hipStream_t s, int w0) {
        WindowInput in;
        in.frame_tokens = tokptr;
        in.pos = pos_;
        in.readout = readout_;
        seq_->run(in, B, logits, s, *this, dump_dir_, w0, cur_ws(), ws_floats_);
    }
};

}  // namespace

namespace {
// Device memory for one call, released when the call leaves (by return or exception) once the stream it was used
// on has drained, since kernels queued on it may still read it.
class CallBuffer {
public:
    CallBuffer(size_t bytes, hipStream_t s) : s_(s) { SHV_HIP_CHECK(hipMalloc(&p_, bytes)); }
    ~CallBuffer() {
        (void)hipStreamSynchronize(s_);
        (void)hipFree(p_);
    }
    CallBuffer(const CallBuffer&) = delete;
    CallBuffer& operator=(const CallBuffer&) = delete;
    void* get() const { return p_; }

private:
    void* p_ = nullptr;
    hipStream_t s_;
};
}  // namespace

void run_delta_rule(Precision p, const float* Q, const float* K, const float* V, const float* dec, const float* beta,
                    int n_windows, float* O, int variant, hipStream_t s) {
    const DeltaKernel kern = delta_rule_kernel(p, Q, K, V, dec, beta, n_windows, O, variant);
    if (kern != DeltaKernel::Chunked) {
        launch_delta(Q, K, V, dec, beta, O, n_windows, kern == DeltaKernel::Reference, s);
        SHV_HIP_CHECK(hipGetLastError());
        return;
    }
    const CallBuffer buf(delta_chunk_floats(n_windows) * sizeof(float), s);
    float* work = static_cast<float*>(buf.get());
    if (p == Precision::BF16) launch_delta_chunked<bf16>(Q, K, V, dec, beta, O, work, n_windows, s);
    else if (p == Precision::FP16) launch_delta_chunked<f16>(Q, K, V, dec, beta, O, work, n_windows, s);
    else launch_delta_chunked<float>(Q, K, V, dec, beta, O, work, n_windows, s);
    SHV_HIP_CHECK(hipGetLastError());
    SHV_HIP_CHECK(hipStreamSynchronize(s));
}

PwGemm::PwGemm(Precision p, int N, int K, const float* d_w, hipStream_t s) : prec_(p), N_(N), K_(K) {
    if (N < 1 || K < 1 || !d_w) throw std::runtime_error("gemm: bad weight shape or null weights");
    const int parts = p == Precision::FP32 ? 1 : p == Precision::BF16 ? weight_parts<bf16>() : weight_parts<f16>();
    const size_t esz = p == Precision::FP32 ? 4 : 2;
    wstride_ = (long long)N * K;
    // fp16: the weight pre-scaled by a power of two as the engine stores its 1x1 convolutions (a scaled copy of the
    // caller's weights is repacked from a call-local buffer)
    const float* src = d_w;
    std::vector<float> h;   // held until the stream is synchronised below
    std::unique_ptr<CallBuffer> scaled;
    if (p == Precision::FP16) {
        h.resize(size_t(N) * size_t(K));
        SHV_HIP_CHECK(hipMemcpy(h.data(), d_w, h.size() * sizeof(float), hipMemcpyDeviceToHost));
        const int S = Uploader::prescale_exp<f16>(h);
        if (S != 0) {
            for (float& v : h) v = std::ldexp(v, S);
            scaled.reset(new CallBuffer(h.size() * sizeof(float), s));
            SHV_HIP_CHECK(hipMemcpyAsync(scaled->get(), h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice, s));
            src = static_cast<const float*>(scaled->get());
        }
        wscale_ = std::ldexp(1.0f, -S);
    }
    SHV_HIP_CHECK(hipMalloc(&w_, size_t(parts) * size_t(wstride_) * esz));
    switch (p) {
    case Precision::FP32: launch_repack<float>(src, static_cast<float*>(w_), N, K, 0, 1, s); break;
    case Precision::BF16: launch_repack<bf16>(src, static_cast<bf16*>(w_), N, K, 0, parts, s); break;
    case Precision::FP16: launch_repack<f16>(src, static_cast<f16*>(w_), N, K, 0, parts, s); break;
    }
    const hipError_t le = hipGetLastError();
    const hipError_t se = hipStreamSynchronize(s);
    if (le != hipSuccess || se != hipSuccess) {
        (void)hipFree(w_);
        throw std::runtime_error(std::string("gemm: weight repack failed: ") +
                                 hipGetErrorString(le != hipSuccess ? le : se));
    }
}
PwGemm::~PwGemm() { (void)hipFree(w_); }
void PwGemm::run(const float* A, long long M, const float* bias, int act, float* C, int variant, hipStream_t s) const {
    if (M < 1 || M > (1ll << 30) || !A || !C) throw std::runtime_error("gemm: bad M or null operand");
    // the reference's activation codes (engine/cuda/common.cuh:69) -> this engine's
    static const int kAct[5] = {ACT_NONE, ACT_RELU, ACT_HS, ACT_SILU, ACT_HSIG};
    if (act < 0 || act > 4) throw std::runtime_error("gemm: unknown activation code");
    GemmArgs p;
    p.M = int(M); p.N = N_; p.K = K_;
    p.A = A; p.lda = K_;
    p.W = w_; p.ldw = K_; p.wstride = wstride_; p.wscale = wscale_;
    p.bias = bias; p.act = kAct[act];
    p.C = C; p.ldc = N_;
    if (prec_ == Precision::FP32 && variant == 4) {
        gemm_f32_mfma(p, s);
        SHV_HIP_CHECK(hipGetLastError());
        return;
    }
    if (prec_ == Precision::FP32 && variant == 3) {   // K blocks in parallel: a workspace for this call
        const size_t ws = size_t((K_ + 63) / 64) * size_t(M) * size_t(N_);
        const CallBuffer buf(ws * sizeof(float), s);
        p.ws = static_cast<float*>(buf.get());
        p.ws_floats = (long long)ws;
        gemm_f32_variant(p, s, variant);
        SHV_HIP_CHECK(hipGetLastError());
        SHV_HIP_CHECK(hipStreamSynchronize(s));
        return;
    }
    switch (prec_) {
    case Precision::FP32: gemm_f32_variant(p, s, variant); break;
    case Precision::BF16: gemm_mfma_variant<bf16>(p, s, variant); break;
    case Precision::FP16: gemm_mfma_variant<f16>(p, s, variant); break;
    }
    SHV_HIP_CHECK(hipGetLastError());
}

// One engine flavour per precision: the exact VALU tier, or the split-operand MFMA tiers with two (fp16) or three
// (bf16) operand parts.
template <typename G> std::unique_ptr<Engine> engine_of(const HostModel& hm, Precision p, const EngineConfig& cfg) {
    return std::unique_ptr<Engine>(new EngineT<G>(hm, p, cfg));
}

std::unique_ptr<Engine> make_engine(const HostModel& hm, Precision p, const EngineConfig& cfg) {
    using Factory = std::unique_ptr<Engine> (*)(const HostModel&, Precision, const EngineConfig&);
    struct Flavour { Precision p; Factory make; };
    static const Flavour flavours[] = {{Precision::FP32, engine_of<float>},
                                       {Precision::BF16, engine_of<bf16>},
                                       {Precision::FP16, engine_of<f16>}};
    for (const Flavour& f : flavours)
        if (f.p == p) return f.make(hm, p, cfg);
    throw std::runtime_error("engine: no kernel flavour for precision code " + std::to_string(int(p)));
}

}  // namespace shv
