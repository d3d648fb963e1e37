// Device-side pieces shared by the SHIELD-V engine and the SHIELD-A sequence engine: device memory, weight upload
// and GPU repacking, the GEMM dispatcher with its profiling families, debug dumps, and SeqStack -- the sequence
// stages both models run (GDN-A, GDN-B twice, SISA on the last row, head) on one set of kernels.  Included by the
// HIP sources only.
#pragma once
#include "engine.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <cstdio>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

namespace shv {

inline void check_launch() { SHV_HIP_CHECK(hipGetLastError()); }

// G selects how GEMM operands reach the multipliers: float = fp32 (matrix cores, or the reference's VALU order),
// f16 / bf16 = split-operand MFMA
template <typename G> inline void gemm_t(const GemmArgs& p, hipStream_t s, bool cpu_order);
template <> inline void gemm_t<float>(const GemmArgs& p, hipStream_t s, bool cpu_order) {
    if (cpu_order) gemm_f32(p, s);
    else gemm_f32_mfma(p, s);
}
template <> inline void gemm_t<f16>(const GemmArgs& p, hipStream_t s, bool) { gemm_mfma<f16>(p, s); }
template <> inline void gemm_t<bf16>(const GemmArgs& p, hipStream_t s, bool) { gemm_mfma<bf16>(p, s); }

inline double gemm_bytes(long long M, int N, int K, int ta, int tw, int tc, int tr) {
    return double(M) * K * ta + double(N) * K * tw + double(M) * N * tc + (tr ? double(M) * N * tr : 0.0);
}

// a GEMM weight on the device: `parts` arrays of N*K elements of the flavour's type, `stride` elements apart; each
// row-major [N][K] (ld 0: the caller's ldw), or group-major (ld 32, 32-column groups kstride = N * 32 apart)
struct DevW {
    const void* w = nullptr;
    long long stride = 0;
    long long ld = 0, kstride = 32;
    // the parts hold w * 2^S (exact); the GEMM multiplies its sums by scale = 2^-S (1 unless pre-scaled)
    float scale = 1.0f;
};

// owner of device allocations
class DevMem {
public:
    DevMem() = default;
    DevMem(const DevMem&) = delete;
    DevMem& operator=(const DevMem&) = delete;
    ~DevMem() { release(); }
    void release() {
        for (void* p : ptrs_) (void)hipFree(p);
        ptrs_.clear();
        bytes_ = 0;
    }
    template <class U> U* make(size_t n) {
        void* p = nullptr;
        const size_t bytes = std::max<size_t>(n * sizeof(U), 256);
        SHV_HIP_CHECK(hipMalloc(&p, bytes));
        ptrs_.push_back(p);
        bytes_ += bytes;
        return static_cast<U*>(p);
    }
    size_t bytes() const { return bytes_; }

private:
    std::vector<void*> ptrs_;
    size_t bytes_ = 0;
};

// Weight upload at load time: fp32 arrays copied to `wmem`, GEMM operands converted on the GPU (repack kernels on
// `s`) from fp32 copies in `staging`, which finish() frees.
class Uploader {
public:
    Uploader(DevMem& wmem, hipStream_t s) : wmem_(wmem), s_(s) {}
    const float* up(const float* src, size_t n) {
        float* d = wmem_.make<float>(n);
        SHV_HIP_CHECK(hipMemcpy(d, src, n * sizeof(float), hipMemcpyHostToDevice));
        return d;
    }
    const float* up(const std::vector<float>& v) { return up(v.data(), v.size()); }
    // fp32 [N][K] rows -> device parts of U with a row permutation, converted by the repack kernel on the GPU;
    // group_major: parts in the group-major GEMM operand layout
    // prescale (fp16 parts only): the parts hold w * 2^S with S such that max |w| * 2^S lies in [2^13, 2^14), and
    // DevW::scale = 2^-S.  fp16 has 5 exponent bits: at He-init magnitudes (|w| ~ 0.05) the lo part of an unscaled
    // weight is subnormal, quantised to 2^-24 in absolute terms, so hi + lo holds the weight to ~1e-6 of its size
    // instead of ~2^-22; scaled, both parts of every weight above max |w| * 2^-16 are normal.  A power of two leaves
    // the weight's digits unchanged, and the GEMM's sums scale back exactly.
    template <typename U>
    DevW repack(const std::vector<float>& src, int N, int K, int perm, bool group_major = false,
                bool prescale = false) {
        const int parts = weight_parts<U>();
        const int S = prescale ? prescale_exp<U>(src) : 0;
        float* st = stage(src, S);
        U* d = wmem_.make<U>(size_t(parts) * N * K);
        launch_repack<U>(st, d, N, K, perm, parts, s_, group_major);
        check_launch();
        DevW w{d, (long long)N * K};
        w.scale = std::ldexp(1.0f, -S);
        if (group_major) {
            w.ld = 32;
            w.kstride = (long long)N * 32;
        }
        return w;
    }
    template <typename U>
    DevW repack_pad(const std::vector<float>& src, int N, int K, int Np, int Kp, bool prescale = false) {
        const int parts = weight_parts<U>();
        const int S = prescale ? prescale_exp<U>(src) : 0;
        float* st = stage(src, S);
        U* d = wmem_.make<U>(size_t(parts) * Np * Kp);
        launch_repack_pad<U>(st, d, N, K, Np, Kp, parts, s_);
        check_launch();
        DevW w{d, (long long)Np * Kp};
        w.scale = std::ldexp(1.0f, -S);
        return w;
    }
    // the exponent S of a prescaled repack (0 for the other part types, an all-zero or non-finite tensor)
    template <typename U> static int prescale_exp(const std::vector<float>& src) {
        if (!std::is_same<U, f16>::value) return 0;
        float mx = 0.0f;
        for (float v : src) mx = std::max(mx, std::fabs(v));
        if (!(mx > 0.0f) || !std::isfinite(mx)) return 0;
        int e = 0;
        std::frexp(mx, &e);   // mx in [2^(e-1), 2^e)
        return std::max(-100, std::min(100, 14 - e));
    }
    // [rows][n] -> [rows][np], zero padded
    const float* up_pad(const std::vector<float>& v, int rows, int n, int np) {
        std::vector<float> o(size_t(rows) * np, 0.0f);
        for (int r = 0; r < rows; ++r)
            for (int j = 0; j < n; ++j) o[size_t(r) * np + j] = v[size_t(r) * n + j];
        return up(o);
    }
    // src * 2^S into the staging buffer (exact: a power of two)
    float* stage(const std::vector<float>& src, int S) {
        float* st = staging_.make<float>(src.size());
        if (S == 0) {
            SHV_HIP_CHECK(hipMemcpy(st, src.data(), src.size() * sizeof(float), hipMemcpyHostToDevice));
        } else {
            std::vector<float> v(src.size());
            for (size_t i = 0; i < v.size(); ++i) v[i] = std::ldexp(src[i], S);
            SHV_HIP_CHECK(hipMemcpy(st, v.data(), v.size() * sizeof(float), hipMemcpyHostToDevice));
        }
        return st;
    }
    void finish() {
        SHV_HIP_CHECK(hipStreamSynchronize(s_));
        staging_.release();
    }
    static std::vector<float> concat(const Linear& a, const Linear& b) {
        std::vector<float> v(a.w);
        v.insert(v.end(), b.w.begin(), b.w.end());
        return v;
    }

private:
    DevMem& wmem_;
    DevMem staging_;
    hipStream_t s_;
};

// Debug dump (window 0 / frame 0; debug runs only, it synchronises s): n values at dev, read back on s itself so
// that they are exactly what the launches queued before on s wrote, stored as fp32 in "<dir>/<name>.f32".
template <typename U> void dump_f32(const std::string& dir, const char* name, const U* dev, size_t n, hipStream_t s) {
    if (dir.empty()) return;
    std::vector<U> raw(n);
    SHV_HIP_CHECK(hipMemcpyAsync(raw.data(), dev, n * sizeof(U), hipMemcpyDeviceToHost, s));
    SHV_HIP_CHECK(hipStreamSynchronize(s));
    std::vector<float> vals(raw.begin(), raw.end());
    const std::string path = dir + "/" + name + ".f32";
    std::FILE* fp = std::fopen(path.c_str(), "wb");
    if (!fp) throw std::runtime_error("dump: cannot open " + path);
    const size_t put = n ? std::fwrite(vals.data(), sizeof(float), n, fp) : 0;
    const bool closed = std::fclose(fp) == 0;
    if (put != n || !closed) throw std::runtime_error("dump: short write to " + path);
}

// GEMM launches of one engine flavour G, timed under "<role>:<kernel template>" when profiling
template <typename G> struct GemmRunner {
    static constexpr bool kF32 = std::is_same<G, float>::value;
    Profiler& pf;
    float* ws = nullptr;   // the exact GEMM's small-M workspace (gemm_f32), null when the caller has none free
    long long ws_floats = 0;
    bool cpu_order = false;   // fp32 tier: the reference CPU order instead of the fp32 matrix cores
    std::string family(const char* role, const GemmArgs& p, bool f32) const {
        if (!pf.profiling()) return std::string();
        if constexpr (!kF32) {
            if (!f32) return std::string(role) + ":" + gemm_mfma_kernel<G>(p);
        } else {
            if (!f32 && !cpu_order) return std::string(role) + ":" + gemm_f32_mfma_kernel_name(p);
        }
        return std::string(role) + ":" + gemm_f32_kernel(p);
    }
    // in this flavour's arithmetic; A is read pre-split where the producer wrote parts, else as fp32
    void gemm(const char* role, GemmArgs p, const DevW& w, hipStream_t s) const {
        if constexpr (kF32) {
            p.ws = ws;
            p.ws_floats = ws_floats;
        }
        p.W = w.w;
        p.wstride = w.stride;
        p.wscale = w.scale;
        if (w.ld) {
            p.ldw = w.ld;
            p.wkstride = w.kstride;
        }
        const int abytes = (p.Ah && !kF32) ? int(sizeof(G)) * weight_parts<G>() : 4;
        const double bytes = gemm_bytes(p.M, p.N, p.K, abytes, kF32 ? 4 : int(sizeof(G)) * weight_parts<G>(),
                                        p.swiglu ? (p.Ch ? int(sizeof(G)) * weight_parts<G>() / 2 : 2) : 4,
                                        p.res ? 4 : 0);
        pf.timed(family(role, p, false), bytes, s, [&] { gemm_t<G>(p, s, cpu_order); }, 2.0 * p.M * p.N * p.K);
        check_launch();
    }
    // the exact fp32 VALU kernel (layers kept in fp32 in every tier)
    void gemm32(const char* role, const GemmArgs& p0, hipStream_t s) const {
        GemmArgs p = p0;
        p.ws = ws;
        p.ws_floats = ws_floats;
        pf.timed(family(role, p, true), gemm_bytes(p.M, p.N, p.K, 4, 4, p.swiglu ? 2 : 4, p.res ? 4 : 0), s,
                 [&] { gemm_f32(p, s); }, 2.0 * p.M * p.N * p.K);
        check_launch();
    }
};

// How one model runs the shared sequence stages.
struct SeqSpec {
    int T;               // tokens per window, readout last: 321 (SHIELD-V) or 126 (SHIELD-A)
    bool audio;          // SHIELD-A arithmetic in the GDN prep, gated norm and head kernels
    int gdn_b_res;       // GEMM residual mode of GDN-B's mixer passes: 2 R + v / sqrt(2), 3 R + 0.70710678 v
    const char* dump[5]; // dump names: input, after GDN-A, after GDN-B, SISA last row, logit
};

// The sequence stages on the device: weights, activations for max_windows windows, and the forward from the
// windows' token rows (WindowInput) to one logit per window.  Activations are fp32 in HBM in every tier;
// G picks the GEMM arithmetic (float: exact VALU order; f16 / bf16: split-operand MFMA with the GEMM A operands
// written pre-split by their producers).
template <typename G> class SeqStack {
    static constexpr bool kF32 = std::is_same<G, float>::value;
    static constexpr int kAS = kF32 ? 4 : int(sizeof(G)) * weight_parts<G>();   // bytes per A value

public:
    SeqStack(const SeqSpec& spec, const GdnHost (&gdn)[2], const SisaHost& S, const std::vector<float>& final_norm_w,
             const Linear& head0, const std::vector<float>& head2_w, float head2_b, int max_windows, Uploader& up,
             DevMem& amem)
        : spec_(spec) {
        cpu_order_ = kF32 && f32_cpu_order_requested();
        const int swiglu_perm = cpu_order_ ? 1 : 2;   // VALU pairs (2j, 2j + 1) or MFMA 16-row panels
        for (int g = 0; g < 2; ++g) {
            const GdnHost& gh = gdn[g];
            Gdn& d = gdn_[g];
            d.norm_w = up.up(gh.norm_w);
            d.ffn_norm_w = up.up(gh.ffn_norm_w);
            d.conv_w = up.up(gh.conv_w);
            d.conv_b = up.up(gh.conv_b);
            d.neg_rate = up.up(gh.neg_rate, kHeads);
            d.dt_bias = up.up(gh.dt_bias, kHeads);
            d.o_norm_w = up.up(gh.o_norm_w);
            d.in_w = up.repack<G>(gh.in.w, gh.in.N, gh.in.K, 0, !kF32);
            d.out_w = up.repack<G>(gh.out.w, gh.out.N, gh.out.K, 0, !kF32);
            d.up_w = up.repack<G>(Uploader::concat(gh.gate, gh.up), 2 * kFF, kD, swiglu_perm, !kF32);
            d.down_w = up.repack<G>(gh.down.w, gh.down.N, gh.down.K, 0, !kF32);
        }
        s_attn_norm_ = up.up(S.attn_norm_w);
        s_ffn_norm_ = up.up(S.ffn_norm_w);
        s_in_w_ = up.repack<G>(S.in.w, S.in.N, S.in.K, 0, !kF32);
        s_in_b_ = up.up(S.in.b);
        s_qc_w_ = up.up(Uploader::concat(S.q, S.c));   // [576][384]: W_Q rows then W_C rows
        s_o_w_ = up.up(S.o.w);
        s_up_w_ = static_cast<const float*>(up.repack<float>(Uploader::concat(S.gate, S.up), 2 * kFF, kD, 1).w);
        s_down_w_ = up.up(S.down.w);
        s_lam_ = up.up(S.lam, kHeads);
        fn_w_ = up.up(final_norm_w);
        h_w0_ = up.up(head0.w);
        h_b0_ = up.up(head0.b);
        h_w2_ = up.up(head2_w);
        h_b2_ = head2_b;

        const size_t Bm = size_t(max_windows), Mm = Bm * size_t(spec_.T);
        H_ = amem.make<float>(Mm * kD);
        P_ = amem.make<float>(Mm * kGld);
        Q_ = amem.make<float>(Mm * kD);
        K_ = amem.make<float>(Mm * kD);
        V_ = amem.make<float>(Mm * kVD);
        dec_ = amem.make<float>(Mm * 8);
        beta_ = amem.make<float>(Mm * 8);
        O_ = amem.make<float>(Mm * kVD);
        // half tiers: the chunked delta-rule scan (SHV_HIP_DELTA_SEQ=1 keeps the token-by-token kernel, for A/B runs)
        const char* ds = std::getenv("SHV_HIP_DELTA_SEQ");
        delta_chunked_ = !cpu_order_ && !(ds && *ds && std::strcmp(ds, "0") != 0);
        if (delta_chunked_) dwork_ = amem.make<float>(delta_chunk_floats(int(Bm), spec_.T));
        mrows_ = (long long)Mm;
        if constexpr (kF32) {
            XN_ = amem.make<float>(Mm * kD);
            ON_ = amem.make<float>(Mm * kVD);
            HID_ = amem.make<float>(Mm * kFF);
        } else {
            XNh_ = amem.make<G>(weight_parts<G>() * Mm * kD);
            ONh_ = amem.make<G>(weight_parts<G>() * Mm * kVD);
            HIDh_ = amem.make<G>(weight_parts<G>() * Mm * kFF);
        }
        XL_ = amem.make<float>(Bm * kD);
        QC_ = amem.make<float>(Bm * 576);
        Y_ = amem.make<float>(Bm * kD);
        X1_ = amem.make<float>(Bm * kD);
        X2_ = amem.make<float>(Bm * kD);
        HIDL_ = amem.make<float>(Bm * kFF);
    }

    // the residual stream [max_windows * T][384], from window w0 on
    float* h(int w0 = 0) const { return H_ + size_t(w0) * spec_.T * kD; }

    // B windows read from `in` -> logits[B], in windows [w0, w0 + B) of every buffer (disjoint window ranges can
    // run at once on different streams)
    void run(const WindowInput& in, int B, float* logits, hipStream_t s, Profiler& pf, const std::string& dump_dir,
             int w0 = 0, float* ws = nullptr, long long ws_floats = 0) {
        const int T = spec_.T, M = B * T;
        const GemmRunner<G> gr{pf, ws, ws_floats, cpu_order_};
        const size_t r0 = size_t(w0) * T;   // first row
        float *H = this->H_ + r0 * kD, *P = this->P_ + r0 * kGld, *Q = this->Q_ + r0 * kD,
              *K = this->K_ + r0 * kD, *V = this->V_ + r0 * kVD, *dec = this->dec_ + r0 * 8,
              *beta = this->beta_ + r0 * 8, *O = this->O_ + r0 * kVD;
        float* work = this->dwork_ ? this->dwork_ + delta_chunk_floats(w0, T) : nullptr;
        float *XN = nullptr, *ON = nullptr, *HID = nullptr;
        G *XNh = nullptr, *ONh = nullptr, *HIDh = nullptr;
        if constexpr (kF32) {
            XN = this->XN_ + r0 * kD;
            ON = this->ON_ + r0 * kVD;
            HID = this->HID_ + r0 * kFF;
        } else {
            XNh = this->XNh_ + r0 * 32;
            ONh = this->ONh_ + r0 * 32;
            HIDh = this->HIDh_ + r0 * 32;
        }
        float *XL = this->XL_ + size_t(w0) * kD, *QC = this->QC_ + size_t(w0) * 576, *Y = this->Y_ + size_t(w0) * kD,
              *X1 = this->X1_ + size_t(w0) * kD, *X2 = this->X2_ + size_t(w0) * kD,
              *HIDL = this->HIDL_ + size_t(w0) * kFF;
        // the A operand of a sequence GEMM: fp32 (exact tier) or the producer's split parts (MFMA tiers, group-major)
        const auto set_a = [&](GemmArgs& p, const float* a32, const G* ah, int width) {
            if constexpr (kF32) {
                p.A = a32;
                p.lda = width;
            } else {
                p.Ah = ah;
                p.lda = 32;
                p.akstride = mrows_ * 32;
                p.astride = mrows_ * width;
            }
            (void)a32; (void)ah;
        };
        // the residual stream's RMSNorm into the A operand of the next GEMM
        const auto rmsnorm_all = [&](const float* w) {
            pf.timed("rmsnorm", double(M) * kD * (4 + kAS), s, [&] {
                if constexpr (kF32) launch_rmsnorm<float>(H, kD, w, XN, kD, M, s);
                else launch_rmsnorm<G>(H, kD, w, XNh, 32, M, s, mrows_ * kD, mrows_ * 32);
            });
            check_launch();
        };
        // the windows' rows into h, normalised for GDN-A's in-projection in the same pass
        pf.timed("window_input", double(M) * kD * (4 + 4 + kAS), s, [&] {
            if constexpr (kF32) launch_window_input<float>(in, gdn_[0].norm_w, H, XN, kD, B, T, s);
            else launch_window_input<G>(in, gdn_[0].norm_w, H, XNh, 32, B, T, s, mrows_ * kD, mrows_ * 32);
        });
        check_launch();
        dump_f32(dump_dir, spec_.dump[0], H, size_t(T) * kD, s);
        for (int st = 0; st < 2; ++st) {
            const Gdn& gd = gdn_[st];
            const int reps = st == 0 ? 1 : 2;
            for (int r = 0; r < reps; ++r) {
                if (st || r) rmsnorm_all(gd.norm_w);
                GemmArgs pi;
                pi.M = M; pi.N = kGn; pi.K = kD;
                set_a(pi, XN, XNh, kD); pi.ldw = kD;
                pi.C = P; pi.ldc = kGld;
                gr.gemm("gemm_seq", pi, gd.in_w, s);
                pf.timed("gdn_prep", double(M) * (4.0 * 1548 * 4 + 4.0 * (2 * kD + kVD + 16)), s, [&] {
                    launch_gdn_prep(P, gd.conv_w, gd.conv_b, gd.neg_rate, gd.dt_bias, Q, K, V, dec, beta, B, s,
                                    T, spec_.audio, !kF32);
                });
                check_launch();
                pf.timed("delta", double(M) * 4.0 * (2 * kD + 2 * kVD + 16), s, [&] {
                    if (delta_chunked_) {
                        launch_delta_chunked<G>(Q, K, V, dec, beta, O, work, B, s, T);
                        return;
                    }
                    launch_delta(Q, K, V, dec, beta, O, B, cpu_order_, s, T);
                }, 2.0 * B * T * kHeads * 4.0 * kDK * kDV);   // per token and head: decay, S^T k, k u^T, S^T q
                check_launch();
                pf.timed("gated_norm", double(M) * (4.0 * 2 * kVD + kAS * kVD), s, [&] {
                    if constexpr (kF32) launch_gated_norm<float>(O, P, gd.o_norm_w, ON, M, s, 0, spec_.audio);
                    else launch_gated_norm<G>(O, P, gd.o_norm_w, ONh, M, s, mrows_ * kVD, spec_.audio, 32, mrows_ * 32);
                });
                check_launch();
                GemmArgs po;
                po.M = M; po.N = kD; po.K = kVD;
                set_a(po, ON, ONh, kVD); po.ldw = kVD;
                po.C = H; po.ldc = kD;
                po.R = H; po.ldr = kD; po.res = reps == 2 ? spec_.gdn_b_res : 1;
                gr.gemm("gemm_seq", po, gd.out_w, s);
            }
            rmsnorm_all(gd.ffn_norm_w);
            GemmArgs pu;
            pu.M = M; pu.N = 2 * kFF; pu.K = kD;
            set_a(pu, XN, XNh, kD); pu.ldw = kD;
            pu.swiglu = 1;
            if constexpr (kF32) {
                pu.C = HID;
                pu.ldc = kFF;
            } else {
                pu.Ch = HIDh;
                pu.ldc = 32;
                pu.ckstride = mrows_ * 32;
                pu.cstride = mrows_ * kFF;
            }
            gr.gemm("gemm_seq", pu, gd.up_w, s);
            GemmArgs pd;
            pd.M = M; pd.N = kD; pd.K = kFF;
            set_a(pd, HID, HIDh, kFF); pd.ldw = kFF;
            pd.C = H; pd.ldc = kD;
            pd.R = H; pd.ldr = kD; pd.res = 1;
            gr.gemm("gemm_seq", pd, gd.down_w, s);
            dump_f32(dump_dir, spec_.dump[1 + st], H, size_t(T) * kD, s);
        }
        // SISA block, last row only: all-row K/V/B/theta/alpha/forget projection, last-row Q|C in fp32
        rmsnorm_all(s_attn_norm_);
        GemmArgs pa;
        pa.M = M; pa.N = kSn; pa.K = kD;
        set_a(pa, XN, XNh, kD); pa.ldw = kD;
        pa.bias = s_in_b_;
        pa.C = P; pa.ldc = kSld;
        gr.gemm("gemm_seq", pa, s_in_w_, s);
        const float* hlast = H + size_t(T - 1) * kD;
        const long long ldlast = (long long)T * kD;
        pf.timed("rmsnorm", double(B) * kD * 8, s,
                 [&] { launch_rmsnorm<float>(hlast, ldlast, s_attn_norm_, XL, kD, B, s); });
        check_launch();
        GemmArgs pq;
        pq.M = B; pq.N = 576; pq.K = kD;
        pq.A = XL; pq.lda = kD; pq.W = s_qc_w_; pq.ldw = kD;
        pq.C = QC; pq.ldc = 576;
        gr.gemm32("gemm_f32_small", pq, s);
        pf.timed("sisa", double(B) * T * kSn * 4, s, [&] { launch_sisa(P, QC, s_lam_, Y, B, s, T); });
        check_launch();
        GemmArgs pw;
        pw.M = B; pw.N = kD; pw.K = kD;
        pw.A = Y; pw.lda = kD; pw.W = s_o_w_; pw.ldw = kD;
        pw.C = X1; pw.ldc = kD;
        pw.R = hlast; pw.ldr = ldlast; pw.res = 1;
        gr.gemm32("gemm_f32_small", pw, s);
        pf.timed("rmsnorm", double(B) * kD * 8, s,
                 [&] { launch_rmsnorm<float>(X1, kD, s_ffn_norm_, XL, kD, B, s); });
        check_launch();
        GemmArgs pu;
        pu.M = B; pu.N = 2 * kFF; pu.K = kD;
        pu.A = XL; pu.lda = kD; pu.W = s_up_w_; pu.ldw = kD;
        pu.C = HIDL; pu.ldc = kFF; pu.swiglu = 1;
        gr.gemm32("gemm_f32_small", pu, s);
        GemmArgs pd;
        pd.M = B; pd.N = kD; pd.K = kFF;
        pd.A = HIDL; pd.lda = kFF; pd.W = s_down_w_; pd.ldw = kFF;
        pd.C = X2; pd.ldc = kD;
        pd.R = X1; pd.ldr = kD; pd.res = 1;
        gr.gemm32("gemm_f32_small", pd, s);
        dump_f32(dump_dir, spec_.dump[3], X2, kD, s);
        pf.timed("head", double(B) * kD * 4, s,
                 [&] { launch_head(X2, fn_w_, h_w0_, h_b0_, h_w2_, h_b2_, logits, B, s, spec_.audio); });
        check_launch();
        dump_f32(dump_dir, spec_.dump[4], logits, 1, s);
    }

private:
    SeqSpec spec_;
    struct Gdn {
        const float *norm_w, *ffn_norm_w, *conv_w, *conv_b, *neg_rate, *dt_bias, *o_norm_w;
        DevW in_w, out_w, up_w, down_w;   // up_w: SwiGLU gate/up interleaved, 1920 rows
    };
    Gdn gdn_[2]{};
    const float *s_attn_norm_ = nullptr, *s_ffn_norm_ = nullptr, *s_in_b_ = nullptr, *s_lam_ = nullptr;
    DevW s_in_w_;
    const float *s_qc_w_ = nullptr, *s_o_w_ = nullptr, *s_up_w_ = nullptr, *s_down_w_ = nullptr;
    const float *fn_w_ = nullptr, *h_w0_ = nullptr, *h_b0_ = nullptr, *h_w2_ = nullptr;
    float h_b2_ = 0.0f;

    float *H_ = nullptr, *P_ = nullptr, *Q_ = nullptr, *K_ = nullptr, *V_ = nullptr, *dec_ = nullptr, *beta_ = nullptr,
          *O_ = nullptr;
    float* dwork_ = nullptr;     // half tiers: the chunked delta rule's per-chunk products
    bool delta_chunked_ = false;
    bool cpu_order_ = false;     // fp32 tier in the reference CPU order (f32_cpu_order_requested at load)
    float *XN_ = nullptr, *ON_ = nullptr, *HID_ = nullptr;   // fp32 tier: the sequence GEMMs' A operands
    // MFMA tiers: the same, written pre-split by their producers in the group-major layout (part q, 32-column group
    // j, row r at q * mrows_ * width + j * mrows_ * 32 + r * 32), so that each DMA load of the direct-to-LDS GEMM
    // reads a 16 x 32 fragment block as 1 KB of contiguous memory (the sequence weights are laid out the same way)
    G *XNh_ = nullptr, *ONh_ = nullptr, *HIDh_ = nullptr;
    long long mrows_ = 0;                                     // rows of those buffers
    float *XL_ = nullptr, *QC_ = nullptr, *Y_ = nullptr, *X1_ = nullptr, *X2_ = nullptr, *HIDL_ = nullptr;

};

}  // namespace shv
