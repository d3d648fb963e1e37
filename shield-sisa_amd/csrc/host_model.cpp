// SHLDV001 loader: strict parsing (engine/cuda/model.cpp:137-179 and engine/model/runtime.cpp:95-134 state the
// format rules), sidecar validation (engine/cuda/api.cu:397-421, engine/model/runtime.cpp:139-166), BatchNorm
// folding in double (runtime.cpp:188-203) and the fused host layouts of the sequence stages (runtime.cpp:329-428).
// Compiled with -ffp-contract=off: the position table must be float32 (time + row) + col without contraction.
#include "host_model.hpp"

#include "sha256.h"

#include <cmath>
#include <cstring>
#include <fstream>
#include <map>
#include <set>
#include <sstream>
#include <stdexcept>

namespace shv {

const BlockCfg kBlocks[15] = {
    {16, 3, 16, 16, 0, 0, 1},    {16, 3, 64, 24, 0, 0, 2},    {24, 3, 72, 24, 0, 0, 1},
    {24, 5, 72, 40, 1, 0, 2},    {40, 5, 120, 40, 1, 0, 1},   {40, 5, 120, 40, 1, 0, 1},
    {40, 3, 240, 80, 0, 1, 2},   {80, 3, 200, 80, 0, 1, 1},   {80, 3, 184, 80, 0, 1, 1},
    {80, 3, 184, 80, 0, 1, 1},   {80, 3, 480, 112, 1, 1, 1},  {112, 3, 672, 112, 1, 1, 1},
    {112, 5, 672, 160, 1, 1, 2}, {160, 5, 960, 160, 1, 1, 1}, {160, 5, 960, 160, 1, 1, 1}};

namespace {

struct Tensor {
    std::vector<int> shape;
    std::vector<float> data;
};

class TensorSet {
public:
    std::map<std::string, Tensor> all;
    std::set<std::string> taken;

    const std::vector<float>& get(const std::string& name, std::initializer_list<int> shape) {
        auto it = all.find(name);
        if (it == all.end()) throw std::runtime_error("weights: missing tensor " + name);
        if (it->second.shape != std::vector<int>(shape)) {
            std::ostringstream o;
            o << "weights: tensor " << name << " has shape [";
            for (size_t i = 0; i < it->second.shape.size(); ++i) o << (i ? "," : "") << it->second.shape[i];
            o << "], expected [";
            size_t i = 0;
            for (int d : shape) o << (i++ ? "," : "") << d;
            o << "]";
            throw std::runtime_error(o.str());
        }
        taken.insert(name);
        return it->second.data;
    }
    int dim0(const std::string& name) const {
        auto it = all.find(name);
        if (it == all.end() || it->second.shape.empty()) throw std::runtime_error("weights: missing tensor " + name);
        return it->second.shape[0];
    }
};

class Reader {
public:
    explicit Reader(const std::string& path) : in_(path, std::ios::binary) {
        if (!in_) throw std::runtime_error("cannot open weights: " + path);
        shv_sha256_init(&h_);
    }
    void read(void* dst, size_t n, const char* what) {
        in_.read(static_cast<char*>(dst), std::streamsize(n));
        if (size_t(in_.gcount()) != n) throw std::runtime_error(std::string("weights: truncated file (") + what + ")");
        shv_sha256_update(&h_, dst, n);
        bytes_ += n;
    }
    template <class U> U scalar(const char* what) {
        U x{};
        read(&x, sizeof x, what);
        return x;
    }
    bool at_end() { return in_.peek() == std::char_traits<char>::eof(); }
    std::string hex() {
        uint8_t d[32];
        char out[65];
        shv_sha256_final(&h_, d);
        shv_sha256_hex(d, out);
        return out;
    }
    size_t bytes() const { return bytes_; }

private:
    std::ifstream in_;
    shv_sha256 h_{};
    size_t bytes_ = 0;
};

void parse(const std::string& path, TensorSet& ts, std::string& sha, size_t& file_bytes) {
    Reader r(path);
    char magic[8];
    r.read(magic, 8, "magic");
    if (std::memcmp(magic, "SHLDV001", 8)) throw std::runtime_error("weights: not a SHLDV001 file: " + path);
    const uint32_t count = r.scalar<uint32_t>("count");
    if (count == 0 || count > 10000) throw std::runtime_error("weights: invalid tensor count");
    uint64_t total = 0;
    for (uint32_t i = 0; i < count; ++i) {
        const uint32_t nl = r.scalar<uint32_t>("name length");
        if (nl == 0 || nl > 4096) throw std::runtime_error("weights: invalid tensor name length");
        std::string name(nl, '\0');
        r.read(&name[0], nl, "name");
        const uint32_t rank = r.scalar<uint32_t>("rank");
        if (rank > 8) throw std::runtime_error("weights: invalid tensor rank");
        Tensor t;
        uint64_t elements = 1;
        for (uint32_t d = 0; d < rank; ++d) {
            const uint32_t dim = r.scalar<uint32_t>("shape");
            if (dim == 0 || dim > 10000000u || elements > 100000000u / dim)
                throw std::runtime_error("weights: invalid shape of " + name);
            t.shape.push_back(int(dim));
            elements *= dim;
        }
        const uint64_t declared = r.scalar<uint64_t>("element count");
        total += elements;
        if (declared != elements || total > 100000000u) throw std::runtime_error("weights: invalid tensor size of " + name);
        t.data.resize(size_t(elements));
        r.read(t.data.data(), size_t(elements) * sizeof(float), name.c_str());
        for (float v : t.data)
            if (!std::isfinite(v)) throw std::runtime_error("weights: non-finite value in " + name);
        if (!ts.all.emplace(name, std::move(t)).second) throw std::runtime_error("weights: duplicate tensor " + name);
    }
    if (!r.at_end()) throw std::runtime_error("weights: trailing data after the last tensor");
    sha = r.hex();
    file_bytes = r.bytes();
}

std::string json_string(const std::string& s, const std::string& key) {
    const size_t k = s.find("\"" + key + "\"");
    if (k == std::string::npos) return "";
    const size_t c = s.find(':', k);
    if (c == std::string::npos) return "";
    const size_t q0 = s.find('"', c + 1);
    if (q0 == std::string::npos) return "";
    const size_t q1 = s.find('"', q0 + 1);
    if (q1 == std::string::npos) return "";
    return s.substr(q0 + 1, q1 - q0 - 1);
}

double read_sidecar(const std::string& path, const std::string& sha) {
    const std::string jp = path + ".json";
    std::ifstream in(jp);
    if (!in) throw std::runtime_error("cannot open " + jp + " (threshold)");
    std::stringstream ss;
    ss << in.rdbuf();
    const std::string s = ss.str();
    const std::string got = json_string(s, "output_sha256");
    if (got.empty()) throw std::runtime_error("no output_sha256 in " + jp + " (the sidecar must name its weight file)");
    if (got != sha)
        throw std::runtime_error(jp + " output_sha256 " + got + " does not match the weights' SHA-256 " + sha +
                                 " (sidecar of another export)");
    const size_t k = s.find("\"threshold\"");
    if (k == std::string::npos) throw std::runtime_error("no threshold in " + jp);
    const size_t c = s.find(':', k);
    if (c == std::string::npos) throw std::runtime_error("bad threshold in " + jp);
    const char* b = s.c_str() + c + 1;
    char* e = nullptr;
    const double v = std::strtod(b, &e);
    if (e == b) throw std::runtime_error("bad threshold in " + jp);
    if (!(v > 0.0 && v < 1.0)) throw std::runtime_error("threshold out of (0,1) in " + jp);
    return v;
}

// conv weight [out][per] followed by BatchNorm2d(eps 1e-3): scale s = gamma / sqrt(var + eps) in double
void fold_bn(TensorSet& ts, const std::vector<float>& w, int out, int per, const std::string& bn,
             std::vector<float>& wf, std::vector<float>& bf) {
    const auto& g = ts.get(bn + ".weight", {out});
    const auto& beta = ts.get(bn + ".bias", {out});
    const auto& mean = ts.get(bn + ".running_mean", {out});
    const auto& var = ts.get(bn + ".running_var", {out});
    wf.assign(size_t(out) * per, 0.0f);
    bf.assign(size_t(out), 0.0f);
    for (int o = 0; o < out; ++o) {
        const double s = double(g[o]) / std::sqrt(double(var[o]) + 1e-3);
        for (int e = 0; e < per; ++e) wf[size_t(o) * per + e] = float(double(w[size_t(o) * per + e]) * s);
        bf[o] = float(double(beta[o]) - double(mean[o]) * s);
    }
}

Linear linear(const std::vector<float>& w, int N, int K, const std::vector<float>* b = nullptr) {
    Linear L;
    L.N = N;
    L.K = K;
    L.w = w;
    if (b) L.b = *b;
    return L;
}

float softplus_host(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

}  // namespace

std::string sha256_file(const std::string& path) {
    std::ifstream in(path, std::ios::binary);
    if (!in) throw std::runtime_error("cannot open " + path);
    shv_sha256 h;
    shv_sha256_init(&h);
    std::vector<char> buf(1 << 20);
    while (in) {
        in.read(buf.data(), std::streamsize(buf.size()));
        if (in.gcount() > 0) shv_sha256_update(&h, buf.data(), size_t(in.gcount()));
    }
    uint8_t d[32];
    char out[65];
    shv_sha256_final(&h, d);
    shv_sha256_hex(d, out);
    return out;
}

HostModel load_host_model(const std::string& path) {
    HostModel hm;
    hm.path = path;
    TensorSet ts;
    parse(path, ts, hm.sha256, hm.file_bytes);
    hm.threshold = read_sidecar(path, hm.sha256);

    // uint8 -> ((v / 255) - mean) / std, float32 (runtime.cpp:224-230, prepare_clips)
    const float mean[3] = {0.485f, 0.456f, 0.406f}, stdv[3] = {0.229f, 0.224f, 0.225f};
    for (int c = 0; c < 3; ++c)
        for (int v = 0; v < 256; ++v) {
            volatile float x = float(v) / 255.0f;
            volatile float y = x - mean[c];
            hm.lut[c][v] = y / stdv[c];
        }

    std::vector<float> wf, bf;
    fold_bn(ts, ts.get("cnn.0.0.weight", {16, 3, 3, 3}), 16, 27, "cnn.0.1", wf, bf);
    hm.stem_w.assign(27 * 16, 0.0f);
    for (int o = 0; o < 16; ++o)
        for (int c = 0; c < 3; ++c)
            for (int dy = 0; dy < 3; ++dy)
                for (int dx = 0; dx < 3; ++dx) hm.stem_w[((dy * 3 + dx) * 3 + c) * 16 + o] = wf[o * 27 + c * 9 + dy * 3 + dx];
    hm.stem_b = bf;

    int H = 90, W = 160;
    for (int i = 0; i < 15; ++i) {
        const BlockCfg& c = kBlocks[i];
        BlockHost& B = hm.blocks[i];
        B.cfg = c;
        B.pad = (c.k - 1) / 2;
        B.H = H;
        B.W = W;
        B.Ho = (H + 2 * B.pad - c.k) / c.stride + 1;
        B.Wo = (W + 2 * B.pad - c.k) / c.stride + 1;
        B.has_expand = c.cexp != c.cin;
        B.residual = c.stride == 1 && c.cin == c.cout;
        const std::string pre = "cnn." + std::to_string(i + 1) + ".block.";
        int j = 0;
        if (B.has_expand) {
            const std::string p = pre + std::to_string(j++);
            fold_bn(ts, ts.get(p + ".0.weight", {c.cexp, c.cin, 1, 1}), c.cexp, c.cin, p + ".1", wf, bf);
            B.expand = linear(wf, c.cexp, c.cin, &bf);
        }
        {
            const std::string p = pre + std::to_string(j++);
            fold_bn(ts, ts.get(p + ".0.weight", {c.cexp, 1, c.k, c.k}), c.cexp, c.k * c.k, p + ".1", wf, bf);
            B.dw_w.assign(size_t(c.k) * c.k * c.cexp, 0.0f);
            for (int ch = 0; ch < c.cexp; ++ch)
                for (int t = 0; t < c.k * c.k; ++t) B.dw_w[size_t(t) * c.cexp + ch] = wf[size_t(ch) * c.k * c.k + t];
            B.dw_b = bf;
        }
        if (c.se) {
            const std::string p = pre + std::to_string(j++);
            B.csq = ts.dim0(p + ".fc1.weight");  // squeeze width from the file (torchvision make_divisible)
            const auto& w1 = ts.get(p + ".fc1.weight", {B.csq, c.cexp, 1, 1});
            const auto& b1 = ts.get(p + ".fc1.bias", {B.csq});
            const auto& w2 = ts.get(p + ".fc2.weight", {c.cexp, B.csq, 1, 1});
            const auto& b2 = ts.get(p + ".fc2.bias", {c.cexp});
            B.se1 = linear(w1, B.csq, c.cexp, &b1);
            B.se2 = linear(w2, c.cexp, B.csq, &b2);
        }
        {
            const std::string p = pre + std::to_string(j++);
            fold_bn(ts, ts.get(p + ".0.weight", {c.cout, c.cexp, 1, 1}), c.cout, c.cexp, p + ".1", wf, bf);
            B.project = linear(wf, c.cout, c.cexp, &bf);
        }
        H = B.Ho;
        W = B.Wo;
    }
    if (H != 6 || W != 10) throw std::runtime_error("internal: unexpected CNN map size");
    fold_bn(ts, ts.get("cnn.16.0.weight", {960, 160, 1, 1}), 960, 160, "cnn.16.1", wf, bf);
    hm.last = linear(wf, 960, 160, &bf);
    hm.proj = linear(ts.get("projection.weight", {kD, 960}), kD, 960);

    {
        const auto& te = ts.get("time_embedding", {20, kD});
        const auto& re = ts.get("row_embedding", {4, kD});
        const auto& ce = ts.get("col_embedding", {4, kD});
        hm.pos.assign(size_t(320) * kD, 0.0f);
        for (int t = 0; t < 20; ++t)
            for (int r = 0; r < 4; ++r)
                for (int c = 0; c < 4; ++c)
                    for (int d = 0; d < kD; ++d) {
                        volatile float a = te[size_t(t) * kD + d] + re[size_t(r) * kD + d];
                        hm.pos[(size_t(t) * 16 + r * 4 + c) * kD + d] = a + ce[size_t(c) * kD + d];
                    }
        hm.readout = ts.get("readout", {1, 1, kD});
    }

    for (int g = 0; g < 2; ++g) {
        GdnHost& G = hm.gdn[g];
        const std::string p = g == 0 ? "gdn_a." : "gdn_b.";
        const std::string x = p + "mixer.";
        G.norm_w = ts.get(p + "norm.weight", {kD});
        G.ffn_norm_w = ts.get(p + "ffn_norm.weight", {kD});
        std::vector<float> w(size_t(kGn) * kD, 0.0f);
        auto put = [&](const char* n, int rows, int at) {
            const auto& src = ts.get(x + n, {rows, kD});
            std::memcpy(&w[size_t(at) * kD], src.data(), sizeof(float) * size_t(rows) * kD);
        };
        put("q_proj.weight", 384, kGq);
        put("k_proj.weight", 384, kGk);
        put("v_proj.weight", 768, kGv);
        put("g_proj.weight", 768, kGg);
        put("a_proj.weight", 6, kGa);
        put("b_proj.weight", 6, kGb);
        G.in = linear(w, kGn, kD);
        G.conv_w.assign(4 * 1536, 0.0f);
        G.conv_b.assign(1536, 0.0f);
        const char* convs[3] = {"q_conv1d", "k_conv1d", "v_conv1d"};
        const int widths[3] = {384, 384, 768}, offs[3] = {0, 384, 768};
        for (int i = 0; i < 3; ++i) {
            const auto& wt = ts.get(x + convs[i] + ".weight", {widths[i], 1, 4});
            const auto& bt = ts.get(x + convs[i] + ".bias", {widths[i]});
            for (int c = 0; c < widths[i]; ++c) {
                for (int j = 0; j < 4; ++j) G.conv_w[size_t(j) * 1536 + offs[i] + c] = wt[size_t(c) * 4 + j];
                G.conv_b[size_t(offs[i]) + c] = bt[c];
            }
        }
        const auto& al = ts.get(x + "A_log", {kHeads});
        const auto& dt = ts.get(x + "dt_bias", {kHeads});
        for (int h = 0; h < kHeads; ++h) {
            G.neg_rate[h] = -expf(al[h]);
            G.dt_bias[h] = dt[h];
        }
        G.o_norm_w = ts.get(x + "o_norm.weight", {kDV});
        G.out = linear(ts.get(x + "o_proj.weight", {kD, kVD}), kD, kVD);
        G.gate = linear(ts.get(p + "ffn.gate.weight", {kFF, kD}), kFF, kD);
        G.up = linear(ts.get(p + "ffn.up.weight", {kFF, kD}), kFF, kD);
        G.down = linear(ts.get(p + "ffn.down.weight", {kD, kFF}), kD, kFF);
    }

    {
        SisaHost& S = hm.sisa;
        const std::string a = "sisa.attn.";
        S.attn_norm_w = ts.get("sisa.attn_norm.weight", {kD});
        S.ffn_norm_w = ts.get("sisa.ffn_norm.weight", {kD});
        std::vector<float> w(size_t(kSn) * kD, 0.0f), b(kSn, 0.0f);
        auto put = [&](const char* n, int rows, int at) {
            const auto& src = ts.get(a + n, {rows, kD});
            std::memcpy(&w[size_t(at) * kD], src.data(), sizeof(float) * size_t(rows) * kD);
        };
        put("W_K.weight", 384, kSk);
        put("W_V.weight", 384, kSv);
        put("W_B.weight", 192, kSb);
        put("theta_proj.weight", 96, kSth);
        put("alpha_proj.weight", 6, kSal);
        put("forget_proj.weight", 6, kSfg);
        const auto& ab = ts.get(a + "alpha_proj.bias", {kHeads});
        const auto& fb = ts.get(a + "forget_proj.bias", {kHeads});
        for (int h = 0; h < kHeads; ++h) {
            b[size_t(kSal) + h] = ab[h];
            b[size_t(kSfg) + h] = fb[h];
        }
        S.in = linear(w, kSn, kD, &b);
        S.q = linear(ts.get(a + "W_Q.weight", {kD, kD}), kD, kD);
        S.c = linear(ts.get(a + "W_C.weight", {192, kD}), 192, kD);
        S.o = linear(ts.get(a + "W_O.weight", {kD, kD}), kD, kD);
        const auto& lr = ts.get(a + "lambda_raw", {kHeads});
        for (int h = 0; h < kHeads; ++h) S.lam[h] = softplus_host(lr[h]);
        S.gate = linear(ts.get("sisa.ffn.w_gate.weight", {kFF, kD}), kFF, kD);
        S.up = linear(ts.get("sisa.ffn.w_up.weight", {kFF, kD}), kFF, kD);
        S.down = linear(ts.get("sisa.ffn.w_down.weight", {kD, kFF}), kD, kFF);
    }
    hm.final_norm_w = ts.get("final_norm.weight", {kD});
    {
        const auto& b0 = ts.get("head.0.bias", {128});
        hm.head0 = linear(ts.get("head.0.weight", {128, kD}), 128, kD, &b0);
    }
    hm.head2_w = ts.get("head.2.weight", {1, 128});
    hm.head2_b = ts.get("head.2.bias", {1})[0];

    for (const auto& kv : ts.all)
        if (!ts.taken.count(kv.first)) throw std::runtime_error("weights: unexpected tensor " + kv.first);
    return hm;
}

}  // namespace shv
