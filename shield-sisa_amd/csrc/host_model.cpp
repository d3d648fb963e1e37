// SHLDV001 loader: strict parsing (engine/cuda/model.cpp:137-179 and engine/model/runtime.cpp:95-134 state the
// format rules), sidecar validation (engine/cuda/api.cu:397-421, engine/model/runtime.cpp:139-166), BatchNorm
// folding in double (runtime.cpp:188-203) and the fused host layouts of the sequence stages (runtime.cpp:329-428).
// Compiled with -ffp-contract=off: the position table must be float32 (time + row) + col without contraction.
#include "host_model.hpp"

#include "sha256.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iterator>
#include <map>
#include <memory>
#include <stdexcept>
#include <unordered_map>

namespace shv {

const BlockCfg kBlocks[15] = {
    {16, 3, 16, 16, 0, 0, 1},    {16, 3, 64, 24, 0, 0, 2},    {24, 3, 72, 24, 0, 0, 1},
    {24, 5, 72, 40, 1, 0, 2},    {40, 5, 120, 40, 1, 0, 1},   {40, 5, 120, 40, 1, 0, 1},
    {40, 3, 240, 80, 0, 1, 2},   {80, 3, 200, 80, 0, 1, 1},   {80, 3, 184, 80, 0, 1, 1},
    {80, 3, 184, 80, 0, 1, 1},   {80, 3, 480, 112, 1, 1, 1},  {112, 3, 672, 112, 1, 1, 1},
    {112, 5, 672, 160, 1, 1, 2}, {160, 5, 960, 160, 1, 1, 1}, {160, 5, 960, 160, 1, 1, 1}};

namespace {

// ------------------------------------------------------------------------------------------ SHLDV001 / SHLDA001
// container: the 8-byte magic, u32 tensor count, then per tensor: u32 name length, name bytes, u32 rank, u32 dims[rank],
// u64 element count, fp32 values (little endian); nothing after the last tensor (tools/export_v.py:3-8;
// the audio file alike, engine/audio/weights.cpp:16-48).
class Cursor {
public:
    Cursor(const std::vector<uint8_t>& buf) : p_(buf.data()), end_(buf.data() + buf.size()) {}
    const uint8_t* bytes(size_t n, const char* what) {
        if (size_t(end_ - p_) < n) throw std::runtime_error(std::string("weights: truncated file (") + what + ")");
        const uint8_t* at = p_;
        p_ += n;
        return at;
    }
    template <class U> U number(const char* what) {
        U v;
        std::memcpy(&v, bytes(sizeof v, what), sizeof v);
        return v;
    }
    bool done() const { return p_ == end_; }

private:
    const uint8_t* p_;
    const uint8_t* end_;
};

// Every tensor of the file, by name; each must be claimed exactly once with its expected shape.
class Weights {
public:
    Weights(const std::string& path, const char* magic) {
        std::ifstream in(path, std::ios::binary | std::ios::ate);
        if (!in) throw std::runtime_error("cannot open weights: " + path);
        const std::streamoff size = in.tellg();
        file_.resize(size_t(size));
        in.seekg(0);
        if (size > 0 && !in.read(reinterpret_cast<char*>(file_.data()), size))
            throw std::runtime_error("cannot read weights: " + path);
        uint8_t digest[32];
        char hex[65];
        shv_sha256 h;
        shv_sha256_init(&h);
        shv_sha256_update(&h, file_.data(), file_.size());
        shv_sha256_final(&h, digest);
        shv_sha256_hex(digest, hex);
        sha_ = hex;
        index(path, magic);
    }
    const std::string& sha256() const { return sha_; }
    size_t file_bytes() const { return file_.size(); }

    // the values of `name`, which must have exactly the shape `dims`
    std::vector<float> take(const std::string& name, std::initializer_list<int> dims) {
        Entry& e = find(name);
        if (!std::equal(e.dims.begin(), e.dims.end(), dims.begin(), dims.end()))
            throw std::runtime_error("weights: tensor " + name + " has shape " + shape_text(e.dims.begin(), e.dims.end()) +
                                     ", expected " + shape_text(dims.begin(), dims.end()));
        e.claimed = true;
        std::vector<float> v(e.count);
        std::memcpy(v.data(), e.data, e.count * sizeof(float));
        return v;
    }
    // the leading dimension of `name` (for widths the file decides, e.g. the SE squeeze)
    int leading(const std::string& name) {
        Entry& e = find(name);
        if (e.dims.empty()) throw std::runtime_error("weights: tensor " + name + " is a scalar");
        return e.dims[0];
    }
    void expect_all_claimed() const {
        for (const auto& kv : table_)
            if (!kv.second.claimed) throw std::runtime_error("weights: unexpected tensor " + kv.first);
    }

private:
    struct Entry {
        std::vector<int> dims;
        const uint8_t* data = nullptr;   // unaligned fp32 values inside file_
        size_t count = 0;
        bool claimed = false;
    };
    std::vector<uint8_t> file_;
    std::string sha_;
    std::unordered_map<std::string, Entry> table_;

    template <class It> static std::string shape_text(It b, It e) {
        std::string s = "[";
        for (It i = b; i != e; ++i) s += (i == b ? "" : ",") + std::to_string(*i);
        return s + "]";
    }
public:
    bool has(const std::string& name) const { return table_.count(name) != 0; }

private:
    Entry& find(const std::string& name) {
        auto it = table_.find(name);
        if (it == table_.end()) throw std::runtime_error("weights: missing tensor " + name);
        return it->second;
    }
    void index(const std::string& path, const char* magic) {
        Cursor c(file_);
        if (std::memcmp(c.bytes(8, "magic"), magic, 8) != 0)
            throw std::runtime_error(std::string("weights: not a ") + magic + " file: " + path);
        const uint32_t n = c.number<uint32_t>("tensor count");
        if (n < 1 || n > 10000) throw std::runtime_error("weights: invalid tensor count");
        uint64_t values = 0;
        for (uint32_t t = 0; t < n; ++t) {
            const uint32_t len = c.number<uint32_t>("name length");
            if (len < 1 || len > 4096) throw std::runtime_error("weights: invalid tensor name length");
            const uint8_t* nm = c.bytes(len, "name");
            std::string name(reinterpret_cast<const char*>(nm), len);
            const uint32_t rank = c.number<uint32_t>("rank");
            if (rank > 8) throw std::runtime_error("weights: invalid tensor rank");
            Entry e;
            uint64_t count = 1;
            for (uint32_t d = 0; d < rank; ++d) {
                const uint32_t dim = c.number<uint32_t>("shape");
                if (dim < 1 || dim > 10000000u || count * dim > 100000000u)
                    throw std::runtime_error("weights: invalid shape of " + name);
                count *= dim;
                e.dims.push_back(int(dim));
            }
            if (c.number<uint64_t>("element count") != count)
                throw std::runtime_error("weights: invalid tensor size of " + name);
            values += count;
            if (values > 100000000u) throw std::runtime_error("weights: invalid tensor size of " + name);
            e.count = size_t(count);
            e.data = c.bytes(e.count * sizeof(float), name.c_str());
            for (size_t i = 0; i < e.count; ++i) {
                float v;
                std::memcpy(&v, e.data + i * sizeof(float), sizeof v);
                if (!std::isfinite(v)) throw std::runtime_error("weights: non-finite value in " + name);
            }
            if (!table_.emplace(std::move(name), std::move(e)).second)
                throw std::runtime_error("weights: duplicate tensor " + std::string(reinterpret_cast<const char*>(nm), len));
        }
        if (!c.done()) throw std::runtime_error("weights: trailing data after the last tensor");
    }
};

// ------------------------------------------------------------------------------------------ sidecar JSON
// The top-level members of a JSON object: strings and numbers kept, nested values skipped.
class JsonTop {
public:
    explicit JsonTop(const std::string& text) : s_(text) {
        ws();
        expect('{');
        ws();
        if (peek() == '}') return;
        for (;;) {
            ws();
            const std::string key = string_value();
            ws();
            expect(':');
            ws();
            const char c = peek();
            if (c == '"') strings_[key] = string_value();
            else if (c == '-' || (c >= '0' && c <= '9')) numbers_[key] = number_value();
            else skip_value();
            ws();
            if (peek() == ',') { ++i_; continue; }
            expect('}');
            return;
        }
    }
    const std::string* str(const std::string& k) const {
        auto it = strings_.find(k);
        return it == strings_.end() ? nullptr : &it->second;
    }
    bool has(const std::string& k) const { return numbers_.count(k) || strings_.count(k); }
    const double* num(const std::string& k) const {
        auto it = numbers_.find(k);
        return it == numbers_.end() ? nullptr : &it->second;
    }

private:
    const std::string& s_;
    size_t i_ = 0;
    std::map<std::string, std::string> strings_;
    std::map<std::string, double> numbers_;

    char peek() const { return i_ < s_.size() ? s_[i_] : '\0'; }
    void ws() {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t')) ++i_;
    }
    void expect(char c) {
        if (peek() != c) throw std::runtime_error(std::string("malformed JSON (expected '") + c + "')");
        ++i_;
    }
    std::string string_value() {
        expect('"');
        std::string out;
        while (i_ < s_.size() && s_[i_] != '"') {
            char c = s_[i_++];
            if (c == '\\') {
                if (i_ >= s_.size()) break;
                const char e = s_[i_++];
                if (e == 'u') { i_ += 4; c = '?'; }   // keys and values used here are ASCII
                else c = e == 'n' ? '\n' : e == 't' ? '\t' : e == 'r' ? '\r' : e == 'b' ? '\b' : e == 'f' ? '\f' : e;
            }
            out.push_back(c);
        }
        expect('"');
        return out;
    }
    double number_value() {
        const char* b = s_.c_str() + i_;
        char* e = nullptr;
        const double v = std::strtod(b, &e);
        if (e == b) throw std::runtime_error("malformed JSON number");
        i_ += size_t(e - b);
        return v;
    }
    void skip_value() {
        const char c = peek();
        if (c == '"') { string_value(); return; }
        if (c == '{' || c == '[') {
            const char close = c == '{' ? '}' : ']';
            ++i_;
            ws();
            if (peek() == close) { ++i_; return; }
            for (;;) {
                ws();
                if (c == '{') { string_value(); ws(); expect(':'); ws(); }
                skip_value();
                ws();
                if (peek() == ',') { ++i_; continue; }
                expect(close);
                return;
            }
        }
        if (c == '-' || (c >= '0' && c <= '9')) { number_value(); return; }
        for (const char* lit : {"true", "false", "null"})
            if (s_.compare(i_, std::strlen(lit), lit) == 0) { i_ += std::strlen(lit); return; }
        throw std::runtime_error("malformed JSON value");
    }
};

// "<weights>.json": output_sha256 must name this file, threshold must be finite in (0, 1).  Returns the threshold.
double check_sidecar(const std::string& weights, const std::string& sha) {
    const std::string path = weights + ".json";
    std::ifstream in(path);
    if (!in) throw std::runtime_error("cannot open " + path + " (threshold)");
    const std::string text((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
    std::unique_ptr<JsonTop> js;
    try {
        js.reset(new JsonTop(text));
    } catch (const std::exception& e) {
        throw std::runtime_error(path + ": " + e.what());
    }
    const std::string* named = js->str("output_sha256");
    if (!named) throw std::runtime_error("no output_sha256 in " + path + " (the sidecar must name its weight file)");
    if (*named != sha)
        throw std::runtime_error(path + " output_sha256 " + *named + " does not match the weights' SHA-256 " + sha +
                                 " (sidecar of another export)");
    if (!js->has("threshold")) throw std::runtime_error("no threshold in " + path);
    const double* t = js->num("threshold");
    if (!t) throw std::runtime_error("bad threshold in " + path);
    if (!(*t > 0.0 && *t < 1.0)) throw std::runtime_error("threshold out of (0,1) in " + path);
    return *t;
}

// conv weight [out][per] followed by BatchNorm2d(eps 1e-3): scale s = gamma / sqrt(var + eps) in double
void fold_bn(Weights& ts, const std::vector<float>& w, int out, int per, const std::string& bn,
             std::vector<float>& wf, std::vector<float>& bf) {
    const auto& g = ts.take(bn + ".weight", {out});
    const auto& beta = ts.take(bn + ".bias", {out});
    const auto& mean = ts.take(bn + ".running_mean", {out});
    const auto& var = ts.take(bn + ".running_var", {out});
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

// Tensor names that differ between the two models' GDN blocks (engine/model/runtime.cpp:329-380 and
// engine/audio/sequence.cpp:299-310); the mixer tensors are named alike.
struct GdnNames { const char *norm, *gate, *up, *down; };
constexpr GdnNames kVideoGdn{"norm.weight", "ffn.gate.weight", "ffn.up.weight", "ffn.down.weight"};
constexpr GdnNames kAudioGdn{"mixer_norm.weight", "ffn.w_gate.weight", "ffn.w_up.weight", "ffn.w_down.weight"};

// One GDN block: in-projection fused [q|k|v|g|a|b] (kGq..kGb), short-conv taps transposed to [tap][1536],
// neg_rate = -expf(A_log).
void load_gdn(Weights& ts, const std::string& p, const GdnNames& nm, GdnHost& G) {
    const std::string x = p + "mixer.";
    G.norm_w = ts.take(p + nm.norm, {kD});
    G.ffn_norm_w = ts.take(p + "ffn_norm.weight", {kD});
    std::vector<float> w(size_t(kGn) * kD, 0.0f);
    auto put = [&](const char* n, int rows, int at) {
        const auto& src = ts.take(x + n, {rows, kD});
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
        const auto& wt = ts.take(x + convs[i] + ".weight", {widths[i], 1, 4});
        const auto& bt = ts.take(x + convs[i] + ".bias", {widths[i]});
        for (int c = 0; c < widths[i]; ++c) {
            for (int j = 0; j < 4; ++j) G.conv_w[size_t(j) * 1536 + offs[i] + c] = wt[size_t(c) * 4 + j];
            G.conv_b[size_t(offs[i]) + c] = bt[c];
        }
    }
    const auto& al = ts.take(x + "A_log", {kHeads});
    const auto& dt = ts.take(x + "dt_bias", {kHeads});
    for (int h = 0; h < kHeads; ++h) {
        G.neg_rate[h] = -expf(al[h]);
        G.dt_bias[h] = dt[h];
    }
    G.o_norm_w = ts.take(x + "o_norm.weight", {kDV});
    G.out = linear(ts.take(x + "o_proj.weight", {kD, kVD}), kD, kVD);
    G.gate = linear(ts.take(p + nm.gate, {kFF, kD}), kFF, kD);
    G.up = linear(ts.take(p + nm.up, {kFF, kD}), kFF, kD);
    G.down = linear(ts.take(p + nm.down, {kD, kFF}), kD, kFF);
}

// The SISA block: all-row projection fused [K|V|B|theta|alpha|forget] with the alpha / forget biases,
// lam = softplus(lambda_raw).  Both models name these tensors alike.
void load_sisa(Weights& ts, SisaHost& S) {
    const std::string a = "sisa.attn.";
    S.attn_norm_w = ts.take("sisa.attn_norm.weight", {kD});
    S.ffn_norm_w = ts.take("sisa.ffn_norm.weight", {kD});
    std::vector<float> w(size_t(kSn) * kD, 0.0f), b(kSn, 0.0f);
    auto put = [&](const char* n, int rows, int at) {
        const auto& src = ts.take(a + n, {rows, kD});
        std::memcpy(&w[size_t(at) * kD], src.data(), sizeof(float) * size_t(rows) * kD);
    };
    put("W_K.weight", 384, kSk);
    put("W_V.weight", 384, kSv);
    put("W_B.weight", 192, kSb);
    put("theta_proj.weight", 96, kSth);
    put("alpha_proj.weight", 6, kSal);
    put("forget_proj.weight", 6, kSfg);
    const auto& ab = ts.take(a + "alpha_proj.bias", {kHeads});
    const auto& fb = ts.take(a + "forget_proj.bias", {kHeads});
    for (int h = 0; h < kHeads; ++h) {
        b[size_t(kSal) + h] = ab[h];
        b[size_t(kSfg) + h] = fb[h];
    }
    S.in = linear(w, kSn, kD, &b);
    S.q = linear(ts.take(a + "W_Q.weight", {kD, kD}), kD, kD);
    S.c = linear(ts.take(a + "W_C.weight", {192, kD}), 192, kD);
    S.o = linear(ts.take(a + "W_O.weight", {kD, kD}), kD, kD);
    const auto& lr = ts.take(a + "lambda_raw", {kHeads});
    for (int h = 0; h < kHeads; ++h) S.lam[h] = softplus_host(lr[h]);
    S.gate = linear(ts.take("sisa.ffn.w_gate.weight", {kFF, kD}), kFF, kD);
    S.up = linear(ts.take("sisa.ffn.w_up.weight", {kFF, kD}), kFF, kD);
    S.down = linear(ts.take("sisa.ffn.w_down.weight", {kD, kFF}), kD, kFF);
}

// Final norm + Linear(384, 128) + Linear(128, 1)
void load_head(Weights& ts, const char* norm, const std::string& out, std::vector<float>& norm_w, Linear& head0,
               std::vector<float>& head2_w, float& head2_b) {
    norm_w = ts.take(norm, {kD});
    const auto& b0 = ts.take("head.0.bias", {128});
    head0 = linear(ts.take("head.0.weight", {128, kD}), 128, kD, &b0);
    head2_w = ts.take(out + ".weight", {1, 128});
    head2_b = ts.take(out + ".bias", {1})[0];
}

}  // namespace

HostModel load_host_model(const std::string& path) {

    HostModel hm;
    hm.path = path;
    Weights ts(path, "SHLDV001");
    hm.sha256 = ts.sha256();
    hm.file_bytes = ts.file_bytes();
    hm.threshold = check_sidecar(path, hm.sha256);

    // uint8 -> ((v / 255) - mean) / std, float32 (runtime.cpp:224-230, prepare_clips)
    const float mean[3] = {0.485f, 0.456f, 0.406f}, stdv[3] = {0.229f, 0.224f, 0.225f};
    for (int c = 0; c < 3; ++c)
        for (int v = 0; v < 256; ++v) {
            volatile float x = float(v) / 255.0f;
            volatile float y = x - mean[c];
            hm.lut[c][v] = y / stdv[c];
        }

    std::vector<float> wf, bf;
    fold_bn(ts, ts.take("cnn.0.0.weight", {16, 3, 3, 3}), 16, 27, "cnn.0.1", wf, bf);
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
            fold_bn(ts, ts.take(p + ".0.weight", {c.cexp, c.cin, 1, 1}), c.cexp, c.cin, p + ".1", wf, bf);
            B.expand = linear(wf, c.cexp, c.cin, &bf);
        }
        {
            const std::string p = pre + std::to_string(j++);
            fold_bn(ts, ts.take(p + ".0.weight", {c.cexp, 1, c.k, c.k}), c.cexp, c.k * c.k, p + ".1", wf, bf);
            B.dw_w.assign(size_t(c.k) * c.k * c.cexp, 0.0f);
            for (int ch = 0; ch < c.cexp; ++ch)
                for (int t = 0; t < c.k * c.k; ++t) B.dw_w[size_t(t) * c.cexp + ch] = wf[size_t(ch) * c.k * c.k + t];
            B.dw_b = bf;
        }
        if (c.se) {
            const std::string p = pre + std::to_string(j++);
            B.csq = ts.leading(p + ".fc1.weight");  // squeeze width from the file (torchvision make_divisible)
            const auto& w1 = ts.take(p + ".fc1.weight", {B.csq, c.cexp, 1, 1});
            const auto& b1 = ts.take(p + ".fc1.bias", {B.csq});
            const auto& w2 = ts.take(p + ".fc2.weight", {c.cexp, B.csq, 1, 1});
            const auto& b2 = ts.take(p + ".fc2.bias", {c.cexp});
            B.se1 = linear(w1, B.csq, c.cexp, &b1);
            B.se2 = linear(w2, c.cexp, B.csq, &b2);
        }
        {
            const std::string p = pre + std::to_string(j++);
            fold_bn(ts, ts.take(p + ".0.weight", {c.cout, c.cexp, 1, 1}), c.cout, c.cexp, p + ".1", wf, bf);
            B.project = linear(wf, c.cout, c.cexp, &bf);
        }
        H = B.Ho;
        W = B.Wo;
    }
    if (H != 6 || W != 10) throw std::runtime_error("internal: unexpected CNN map size");
    fold_bn(ts, ts.take("cnn.16.0.weight", {960, 160, 1, 1}), 960, 160, "cnn.16.1", wf, bf);
    hm.last = linear(wf, 960, 160, &bf);
    hm.proj = linear(ts.take("projection.weight", {kD, 960}), kD, 960);

    {
        const auto& te = ts.take("time_embedding", {20, kD});
        const auto& re = ts.take("row_embedding", {4, kD});
        const auto& ce = ts.take("col_embedding", {4, kD});
        hm.pos.assign(size_t(320) * kD, 0.0f);
        for (int t = 0; t < 20; ++t)
            for (int r = 0; r < 4; ++r)
                for (int c = 0; c < 4; ++c)
                    for (int d = 0; d < kD; ++d) {
                        volatile float a = te[size_t(t) * kD + d] + re[size_t(r) * kD + d];
                        hm.pos[(size_t(t) * 16 + r * 4 + c) * kD + d] = a + ce[size_t(c) * kD + d];
                    }
        hm.readout = ts.take("readout", {1, 1, kD});
    }

    for (int g = 0; g < 2; ++g) load_gdn(ts, g == 0 ? "gdn_a." : "gdn_b.", kVideoGdn, hm.gdn[g]);
    load_sisa(ts, hm.sisa);
    load_head(ts, "final_norm.weight", "head.2", hm.final_norm_w, hm.head0, hm.head2_w, hm.head2_b);

    ts.expect_all_claimed();
    return hm;
}

namespace {

// BatchNorm `bn` of c channels as the reference folds it for its frontend, in float (frontend.cpp:136-144)
void audio_bn(Weights& ts, const std::string& bn, int c, std::vector<float>& scale, std::vector<float>& shift) {
    const auto& g = ts.take(bn + ".weight", {c});
    const auto& beta = ts.take(bn + ".bias", {c});
    const auto& mean = ts.take(bn + ".running_mean", {c});
    const auto& var = ts.take(bn + ".running_var", {c});
    scale.assign(size_t(c), 0.0f);
    shift.assign(size_t(c), 0.0f);
    for (int j = 0; j < c; ++j) {
        const float sd = std::sqrt(var[j] + 1e-5f);
        scale[j] = g[j] / sd;
        const float ms = mean[j] * scale[j];
        shift[j] = beta[j] - ms;
    }
}

// a 1x1 layer [out][in] followed by BatchNorm, the scale folded into the rows and the shift as the bias
Linear audio_pointwise(Weights& ts, const std::string& name, int out, int in) {
    const auto& w = ts.take(name + ".0.weight", {out, in, 1, 1});
    std::vector<float> scale, shift;
    audio_bn(ts, name + ".1", out, scale, shift);
    std::vector<float> wf(w.size());
    for (int o = 0; o < out; ++o)
        for (int k = 0; k < in; ++k) wf[size_t(o) * in + k] = w[size_t(o) * in + k] * scale[o];
    return linear(wf, out, in, &shift);
}

void load_audio_front(Weights& ts, AudioFrontHost& F) {
    constexpr int kBins = 257;
    F.mean = ts.take("frontend.mean", {80});
    F.stdv = ts.take("frontend.std", {80});
    // the export writes the window and the filterbank (engine/audio/export.py:35); without them the reference's
    // own definitions apply (frontend.cpp:127-135): periodic Hann, HTK mel triangles from 20 to 7600 Hz
    if (ts.has("frontend.window")) {
        F.window = ts.take("frontend.window", {400});
    } else {
        F.window.assign(400, 0.0f);
        for (int j = 0; j < 400; ++j) F.window[j] = 0.5f * (1.f - std::cos(float(2. * M_PI * j / 400.)));
    }
    std::vector<float> fb;
    if (ts.has("frontend.fb")) {
        fb = ts.take("frontend.fb", {80, kBins});
    } else {
        fb.assign(size_t(80) * kBins, 0.0f);
        double hz[82];
        const double m0 = 2595. * std::log10(1. + 20. / 700.), m1 = 2595. * std::log10(1. + 7600. / 700.);
        for (int j = 0; j < 82; ++j) hz[j] = 700. * (std::pow(10., (m0 + (m1 - m0) * j / 81.) / 2595.) - 1.);
        for (int m = 0; m < 80; ++m)
            for (int k = 0; k < kBins; ++k)
                fb[size_t(m) * kBins + k] = float(std::max(0., std::min((k * 31.25 - hz[m]) / (hz[m + 1] - hz[m]),
                                                                       (hz[m + 2] - k * 31.25) / (hz[m + 2] - hz[m + 1]))));
    }
    F.fb_off.assign(1, 0);
    for (int m = 0; m < 80; ++m) {
        for (int k = 0; k < kBins; ++k)
            if (fb[size_t(m) * kBins + k] != 0.0f) {
                F.fb_k.push_back(k);
                F.fb_w.push_back(fb[size_t(m) * kBins + k]);
            }
        F.fb_off.push_back(int(F.fb_k.size()));
    }
    F.wr.assign(256, 0.0f);
    F.wi.assign(256, 0.0f);
    for (int j = 0; j < 256; ++j) {
        F.wr[j] = float(std::cos(-2. * M_PI * j / 512.));
        F.wi[j] = float(std::sin(-2. * M_PI * j / 512.));
    }
    F.stem_w = ts.take("cnn.stem.0.weight", {32, 1, 3, 3});
    audio_bn(ts, "cnn.stem.1", 32, F.stem_scale, F.stem_shift);
    static const int kChannels[4] = {48, 96, 160, 192};
    int ci = 32;
    for (int st = 0; st < 4; ++st)
        for (int b = 0; b < 2; ++b) {
            AudioBlockHost& B = F.blocks[st * 2 + b];
            const std::string base = "cnn.stages." + std::to_string(st) + "." + std::to_string(b);
            B.ci = ci;
            B.hid = 2 * ci;
            B.co = kChannels[st];
            B.sf = b == 0 && st < 2 ? 2 : 1;   // frontend.cpp:216-218: stage 0 / 1 first blocks stride 2 in
            B.st = b == 0 && st < 3 ? 2 : 1;   // frequency, stages 0-2 first blocks stride 2 in time
            B.residual = B.ci == B.co && B.sf == 1 && B.st == 1;
            B.pw1 = audio_pointwise(ts, base + ".pw1", B.hid, B.ci);
            const auto& dw = ts.take(base + ".dw.0.weight", {B.hid, 1, 3, 3});
            B.dw_w.assign(size_t(9) * B.hid, 0.0f);
            for (int c = 0; c < B.hid; ++c)
                for (int k = 0; k < 9; ++k) B.dw_w[size_t(k) * B.hid + c] = dw[size_t(c) * 9 + k];
            audio_bn(ts, base + ".dw.1", B.hid, B.dw_scale, B.dw_shift);
            B.pw2 = audio_pointwise(ts, base + ".pw2", B.co, B.hid);
            ci = B.co;
        }
    F.fa_w = ts.take("cnn.freq_attn.weight", {1, 192, 1, 1});
    F.fa_b = ts.take("cnn.freq_attn.bias", {1})[0];
    F.proj = linear(ts.take("cnn.proj.weight", {kD, 192}), kD, 192);
    F.present = true;
}

}  // namespace

AudioHost load_audio_host(const std::string& path) {
    AudioHost ah;
    ah.path = path;
    Weights ts(path, "SHLDA001");
    ah.sha256 = ts.sha256();
    ah.file_bytes = ts.file_bytes();
    ah.readout = ts.take("readout", {1, 1, kD});
    for (int g = 0; g < 2; ++g) load_gdn(ts, g == 0 ? "gdn_a." : "gdn_b.", kAudioGdn, ah.gdn[g]);
    load_sisa(ts, ah.sisa);
    load_head(ts, "head_norm.weight", "head.3", ah.final_norm_w, ah.head0, ah.head2_w, ah.head2_b);
    if (ts.has("frontend.mean")) load_audio_front(ts, ah.front);
    return ah;
}

}  // namespace shv
