// SHIELD-V host model: the parsed and validated SHLDV001 weight file, BatchNorm folded, in plain fp32 host
// layouts.  The engine uploads these arrays once and repacks the GEMM operands on the GPU.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

namespace shv {

constexpr int kImgH = 180, kImgW = 320, kFrames = 20, kTokPerFrame = 16, kD = 384, kT = 321;
constexpr int kTAudio = 126;   // SHIELD-A windows: 125 frontend tokens + the readout (engine/audio/sequence.cpp:19)
constexpr int kHeads = 6, kDK = 64, kDV = 128, kVD = 768, kFF = 960, kPairs = 16, kCnnOut = 960;
constexpr size_t kFrameBytes = size_t(kImgH) * kImgW * 3;   // 172800
constexpr size_t kTokenFloats = size_t(kTokPerFrame) * kD;   // 6144
// fused GDN in-projection columns [q 384 | k 384 | v 768 | g 768 | a 6 | b 6] (engine/model/net.hpp:13)
constexpr int kGq = 0, kGk = 384, kGv = 768, kGg = 1536, kGa = 2304, kGb = 2310, kGn = 2316, kGld = 2320;
// fused SISA all-row projection [K 384 | V 384 | B 192 | theta 96 | alpha 6 | forget 6] (net.hpp:15)
constexpr int kSk = 0, kSv = 384, kSb = 768, kSth = 960, kSal = 1056, kSfg = 1062, kSn = 1068, kSld = 1072;

// MobileNetV3-Large features[1..15] (engine/model/runtime.cpp:212-216)
struct BlockCfg { int cin, k, cexp, cout, se, hs, stride; };
extern const BlockCfg kBlocks[15];

struct Linear {            // y = x W^T (+ b); W row-major [N][K]
    int N = 0, K = 0;
    std::vector<float> w, b;
};

struct BlockHost {
    BlockCfg cfg{};
    int H = 0, W = 0, Ho = 0, Wo = 0, pad = 0, csq = 0;
    bool has_expand = false, residual = false;
    Linear expand, project, se1, se2;
    std::vector<float> dw_w;  // [k*k][cexp]
    std::vector<float> dw_b;  // [cexp]
};

struct GdnHost {
    std::vector<float> norm_w, ffn_norm_w;
    Linear in;                           // [2316][384]
    std::vector<float> conv_w, conv_b;   // conv_w [4 taps][1536] (tap 0 pairs with t-3), conv_b [1536]
    float neg_rate[kHeads] = {}, dt_bias[kHeads] = {};   // neg_rate = -expf(A_log)
    std::vector<float> o_norm_w;         // [128]
    Linear out, gate, up, down;          // o_proj [384][768], ffn gate/up [960][384], down [384][960]
};

struct SisaHost {
    std::vector<float> attn_norm_w, ffn_norm_w;
    Linear in;                           // [1068][384] + bias (alpha/forget biases at 1056/1062)
    Linear q, c, o;                      // W_Q [384][384], W_C [192][384], W_O [384][384]
    float lam[kHeads] = {};              // softplus(lambda_raw)
    Linear gate, up, down;
};

struct HostModel {
    std::string path, sha256;
    double threshold = 0.0;
    size_t file_bytes = 0;
    float lut[3][256] = {};
    std::vector<float> stem_w;           // [27 taps (dy,dx,c)][16]
    std::vector<float> stem_b;           // [16]
    BlockHost blocks[15];
    Linear last;                         // 160 -> 960 (+bias), hardswish
    Linear proj;                         // 960 -> 384, no bias
    std::vector<float> pos;              // [320][384] = (time + row) + col
    std::vector<float> readout;          // [384]
    GdnHost gdn[2];
    SisaHost sisa;
    std::vector<float> final_norm_w;
    Linear head0;                        // 384 -> 128 (+bias)
    std::vector<float> head2_w;          // [128]
    float head2_b = 0.0f;
};

// Parses and validates "path" (every tensor of the architecture present with its shape, finite values, no extra
// tensors, no trailing bytes), hashes it, validates the sidecar "<path>.json" (output_sha256 == file SHA-256,
// threshold finite in (0,1)) and folds BatchNorm (eps 1e-3) in double.  Throws std::runtime_error.
HostModel load_host_model(const std::string& path);

// SHIELD-A's sequence stages (engine/audio/sequence.cpp:290-317): the tensors of a SHLDA001 file that the stages
// read, in the same host layouts as SHIELD-V's (final norm = head_norm, head2 = head.3).  The file's frontend
// tensors are indexed and left alone.  Throws std::runtime_error.
// SHIELD-A frontend (engine/audio/frontend.cpp): log-mel tables, the stem, eight inverted blocks (4 stages x 2),
// frequency attention and the token projection.  BatchNorm is kept as the reference computes it (float scale =
// gamma / sqrt(var + 1e-5f), shift = beta - mean * scale, frontend.cpp:136-144); the 1x1 layers carry it folded into
// their weights (w * scale per output row, bias = shift).
struct AudioBlockHost {
    int ci = 0, hid = 0, co = 0, sf = 1, st = 1;
    bool residual = false;
    Linear pw1, pw2;                                  // [hid][ci], [co][hid], BatchNorm folded
    std::vector<float> dw_w, dw_scale, dw_shift;      // [9][hid] (tap 3 kf + kt), [hid], [hid]
};
struct AudioFrontHost {
    bool present = false;
    std::vector<float> mean, stdv, window, wr, wi;    // [80], [80], [400], [256], [256]
    std::vector<int> fb_off, fb_k;                    // [81], nonzero taps of each filter in increasing k
    std::vector<float> fb_w;
    std::vector<float> stem_w, stem_scale, stem_shift;   // [32][9] (tap 3 kf + kt), [32], [32]
    AudioBlockHost blocks[8];
    std::vector<float> fa_w;                          // [192]
    float fa_b = 0.0f;
    Linear proj;                                      // [384][192]
};

struct AudioHost {
    std::string path, sha256;
    size_t file_bytes = 0;
    AudioFrontHost front;                // present when the file carries the frontend's tensors
    std::vector<float> readout;          // [384]
    GdnHost gdn[2];
    SisaHost sisa;
    std::vector<float> final_norm_w;
    Linear head0;
    std::vector<float> head2_w;
    float head2_b = 0.0f;
};
AudioHost load_audio_host(const std::string& path);

}  // namespace shv
