// Launchers of the gfx950 kernels (host-callable).  Activations are fp32 in HBM in every mode; the mode only
// selects how GEMM operands reach the multipliers (exact VALU order, or split fp16 / bf16 parts on MFMA).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <type_traits>

#include "host_model.hpp"


namespace shv {

typedef _Float16 f16;   // same storage types as the device code (host-visible)
typedef __bf16 bf16;

// C[m][n] = epilogue(sum_k A[m][k] * W[n][k]); A, C, R fp32 row-major; W row-major [N][K] (PyTorch Linear /
// 1x1 conv layout).  Epilogue, per element in this order: * wscale (the inverse of the power of two a pre-scaled
// weight was stored at; 1 leaves the sum unchanged); + bias[n]; activation; residual (res 1: R + v,
// res 2: R + v / 1.41421356f, res 3: R + 0.70710678f * v); stored fp32.  swiglu: fp32 tier -- W rows (2j, 2j+1) = (gate_j, up_j); MFMA tiers --
// W rows in 16-row panels (gate panel, up panel, ...); out[m][j] = silu(gate) * up.
// Optional SE prologue: A[m][k] := scale[(m / scale_rows) * ld_scale + k] * A[m][k].
// MFMA tiers: W holds the weight's parts (fp16: hi, lo; bf16: hi, mid, lo) wstride elements apart.
struct GemmArgs {
    int M = 0, N = 0, K = 0;
    const float* A = nullptr; long long lda = 0;
    const void* W = nullptr; long long ldw = 0; long long wstride = 0; float wscale = 1.0f;
    const float* scale = nullptr; int scale_rows = 1; int ld_scale = 0;
    const float* bias = nullptr; int act = 0;
    float* C = nullptr; long long ldc = 0;
    const float* R = nullptr; long long ldr = 0; int res = 0;
    int swiglu = 0;
    // MFMA tiers: A given pre-split (parts of the tier's type, part stride astride elements) instead of fp32 A; and a
    // SwiGLU output written pre-split (parts, part stride cstride) instead of fp32 C.  The split is a function of each
    // fp32 value, so both give results bitwise equal to the fp32 forms.
    const void* Ah = nullptr; long long astride = 0;
    void* Ch = nullptr; long long cstride = 0;
    // Layout of each part of the pre-split operands (W, Ah, Ch): element (row, col) at (col / 32) * kstride +
    // row * ld + col % 32 (ld = ldw, lda, ldc).  32 (the default) is plain row-major; group-major operands (ld 32,
    // kstride >= rows * 32: each 16 x 32 fragment block 1 KB contiguous) are read by the small-M, LDS-staged and
    // direct-to-LDS kernels (the sequence GEMMs); the other kernels take the default only.
    long long wkstride = 32, akstride = 32, ckstride = 32;
    // Exact tier: device workspace of ws_floats floats the GEMM may use for its K-block sums when M is small (the
    // caller guarantees no other launch uses it meanwhile); null: never.
    float* ws = nullptr; long long ws_floats = 0;
};

// fp32 tier: VALU GEMM, each output accumulated in K blocks of 64 (fma chain from +0 per block, block sums added
// in order) exactly as the reference CPU engine (engine/model/isa_impl.hpp:188-317).
void gemm_f32(const GemmArgs& p, hipStream_t s);
// fp32 tier, all-row sequence GEMMs: v_mfma_f32_16x16x4_f32 (fp32 operands, products and accumulation).  Per
// output, K in steps of 16 dealt round robin over four partial sums (each from +0, in increasing k, four MFMAs per
// step), added as (p0 + p1) + (p2 + p3): the same for every tile, M and batch (row independence).  SwiGLU weights in
// 16-row gate / up panels (repack perm 2).
void gemm_f32_mfma(const GemmArgs& p, hipStream_t s);
std::string gemm_f32_mfma_kernel_name(const GemmArgs& p);
// fp16 / bf16 tiers: MFMA 16x16x32 on split operands (fp16 2 parts / 3 products, bf16 3 parts / 6 products) with
// fp32 accumulation, K consumed in 32-wide steps in increasing order (no split-K): a row's outputs do not depend
// on M, the tile, or other rows.
template <typename T> void gemm_mfma(const GemmArgs& p, hipStream_t s);
// Kernel variants, for the GEMM microbench and its bitwise variant check (every variant performs the same operation
// sequence per output, so all give bitwise equal results).  fp32: 0 automatic, 1 GEMV, 2 tiled, 3 K blocks in
// parallel (needs ws for ceil(K / 64) * M * N floats), 5 narrow (the (K, N) shapes of blocks 1-6 only), 6 column
// chunks (K <= 1024, K % 4 == 0).  MFMA tiers:
// 0 automatic, 1 small-M, 2..6 direct with 1..5 column tiles per wave, 7 LDS-staged 128 x 128, 8 streaming (N <= 160,
// every column in one workgroup; the SE projects' kernel), 9 wide (K <= 256: 64 rows' A split once into LDS, every
// column chunk of them; no SE scale).
void gemm_f32_variant(const GemmArgs& p, hipStream_t s, int variant);
// The kernel (template name) that gemm_f32 / gemm_mfma run for these arguments: the profiler's family names.
std::string gemm_f32_kernel(const GemmArgs& p);
template <typename T> std::string gemm_mfma_kernel(const GemmArgs& p);
template <typename T> void gemm_mfma_variant(const GemmArgs& p, hipStream_t s, int variant);
// half tiers: last 1x1 (x [F*60][160] fp32, pre-split weight parts [960][160], * wscale, + bias, hardswish) fused
// with the 4x4 pool -> pooled [F][16][960] fp32, bitwise equal to gemm_mfma + launch_pool
template <typename T>
void launch_tail_pool(const float* x, const void* w, long long wstride, float wscale, const float* bias,
                      float* pooled, int F, hipStream_t s);
// number of weight parts an MFMA tier stores
template <typename T> constexpr int weight_parts() { return sizeof(T) == 4 ? 1 : (std::is_same<T, bf16>::value ? 3 : 2); }

// ---------------------------------------------------------------- CNN (NHWC)
// uint8 [F][180][320][3] -> T [F][90][160][16]; lut [3][256], w [27][16] (tap (dy,dx,c) major), b [16]
template <typename T>
void launch_stem(const uint8_t* in, T* out, const float* lut, const float* w, const float* b, int F, hipStream_t s);
// depthwise KxK stride S pad (K-1)/2 + bias + act; w [K*K][C], C % 8 == 0
template <typename T>
void launch_dw(const T* in, T* out, const float* w, const float* b, int F, int H, int W, int C, int K, int S, int Ho,
               int Wo, int act, hipStream_t s);
// SE squeeze: pooled[f][c] = mean over the map (row sums left to right, rows in order, / (float)HW)
template <typename T> void launch_se_pool(const T* x, float* pooled, int F, int Ho, int Wo, int C, hipStream_t s);
// 4x4 adaptive average pool of [F][6][10][960] -> [F][16][960]
template <typename T> void launch_pool(const T* in, T* out, int F, hipStream_t s);
// weight repack on the GPU: part q of dst (q < parts, N*K elements apart) holds the q-th rounding residual of
// src[perm(r)][k] in T (T = float: the value itself).  perm 0 identity, 1 SwiGLU pair interleave (rows 2j, 2j+1
// <- gate j, up j of src = [gate; up]), 2 SwiGLU 16-row panel interleave.  Each part row-major [N][K], or with
// group_major (K % 32 == 0) in GemmArgs' group-major layout: (r, k) at (k / 32) * N * 32 + r * 32 + k % 32.
template <typename T>
void launch_repack(const float* src, T* dst, int N, int K, int perm, int parts, hipStream_t s, bool group_major = false);

// padded repack: dst part q is [Np][Kp] (zero outside [N][K]) holding the q-th rounding residual of src [N][K]
template <typename T>
void launch_repack_pad(const float* src, T* dst, int N, int K, int Np, int Kp, int parts, hipStream_t s);

// ---------------------------------------------------------------- fused inverted-residual blocks (half tiers)
// Compile-time shape of block i's fused kernel for the fp16 or bf16 tier (tile; channel counts padded: cinp to 32,
// cexpp to the kernel's chunk width, coutp to 16).
struct IrShape { int cin, cexp, cout, k, stride, se, hs, th, tw, cinp, cexpp, coutp; };
IrShape ir_shape(int block, bool bf16_tier);
// Operands of one fused block over F frames.  Weights are padded and pre-split: wexp parts [cexpp][cinp],
// wproj parts [coutp][cexpp] (wexp_stride / wproj_stride elements apart); bexp, bdw [cexpp]; wdw [k*k][cexpp];
// bproj [coutp].  Non-SE blocks: X [F][H][W][cin] -> Y [F][Ho][Wo][cout] (Y must not alias X).  SE blocks:
// X -> D [F][Ho][Wo][cexp] and part [F][ntiles][cexpp] (per-tile channel sums of D).
struct IrArgs {
    const float* X = nullptr;
    float* Y = nullptr;
    float* D = nullptr;
    float* part = nullptr;
    const void* wexp = nullptr; long long wexp_stride = 0;
    const float* bexp = nullptr;
    const float* wdw = nullptr;
    const float* bdw = nullptr;
    const void* wproj = nullptr; long long wproj_stride = 0;
    const float* bproj = nullptr;
    // powers of two that the expand / project sums are multiplied by before their bias (the inverse of the scale the
    // pre-scaled weight parts were stored at; 1 when they were not)
    float sexp = 1.0f, sproj = 1.0f;
    int H = 0, W = 0, Ho = 0, Wo = 0, tiles_x = 0, ntiles = 0, frames = 0;
    // block 1 with the stem fused in: uint8 frames [F][180][320][3], byte -> float table [3][256], stem weights
    // [27][16] (tap (dy,dx,c) major) and bias [16]; X is then unused
    const uint8_t* img = nullptr;
    const float *lut = nullptr, *stem_w = nullptr, *stem_b = nullptr;
};
template <typename T> void launch_ir_block(int block, const IrArgs& a, int F, hipStream_t s);
// Strip kernels (pixel-per-lane layout): blocks 1-3 one wave per strip, later blocks one workgroup per strip.
// Enabled unless SHV_HIP_NO_STRIP is set (then every block takes the tile kernels).
bool strip_kernels_enabled();
// stem + block 1 in one strip kernel (half tiers): the stem output never reaches HBM; bitwise equal to launch_stem
// followed by block 1's strip kernel
template <typename T> void launch_stem_block1(const IrArgs& a, int F, hipStream_t s);
// the shape of block i's strip kernel when it has one that is not interchangeable with its tile kernel's (the tile
// is then (rows per step, columns per strip), which the SE partial sums are laid out by)
bool ir_strip_shape(int block, bool bf16_tier, IrShape* out);
// launches block i's strip kernel; false when the block has none
template <typename T> bool launch_ir_strip(int block, const IrArgs& a, int F, hipStream_t s);
// SE squeeze from the fused kernel's tile sums: pooled[f][c] = (sum over tiles in order) / (float)hw
void launch_se_reduce(const float* part, int ntiles, int cexpp, int cexp, int hw, float* pooled, int F,
                      hipStream_t s);

// ---------------------------------------------------------------- SHIELD-A frontend (engine/audio/frontend.cpp)
constexpr int kAudioWindowSamples = 160000;              // 10 s of 16 kHz PCM
constexpr int kAudioMelFrames = 997, kAudioMelBins = 80;  // log-mel image [time][freq]
constexpr int kAudioTokensPerWindow = 125;               // CNN time steps = frontend tokens
constexpr int kAudioCnnFreq = 20, kAudioCnnCh = 192;     // CNN output image [125][20][192]
// Device tables of the log-mel step: analysis window [400], FFT twiddles wr, wi [256] (cos, sin of -2 pi k / 512),
// the filterbank's nonzero taps as rows m: entries fb_off[m] .. fb_off[m + 1] of (fb_k, fb_w) in increasing k, and
// the normalisation mean, stdv [80]
struct AudioMelTables {
    const float *window = nullptr, *wr = nullptr, *wi = nullptr;
    const int *fb_off = nullptr, *fb_k = nullptr;
    const float *fb_w = nullptr, *mean = nullptr, *stdv = nullptr;
};
// PCM windows (window w at pcm + w * stride, stride >= 160,000 samples) -> normalised log-mel [n][997][80]
void launch_audio_mel(const float* pcm, long long stride, int n, const AudioMelTables& tb, float* mel, hipStream_t s);
// log-mel [n][997][80] -> stem image [n][997][80][32]: 3x3 conv (w [32][9], tap 3 kf + kt), BatchNorm scale/shift,
// SiLU
void launch_audio_stem(const float* mel, const float* w, const float* scale, const float* shift, float* out, int n,
                       hipStream_t s);
// depthwise 3x3, strides (time st, freq sf) in {1, 2}, padding 1, BatchNorm, SiLU: in [n][T][F][C] ->
// out [n][(T + st - 1) / st][(F + sf - 1) / sf][C]; w [9][C] (tap 3 kf + kt), C % 4 == 0
void launch_audio_dw(const float* in, float* out, const float* w, const float* scale, const float* shift, int n,
                     int T, int F, int C, int st, int sf, hipStream_t s);
// frequency attention: image [n][125][20][192], attention weights w [192] and bias -> pooled [n][125][192]
void launch_audio_freq_pool(const float* h, const float* w, float bias, float* pooled, int n, hipStream_t s);

// ---------------------------------------------------------------- face crops (uint8 RGB, device memory)
struct CropJob {
    const uint8_t* frame;   // native RGB frame (or the I420 Y plane), rows `stride` bytes apart
    int width, height;
    long long stride;
    int x, y, w, h;         // crop rectangle in 320x180 letterbox units (w >= 80, h >= 45)
    const uint8_t *u = nullptr, *v = nullptr;   // I420 chroma planes ((width + 1) / 2 wide)
    long long u_stride = 0, v_stride = 0;
};
// crop i = cv2.resize(canvas(frame_i)[4y:4(y+h), 4x:4(x+w)], (320, 180), INTER_AREA) -> out + i * 172800 (RGB
// frames, or I420 frames converted per pixel); returns after the crops are written (synchronises s)
void native_crops(const CropJob* jobs, int n, uint8_t* out, bool i420, hipStream_t s);

// ---------------------------------------------------------------- sequence (fp32 residual stream)
// Where a batch's windows take their rows: frame_tokens[window * 20 + position] is a frame's 16 x 384 token block
// (SHIELD-V), or token t of window b is at tokens + b * ldw + t * 384 (a SHIELD-V window's 20 frames' tokens back to
// back, ldw 122,880; a SHIELD-A window's 125 tokens).  SHIELD-V (T = 321) adds the position table pos [320][384].
// The last row of every window is the readout vector.
struct WindowInput {
    const float* const* frame_tokens = nullptr;
    const float* pos = nullptr;
    const float* tokens = nullptr;
    long long ldw = 0;
    const float* readout = nullptr;
};
// The residual stream h [B*T][384] of B windows and, in the same pass, its RMSNorm with weights w into out (the
// layout of launch_rmsnorm's output)
template <typename T>
void launch_window_input(const WindowInput& in, const float* w, float* h, T* out, long long ldo, int B, int TT,
                         hipStream_t s, long long pstride = 0, long long kstride = 32);
// out[r] = (x[r] * (1 / sqrt(sum(x^2) / 384 + 1e-6))) * w with the reference's 16-lane sum tree.  T = f16 / bf16:
// out holds the split parts of each value (part stride pstride elements), the pre-split A of the next GEMM, value
// (r, c) of a part at (c / 32) * kstride + r * ldo + c % 32 (GemmArgs' operand layout).
template <typename T>
void launch_rmsnorm(const float* x, long long ldx, const float* w, T* out, long long ldo, int rows, hipStream_t s,
                    long long pstride = 0, long long kstride = 32);
// Every sequence kernel takes the window length T: 321 (SHIELD-V) or 126 (SHIELD-A); others throw.
// short conv4 + SiLU on q|k|v, per-head L2 norm, decay = exp(neg_rate * softplus(a + dt_bias)), beta = sigmoid(b).
// P [rows][2320] -> Q, K [rows][384], V [rows][768], dec, beta [rows][8].  Video: q * (1/sqrt(max(ss,1e-6))) * 0.125;
// audio: q and k * 1/max(sqrt(ss), 1e-12), q unscaled (engine/audio/sequence.cpp:119-124)
// fast: SiLU as silu_fast (the fp16 / bf16 tiers); else the exact tier's Cephes form
void launch_gdn_prep(const float* P, const float* conv_w, const float* conv_b, const float* neg_rate,
                     const float* dt_bias, float* Q, float* K, float* V, float* dec, float* beta, int B,
                     hipStream_t s, int T = kT, bool audio = false, bool fast = false);
// gated delta rule, sequential over T tokens from zero state, fp32; O [rows][768].  exact: the reference's
// 64-key fma chains (fp32 tier); else each column's keys split over 4 lane rows, partial sums added in a fixed order
void launch_delta(const float* Q, const float* K, const float* V, const float* dec, const float* beta, float* O,
                  int B, bool exact, hipStream_t s, int T = kT);
// Half tiers: the same recurrence over chunks of 32 tokens on the split-operand matrix cores (a parallel prep of
// every chunk's state-independent products into `work`, delta_chunk_floats(B, T) floats, then one scan per
// (window, head)); equal to the token-by-token form up to rounding.
size_t delta_chunk_floats(int B, int T = kT);
template <typename T>
void launch_delta_chunked(const float* Q, const float* K, const float* V, const float* dec, const float* beta,
                          float* O, float* work, int B, hipStream_t s, int Tw = kT);
// ((o * rstd) * w) * silu(gate) per (row, head) -> T [rows][768] (T = f16 / bf16: split parts, as launch_rmsnorm,
// with silu_fast; row stride ld, 32-column group stride kstride).
// audio: o * 0.125 first and eps 1e-5 (engine/audio/sequence.cpp:160-171); video eps 1e-6
template <typename T>
void launch_gated_norm(const float* O, const float* P, const float* w, T* out, int rows, hipStream_t s,
                       long long pstride = 0, bool audio = false, long long ld = kVD, long long kstride = 32);
// SISA last-row attention per (window, head): S [rows][1072] (B rotated in place), QC [B][576] -> Y [B][384]
void launch_sisa(float* S, const float* QC, const float* lam, float* Y, int B, hipStream_t s, int T = kT);
// final RMSNorm + Linear(384,128) + activation + Linear(128,1); w0 [128][384]; activation SiLU (video) or
// exact GELU (audio, engine/audio/sequence.cpp:318-330)
void launch_head(const float* X, const float* norm_w, const float* w0, const float* b0, const float* w2, float b2,
                 float* logits, int B, hipStream_t s, bool audio = false);
// Token-slot stores: pairs[2 i] = batch frame, pairs[2 i + 1] = pool slot; the frame's 6144 token floats are
// copied to the slot for every listed pair
void launch_slot_store(const float* tokens, const int32_t* pairs, int n_pairs, float* pool, hipStream_t s);

}  // namespace shv
