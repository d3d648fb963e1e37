// Fused inverted-residual blocks 1-3 of MobileNetV3-Large (3x3 depthwise, ReLU, no squeeze-excite) for the fp16 /
// bf16 tiers, in a pixel-per-lane layout that keeps every intermediate in registers.
//
// Each wave works alone on a column strip of one frame, 16 lanes wide, walking down the map R output rows per
// step.  The expand runs transposed, E^T[ch][px] = Wexp[ch][:] . X^T[:][px], on v_mfma_f32_16x16x16 with split
// operands; its result fragment gives lane (r, g) = (16 g + r) pixel r of the strip and channels 4 g .. 4 g + 3 of
// a 16-channel tile.  In that layout
//   * the depthwise neighbours along x are lanes r - 1 / r + 1 of the same 16-lane row (DPP row shifts), the
//     neighbours along y are other rows held by the same lane, and the tap weights are broadcast from lane t of a
//     register that holds the 9 taps and the bias of the lane row's 4 channels (DPP row_newbcast);
//   * the depthwise result is exactly the B fragment (k = channels 4 g .., column = pixel r) of the projection
//     Y^T = Wproj^T . D^T, whose result is again one pixel per lane with 4 consecutive output channels -- one
//     float4 store into the NHWC output.
// So the expanded tensor never leaves the registers, and nothing but the weights uses LDS.  A 16-lane strip
// yields 14 output columns at stride 1 (lanes 1 .. 14; lanes 0 and 15 only provide the x halo) and 15 at
// stride 2 (the row holds the even input columns in one tile and the odd ones in another; lane 0's odd column is
// the left halo).  Rows outside the map give E = 0 (uniform per step); columns outside the map give E = 0
// because the expand accumulator starts at -inf there (ReLU(-inf) = 0).
//
// Numerics: the same split-operand products as the other fused kernels; expand and project accumulators start
// from their bias, the depthwise chain runs over (dy, dx) in order and adds its bias last.  Per-element results
// therefore differ from the layer path by accumulation rounding only.
#include "dev_common.hpp"
#include "kernels.hpp"
#include "mfma.hpp"

#include <algorithm>
#include <cstdlib>
#include <stdexcept>
#include <type_traits>

namespace shv {
namespace {

constexpr int ST_THREADS = 256;   // 4 independent waves; the workgroup shares the LDS copy of the weights

// Workgroup barrier that waits for LDS traffic only (global loads issued before it stay in flight).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// The expanded values of an input row outside the map (zero).  Made opaque so that the compiler materialises them only
// on that (rare, wave-uniform) path instead of hoisting four register moves per row into the common path.
__device__ __forceinline__ f32x4 zero_rows() {
    f32x4 z = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    asm volatile("" : "+v"(z));
    return z;
}

// v_mfma_f32_16x16x16 fragments (lane l = 16 g + r): A row r, k = 4 g .. 4 g + 3; B column r, k = 4 g ..
// 4 g + 3; C column r, rows 4 g .. 4 g + 3.  Products as in Split<T> (smallest first).
template <typename T> struct Split16;
template <> struct Split16<f16> {
    typedef _Float16 V4 __attribute__((ext_vector_type(4)));
    static __device__ __forceinline__ f32x4 mfma(V4 a, V4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ _Float16 bits(f16 x) { return x; }
};
template <> struct Split16<bf16> {
    typedef short V4 __attribute__((ext_vector_type(4)));
    static __device__ __forceinline__ f32x4 mfma(V4 a, V4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ short bits(bf16 x) { return __builtin_bit_cast(short, x); }
};

// float4 -> the P part fragments (k = the 4 values)
template <typename T> __device__ __forceinline__ void split4(const float4 v, typename Split16<T>::V4* parts) {
    const float x[4] = {v.x, v.y, v.z, v.w};
    uint2 four[Split<T>::P];
    split4_packed<T>(x, four);
#pragma unroll
    for (int q = 0; q < Split<T>::P; ++q) parts[q] = __builtin_bit_cast(typename Split16<T>::V4, four[q]);
}
// acc += W . A over the split products; w = weight parts (A operand), x = activation parts (B operand)
template <typename T>
__device__ __forceinline__ f32x4 mfma_split16(const typename Split16<T>::V4* w, const typename Split16<T>::V4* x,
                                              f32x4 acc) {
#pragma unroll
    for (int i = 0; i < Split<T>::NPROD; ++i) acc = Split16<T>::mfma(w[Split<T>::wp(i)], x[Split<T>::ap(i)], acc);
    return acc;
}

// 8 bytes of LDS -> one part fragment
template <typename T> __device__ __forceinline__ typename Split16<T>::V4 lds_frag(const T* p) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    return __builtin_bit_cast(typename Split16<T>::V4, u);
}

__device__ __forceinline__ float row_shr1(float v) {   // lane r <- lane r - 1 of its 16-lane row (lane 0 <- 0)
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x111, 0xf, 0xf, true));
}
__device__ __forceinline__ float row_shl1(float v) {   // lane r <- lane r + 1 of its 16-lane row (lane 15 <- 0)
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x101, 0xf, 0xf, true));
}

// 3x3 depthwise output: ((e0 w0 + e1 w1) + ... + e8 w8) + bias as an fma chain, with tap t's weight taken from
// lane t and the bias from lane 9 of wv's 16-lane row.  The leading s_nop covers the two wait states a DPP read
// needs after a VALU write of its source register.
__device__ __forceinline__ float dw9(float wv, float e0, float e1, float e2, float e3, float e4, float e5, float e6,
                                     float e7, float e8) {
    float acc;
    asm("s_nop 1\n\t"
        "v_mul_f32_dpp %0, %1, %2 row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %3 row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %4 row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %5 row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %6 row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %7 row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %8 row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %9 row_newbcast:7 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %10 row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %0, %1, %0 row_newbcast:9 row_mask:0xf bank_mask:0xf"
        : "=&v"(acc)
        : "v"(wv), "v"(e0), "v"(e1), "v"(e2), "v"(e3), "v"(e4), "v"(e5), "v"(e6), "v"(e7), "v"(e8));
    return acc;
}

template <int CIN_, int CEXP_, int COUT_, int S_, int R_, int MINB_ = 1>
struct StripCfg {
    static constexpr int CIN = CIN_, CEXP = CEXP_, COUT = COUT_, S = S_, R = R_;
    static constexpr int MINB = MINB_;   // workgroups per CU the register allocation must allow
    static constexpr bool EXPAND = CIN != CEXP;
    static constexpr bool RES = S == 1 && CIN == COUT;
    static constexpr int KSI = (CIN + 15) / 16;              // expand K steps
    static constexpr int CT = (CEXP + 15) / 16;              // expanded-channel tiles
    static constexpr int OT = (COUT + 15) / 16;              // output-channel tiles
    static constexpr int VALID = S == 1 ? 14 : 15;           // output columns per strip (lanes 1 .. VALID)
    static constexpr int NT = S;                             // pixel tiles per input row (stride 2: even, odd)
    static constexpr int IR = S == 1 ? R + 2 : 2 * R + 1;    // input rows per step
    static constexpr int KP = KSI * 16 + 4;                  // LDS row stride (elements) of the expand weights
    static constexpr int CP = CT * 16 + 4;                   // LDS row stride of the project weights
    static_assert(CIN % 4 == 0 && COUT % 4 == 0, "channel counts must be multiples of 4");
    static_assert(EXPAND || (CT == 1 && KSI == 1), "blocks without expand have one 16-channel tile");
};

//                  cin cexp cout s  R  workgroups per CU
typedef StripCfg<16, 16, 16, 1, 6, 3> S1; // 90x160 (three workgroups per CU: stem + block 1 1.72 -> 1.27 ms, 1 spill)
typedef StripCfg<16, 64, 24, 2, 2, 3> S2; // 90x160 -> 45x80 (R 2 in three per CU: 6% slower alone, forward -0.5%)
typedef StripCfg<16, 64, 24, 2, 1> S2B;   // bf16 (R 2 in three per CU spills)
typedef StripCfg<24, 72, 24, 1, 3, 3> S3; // 45x80 (R 3 in 164 VGPRs, three workgroups per CU: 1.12 -> 0.97 ms)
typedef StripCfg<24, 72, 24, 1, 4> S3B;   // bf16 (three operand parts: R 3 in three workgroups per CU spills)

template <typename T, class C> struct StripLds {
    static constexpr int P = Split<T>::P;
    static constexpr int WE = C::EXPAND ? P * C::CT * 16 * C::KP : 0;   // T elements
    static constexpr int WP = P * C::OT * 16 * C::CP;
    static constexpr int BE = C::EXPAND ? 2 * C::CT * 16 : 0;           // floats: expand bias, then -inf
    static constexpr int BYTES = (WE + WP) * (int)sizeof(T) + BE * 4;
};

// Stem fused into block 1 (STEM): per step a wave needs stem rows iy0 .. iy0 + 7 at its 16 columns, i.e. frame rows
// 2 iy0 - 1 .. 2 iy0 + 15 (17) and frame columns 2 x - 1 .. 2 x + 1 of the strip's stem columns x (33 frame pixels).
// The stem convolution runs on the matrix cores in the same transposed form as the expand layers: with the K order
// k = 4 tap + channel (channel 3 a zero pad; taps 9 .. 11 zero weights), the B fragment of lane (r, g) for K chunk
// q is the 4 channels of frame pixel (2 j + dy, 2 r + dx), tap 4 q + g = (dy, dx), and the result fragment is
// already the pixel-per-lane layout of block 1's input rows (pixel r, channels 4 g ..).  The wave stages its frame
// pixels in a private LDS tile [part][17][33][4], each byte mapped through a table that holds the split parts of
// the byte -> float value, so no split arithmetic runs per pixel; pixels outside the frame stage as 0.  Per stem row:
// 3 K chunks x the split products, + bias, hardswish.  Split operands keep fp32-level operand precision; the result
// differs from the fp32 stem kernel by accumulation rounding.  The tile is private to the wave: in-order LDS
// execution plus a wait on the wave's own LDS traffic separates staging from use.
constexpr int STEM_FR = 17, STEM_FC = 33 * 3;    // staged frame rows, bytes per staged row
constexpr int STEM_TILE = STEM_FR * 33 * 4;      // T elements of one part of a wave's tile
// byte -> parts table of one part: the three channels' 256 entries, then 256 zeros that bytes outside the frame
// are looked up in (a row offset chosen per lane and row instead of a select per staged element and part)
constexpr int STEM_LUT = 4 * 256, STEM_ZERO = 3 * 256;
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// Lane l stages byte columns l and l + 64 (the latter for l < STEM_FC - 64) of the step's 17 frame rows.  Addresses
// are clamped into the frame so that every load is unconditional and all are in flight together; bytes outside the
// frame are masked when staged.
constexpr int STEM_NB = 2 * STEM_FR;
__device__ __forceinline__ void stem_fetch(const uint8_t* img, long long f, int fy0, int fb0, int lane,
                                           int (&bytes)[STEM_NB]) {
    const uint8_t* fr = img + f * (180 * 320 * 3);
    // unsigned 32-bit offsets from the frame's (scalar) base address
    const unsigned b0 = min(max(fb0 + lane, 0), 320 * 3 - 1), b1 = min(max(fb0 + lane + 64, 0), 320 * 3 - 1);
#pragma unroll
    for (int u = 0; u < STEM_FR; ++u) {
        const unsigned row = unsigned(min(max(fy0 + u, 0), 179)) * (320 * 3);
        bytes[2 * u] = fr[row + b0];
        bytes[2 * u + 1] = fr[row + b1];
    }
}

template <typename T, class C, bool STEM = false>
// segs: each strip's output rows are dealt over segs items of seg_rows rows (a multiple of R) when frames are few;
// every step reads its own input rows, so the split changes no result.
__global__ void __launch_bounds__(ST_THREADS, C::MINB) ir_strip_kernel(IrArgs a, int strips, int items, int segs, int seg_rows,
                                                              const float* __restrict__ stem_w,
                                                              const float* __restrict__ stem_b) {
    typedef Split16<T> S16;
    typedef typename S16::V4 V4;
    typedef StripLds<T, C> L;
    constexpr int P = Split<T>::P;
    static_assert(!STEM || (!C::EXPAND && C::S == 1 && C::CIN == 16 && C::IR == 8), "the stem feeds block 1 only");
    __shared__ __attribute__((aligned(16))) unsigned char lds_raw[(L::BYTES + 15) / 16 * 16];
    // STEM: the waves' frame tiles [wave][part][STEM_TILE], then the byte -> parts table [part][STEM_LUT]
    __shared__ __attribute__((aligned(16))) T stem_lds[STEM ? (ST_THREADS / 64) * P * STEM_TILE + P * STEM_LUT : 1];
    T* We = reinterpret_cast<T*>(lds_raw);                               // [P][CT*16][KP]
    T* Wp = We + L::WE;                                                  // [P][OT*16][CP]
    float* Be = reinterpret_cast<float*>(lds_raw + (L::WE + L::WP) * sizeof(T));   // [2][CT*16]
    const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: item and frame math stays scalar

    // ---- weights -> LDS (the only workgroup-wide step)
    {
        const T* wexp = static_cast<const T*>(a.wexp);
        const T* wproj = static_cast<const T*>(a.wproj);
        constexpr int CEXPP = (C::CEXP + 31) / 32 * 32, CINP = (C::CIN + 31) / 32 * 32, COUTP = C::OT * 16;
        if constexpr (C::EXPAND) {
            for (int i = tid; i < P * C::CT * 16 * C::KSI * 16; i += ST_THREADS) {
                const int k = i % (C::KSI * 16), rest = i / (C::KSI * 16);
                const int c = rest % (C::CT * 16), q = rest / (C::CT * 16);
                We[(q * C::CT * 16 + c) * C::KP + k] = wexp[q * a.wexp_stride + (long long)c * CINP + k];
            }
            // the expand sums run at the pre-scaled weights' scale 1 / sexp from a bias at that scale (exact:
            // powers of two) and are scaled back before the activation
            const float einv = 1.0f / a.sexp;
            for (int i = tid; i < C::CT * 16; i += ST_THREADS) {
                Be[i] = a.bexp[i] * einv;
                Be[C::CT * 16 + i] = -__builtin_inff();
            }
        }
        for (int i = tid; i < P * COUTP * C::CT * 16; i += ST_THREADS) {
            const int k = i % (C::CT * 16), rest = i / (C::CT * 16);
            const int o = rest % COUTP, q = rest / COUTP;
            Wp[(q * COUTP + o) * C::CP + k] = wproj[q * a.wproj_stride + (long long)o * CEXPP + k];
        }
        (void)CEXPP;
        if constexpr (STEM) {
            for (int i = tid; i < (ST_THREADS / 64) * P * STEM_TILE; i += ST_THREADS) stem_lds[i] = T(0.0f);
            for (int i = tid; i < STEM_LUT; i += ST_THREADS) {
                T part[P];
                Split<T>::split(i < STEM_ZERO ? a.lut[i] : 0.0f, part);
#pragma unroll
                for (int q = 0; q < P; ++q) stem_lds[(ST_THREADS / 64) * P * STEM_TILE + q * STEM_LUT + i] = part[q];
            }
        }
    }
    __syncthreads();
    T* const stile = stem_lds + (STEM ? wave * P * STEM_TILE : 0);
    const T* const stab = stem_lds + (STEM ? (ST_THREADS / 64) * P * STEM_TILE : 0);
    // STEM: stem weight fragments (A row r = output channel r, k = 4 tap + channel), bias, per-lane tile offsets
    V4 sw[STEM ? 3 : 1][P];
    float sbias[4];
    int soff[STEM ? 3 : 1];
    if constexpr (STEM) {
#pragma unroll
        for (int qc = 0; qc < 3; ++qc) {
            const int t = 4 * qc + g;
            float w4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) w4[i] = t < 9 && i < 3 ? stem_w[(t * 3 + i) * 16 + r] : 0.0f;
            split4<T>(make_float4(w4[0], w4[1], w4[2], w4[3]), sw[qc]);
            const int tt = min(t, 8), dy = tt / 3, dx = tt - 3 * dy;   // taps 9 .. 11 read tap 8 (zero weights)
            soff[qc] = (dy * 33 + 2 * r + dx) * 4;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) sbias[i] = stem_b[4 * g + i];
    }

    // ---- per-lane constants: depthwise taps + bias (lane r <= 9 of each row: tap r, bias), project bias.  The
    // expand sums leave the matrix cores at the scale 1 / sexp (a power of two) and go through ReLU unscaled: as
    // relu(sexp * x) = sexp * relu(x) and scaling by a power of two is exact, the taps multiplied by sexp give every
    // depthwise product bitwise the value of scaling each expanded element first, for one multiply per tap register
    // instead of one per element
    constexpr int CEXPP_DW = (C::CEXP + 31) / 32 * 32;
    float wdw[C::CT][4];
    const float tap_scale = C::EXPAND && r < 9 ? a.sexp : 1.0f;
#pragma unroll
    for (int ct = 0; ct < C::CT; ++ct) {
        const int c = ct * 16 + 4 * g;
        const float* src = r < 9 ? a.wdw + r * CEXPP_DW + c : a.bdw + c;
        const float4 v = *reinterpret_cast<const float4*>(src);
        wdw[ct][0] = v.x * tap_scale; wdw[ct][1] = v.y * tap_scale; wdw[ct][2] = v.z * tap_scale;
        wdw[ct][3] = v.w * tap_scale;
    }
    f32x4 pb[C::OT];
#pragma unroll
    for (int ot = 0; ot < C::OT; ++ot) {
        const float4 v = *reinterpret_cast<const float4*>(a.bproj + ot * 16 + 4 * g);
        const float pinv = 1.0f / a.sproj;   // the project sums run at the weights' scale, from the bias at it
        pb[ot] = f32x4{v.x * pinv, v.y * pinv, v.z * pinv, v.w * pinv};
    }

    const int H = a.H, W = a.W, Ho = a.Ho, Wo = a.Wo;
    for (int item = blockIdx.x * (ST_THREADS / 64) + wave; item < items; item += gridDim.x * (ST_THREADS / 64)) {
        const int seg = item % segs, fs = item / segs;
        const int strip = fs % strips;
        const long long f = fs / strips;
        const int oyA = seg * seg_rows, oyB = min(Ho, oyA + seg_rows);   // this item's output rows
        const int ox = strip * C::VALID + r - 1;                   // this lane's output column
        int ixc[C::NT];
        bool pin[C::NT];
#pragma unroll
        for (int t = 0; t < C::NT; ++t) {
            const int ix = C::S == 1 ? ox : 2 * ox + t;
            pin[t] = ix >= 0 && ix < W;
            ixc[t] = min(max(ix, 0), W - 1);
        }
        const bool store_lane = r >= 1 && r <= C::VALID && ox < Wo;
        const float* Xf = a.X + f * H * W * C::CIN;
        float* Yf = a.Y + f * Ho * Wo * C::COUT;
        // expand accumulator start: the bias, or -inf for columns outside the map
        int be_off[C::NT];
#pragma unroll
        for (int t = 0; t < C::NT; ++t) be_off[t] = pin[t] ? 0 : C::CT * 16;

        int sbytes[STEM ? STEM_NB : 1];   // STEM: the step's staged frame bytes
        for (int oy0 = oyA; oy0 < oyB; oy0 += C::R) {
            const int iy0 = C::S * oy0 - 1;
            // ---- the step's input rows: fp32 (no expand) or split into B fragments
            V4 xf[C::EXPAND ? C::IR : 1][C::NT][C::KSI][P];
            float4 xe[C::EXPAND ? 1 : C::IR];
            bool rin[C::IR];
            float4 sx[STEM ? C::IR : 1];   // STEM: the step's stem rows (pixel r, channels 4 g ..)
            if constexpr (STEM) {
                const int fy0 = 2 * iy0 - 1, fb0 = (2 * (strip * C::VALID - 1) - 1) * 3;   // first row, first byte
                if (oy0 == oyA) stem_fetch(a.img, f, fy0, fb0, lane, sbytes);
                wave_lds_sync();   // the previous step's reads of the tile are done
                {
                    const int e1 = lane + 64;
                    const bool c0 = fb0 + lane >= 0 && fb0 + lane < 320 * 3, c1 = e1 < STEM_FC && fb0 + e1 < 320 * 3;
                    // tile slots; lanes past the row's bytes store a zero into a channel-3 pad slot (zero anyway)
                    // rather than branch around the store
                    const int d0 = (lane / 3) * 4 + lane % 3;
                    const int d1 = e1 < STEM_FC ? (e1 / 3) * 4 + e1 % 3 : ((e1 - STEM_FC) % 33) * 4 + 3;
                    // table rows: the byte's channel, or the zeros for bytes outside the frame
                    const int t0 = c0 ? (lane % 3) * 256 : STEM_ZERO, t1 = c1 ? (e1 % 3) * 256 : STEM_ZERO;
#pragma unroll
                    for (int u = 0; u < STEM_FR; ++u) {
                        const bool rin_u = fy0 + u >= 0 && fy0 + u < 180;   // uniform
                        const int i0 = (rin_u ? t0 : STEM_ZERO) + sbytes[2 * u];
                        const int i1 = (rin_u ? t1 : STEM_ZERO) + sbytes[2 * u + 1];
#pragma unroll
                        for (int q = 0; q < P; ++q) {
                            stile[q * STEM_TILE + u * 132 + d0] = stab[q * STEM_LUT + i0];
                            stile[q * STEM_TILE + u * 132 + d1] = stab[q * STEM_LUT + i1];
                        }
                    }
                }
                // the next step's bytes load while this step computes
                if (oy0 + C::R < oyB) stem_fetch(a.img, f, fy0 + 2 * C::R, fb0, lane, sbytes);
                wave_lds_sync();
#pragma unroll
                for (int j = 0; j < C::IR; ++j) {
                    f32x4 acc = f32x4{sbias[0], sbias[1], sbias[2], sbias[3]};
#pragma unroll
                    for (int qc = 0; qc < 3; ++qc) {
                        V4 xf[P];
#pragma unroll
                        for (int q = 0; q < P; ++q) xf[q] = lds_frag<T>(stile + q * STEM_TILE + 2 * j * 132 + soff[qc]);
                        acc = mfma_split16<T>(sw[qc], xf, acc);
                    }
                    sx[j] = make_float4(hswish_nb(acc[0]), hswish_nb(acc[1]), hswish_nb(acc[2]), hswish_nb(acc[3]));
                }
            }
#pragma unroll
            for (int j = 0; j < C::IR; ++j) {
                const int iy = iy0 + j;
                rin[j] = iy >= 0 && iy < H;
                const int iyc = min(max(iy, 0), H - 1);
#pragma unroll
                for (int t = 0; t < C::NT; ++t)
#pragma unroll
                    for (int ks = 0; ks < C::KSI; ++ks) {
                        const int ch = min(ks * 16 + 4 * g, C::CIN - 4);
                        const float4 v =
                            STEM ? sx[j]
                                 : *reinterpret_cast<const float4*>(Xf + ((long long)iyc * W + ixc[t]) * C::CIN + ch);
                        if constexpr (C::EXPAND) {
                            split4<T>(v, xf[j][t][ks]);
                        } else {
                            const bool ok = rin[j] && pin[0];
                            xe[j] = ok ? v : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                        }
                    }
            }
            f32x4 y[C::R][C::OT];
#pragma unroll
            for (int q = 0; q < C::R; ++q)
#pragma unroll
                for (int ot = 0; ot < C::OT; ++ot) y[q][ot] = pb[ot];

#pragma unroll
            for (int ct = 0; ct < C::CT; ++ct) {
                // ---- expanded rows of this channel tile (fp32, zero outside the map)
                f32x4 e[C::IR][C::NT];
                if constexpr (C::EXPAND) {
                    V4 wf[C::KSI][P];
#pragma unroll
                    for (int ks = 0; ks < C::KSI; ++ks)
#pragma unroll
                        for (int q = 0; q < P; ++q)
                            wf[ks][q] = lds_frag<T>(We + (q * C::CT * 16 + ct * 16 + r) * C::KP + ks * 16 + 4 * g);
                    f32x4 init[C::NT];
#pragma unroll
                    for (int t = 0; t < C::NT; ++t) {
                        const float4 b = *reinterpret_cast<const float4*>(Be + be_off[t] + ct * 16 + 4 * g);
                        init[t] = f32x4{b.x, b.y, b.z, b.w};
                    }
#pragma unroll
                    for (int j = 0; j < C::IR; ++j)
#pragma unroll
                        for (int t = 0; t < C::NT; ++t) {
                            f32x4 acc;
                            if (rin[j]) {   // uniform: the whole wave is on the same input row
                                acc = init[t];
#pragma unroll
                                for (int ks = 0; ks < C::KSI; ++ks) acc = mfma_split16<T>(wf[ks], xf[j][t][ks], acc);
#pragma unroll
                                for (int i = 0; i < 4; ++i) acc[i] = relu_nb(acc[i]);   // sexp: in the taps
                            } else {
                                acc = zero_rows();
                            }
                            e[j][t] = acc;
                        }
                } else {
#pragma unroll
                    for (int j = 0; j < C::IR; ++j) e[j][0] = f32x4{xe[j].x, xe[j].y, xe[j].z, xe[j].w};
                }
                // ---- left / right neighbours along x
                f32x4 el[C::IR], er[C::S == 1 ? C::IR : 1];
#pragma unroll
                for (int j = 0; j < C::IR; ++j)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if constexpr (C::S == 1) {
                            el[j][i] = row_shr1(e[j][0][i]);
                            er[j][i] = row_shl1(e[j][0][i]);
                        } else {
                            el[j][i] = row_shr1(e[j][1][i]);
                        }
                    }
                V4 wp[C::OT][P];
#pragma unroll
                for (int ot = 0; ot < C::OT; ++ot)
#pragma unroll
                    for (int q = 0; q < P; ++q)
                        wp[ot][q] = lds_frag<T>(Wp + (q * C::OT * 16 + ot * 16 + r) * C::CP + ct * 16 + 4 * g);
                // ---- depthwise + ReLU, then the projection of this channel tile, one output row at a time
#pragma unroll
                for (int qr = 0; qr < C::R; ++qr) {
                    const int j0 = C::S * qr;
                    float d[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        float v;
                        if constexpr (C::S == 1)
                            v = dw9(wdw[ct][i], el[j0][i], e[j0][0][i], er[j0][i], el[j0 + 1][i], e[j0 + 1][0][i],
                                    er[j0 + 1][i], el[j0 + 2][i], e[j0 + 2][0][i], er[j0 + 2][i]);
                        else
                            v = dw9(wdw[ct][i], el[j0][i], e[j0][0][i], e[j0][1][i], el[j0 + 1][i], e[j0 + 1][0][i],
                                    e[j0 + 1][1][i], el[j0 + 2][i], e[j0 + 2][0][i], e[j0 + 2][1][i]);
                        d[i] = relu_nb(v);
                    }
                    V4 df[P];
                    split4<T>(make_float4(d[0], d[1], d[2], d[3]), df);
#pragma unroll
                    for (int ot = 0; ot < C::OT; ++ot) y[qr][ot] = mfma_split16<T>(wp[ot], df, y[qr][ot]);
                }
            }

            // ---- epilogue: (+ residual) and one float4 per (row, output tile) per lane.  Expand blocks re-read
            // the residual (clamped) before the first store: the memory counter retires in order, so a load issued
            // after a store would wait for that store.
            float4 res[C::RES ? C::R : 1][C::OT];
            if constexpr (C::RES) {
#pragma unroll
                for (int qr = 0; qr < C::R; ++qr)
#pragma unroll
                    for (int ot = 0; ot < C::OT; ++ot) {
                        if constexpr (C::EXPAND) {
                            const int oyc = min(oy0 + qr, Ho - 1), oxc = min(max(ox, 0), Wo - 1);
                            const int n = min(ot * 16 + 4 * g, C::COUT - 4);
                            res[qr][ot] = *reinterpret_cast<const float4*>(Xf + ((long long)oyc * W + oxc) * C::CIN + n);
                        } else {
                            res[qr][ot] = xe[qr + 1];
                        }
                    }
            }
#pragma unroll
            for (int qr = 0; qr < C::R; ++qr) {
                const int oy = oy0 + qr;
                if (oy >= Ho) break;
#pragma unroll
                for (int ot = 0; ot < C::OT; ++ot) {
                    const int n = ot * 16 + 4 * g;
                    if (!store_lane || n >= C::COUT) continue;
                    float4 v = make_float4(y[qr][ot][0] * a.sproj, y[qr][ot][1] * a.sproj, y[qr][ot][2] * a.sproj,
                                           y[qr][ot][3] * a.sproj);
                    if constexpr (C::RES) {
                        const float4 x = res[qr][ot];
                        v.x = x.x + v.x; v.y = x.y + v.y; v.z = x.z + v.z; v.w = x.w + v.w;
                    }
                    *reinterpret_cast<float4*>(Yf + ((long long)oy * Wo + ox) * C::COUT + n) = v;
                }
            }
        }
    }
}

template <typename T, class C, bool STEM = false> void launch_strip(int block, const IrArgs& a, int F, hipStream_t s) {
    // the engine pads the weights to the block's IrShape; the kernel reads them with these paddings
    const IrShape sh = ir_shape(block, std::is_same<T, bf16>::value);
    if (sh.cin != C::CIN || sh.cexp != C::CEXP || sh.cout != C::COUT || sh.k != 3 || sh.stride != C::S || sh.se ||
        sh.hs || sh.cinp != (C::CIN + 31) / 32 * 32 || sh.cexpp != (C::CEXP + 31) / 32 * 32 || sh.coutp != C::OT * 16)
        throw std::runtime_error("ir_strip: weight padding disagrees with the block shape");
    const int strips = (a.Wo + C::VALID - 1) / C::VALID;
    if ((C::S == 1 && (a.Ho != a.H || a.Wo != a.W)) || (C::S == 2 && (a.Ho != (a.H + 1) / 2 || a.Wo != (a.W + 1) / 2)))
        throw std::runtime_error("ir_strip: map shape does not match the stride");
    if (a.frames != F || (long long)F * strips > (1ll << 30)) throw std::runtime_error("ir_strip: bad frame count");
    // persistent workgroups: as many as the device holds at once (per-instantiation occupancy, cached)
    static const int resident = [] {
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, ir_strip_kernel<T, C, STEM>, ST_THREADS, 0) !=
                hipSuccess)
            throw std::runtime_error("ir_strip: cannot query the device occupancy");
        return std::max(1, cus) * std::max(1, per_cu);
    }();
    const int waves_per_wg = ST_THREADS / 64;
    // fewer (frame, strip) items than resident waves: deal each strip's steps over row segments
    const int steps = (a.Ho + C::R - 1) / C::R;
    int seg_steps = steps;
    if ((long long)F * strips < (long long)resident * waves_per_wg) {
        const int want = std::min<long long>(steps, (long long)resident * waves_per_wg / ((long long)F * strips));
        seg_steps = (steps + want - 1) / want;
    }
    const int segs = (steps + seg_steps - 1) / seg_steps;
    if ((long long)F * strips * segs > (1ll << 30)) throw std::runtime_error("ir_strip: too many items");
    const int items = F * strips * segs;
    const int grid = std::min((items + waves_per_wg - 1) / waves_per_wg, resident);
    hipLaunchKernelGGL((ir_strip_kernel<T, C, STEM>), dim3(grid), dim3(ST_THREADS), 0, s, a, strips, items, segs,
                       seg_steps * C::R, a.stem_w, a.stem_b);
}


// ------------------------------------------------------------------------------------------------------------
// Workgroup strip kernel (blocks 4-15: wider channel counts, 5x5 taps, hardswish, squeeze-excite).
//
// The 4 waves of a workgroup share one strip (16 lanes = 16 pixel columns) of one frame and walk down it R output
// rows per step.  Each step's input rows are staged once in LDS, already split into the operand parts; each wave
// then takes the 16-channel tiles ct = wave, wave + 4, ... and, per tile, computes the expanded rows (transposed
// split MFMA 16x16x32, K = input channels), the depthwise outputs and either
//   * (squeeze-excite blocks) the D rows to HBM and the step's channel sums, or
//   * (other blocks) its share of the projection Y^T += Wproj^T[:, tile] . D^T (16x16x16), the 4 wave partials
//     being added in wave order through LDS at the end of the step (+ bias, + residual).
// The depthwise streams over the step's input rows in order, adding each row's taps to every output row that uses
// it, so each output is still one fma chain over (dy, dx) in order, then + bias.  Tap weights are broadcast from
// lane t (tap t < 16) of a first register and lane t - 16 of a second one (5x5), the bias from the lane after the
// last tap.  Columns outside the map expand from -1e30 (ReLU and hardswish both give 0 there), rows outside the
// map are skipped (E = 0).
template <int CIN_, int CEXP_, int COUT_, int KS_, int S_, int HS_, int SE_, int R_, int MINB_ = 1, int ROLLK_ = 0,
          int NOPF_ = 0, int WHOLE_H_ = 0, int NPOS_ = 16, int YBA_ = 0, int WAVES_ = 4, int RING_ = 0>
struct WgCfg {
    static constexpr int CIN = CIN_, CEXP = CEXP_, COUT = COUT_, KS = KS_, S = S_, R = R_;
    static constexpr int MINB = MINB_;   // workgroups per CU the register allocation must allow
    // waves of a workgroup sharing one staged step (channel tiles ct = wave, wave + WAVES, ...); the projection
    // blocks add their wave partials in four-wave order and keep 4
    static constexpr int WAVES = WAVES_, THREADS = 64 * WAVES_;
    // ROLLK: the expand runs K-step-outer in a rolled loop (weight parts loaded per K step, one step ahead), so only
    // one K step's fragments are live -- for wide inputs, where the unrolled form holds every row's fragments
    static constexpr bool ROLLK = ROLLK_ != 0;
    // NOPF: a step's input rows are staged at the start of the step (NOPF_ float4 per thread at a time, 4 for
    // NOPF_ = 1) instead of being held in registers during the previous step -- for wide inputs with long steps,
    // where those registers would cost occupancy and an exposed load per step is cheap
    static constexpr bool NOPF = NOPF_ != 0;
    static constexpr int NOPF_CHUNK = NOPF_ > 1 ? NOPF_ : 4;
    // WHOLE_H (one step covers the map's WHOLE_H rows): only the map's own rows are staged -- the padding rows above
    // and below are never read, the expand skips them -- so LDS holds WHOLE_H rows instead of IR
    static constexpr int XR0 = WHOLE_H_ ? KS_ / 2 : 0;     // first staged input row of a step (relative)
    static constexpr int XRN = WHOLE_H_ ? WHOLE_H_ : S_ * (R_ - 1) + KS_;
    static_assert(!WHOLE_H_ || S_ * R_ >= WHOLE_H_, "whole-map staging: one step per map");
    static constexpr bool HS = HS_ != 0, SE = SE_ != 0, PROJ = !SE;
    static constexpr int ACT = HS ? ACT_HS : ACT_RELU;
    static constexpr int PADK = KS / 2;
    static constexpr int KS32 = (CIN + 31) / 32, CINP = KS32 * 32, XLD = CINP + 8;
    static constexpr int CEXPP = (CEXP + 31) / 32 * 32;     // weight padding of the engine (IrShape cexpp)
    static constexpr int CT = (CEXP + 15) / 16, OT = (COUT + 15) / 16, COUTP = OT * 16;
    static constexpr int NT = S, IR = S * (R - 1) + KS;
    static constexpr int VALID = S == 1 ? 16 - 2 * PADK : (KS == 3 ? 15 : 14);
    static constexpr int LO = S == 1 ? PADK : 1;            // first output lane
    // NPOS < 16 (one strip covers the map): only the NPOS pixel positions of a tile from lane POS0 on are staged --
    // the map's columns; the other lanes are outside the map (their expand starts at -1e30) and read a clamped one
    static constexpr int NPOS = NPOS_, POS0 = NPOS_ == 16 ? 0 : LO;
    // YBA (projection blocks): the wave partials of the projection share LDS with the staged rows (two more
    // barriers per step: before the partials are written, and before the next step's rows are staged)
    static constexpr bool YBA = YBA_ != 0;
    // RING (squeeze-excite blocks stepping down the map): the HALO = KS - S input rows a step shares with the next
    // stay staged.  LDS holds the IR rows as a ring, row j of step st in slot (st * ADV + j) mod IR, and every step
    // but a segment's first stages only its ADV = S * R new rows (a staged row depends on its map row alone)
    static constexpr int ADV = S * R, HALO = IR - ADV;
    static constexpr bool RING = RING_ != 0 && SE && !WHOLE_H_ && !YBA && HALO > 0;
    static_assert(!RING || (XR0 == 0 && XRN == IR), "the ring holds a step's IR input rows");
    static_assert(NPOS >= 1 && NPOS <= 16 && POS0 + NPOS <= 16, "staged positions within the 16 lanes");
    static constexpr bool RES = PROJ && S == 1 && CIN == COUT;
    static constexpr int NWR = (KS * KS + 1 + 15) / 16;    // depthwise weight registers per value (taps + bias)
    static_assert(CIN % 4 == 0 && CEXP % 4 == 0 && COUT % 4 == 0, "channel counts must be multiples of 4");
    static_assert(KS == 3 || KS == 5, "3x3 or 5x5 depthwise");
    static_assert(WAVES == 4 || (SE && (WAVES == 8)), "projection blocks: four waves; squeeze-excite blocks: 4 or 8");
};

template <typename T, class C> struct WgLds {
    static constexpr int P = Split<T>::P;
    static constexpr int XS = C::XRN * C::NT * P * C::NPOS * C::XLD;    // T elements
    static constexpr int YB = C::PROJ ? 4 * C::R * C::OT * 64 : 0;  // float4s
    static constexpr int BYTES = C::YBA ? (XS * (int)sizeof(T) > YB * 16 ? XS * (int)sizeof(T) : YB * 16)
                                        : XS * (int)sizeof(T) + YB * 16;
};

// acc (op)= the KS taps of one input row: first row of an output starts the chain with a product
template <bool FIRST, int L0, int L1, int L2>
__device__ __forceinline__ float taps3(float acc, float w0, float w1, float w2, float e0, float e1, float e2) {
    if constexpr (FIRST)
        asm("s_nop 1\n\t"
            "v_mul_f32_dpp %0, %1, %4 row_newbcast:%7 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %0, %2, %5 row_newbcast:%8 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %0, %3, %6 row_newbcast:%9 row_mask:0xf bank_mask:0xf"
            : "=&v"(acc)
            : "v"(w0), "v"(w1), "v"(w2), "v"(e0), "v"(e1), "v"(e2), "i"(L0), "i"(L1), "i"(L2));
    else
        asm("s_nop 1\n\t"
            "v_fmac_f32_dpp %0, %1, %4 row_newbcast:%7 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %0, %2, %5 row_newbcast:%8 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %0, %3, %6 row_newbcast:%9 row_mask:0xf bank_mask:0xf"
            : "+v"(acc)
            : "v"(w0), "v"(w1), "v"(w2), "v"(e0), "v"(e1), "v"(e2), "i"(L0), "i"(L1), "i"(L2));
    return acc;
}
template <bool FIRST, int L0, int L1, int L2, int L3, int L4>
__device__ __forceinline__ float taps5(float acc, float w0, float w1, float w2, float w3, float w4, float e0, float e1,
                                       float e2, float e3, float e4) {
    if constexpr (FIRST)
        asm("s_nop 1\n\t"
            "v_mul_f32_dpp %0, %1, %6 row_newbcast:%11 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %0, %2, %7 row_newbcast:%12 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %0, %3, %8 row_newbcast:%13 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %0, %4, %9 row_newbcast:%14 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %0, %5, %10 row_newbcast:%15 row_mask:0xf bank_mask:0xf"
            : "=&v"(acc)
            : "v"(w0), "v"(w1), "v"(w2), "v"(w3), "v"(w4), "v"(e0), "v"(e1), "v"(e2), "v"(e3), "v"(e4), "i"(L0),
              "i"(L1), "i"(L2), "i"(L3), "i"(L4));
    else
        asm("s_nop 1\n\t"
            "v_fmac_f32_dpp %0, %1, %6 row_newbcast:%11 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %0, %2, %7 row_newbcast:%12 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %0, %3, %8 row_newbcast:%13 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %0, %4, %9 row_newbcast:%14 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %0, %5, %10 row_newbcast:%15 row_mask:0xf bank_mask:0xf"
            : "+v"(acc)
            : "v"(w0), "v"(w1), "v"(w2), "v"(w3), "v"(w4), "v"(e0), "v"(e1), "v"(e2), "v"(e3), "v"(e4), "i"(L0),
              "i"(L1), "i"(L2), "i"(L3), "i"(L4));
    return acc;
}
// v + (lane L of wv's row)
template <int L> __device__ __forceinline__ float add_bcast(float v, float wv) {
    float out;
    asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf" : "=v"(out) : "v"(wv), "v"(v), "i"(L));
    return out;
}
// lane r <- lane r + D of its 16-lane row (0 where that is outside the row)
template <int D> __device__ __forceinline__ float lane_shift(float v) {
    if constexpr (D == 0) return v;
    else if constexpr (D > 0)
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x100 + D, 0xf, 0xf, true));
    else
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x110 - D, 0xf, 0xf, true));
}
// transposed split product: acc += W . X with W the A operand (weight parts), X the B operand (activation parts)
template <typename T>
__device__ __forceinline__ f32x4 mfma_wx(const typename Split<T>::V8* w, const typename Split<T>::V8* x, f32x4 acc) {
#pragma unroll
    for (int i = 0; i < Split<T>::NPROD; ++i) acc = Split<T>::mfma(w[Split<T>::wp(i)], x[Split<T>::ap(i)], acc);
    return acc;
}

// the staged pixel position a lane's B fragments come from (its own, or the nearest staged one: NPOS < 16)
template <class C> __device__ __forceinline__ int staged_pos(int r) {
    if constexpr (C::NPOS == 16) return r;
    else return min(max(r - C::POS0, 0), C::NPOS - 1);
}

// one input row's taps (weights of kernel row DY) into an output accumulator, per value i of the lane
template <class C, bool FIRST, int DY>
__device__ __forceinline__ float row_taps(float acc, const float (&wd)[C::NWR], const float* v) {
    constexpr int t0 = DY * C::KS;
    if constexpr (C::KS == 3) {
        return taps3<FIRST, t0 % 16, (t0 + 1) % 16, (t0 + 2) % 16>(acc, wd[t0 / 16], wd[(t0 + 1) / 16], wd[(t0 + 2) / 16],
                                                                  v[0], v[1], v[2]);
    } else {
        return taps5<FIRST, t0 % 16, (t0 + 1) % 16, (t0 + 2) % 16, (t0 + 3) % 16, (t0 + 4) % 16>(
            acc, wd[t0 / 16], wd[(t0 + 1) / 16], wd[(t0 + 2) / 16], wd[(t0 + 3) / 16], wd[(t0 + 4) / 16], v[0], v[1],
            v[2], v[3], v[4]);
    }
}

template <class C, int J, int Q>
__device__ __forceinline__ void accum_row(f32x4 (&acc)[C::R], const float (&wd)[4][C::NWR], const f32x4 (&v)[C::KS]) {
    if constexpr (Q < C::R) {
        constexpr int DY = J - C::S * Q;
        if constexpr (DY >= 0 && DY < C::KS) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float vi[C::KS];
#pragma unroll
                for (int dx = 0; dx < C::KS; ++dx) vi[dx] = v[dx][i];
                acc[Q][i] = row_taps<C, DY == 0, DY>(acc[Q][i], wd[i], vi);
            }
        }
        accum_row<C, J, Q + 1>(acc, wd, v);
    }
}

// the LDS slot of a step's staged row j (j counted from XR0; rb: the ring slot of the step's row 0)
template <class C> __device__ __forceinline__ int row_slot(int j, int rb) {
    if constexpr (C::RING) return rb + j < C::IR ? rb + j : rb + j - C::IR;
    else return j;
}

template <typename T, class C, int J>
__device__ __forceinline__ void wg_rows(f32x4 (&acc)[C::R], const float (&wd)[4][C::NWR], const typename Split<T>::V8 (&wf)[C::KS32][Split<T>::P],
                                        const f32x4 (&init)[C::NT], const T* Xs, int r, int g, int iy0, int H,
                                        float es, int rb) {
    if constexpr (J < C::IR) {
        typedef typename Split<T>::V8 V8;
        constexpr int P = Split<T>::P;
        f32x4 e[C::NT];
        const int iy = iy0 + J;
        if (iy >= 0 && iy < H) {   // uniform
            const T* Xr = Xs + row_slot<C>(J - C::XR0, rb) * (C::NT * P * C::NPOS * C::XLD);
#pragma unroll
            for (int t = 0; t < C::NT; ++t) {
                f32x4 x = init[t];
#pragma unroll
                for (int ks = 0; ks < C::KS32; ++ks) {
                    V8 xf[P];
#pragma unroll
                    for (int q = 0; q < P; ++q)
                        xf[q] = *reinterpret_cast<const V8*>(Xr + ((t * P + q) * C::NPOS + staged_pos<C>(r)) * C::XLD + ks * 32 + g * 8);
                    x = mfma_wx<T>(wf[ks], xf, x);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) x[i] = apply_act_nb(C::HS ? x[i] * es : x[i], C::ACT);
                e[t] = x;
            }
        } else {
#pragma unroll
            for (int t = 0; t < C::NT; ++t) e[t] = zero_rows();
        }
        // tap variants dx = 0 .. KS-1 of this row for the lane's output column
        f32x4 v[C::KS];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (C::S == 1) {
#pragma unroll
                for (int dx = 0; dx < C::KS; ++dx) {
                    if constexpr (C::KS == 3) {
                        if (dx == 0) v[dx][i] = lane_shift<-1>(e[0][i]);
                        else if (dx == 1) v[dx][i] = e[0][i];
                        else v[dx][i] = lane_shift<1>(e[0][i]);
                    } else {
                        if (dx == 0) v[dx][i] = lane_shift<-2>(e[0][i]);
                        else if (dx == 1) v[dx][i] = lane_shift<-1>(e[0][i]);
                        else if (dx == 2) v[dx][i] = e[0][i];
                        else if (dx == 3) v[dx][i] = lane_shift<1>(e[0][i]);
                        else v[dx][i] = lane_shift<2>(e[0][i]);
                    }
                }
            } else if constexpr (C::KS == 3) {   // even tile 0, odd tile 1: cols 2ox-1, 2ox, 2ox+1
                v[0][i] = lane_shift<-1>(e[1][i]);
                v[1][i] = e[0][i];
                v[2][i] = e[1][i];
            } else {                             // cols 2ox-2 .. 2ox+2
                v[0][i] = lane_shift<-1>(e[0][i]);
                v[1][i] = lane_shift<-1>(e[1][i]);
                v[2][i] = e[0][i];
                v[3][i] = e[1][i];
                v[4][i] = lane_shift<1>(e[0][i]);
            }
        }
        accum_row<C, J, 0>(acc, wd, v);
        wg_rows<T, C, J + 1>(acc, wd, wf, init, Xs, r, g, iy0, H, es, rb);
    }
}

// ROLLK expand: ea[staged row][tile] = init + W . X over the K steps in order (rows outside the map left at init,
// unused); staged row j holds input row XR0 + j of the step
template <typename T, class C>
__device__ __forceinline__ void wg_expand_rolled(f32x4 (&ea)[C::XRN][C::NT], const T* wexp, long long wstride, int ct,
                                                 const f32x4 (&init)[C::NT], const T* Xs, int r, int g, int iy0,
                                                 int H, int rb) {
    typedef typename Split<T>::V8 V8;
    constexpr int P = Split<T>::P;
#pragma unroll
    for (int j = 0; j < C::XRN; ++j)
#pragma unroll
        for (int t = 0; t < C::NT; ++t) ea[j][t] = init[t];
    const T* wrow = wexp + (long long)(ct * 16 + r) * C::CINP + g * 8;
    V8 wn[P];
#pragma unroll
    for (int q = 0; q < P; ++q) wn[q] = load_part8<T>(wrow + q * wstride);
#pragma unroll 1
    for (int ks = 0; ks < C::KS32; ++ks) {
        V8 w[P];
#pragma unroll
        for (int q = 0; q < P; ++q) w[q] = wn[q];
        if (ks + 1 < C::KS32) {
#pragma unroll
            for (int q = 0; q < P; ++q) wn[q] = load_part8<T>(wrow + q * wstride + (ks + 1) * 32);
        }
#pragma unroll
        for (int j = 0; j < C::XRN; ++j) {
            const int iy = iy0 + C::XR0 + j;
            if (iy >= 0 && iy < H) {   // uniform
#pragma unroll
                for (int t = 0; t < C::NT; ++t) {
                    V8 xf[P];
#pragma unroll
                    for (int q = 0; q < P; ++q)
                        xf[q] = *reinterpret_cast<const V8*>(Xs + (((row_slot<C>(j, rb) * C::NT + t) * P + q) * C::NPOS + staged_pos<C>(r)) * C::XLD + ks * 32 + g * 8);
                    ea[j][t] = mfma_wx<T>(w, xf, ea[j][t]);
                }
            }
        }
    }
}

// tap variants dx = 0 .. KS-1 of one input row (E tiles e) for the lane's output column
template <class C>
__device__ __forceinline__ void tap_variants(const f32x4 (&e)[C::NT], f32x4 (&v)[C::KS]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (C::S == 1) {
            if constexpr (C::KS == 3) {
                v[0][i] = lane_shift<-1>(e[0][i]);
                v[1][i] = e[0][i];
                v[2][i] = lane_shift<1>(e[0][i]);
            } else {
                v[0][i] = lane_shift<-2>(e[0][i]);
                v[1][i] = lane_shift<-1>(e[0][i]);
                v[2][i] = e[0][i];
                v[3][i] = lane_shift<1>(e[0][i]);
                v[4][i] = lane_shift<2>(e[0][i]);
            }
        } else if constexpr (C::KS == 3) {   // even tile 0, odd tile 1: cols 2ox-1, 2ox, 2ox+1
            v[0][i] = lane_shift<-1>(e[1][i]);
            v[1][i] = e[0][i];
            v[2][i] = e[1][i];
        } else {                             // cols 2ox-2 .. 2ox+2
            v[0][i] = lane_shift<-1>(e[0][i]);
            v[1][i] = lane_shift<-1>(e[1][i]);
            v[2][i] = e[0][i];
            v[3][i] = e[1][i];
            v[4][i] = lane_shift<1>(e[0][i]);
        }
    }
}

// the depthwise over rows whose expand accumulators are ready (ROLLK)
template <class C, int J>
__device__ __forceinline__ void wg_rows_acc(f32x4 (&acc)[C::R], const float (&wd)[4][C::NWR],
                                            const f32x4 (&ea)[C::XRN][C::NT], int iy0, int H, float es) {
    if constexpr (J < C::IR) {
        f32x4 e[C::NT];
        if constexpr (J >= C::XR0 && J < C::XR0 + C::XRN) {
            const int iy = iy0 + J;
            // rows outside the map become +0 through an all-ones / all-zeros mask that the compiler
            // cannot see through: as a select it turned each element into its own branch around the activation
            int keep = iy >= 0 && iy < H ? -1 : 0;
            asm("" : "+v"(keep));
#pragma unroll
            for (int t = 0; t < C::NT; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    e[t][i] = __int_as_float(
                        __float_as_int(apply_act_nb(C::HS ? ea[J - C::XR0][t][i] * es : ea[J - C::XR0][t][i], C::ACT)) &
                        keep);
        } else {   // never staged: outside the map (whole-map staging)
#pragma unroll
            for (int t = 0; t < C::NT; ++t) e[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        f32x4 v[C::KS];
        tap_variants<C>(e, v);
        accum_row<C, J, 0>(acc, wd, v);
        wg_rows_acc<C, J + 1>(acc, wd, ea, iy0, H, es);
    }
}

template <typename T, class C>
// csplit (squeeze-excite blocks; 1 otherwise): the channel tiles of a (frame, strip) are dealt over csplit
// workgroups, and segs: its steps over segs items of seg_steps steps, so that few frames still fill the device
// (item = ((frame, strip) * segs + segment) * csplit + group).  Every output is computed the same way whichever
// workgroup takes its tile and step.
__global__ void __launch_bounds__(C::THREADS, C::MINB) ir_wgstrip_kernel(IrArgs a, int strips, int steps, int items,
                                                                           int csplit, int segs, int seg_steps) {
    typedef Split<T> S;
    typedef typename S::V8 V8;
    typedef typename Split16<T>::V4 V4;
    typedef WgLds<T, C> L;
    constexpr int P = S::P;
    __shared__ __attribute__((aligned(16))) unsigned char lds_raw[L::BYTES];
    T* Xs = reinterpret_cast<T*>(lds_raw);                                   // [IR][NT][P][16][XLD]
    float4* Yb = reinterpret_cast<float4*>(lds_raw + (C::YBA ? 0 : L::XS * sizeof(T)));    // [4][R][OT][64]
    const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: tile and LDS-slot math stays scalar
    const T* wexp = static_cast<const T*>(a.wexp);
    const T* wproj = static_cast<const T*>(a.wproj);
    const int H = a.H, W = a.W, Ho = a.Ho, Wo = a.Wo;

    // staging of a step's input rows: float4 i -> (row j, tile t, pixel p, channel quad c4).  The loads read clamped,
    // always valid addresses unconditionally (32-bit offsets from the frame's base); what lies outside the map or
    // past cin is zeroed when the rows are split into LDS, so no load waits on a predicate.  A full staging covers
    // the step's XRN rows; with the ring a continuing step stages its ADV new rows (j = HALO ..) only
    constexpr int XQ = C::CINP / 4;
    constexpr int XROW = C::NT * C::NPOS * XQ;               // float4s of one staged input row
    constexpr int XN = C::XRN * XROW, XNC = C::RING ? C::ADV * XROW : XN;
    constexpr int XPT_ALL = (XN + C::THREADS - 1) / C::THREADS, XPTC_ALL = (XNC + C::THREADS - 1) / C::THREADS;
    constexpr int XPT = C::NOPF ? (XPT_ALL < C::NOPF_CHUNK ? XPT_ALL : C::NOPF_CHUNK) : XPT_ALL;   // held at a time
    float4 xpre[XPT];
    auto col_of = [&](int strip, int p, int t) {
        return C::S == 1 ? strip * C::VALID - C::PADK + p : 2 * (strip * C::VALID - 1 + p) + t;
    };
    // FULL: std::true_type (every row of the step) or std::false_type (the ring's new rows)
    auto load_step = [&](auto full, int fs, int step, int k0) {
        constexpr bool FULL = decltype(full)::value;
        constexpr int N = FULL ? XN : XNC, J0 = FULL ? 0 : C::XRN - XNC / XROW;
        constexpr int NK = (FULL ? XPT_ALL : XPTC_ALL) < XPT ? (FULL ? XPT_ALL : XPTC_ALL) : XPT;
        const int strip = fs % strips;
        const float* Xf = a.X + (long long)(fs / strips) * (H * W * C::CIN);
        const int iy0 = C::S * step * C::R - C::PADK + C::XR0;
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const int i = min(tid + (k0 + k) * C::THREADS, N - 1);
            const int c4 = i % XQ, rest = i / XQ;
            const int p = rest % C::NPOS, jt = rest / C::NPOS;
            const int t = jt % C::NT, j = J0 + jt / C::NT;
            const int cy = min(max(iy0 + j, 0), H - 1), cx = min(max(col_of(strip, p + C::POS0, t), 0), W - 1);
            const int cc = min(c4, C::CIN / 4 - 1);
            const unsigned byte_off = unsigned(((cy * W + cx) * C::CIN + cc * 4) * 4);   // within one frame
            xpre[k] = *reinterpret_cast<const float4*>(reinterpret_cast<const char*>(Xf) + byte_off);
        }
    };
    auto store_step = [&](auto full, int strip, int step, int k0) {
        constexpr bool FULL = decltype(full)::value;
        constexpr int N = FULL ? XN : XNC, J0 = FULL ? 0 : C::XRN - XNC / XROW;
        constexpr int NK = (FULL ? XPT_ALL : XPTC_ALL) < XPT ? (FULL ? XPT_ALL : XPTC_ALL) : XPT;
        const int iy0 = C::S * step * C::R - C::PADK + C::XR0;
        const int rb = C::RING ? step * C::ADV % C::IR : 0;
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const int i = tid + (k0 + k) * C::THREADS;
            if (i >= N) continue;
            const int c4 = i % XQ, rest = i / XQ;
            const int p = rest % C::NPOS, jt = rest / C::NPOS;
            const int t = jt % C::NT, j = J0 + jt / C::NT;
            const int iy = iy0 + j, ix = col_of(strip, p + C::POS0, t);
            const bool in = iy >= 0 && iy < H && ix >= 0 && ix < W && c4 * 4 < C::CIN;
            const float x[4] = {in ? xpre[k].x : 0.0f, in ? xpre[k].y : 0.0f, in ? xpre[k].z : 0.0f,
                                in ? xpre[k].w : 0.0f};
            uint2 four[P];
            split4_packed<T>(x, four);
            const int jl = row_slot<C>(j, rb) * C::NT + t;
#pragma unroll
            for (int q = 0; q < P; ++q)
                *reinterpret_cast<uint2*>(Xs + ((jl * P + q) * C::NPOS + p) * C::XLD + c4 * 4) = four[q];
        }
    };
    const std::true_type full_rows;
    const std::false_type new_rows;

    // item -> (frame, strip) index, first step of its segment
    auto item_fs = [&](int it) { return it / csplit / segs; };
    auto item_s0 = [&](int it) { return (it / csplit % segs) * seg_steps; };
    if constexpr (!C::NOPF) {
        if ((int)blockIdx.x < items) load_step(full_rows, item_fs(blockIdx.x), item_s0(blockIdx.x), 0);
    }
    for (int item = blockIdx.x; item < items; item += gridDim.x) {
        const int fs = item_fs(item), cgroup = item % csplit;   // (frame, strip) index, channel-tile group
        const int s0 = item_s0(item), s1 = min(steps, s0 + seg_steps);
        const int strip = fs % strips;
        const long long f = fs / strips;
        // this lane's output column and the map columns of its pixel tiles
        const int ox = C::S == 1 ? strip * C::VALID - C::PADK + r : strip * C::VALID - 1 + r;
        const bool out_lane = r >= C::LO && r < C::LO + C::VALID && ox < Wo;
        bool pin[C::NT];
#pragma unroll
        for (int t = 0; t < C::NT; ++t) {
            const int ix = col_of(strip, r, t);
            pin[t] = ix >= 0 && ix < W;
        }
        for (int step = s0; step < s1; ++step) {
            const int oy0 = step * C::R;
            const int rb = C::RING ? step * C::ADV % C::IR : 0;   // ring slot of the step's first row
            if constexpr (C::NOPF) {
                if (!C::RING || step == s0) {
                    for (int k0 = 0; k0 < XPT_ALL; k0 += XPT) {
                        load_step(full_rows, fs, step, k0);
                        store_step(full_rows, strip, step, k0);
                    }
                } else {
                    for (int k0 = 0; k0 < XPTC_ALL; k0 += XPT) {
                        load_step(new_rows, fs, step, k0);
                        store_step(new_rows, strip, step, k0);
                    }
                }
                lds_barrier();
            } else {
                if (!C::RING || step == s0) store_step(full_rows, strip, step, 0);
                else store_step(new_rows, strip, step, 0);
                lds_barrier();
                // the next step's (or next item's first) rows are in flight while this step computes
                if (step + 1 < s1) load_step(new_rows, fs, step + 1, 0);
                else if (item + (int)gridDim.x < items)
                    load_step(full_rows, item_fs(item + gridDim.x), item_s0(item + gridDim.x), 0);
            }

            f32x4 y[C::PROJ ? C::R : 1][C::PROJ ? C::OT : 1];
            if constexpr (C::PROJ) {
#pragma unroll
                for (int ot = 0; ot < C::OT; ++ot) {
                    float4 b = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    if (wave == 0) b = *reinterpret_cast<const float4*>(a.bproj + ot * 16 + 4 * g);
                    const float pinv = 1.0f / a.sproj;   // project sums at the weights' scale (exact)
#pragma unroll
                    for (int q = 0; q < C::R; ++q) y[q][ot] = f32x4{b.x * pinv, b.y * pinv, b.z * pinv, b.w * pinv};
                }
            }
            for (int ct = wave + C::WAVES * cgroup; ct < C::CT; ct += C::WAVES * csplit) {
                const int c = ct * 16 + 4 * g;
                // ---- this tile's weights
                V8 wf[C::ROLLK ? 1 : C::KS32][P];
                if constexpr (!C::ROLLK) {
#pragma unroll
                    for (int ks = 0; ks < C::KS32; ++ks)
#pragma unroll
                        for (int q = 0; q < P; ++q)
                            wf[ks][q] = load_part8<T>(wexp + q * a.wexp_stride + (long long)(ct * 16 + r) * C::CINP + ks * 32 + g * 8);
                }
                // ReLU blocks: the expand scale sexp rides in the taps, relu(sexp * x) = sexp * relu(x) exactly
                // (a power of two); hardswish blocks scale each expanded element before the activation
                float wd[4][C::NWR];
#pragma unroll
                for (int w = 0; w < C::NWR; ++w) {
                    const int t = min(w * 16 + r, C::KS * C::KS);
                    const float* src = t < C::KS * C::KS ? a.wdw + t * C::CEXPP + c : a.bdw + c;
                    const float4 v = *reinterpret_cast<const float4*>(src);
                    const float f = !C::HS && t < C::KS * C::KS ? a.sexp : 1.0f;
                    wd[0][w] = v.x * f; wd[1][w] = v.y * f; wd[2][w] = v.z * f; wd[3][w] = v.w * f;
                }
                // expand sums at the pre-scaled weights' scale 1 / sexp, from the bias at that scale (exact)
                const float4 be = *reinterpret_cast<const float4*>(a.bexp + c);
                const float einv = 1.0f / a.sexp;
                f32x4 init[C::NT];
#pragma unroll
                for (int t = 0; t < C::NT; ++t)
                    init[t] = pin[t] ? f32x4{be.x * einv, be.y * einv, be.z * einv, be.w * einv}
                                     : f32x4{-1e30f, -1e30f, -1e30f, -1e30f};
                V4 pw[C::PROJ ? C::OT : 1][P];
                if constexpr (C::PROJ) {
#pragma unroll
                    for (int ot = 0; ot < C::OT; ++ot)
#pragma unroll
                        for (int q = 0; q < P; ++q) {
                            const uint2 u = *reinterpret_cast<const uint2*>(wproj + q * a.wproj_stride +
                                                                            (long long)(ot * 16 + r) * C::CEXPP + c);
                            pw[ot][q] = __builtin_bit_cast(V4, u);
                        }
                }
                // ---- expand + depthwise, streaming over the step's input rows
                f32x4 acc[C::R];
#pragma unroll
                for (int q = 0; q < C::R; ++q) acc[q] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                if constexpr (C::ROLLK) {
                    f32x4 ea[C::XRN][C::NT];
                    wg_expand_rolled<T, C>(ea, wexp, a.wexp_stride, ct, init, Xs, r, g, C::S * oy0 - C::PADK, H, rb);
                    wg_rows_acc<C, 0>(acc, wd, ea, C::S * oy0 - C::PADK, H, a.sexp);
                } else {
                    wg_rows<T, C, 0>(acc, wd, wf, init, Xs, r, g, C::S * oy0 - C::PADK, H, a.sexp, rb);
                }
                constexpr int BL = C::KS * C::KS;   // bias lane index (taps 0 .. BL-1)
                f32x4 d[C::R];
#pragma unroll
                for (int q = 0; q < C::R; ++q)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        d[q][i] = apply_act_nb(add_bcast<BL % 16>(acc[q][i], wd[i][BL / 16]), C::ACT);
                if constexpr (C::SE) {
                    // D rows -> HBM; channel sums of the step's valid pixels (rows in order, then the 16 lanes)
                    float4 sum = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
                    for (int q = 0; q < C::R; ++q) {
                        const int oy = oy0 + q;
                        if (out_lane && oy < Ho) {
                            const float4 v = make_float4(d[q][0], d[q][1], d[q][2], d[q][3]);
                            if (c < C::CEXP)
                                *reinterpret_cast<float4*>(a.D + ((f * Ho + oy) * Wo + ox) * C::CEXP + c) = v;
                            sum.x = sum.x + v.x; sum.y = sum.y + v.y; sum.z = sum.z + v.z; sum.w = sum.w + v.w;
                        }
                    }
                    sum.x = tree16(sum.x); sum.y = tree16(sum.y); sum.z = tree16(sum.z); sum.w = tree16(sum.w);
                    if (r == 0)
                        *reinterpret_cast<float4*>(a.part + (f * a.ntiles + step * strips + strip) * C::CEXPP + c) = sum;
                } else {
#pragma unroll
                    for (int q = 0; q < C::R; ++q) {
                        V4 df[P];
                        split4<T>(make_float4(d[q][0], d[q][1], d[q][2], d[q][3]), df);
#pragma unroll
                        for (int ot = 0; ot < C::OT; ++ot) y[q][ot] = mfma_split16<T>(pw[ot], df, y[q][ot]);
                    }
                }
            }
            if constexpr (C::PROJ) {
                if constexpr (C::YBA) lds_barrier();   // every wave is done with the staged rows
#pragma unroll
                for (int q = 0; q < C::R; ++q)
#pragma unroll
                    for (int ot = 0; ot < C::OT; ++ot)
                        Yb[((wave * C::R + q) * C::OT + ot) * 64 + lane] = make_float4(y[q][ot][0], y[q][ot][1], y[q][ot][2], y[q][ot][3]);
            }
            lds_barrier();   // Xs free for the next step; the wave partials of Y complete
            if constexpr (C::PROJ) {
                // (row, output tile) pairs round robin over the waves: wave partials added in wave order
                for (int pr = wave; pr < C::R * C::OT; pr += 4) {
                    const int q = pr / C::OT, ot = pr % C::OT;
                    const int oy = oy0 + q, n = ot * 16 + 4 * g;
                    float4 res = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    if constexpr (C::RES) {
                        const int oyc = min(oy, Ho - 1), oxc = min(max(ox, 0), Wo - 1), nc = min(n, C::COUT - 4);
                        res = *reinterpret_cast<const float4*>(a.X + ((f * H + oyc) * W + oxc) * C::CIN + nc);
                    }
                    float4 v = Yb[((0 * C::R + q) * C::OT + ot) * 64 + lane];
#pragma unroll
                    for (int w = 1; w < 4; ++w) {
                        const float4 u = Yb[((w * C::R + q) * C::OT + ot) * 64 + lane];
                        v.x = v.x + u.x; v.y = v.y + u.y; v.z = v.z + u.z; v.w = v.w + u.w;
                    }
                    v.x = v.x * a.sproj; v.y = v.y * a.sproj; v.z = v.z * a.sproj; v.w = v.w * a.sproj;
                    if constexpr (C::RES) {
                        v.x = res.x + v.x; v.y = res.y + v.y; v.z = res.z + v.z; v.w = res.w + v.w;
                    }
                    if (out_lane && oy < Ho && n < C::COUT)
                        *reinterpret_cast<float4*>(a.Y + ((f * Ho + oy) * Wo + ox) * C::COUT + n) = v;
                }
                if constexpr (C::YBA) lds_barrier();   // the partials are read before the next rows are staged
            }
        }
    }
}

//                cin  cexp cout k  s  hs se R  minb
// Blocks 4-6 keep the rows shared by consecutive steps staged (RING; bitwise unchanged): block 4 0.88 -> 0.85 ms,
// blocks 5-6 1.80 -> 1.78 ms per 128 clips alone.  Blocks 11-13 ran slower with it (block 11 0.67 -> 0.83 ms: 165 ->
// 181 VGPRs, two waves per SIMD instead of three; blocks 12, 13 +4%, +1%)
typedef WgCfg<24, 72, 40, 5, 2, 0, 1, 3, 3, 0, 0, 0, 16, 0, 4, 1> G4;   // 45x80 -> 23x40 (R 3, three workgroups per CU: 0.94 -> 0.88 ms)
typedef WgCfg<40, 120, 40, 5, 1, 0, 1, 6, 1, 0, 0, 0, 16, 0, 4, 1> G5;   // 23x40 (b5, b6)
typedef WgCfg<40, 240, 80, 3, 2, 1, 0, 3, 2, 0, 0, 0, 16, 1> G7;    // 23x40 -> 12x20
typedef WgCfg<80, 200, 80, 3, 1, 1, 0, 4, 2, 0, 8, 0, 16, 1> G8;       // 12x20
typedef WgCfg<80, 184, 80, 3, 1, 1, 0, 4, 2, 0, 8, 0, 16, 1> G9;       // 12x20 (b9, b10)
typedef WgCfg<80, 480, 112, 3, 1, 1, 1, 4> G11;       // 12x20
typedef WgCfg<112, 672, 112, 3, 1, 1, 1, 6, 1, 0, 0, 0, 16, 0, 8> G12;   // 12x20, eight waves per staged step
// Blocks 12-15 (squeeze-excite, wide expands) run eight waves on each staged step: the same LDS serves twice the
// waves, so a workgroup holds half the LDS per wave (alone: block 12 1.14 -> 1.06 ms, 13 1.55 -> 1.28, 14-15
// 1.50 -> 1.21 per 128 clips; the concurrent forward unchanged to -0.5%, bf16 async +3%).
// Block 13 takes 2 output rows per step (7 staged input rows, 76 KB of LDS: two workgroups per CU, and room for
// the other branches' kernels): alone 1.43 -> 1.55 ms per 128 clips against the whole-map step (130 KB), but the
// concurrent forward 19.02 -> 18.84 ms; 1 row per step 19.08, 3 rows 19.14.  The bf16 tier runs it too (114 KB
// with three parts, one workgroup per CU): 2.68 -> 1.63 ms against the tile kernel, bf16 forward 27.9 -> 26.5 ms.
typedef WgCfg<112, 672, 160, 5, 2, 1, 1, 2, 2, 1, 16, 0, 10, 0, 8> G13;   // 12x20 -> 6x10, 10 columns/tile, eight waves
typedef WgCfg<160, 960, 160, 5, 1, 1, 1, 6, 1, 1, 1, 6, 16, 0, 8> G14;   // 6x10 (b14, b15), eight waves
// bf16 (three operand parts): fewer rows per step where the fp16 row step leaves LDS room for one workgroup per CU
typedef WgCfg<24, 72, 40, 5, 2, 0, 1, 3, 1, 0, 0, 0, 16, 0, 4, 1> G4B;
typedef WgCfg<40, 240, 80, 3, 2, 1, 0, 2, 2, 0, 0, 0, 16, 1> G7B;
typedef WgCfg<112, 672, 112, 3, 1, 1, 1, 4> G12B;

// the block shape the engine pads weights to and sizes the SE partial sums by: tile = (R rows, VALID columns)
template <class C> IrShape wg_shape() {
    IrShape s;
    s.cin = C::CIN; s.cexp = C::CEXP; s.cout = C::COUT; s.k = C::KS; s.stride = C::S; s.se = C::SE; s.hs = C::HS;
    s.th = C::R; s.tw = C::VALID; s.cinp = C::CINP; s.cexpp = C::CEXPP; s.coutp = C::COUTP;
    return s;
}

template <typename T, class C> void launch_wgstrip(int block, const IrArgs& a, int F, hipStream_t s) {
    const IrShape sh = ir_shape(block, std::is_same<T, bf16>::value);
    if (sh.cin != C::CIN || sh.cexp != C::CEXP || sh.cout != C::COUT || sh.k != C::KS || sh.stride != C::S ||
        sh.se != (int)C::SE || sh.hs != (int)C::HS || sh.cinp != C::CINP || sh.cexpp != C::CEXPP ||
        sh.coutp != C::COUTP)
        throw std::runtime_error("ir_wgstrip: weight padding disagrees with the block shape");
    const int strips = (a.Wo + C::VALID - 1) / C::VALID, steps = (a.Ho + C::R - 1) / C::R;
    if ((C::S == 1 && (a.Ho != a.H || a.Wo != a.W)) || (C::S == 2 && (a.Ho != (a.H + 1) / 2 || a.Wo != (a.W + 1) / 2)))
        throw std::runtime_error("ir_wgstrip: map shape does not match the stride");
    if (a.frames != F || (long long)F * strips > (1ll << 30)) throw std::runtime_error("ir_wgstrip: bad frame count");
    if (C::SE && (a.tiles_x != strips || a.ntiles != strips * steps))
        throw std::runtime_error("ir_wgstrip: SE partial-sum grid mismatch");
    if (C::XRN != C::IR && (steps != 1 || a.H != C::XRN))
        throw std::runtime_error("ir_wgstrip: whole-map staging needs the map in one step");
    if (C::NPOS < 16) {   // the staged positions must hold every map column of both pixel tiles
        const auto col = [](int lane, int t) { return C::S == 1 ? lane - C::PADK : 2 * (lane - 1) + t; };
        if (strips != 1 || col(C::POS0, 0) > 0 || col(C::POS0 + C::NPOS - 1, C::NT - 1) < a.W - 1)
            throw std::runtime_error("ir_wgstrip: staged positions do not cover the map");
    }
    static const int resident = [] {
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, ir_wgstrip_kernel<T, C>, C::THREADS, 0) != hipSuccess)
            throw std::runtime_error("ir_wgstrip: cannot query the device occupancy");
        return std::max(1, cus) * std::max(1, per_cu);
    }();
    // squeeze-excite blocks with fewer (frame, strip) items than resident workgroups deal each item's channel
    // tiles over several workgroups (at least one tile per wave each)
    int csplit = 1;
    if (C::SE && (long long)F * strips < resident)
        csplit = std::max(1, std::min(int(resident / ((long long)F * strips)), C::CT / C::WAVES));
    // still fewer items than resident workgroups: deal each strip's steps over segments as well
    int seg_steps = steps;
    if ((long long)F * strips * csplit < resident) {
        const int want = std::min<long long>(steps, resident / ((long long)F * strips * csplit));
        seg_steps = (steps + want - 1) / want;
    }
    const int segs = (steps + seg_steps - 1) / seg_steps;
    if ((long long)F * strips * csplit * segs > (1ll << 30)) throw std::runtime_error("ir_wgstrip: too many items");
    const int items = F * strips * csplit * segs;
    const int grid = std::min(items, resident);
    hipLaunchKernelGGL((ir_wgstrip_kernel<T, C>), dim3(grid), dim3(C::THREADS), 0, s, a, strips, steps, items,
                       csplit, segs, seg_steps);
}

}  // namespace

bool strip_kernels_enabled() {
    static const bool on = std::getenv("SHV_HIP_NO_STRIP") == nullptr;
    return on;
}

bool ir_strip_shape(int block, bool bf16_tier, IrShape* out) {
    switch (block) {
    case 3: *out = bf16_tier ? wg_shape<G4B>() : wg_shape<G4>(); return true;
    case 4: case 5: *out = wg_shape<G5>(); return true;
    case 6: *out = bf16_tier ? wg_shape<G7B>() : wg_shape<G7>(); return true;
    case 7: *out = wg_shape<G8>(); return true;
    case 8: case 9: *out = wg_shape<G9>(); return true;
    case 10: *out = wg_shape<G11>(); return true;
    case 11: *out = bf16_tier ? wg_shape<G12B>() : wg_shape<G12>(); return true;
    case 12: *out = wg_shape<G13>(); return true;
    case 13: case 14: *out = wg_shape<G14>(); return true;
    default: return false;
    }
}

template <typename T> bool launch_ir_strip(int block, const IrArgs& a, int F, hipStream_t s) {
    constexpr bool IS_BF16 = std::is_same<T, bf16>::value;
    switch (block) {
    case 0: launch_strip<T, S1>(block, a, F, s); return true;
    case 1: launch_strip<T, std::conditional_t<IS_BF16, S2B, S2>>(block, a, F, s); return true;
    case 2: launch_strip<T, std::conditional_t<IS_BF16, S3B, S3>>(block, a, F, s); return true;
    case 3: launch_wgstrip<T, std::conditional_t<IS_BF16, G4B, G4>>(block, a, F, s); return true;
    case 4: case 5: launch_wgstrip<T, G5>(block, a, F, s); return true;
    case 6: launch_wgstrip<T, std::conditional_t<IS_BF16, G7B, G7>>(block, a, F, s); return true;
    case 7: launch_wgstrip<T, G8>(block, a, F, s); return true;
    case 8: case 9: launch_wgstrip<T, G9>(block, a, F, s); return true;
    case 10: launch_wgstrip<T, G11>(block, a, F, s); return true;
    case 11: launch_wgstrip<T, std::conditional_t<IS_BF16, G12B, G12>>(block, a, F, s); return true;
    case 12: launch_wgstrip<T, G13>(block, a, F, s); return true;
    case 13: case 14: launch_wgstrip<T, G14>(block, a, F, s); return true;
    default: return false;
    }
}
template bool launch_ir_strip<f16>(int, const IrArgs&, int, hipStream_t);
template bool launch_ir_strip<bf16>(int, const IrArgs&, int, hipStream_t);

template <typename T> void launch_stem_block1(const IrArgs& a, int F, hipStream_t s) {
    if (!a.img || !a.lut || !a.stem_w || !a.stem_b || a.H != 90 || a.W != 160)
        throw std::runtime_error("stem + block 1: needs the frames, the table, the stem weights and the 90x160 map");
    launch_strip<T, S1, true>(0, a, F, s);
}
template void launch_stem_block1<f16>(const IrArgs&, int, hipStream_t);
template void launch_stem_block1<bf16>(const IrArgs&, int, hipStream_t);

}  // namespace shv
