// MobileNetV3 kernels other than the 1x1 convolutions (those are GEMMs): stem, depthwise, SE squeeze, 4x4 pool,
// and the on-GPU weight repacker.  NHWC fp32 activations.  Every output element is computed by the reference CPU
// engine's sequence of operations (engine/model/isa_impl.hpp:558-643, 757-769, 827-842), so the fp32 tier is bitwise
// equal to it.  The stem and the depthwise stage their inputs in LDS tiles with zeros outside the map, as the
// reference pads its rows.
#include "dev_common.hpp"
#include "kernels.hpp"

#include <stdexcept>
#include <type_traits>

namespace shv {
namespace {

inline unsigned int cdiv(long long a, long long b) { return (unsigned int)((a + b - 1) / b); }

// ------------------------------------------------------------------------------------------------ stem
// A workgroup owns a 6 x 32 tile of output pixels of one frame, one pixel per thread.  The 13 x 65 input patch
// that tile needs (stride 2, pad 1) is normalised through the byte -> float table into LDS once, zeros outside the
// image like the reference's padded rows (isa_impl.hpp:558-600); each pixel's 16 channels are then the fma chain
// over (dy, dx, c) from +0, + bias, hardswish.  The 27 x 16 weights are read at wave-uniform addresses (scalar
// loads into SGPR operands), one tap at a time.
constexpr int kStemTH = 6, kStemTW = 32;
__global__ void __launch_bounds__(kStemTH * kStemTW)
stem_tile_kernel(const uint8_t* __restrict__ in, float* __restrict__ out, const float* __restrict__ lut,
                 const float* __restrict__ w, const float* __restrict__ b) {
    constexpr int IH = 2 * kStemTH + 1, IW3 = (2 * kStemTW + 1) * 3;   // 13 rows x 65 pixels x 3 channels
    constexpr int NT = kStemTH * kStemTW;
    __shared__ float slut[768];
    __shared__ float patch[IH * IW3];
    for (int i = threadIdx.x; i < 768; i += NT) slut[i] = lut[i];
    __syncthreads();
    const int oy0 = blockIdx.y * kStemTH, ox0 = blockIdx.x * kStemTW;
    const uint8_t* img = in + (size_t)blockIdx.z * (180 * 320 * 3);
    const int col0 = (2 * ox0 - 1) * 3;                                 // byte column of patch column 0
    for (int i = threadIdx.x; i < IH * IW3; i += NT) {
        const int r = i / IW3, q = i - r * IW3;                         // q = 3 * patch column + channel
        const int iy = 2 * oy0 - 1 + r, bx = col0 + q;
        float v = 0.0f;
        if (iy >= 0 && iy < 180 && bx >= 0 && bx < 960) v = slut[(q % 3) * 256 + img[iy * 960 + bx]];
        patch[i] = v;
    }
    __syncthreads();
    const int ty = threadIdx.x / kStemTW, tx = threadIdx.x - ty * kStemTW;
    float acc[16];
#pragma unroll
    for (int o = 0; o < 16; ++o) acc[o] = 0.0f;
#pragma unroll 1
    for (int t = 0; t < 9; ++t) {
        const int dy = t / 3, dx = t - dy * 3;
        const float* px = patch + (2 * ty + dy) * IW3 + (2 * tx + dx) * 3;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const float x = px[c];
            const float* wr = w + (t * 3 + c) * 16;
#pragma unroll
            for (int o = 0; o < 16; ++o) acc[o] = __builtin_fmaf(x, wr[o], acc[o]);
        }
    }
    float v[16];
#pragma unroll
    for (int o = 0; o < 16; ++o) v[o] = hswish(acc[o] + b[o]);
    float* dst = out + (((size_t)blockIdx.z * 90 + oy0 + ty) * 160 + ox0 + tx) * 16;
    write8(dst, v);
    write8(dst + 8, v + 8);
}

// ------------------------------------------------------------------------------------------------ depthwise
// Depthwise KS x KS, stride S, fp32.  A workgroup owns TH x 8 output pixels x 32 channels of one frame: it stages
// the input halo [(TH-1)S+KS][7S+KS][32] in LDS with float4 loads (zeros outside the map and beyond C), then each
// thread takes one channel and one output column and walks the TH rows.  Every output is the fma chain over
// (dy, dx) in order from +0 -- padding taps add a zero product to a chain that started at +0, which changes
// nothing, so this equals the reference's chain over zero-padded rows (isa_impl.hpp:603-643) -- + bias, ReLU or
// hardswish.
constexpr int kDwTW = 8, kDwCC = 32;
template <int KS, int S>
__global__ void __launch_bounds__(256)
dw_tile_kernel(const float* __restrict__ in, float* __restrict__ out, const float* __restrict__ w,
               const float* __restrict__ b, int H, int W, int C, int Ho, int Wo, int tiles_x, int act) {
    constexpr int TH = S == 1 ? 8 : 4;
    constexpr int IH = (TH - 1) * S + KS, IW = (kDwTW - 1) * S + KS, P = (KS - 1) / 2;
    __shared__ float4 halo[IH * IW * (kDwCC / 4)];
    const int f = blockIdx.z, c0 = blockIdx.y * kDwCC;
    const int ty0 = (blockIdx.x / tiles_x) * TH, tx0 = (blockIdx.x % tiles_x) * kDwTW;
    const float* src = in + (size_t)f * H * W * C;
    for (int i = threadIdx.x; i < IH * IW * (kDwCC / 4); i += 256) {
        const int quad = i % (kDwCC / 4), pix = i / (kDwCC / 4);
        const int r = pix / IW, cx = pix - r * IW;
        const int iy = ty0 * S - P + r, ix = tx0 * S - P + cx, ch = c0 + 4 * quad;
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (iy >= 0 && iy < H && ix >= 0 && ix < W && ch < C)   // C % 8 == 0: a quad is all in or all out
            v = *reinterpret_cast<const float4*>(src + ((size_t)iy * W + ix) * C + ch);
        halo[i] = v;
    }
    __syncthreads();
    const int lane_c = threadIdx.x % kDwCC, col = threadIdx.x / kDwCC;
    const int ch = c0 + lane_c, ox = tx0 + col;
    if (ch >= C || ox >= Wo) return;
    float wt[KS * KS];
#pragma unroll
    for (int t = 0; t < KS * KS; ++t) wt[t] = w[t * C + ch];
    const float bias = b[ch];
    const float* hs = reinterpret_cast<const float*>(halo);
    float* dst = out + (size_t)f * Ho * Wo * C + ch;
#pragma unroll 1
    for (int yy = 0; yy < TH; ++yy) {
        const int oy = ty0 + yy;
        if (oy >= Ho) break;
        float acc = 0.0f;
#pragma unroll
        for (int dy = 0; dy < KS; ++dy)
#pragma unroll
            for (int dx = 0; dx < KS; ++dx)
                acc = __builtin_fmaf(hs[((yy * S + dy) * IW + col * S + dx) * kDwCC + lane_c], wt[dy * KS + dx], acc);
        dst[((size_t)oy * Wo + ox) * C] = apply_act(acc + bias, act);
    }
}

// ------------------------------------------------------------------------------------------------ SE squeeze
// SE mean in the CPU engine's order (engine/model/isa_impl.hpp:762-772): per channel, each row summed left to right
// from its first element, the row sums added top to bottom from the first row's, the total divided by (float)(Ho*Wo).
// The row sums are independent, so a workgroup (frame, 64 channels) gives each of SP_RG row groups its own rows
// (lanes on consecutive channels: 256-byte loads) and one thread per channel adds the row sums in order from LDS:
// the same operations as one serial loop, with a dependent chain of Wo + Ho adds instead of Ho * Wo.
constexpr int SP_CH = 64, SP_RG = 8, SP_MAXH = 64, SP_U = 8;
template <typename T>
__global__ void __launch_bounds__(SP_CH * SP_RG)
se_pool_kernel(const T* __restrict__ x, float* __restrict__ pooled, int Ho, int Wo, int C) {
    __shared__ float rows[SP_MAXH][SP_CH];
    const int cl = threadIdx.x % SP_CH, rg = threadIdx.x / SP_CH;
    const int c = blockIdx.y * SP_CH + cl;
    const long long f = blockIdx.x;
    const bool live = c < C;
    const T* base = x + f * Ho * Wo * C + (live ? c : 0);
    for (int y = rg; y < Ho; y += SP_RG) {
        const T* row = base + (long long)y * Wo * C;
        float acc = to_f(row[0]);
        for (int x0 = 1; x0 < Wo; x0 += SP_U) {
            float v[SP_U];
#pragma unroll
            for (int i = 0; i < SP_U; ++i) v[i] = x0 + i < Wo ? to_f(row[(long long)(x0 + i) * C]) : 0.0f;
#pragma unroll
            for (int i = 0; i < SP_U; ++i)
                if (x0 + i < Wo) acc = acc + v[i];
        }
        rows[y][cl] = acc;
    }
    __syncthreads();
    if (rg == 0 && live) {
        float tot = rows[0][cl];
        for (int y = 1; y < Ho; ++y) tot = tot + rows[y][cl];
        pooled[f * C + c] = tot / float(Ho * Wo);
    }
}

// ------------------------------------------------------------------------------------------------ 4x4 pool
// Adaptive 6x10 -> 4x4 average pool (overlapping bins: rows {0,1,3,4}[r] + [0,2), columns {0,2,5,7}[c] + [0,3)).
// A workgroup owns one frame and a PL_CH-channel slice: it stages the slice of all 60 pixels in LDS with 16-byte
// loads (every input value leaves HBM once, although the bins overlap), then each thread sums bins from LDS.  Per
// output: +0, then the 6 values row by row, left to right, then (acc / 2) / 3 -- the reference CPU engine's
// operation order (engine/model/isa_impl.hpp:836-842).
constexpr int PL_CH = 240;   // channels per workgroup: 960 / 4, 57.6 KB of LDS
template <typename T>
__global__ void __launch_bounds__(256) pool_kernel(const T* __restrict__ in, T* __restrict__ out) {
    __shared__ float tile[60 * PL_CH];
    const long long f = blockIdx.x;
    const int c0 = blockIdx.y * PL_CH;
    const T* src = in + f * 60 * 960 + c0;
    constexpr int V4 = PL_CH / 4;   // 16-byte pieces per pixel
    for (int i = threadIdx.x; i < 60 * V4; i += 256) {
        const int px = i / V4, q = i % V4;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = to_f(src[px * 960 + q * 4 + e]);
        *reinterpret_cast<float4*>(&tile[px * PL_CH + q * 4]) = make_float4(v[0], v[1], v[2], v[3]);
    }
    __syncthreads();
    T* dst = out + f * 16 * 960 + c0;
    for (int o = threadIdx.x; o < 16 * PL_CH; o += 256) {
        const int tok = o / PL_CH, c = o % PL_CH;
        const int y0 = ((tok >> 2) * 3) >> 1;   // floor(r * 6 / 4)
        const int x0 = ((tok & 3) * 5) >> 1;    // floor(c * 10 / 4)
        float acc = 0.0f;
#pragma unroll
        for (int dy = 0; dy < 2; ++dy)
#pragma unroll
            for (int dx = 0; dx < 3; ++dx) acc = acc + tile[((y0 + dy) * 10 + x0 + dx) * PL_CH + c];
        dst[tok * 960 + c] = from_f<T>((acc / 2.0f) / 3.0f);
    }
}

// ------------------------------------------------------------------------------------------------ repack
template <typename T>
__global__ void __launch_bounds__(256)
repack_kernel(const float* __restrict__ src, T* __restrict__ dst, int N, int K, int perm, int parts, int group_major) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)N * K) return;
    const int r = int(idx / K), k = int(idx % K);
    const int F = N / 2;
    int sr = r;
    if (perm == 1) sr = (r & 1) ? F + (r >> 1) : (r >> 1);
    else if (perm == 2) {
        const int panel = r >> 4, l = r & 15;
        sr = ((panel & 1) ? F : 0) + (panel >> 1) * 16 + l;
    }
    float rest = src[(long long)sr * K + k];
    const long long o = group_major ? (long long)(k >> 5) * N * 32 + r * 32 + (k & 31) : idx;
    for (int q = 0; q < parts; ++q) {   // part q = T(rounding residual left by parts 0..q-1)
        const T v = from_f<T>(rest);
        dst[(long long)q * N * K + o] = v;
        rest = rest - to_f(v);
    }
}

template <typename T>
__global__ void __launch_bounds__(256)
repack_pad_kernel(const float* __restrict__ src, T* __restrict__ dst, int N, int K, int Np, int Kp, int parts) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)Np * Kp) return;
    const int r = int(idx / Kp), k = int(idx % Kp);
    float rest = (r < N && k < K) ? src[(long long)r * K + k] : 0.0f;
    for (int q = 0; q < parts; ++q) {
        const T v = from_f<T>(rest);
        dst[(long long)q * Np * Kp + idx] = v;
        rest = rest - to_f(v);
    }
}

}  // namespace

template <typename T>
void launch_repack_pad(const float* src, T* dst, int N, int K, int Np, int Kp, int parts, hipStream_t s) {
    hipLaunchKernelGGL(repack_pad_kernel<T>, dim3(cdiv((long long)Np * Kp, 256)), dim3(256), 0, s, src, dst, N, K, Np,
                       Kp, parts);
}
template void launch_repack_pad<f16>(const float*, f16*, int, int, int, int, int, hipStream_t);
template void launch_repack_pad<bf16>(const float*, bf16*, int, int, int, int, int, hipStream_t);

template <typename T>
void launch_stem(const uint8_t* in, T* out, const float* lut, const float* w, const float* b, int F, hipStream_t s) {
    static_assert(std::is_same<T, float>::value, "activations are fp32 in every tier");
    hipLaunchKernelGGL(stem_tile_kernel, dim3(160 / kStemTW, 90 / kStemTH, F), dim3(kStemTH * kStemTW), 0, s, in, out,
                       lut, w, b);
}

template <typename T>
void launch_dw(const T* in, T* out, const float* w, const float* b, int F, int H, int W, int C, int K, int S, int Ho,
               int Wo, int act, hipStream_t s) {
    static_assert(std::is_same<T, float>::value, "activations are fp32 in every tier");
    if (C % 8) throw std::runtime_error("depthwise: C % 8 != 0");
    const int th = S == 1 ? 8 : 4;
    const int tiles_x = int(cdiv(Wo, kDwTW)), tiles = tiles_x * int(cdiv(Ho, th));
    const dim3 grid(tiles, cdiv(C, kDwCC), F), blk(256);
    if (K == 3 && S == 1) hipLaunchKernelGGL((dw_tile_kernel<3, 1>), grid, blk, 0, s, in, out, w, b, H, W, C, Ho, Wo, tiles_x, act);
    else if (K == 3 && S == 2) hipLaunchKernelGGL((dw_tile_kernel<3, 2>), grid, blk, 0, s, in, out, w, b, H, W, C, Ho, Wo, tiles_x, act);
    else if (K == 5 && S == 1) hipLaunchKernelGGL((dw_tile_kernel<5, 1>), grid, blk, 0, s, in, out, w, b, H, W, C, Ho, Wo, tiles_x, act);
    else if (K == 5 && S == 2) hipLaunchKernelGGL((dw_tile_kernel<5, 2>), grid, blk, 0, s, in, out, w, b, H, W, C, Ho, Wo, tiles_x, act);
    else throw std::runtime_error("depthwise: unsupported kernel/stride");
}

template <typename T> void launch_se_pool(const T* x, float* pooled, int F, int Ho, int Wo, int C, hipStream_t s) {
    if (Ho > SP_MAXH || Ho < 1 || Wo < 1) throw std::runtime_error("se_pool: map height outside 1..64");
    if (F < 1) return;
    hipLaunchKernelGGL(se_pool_kernel<T>, dim3((unsigned)F, cdiv(C, SP_CH)), dim3(SP_CH * SP_RG), 0, s, x, pooled, Ho,
                       Wo, C);
}

template <typename T> void launch_pool(const T* in, T* out, int F, hipStream_t s) {
    hipLaunchKernelGGL(pool_kernel<T>, dim3((unsigned)F, 960 / PL_CH), dim3(256), 0, s, in, out);
}

template <typename T>
void launch_repack(const float* src, T* dst, int N, int K, int perm, int parts, hipStream_t s, bool group_major) {
    if (group_major && K % 32) throw std::runtime_error("repack: the group-major layout needs K % 32 == 0");
    hipLaunchKernelGGL(repack_kernel<T>, dim3(cdiv((long long)N * K, 256)), dim3(256), 0, s, src, dst, N, K, perm,
                       parts, int(group_major));
}

template void launch_stem<float>(const uint8_t*, float*, const float*, const float*, const float*, int, hipStream_t);
template void launch_dw<float>(const float*, float*, const float*, const float*, int, int, int, int, int, int, int, int,
                               int, hipStream_t);
template void launch_se_pool<float>(const float*, float*, int, int, int, int, hipStream_t);
template void launch_pool<float>(const float*, float*, int, hipStream_t);
template void launch_repack<float>(const float*, float*, int, int, int, int, hipStream_t, bool);
template void launch_repack<f16>(const float*, f16*, int, int, int, int, hipStream_t, bool);
template void launch_repack<bf16>(const float*, bf16*, int, int, int, int, hipStream_t, bool);

}  // namespace shv
