// MobileNetV3 kernels other than the 1x1 convolutions (those are GEMMs): stem, depthwise, SE squeeze, 4x4 pool,
// and the on-GPU weight repacker.  NHWC activations in storage type T, fp32 arithmetic.  Every output element is
// computed by the reference CPU engine's sequence of operations (engine/model/isa_impl.hpp:558-643, 757-769,
// 827-842), so the fp32 tier is bitwise equal to it; padding taps are skipped (adding a zero product changes
// at most the sign of a zero).
#include "dev_common.hpp"
#include "kernels.hpp"

#include <stdexcept>

namespace shv {
namespace {

inline unsigned int cdiv(long long a, long long b) { return (unsigned int)((a + b - 1) / b); }

// ------------------------------------------------------------------------------------------------ stem
// one thread per output pixel: 3x3 stride-2 conv over the LUT-normalised input (fma chain over (dy, dx, c)),
// + bias, hardswish, 16 channels stored as two 16-byte (half) / 32-byte (fp32) vectors
template <typename T>
__global__ void __launch_bounds__(256)
stem_kernel(const uint8_t* __restrict__ in, T* __restrict__ out, const float* __restrict__ lut,
            const float* __restrict__ w, const float* __restrict__ b, int F) {
    // the byte -> float table in LDS (per-lane index); weights and bias are read at wave-uniform constant offsets,
    // which the compiler serves from the scalar data cache into SGPR operands
    __shared__ float slut[768];
    for (int i = threadIdx.x; i < 768; i += blockDim.x) slut[i] = lut[i];
    __syncthreads();
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)F * 90 * 160) return;
    const int ox = int(idx % 160), oy = int((idx / 160) % 90);
    const long long f = idx / (90 * 160);
    float acc[16];
#pragma unroll
    for (int o = 0; o < 16; ++o) acc[o] = 0.0f;
    // taps (dy, dx) in order, one at a time (rolled: one tap's 48 weights live in scalar registers)
#pragma unroll 1
    for (int t = 0; t < 9; ++t) {
        const int dy = t / 3, dx = t - dy * 3;
        const int iy = 2 * oy - 1 + dy, ix = 2 * ox - 1 + dx;
        if (iy < 0 || iy >= 180 || ix < 0 || ix >= 320) continue;
        const uint8_t* px = in + ((f * 180 + iy) * 320 + ix) * 3;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const float x = slut[c * 256 + px[c]];
            const float* wr = w + (t * 3 + c) * 16;
#pragma unroll
            for (int o = 0; o < 16; ++o) acc[o] = __builtin_fmaf(x, wr[o], acc[o]);
        }
    }
    float v[16];
#pragma unroll
    for (int o = 0; o < 16; ++o) v[o] = hswish(acc[o] + b[o]);
    store8(out + idx * 16, v);
    store8(out + idx * 16 + 8, v + 8);
}

// ------------------------------------------------------------------------------------------------ depthwise
// one thread per (output pixel, 8 channels): fma chain over (dy, dx) from +0, + bias, activation
template <typename T, int KS, int S>
__global__ void __launch_bounds__(256)
dw_kernel(const T* __restrict__ in, T* __restrict__ out, const float* __restrict__ w, const float* __restrict__ b,
          int F, int H, int W, int C, int Ho, int Wo, int act) {
    const int CG = C >> 3;
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)F * Ho * Wo * CG) return;
    const int cg = int(idx % CG);
    const long long pix = idx / CG;
    const int ox = int(pix % Wo);
    const long long fy = pix / Wo;
    const int oy = int(fy % Ho);
    const long long f = fy / Ho;
    constexpr int P = (KS - 1) / 2;
    const int c0 = cg * 8;
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int dy = 0; dy < KS; ++dy) {
        const int iy = oy * S - P + dy;
        if (iy < 0 || iy >= H) continue;
#pragma unroll
        for (int dx = 0; dx < KS; ++dx) {
            const int ix = ox * S - P + dx;
            if (ix < 0 || ix >= W) continue;
            float x[8], wv[8];
            load8(in + ((f * H + iy) * W + ix) * C + c0, x);
            load8(w + (dy * KS + dx) * C + c0, wv);
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] = __builtin_fmaf(x[i], wv[i], acc[i]);
        }
    }
    float bb[8], v[8];
    load8(b + c0, bb);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = apply_act(acc[i] + bb[i], act);
    store8(out + pix * C + c0, v);
}

// ------------------------------------------------------------------------------------------------ SE squeeze
// one thread per (frame, channel): row sums left to right, rows added in order, divided by (float)(Ho*Wo)
template <typename T>
__global__ void __launch_bounds__(256)
se_pool_kernel(const T* __restrict__ x, float* __restrict__ pooled, int F, int Ho, int Wo, int C) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)F * C) return;
    const int c = int(idx % C);
    const long long f = idx / C;
    const T* base = x + f * Ho * Wo * C + c;
    float tot = 0.0f;
    for (int y = 0; y < Ho; ++y) {
        const T* row = base + (long long)y * Wo * C;
        float acc = to_f(row[0]);
        for (int xx = 1; xx < Wo; ++xx) acc = acc + to_f(row[(long long)xx * C]);
        tot = y == 0 ? acc : tot + acc;
    }
    pooled[idx] = tot / float(Ho * Wo);
}

// ------------------------------------------------------------------------------------------------ 4x4 pool
// token t = r*4 + c over rows {0,1,3,4}[r]+[0,2), cols {0,2,5,7}[c]+[0,3): sum from +0, then (acc / 2) / 3
template <typename T>
__global__ void __launch_bounds__(256) pool_kernel(const T* __restrict__ in, T* __restrict__ out, int F) {
    constexpr int CG = 960 / 8;
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)F * 16 * CG) return;
    const int cg = int(idx % CG), tok = int((idx / CG) % 16);
    const long long f = idx / (16 * CG);
    const int r0 = ((tok >> 2) * 3) >> 1;   // floor(r * 6 / 4): 0, 1, 3, 4
    const int c0 = ((tok & 3) * 5) >> 1;    // floor(c * 10 / 4): 0, 2, 5, 7
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    for (int y = r0; y < r0 + 2; ++y)
        for (int x = c0; x < c0 + 3; ++x) {
            float v[8];
            load8(in + ((f * 6 + y) * 10 + x) * 960 + cg * 8, v);
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] = acc[i] + v[i];
        }
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = (acc[i] / 2.0f) / 3.0f;
    store8(out + (f * 16 + tok) * 960 + cg * 8, acc);
}

// ------------------------------------------------------------------------------------------------ repack
template <typename T>
__global__ void __launch_bounds__(256)
repack_kernel(const float* __restrict__ src, T* __restrict__ dst, int N, int K, int perm, int parts) {
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
    for (int q = 0; q < parts; ++q) {   // part q = T(rounding residual left by parts 0..q-1)
        const T v = from_f<T>(rest);
        dst[(long long)q * N * K + idx] = v;
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
    hipLaunchKernelGGL(stem_kernel<T>, dim3(cdiv((long long)F * 14400, 256)), dim3(256), 0, s, in, out, lut, w, b, F);
}

template <typename T>
void launch_dw(const T* in, T* out, const float* w, const float* b, int F, int H, int W, int C, int K, int S, int Ho,
               int Wo, int act, hipStream_t s) {
    if (C % 8) throw std::runtime_error("depthwise: C % 8 != 0");
    const dim3 grid(cdiv((long long)F * Ho * Wo * (C / 8), 256)), blk(256);
    if (K == 3 && S == 1) hipLaunchKernelGGL((dw_kernel<T, 3, 1>), grid, blk, 0, s, in, out, w, b, F, H, W, C, Ho, Wo, act);
    else if (K == 3 && S == 2) hipLaunchKernelGGL((dw_kernel<T, 3, 2>), grid, blk, 0, s, in, out, w, b, F, H, W, C, Ho, Wo, act);
    else if (K == 5 && S == 1) hipLaunchKernelGGL((dw_kernel<T, 5, 1>), grid, blk, 0, s, in, out, w, b, F, H, W, C, Ho, Wo, act);
    else if (K == 5 && S == 2) hipLaunchKernelGGL((dw_kernel<T, 5, 2>), grid, blk, 0, s, in, out, w, b, F, H, W, C, Ho, Wo, act);
    else throw std::runtime_error("depthwise: unsupported kernel/stride");
}

template <typename T> void launch_se_pool(const T* x, float* pooled, int F, int Ho, int Wo, int C, hipStream_t s) {
    hipLaunchKernelGGL(se_pool_kernel<T>, dim3(cdiv((long long)F * C, 256)), dim3(256), 0, s, x, pooled, F, Ho, Wo, C);
}

template <typename T> void launch_pool(const T* in, T* out, int F, hipStream_t s) {
    hipLaunchKernelGGL(pool_kernel<T>, dim3(cdiv((long long)F * 16 * 120, 256)), dim3(256), 0, s, in, out, F);
}

template <typename T> void launch_repack(const float* src, T* dst, int N, int K, int perm, int parts, hipStream_t s) {
    hipLaunchKernelGGL(repack_kernel<T>, dim3(cdiv((long long)N * K, 256)), dim3(256), 0, s, src, dst, N, K, perm,
                       parts);
}

template void launch_stem<float>(const uint8_t*, float*, const float*, const float*, const float*, int, hipStream_t);
template void launch_dw<float>(const float*, float*, const float*, const float*, int, int, int, int, int, int, int, int,
                               int, hipStream_t);
template void launch_se_pool<float>(const float*, float*, int, int, int, int, hipStream_t);
template void launch_pool<float>(const float*, float*, int, hipStream_t);
template void launch_repack<float>(const float*, float*, int, int, int, int, hipStream_t);
template void launch_repack<f16>(const float*, f16*, int, int, int, int, hipStream_t);
template void launch_repack<bf16>(const float*, bf16*, int, int, int, int, hipStream_t);

}  // namespace shv
