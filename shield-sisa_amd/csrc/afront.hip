// SHIELD-A frontend kernels for gfx950 (the reference: engine/audio/frontend.cpp): the log-mel frames of a 10 s
// window, the CNN's stem and depthwise layers, and the frequency-attention pooling.  The CNN's 1x1 layers and the
// token projection are GEMMs of the engine's tiers.  Activations are fp32 in HBM, image layout [time][freq][channel].
//
// Per element these kernels perform the reference's IEEE operations in its order (the reference is compiled with
// -ffp-contract=off, and so is this file): the radix-2 FFT's butterflies, the power spectrum, the filterbank fma
// chain, the stem's fma chain over its nine taps, the depthwise sum of products over (kf, kt) skipping the padding
// taps, BatchNorm as a product then a sum, the softmax's running sum.  The transcendental functions (exp in SiLU and
// the softmax, log of the mel energies) are the device's, within an ulp or two of glibc's.
#include "dev_common.hpp"
#include "kernels.hpp"

#include <stdexcept>

namespace shv {
namespace {

inline unsigned int cdiv(long long a, long long b) { return (unsigned int)((a + b - 1) / b); }

// waits for the wave's own LDS accesses: LDS executes one wave's instructions in order, so after this every lane
// sees what every lane of the wave wrote before
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

__device__ __forceinline__ float silu_libm(float y) { return y / (1.0f + expf(0.0f - y)); }

// ---------------------------------------------------------------------------------------------------- log-mel
// One wave per frame, four frames per workgroup.  Frame t's 400 windowed samples pcm[t * 160 + 56 + j] * window[j]
// go to the bit-reversed slots of a 512-point buffer (the rest zero), nine radix-2 stages run in place with the
// twiddles e^{-2 pi i k / 512} (host-computed in double, rounded to float), then |X_k|^2 for k <= 256, each mel bin's
// fma chain over its filter's nonzero taps in increasing k, and (log(e + 1e-6) - mean) / std
// (frontend.cpp:245-256).
constexpr int MEL_WAVES = 4;

__global__ void __launch_bounds__(64 * MEL_WAVES) audio_mel_kernel(const float* __restrict__ pcm, long long stride,
                                                                   AudioMelTables tb, float* __restrict__ mel) {
    __shared__ float re[MEL_WAVES][512], im[MEL_WAVES][512];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x * MEL_WAVES + wave;
    if (t >= kAudioMelFrames) return;   // wave-uniform; no workgroup barrier follows
    const long long win = blockIdx.y;
    float* R = re[wave];
    float* I = im[wave];
    for (int i = lane; i < 512; i += 64) {
        R[i] = 0.0f;
        I[i] = 0.0f;
    }
    wave_lds_sync();
    const float* x = pcm + win * stride + (long long)t * 160;
    for (int n = 56 + lane; n < 456; n += 64) R[__builtin_bitreverse32(unsigned(n)) >> 23] = x[n] * tb.window[n - 56];
    wave_lds_sync();
#pragma unroll 1
    for (int lh = 0; lh < 9; ++lh) {   // half = 2^lh, size = 2 half, twiddle step 256 / half
        const int half = 1 << lh;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int b = lane + 64 * q;                  // butterfly 0..255
            const int j = b & (half - 1), a = ((b >> lh) << (lh + 1)) + j, c = a + half;
            const int k = j << (8 - lh);
            const float wr = tb.wr[k], wi = tb.wi[k];
            const float rb = R[c], ib = I[c], ra = R[a], ia = I[a];
            const float r = wr * rb - wi * ib, ii = wr * ib + wi * rb;
            R[a] = ra + r;
            I[a] = ia + ii;
            R[c] = ra - r;
            I[c] = ia - ii;
        }
        wave_lds_sync();
    }
    for (int k = lane; k <= 256; k += 64) R[k] = R[k] * R[k] + I[k] * I[k];
    wave_lds_sync();
    float* out = mel + (win * kAudioMelFrames + t) * kAudioMelBins;
    for (int m = lane; m < kAudioMelBins; m += 64) {
        float v = 0.0f;
        for (int e = tb.fb_off[m]; e < tb.fb_off[m + 1]; ++e) v = __builtin_fmaf(tb.fb_w[e], R[tb.fb_k[e]], v);
        out[m] = (logf(v + 1e-6f) - tb.mean[m]) / tb.stdv[m];
    }
}

// ---------------------------------------------------------------------------------------------------- stem
// 3x3 convolution 1 -> 32 channels over the [997][80] log-mel image (zero padding), BatchNorm, SiLU
// (frontend.cpp:205-212): per output an fma chain from +0 over the taps q = 3 kf + kt (a padding tap adds a zero
// product, as the reference's zero patch entries do).  Four lanes per pixel, eight channels each.
__global__ void __launch_bounds__(256) audio_stem_kernel(const float* __restrict__ mel, const float* __restrict__ w,
                                                         const float* __restrict__ scale,
                                                         const float* __restrict__ shift, float* __restrict__ out,
                                                         long long pixels) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= pixels * 4) return;
    const long long px = i >> 2;
    const int c0 = int(i & 3) * 8;
    const long long win = px / (kAudioMelFrames * kAudioMelBins);
    const int rem = int(px - win * (kAudioMelFrames * kAudioMelBins));
    const int t = rem / kAudioMelBins, f = rem - t * kAudioMelBins;
    const float* m = mel + win * (kAudioMelFrames * kAudioMelBins);
    float patch[9];
#pragma unroll
    for (int kf = 0; kf < 3; ++kf)
#pragma unroll
        for (int kt = 0; kt < 3; ++kt) {
            const int ti = t + kt - 1, fi = f + kf - 1;
            patch[kf * 3 + kt] =
                (ti >= 0 && ti < kAudioMelFrames && fi >= 0 && fi < kAudioMelBins) ? m[ti * kAudioMelBins + fi] : 0.0f;
        }
    float y[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < 9; ++q) s = __builtin_fmaf(patch[q], w[(c0 + c) * 9 + q], s);
        const float v = s * scale[c0 + c] + shift[c0 + c];
        y[c] = silu_libm(v);
    }
    float4* o = reinterpret_cast<float4*>(out + px * 32 + c0);
    o[0] = make_float4(y[0], y[1], y[2], y[3]);
    o[1] = make_float4(y[4], y[5], y[6], y[7]);
}

// ---------------------------------------------------------------------------------------------------- depthwise
// 3x3 depthwise with strides (time st, freq sf), padding 1, BatchNorm, SiLU (frontend.cpp:32-39, 188-192): per output
// sum = sum + x * w from +0 over kf, then kt, skipping taps outside the image.  A lane takes 4 channels of DW_TO
// consecutive time outputs of one frequency column: the 9 weight quads are loaded once and the input rows the outputs
// share (kt = 2 of output j is kt = 0 of output j + 1 at stride 1) once per kf, while every output still adds its
// products in the (kf, kt) order above.
constexpr int DW_TO = 4;
template <int ST>
__global__ void __launch_bounds__(256) audio_dw_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                       const float* __restrict__ w, const float* __restrict__ scale,
                                                       const float* __restrict__ shift, int T, int F, int C, int sf,
                                                       int To, int Fo, long long total) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int C4 = C >> 2;
    const int c = int(i % C4) * 4;
    const long long px = i / C4;   // (window, time group, frequency column)
    const int fo = int(px % Fo);
    const long long r = px / Fo;
    const int tgroups = (To + DW_TO - 1) / DW_TO;
    const int to0 = int(r % tgroups) * DW_TO;
    const long long win = r / tgroups;
    const float* x = in + win * T * F * C;
    constexpr int NR = ST * (DW_TO - 1) + 3;   // input rows of the group's outputs: ST * to0 - 1 + 0 .. NR - 1
    float4 k[9];
#pragma unroll
    for (int q = 0; q < 9; ++q) k[q] = *reinterpret_cast<const float4*>(w + q * C + c);
    float4 sum[DW_TO];
#pragma unroll
    for (int j = 0; j < DW_TO; ++j) sum[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const int ti0 = ST * to0 - 1;
#pragma unroll
    for (int kf = 0; kf < 3; ++kf) {
        const int fi = fo * sf + kf - 1;
        if (fi < 0 || fi >= F) continue;
        float4 v[NR];
#pragma unroll
        for (int j = 0; j < NR; ++j) {
            const int ti = min(max(ti0 + j, 0), T - 1);   // clamped: rows outside the image are skipped below
            v[j] = *reinterpret_cast<const float4*>(x + ((long long)ti * F + fi) * C + c);
        }
#pragma unroll
        for (int j = 0; j < DW_TO; ++j)
#pragma unroll
            for (int kt = 0; kt < 3; ++kt) {
                const int ti = ti0 + ST * j + kt;
                if (ti < 0 || ti >= T) continue;
                const float4 a = v[ST * j + kt], b = k[kf * 3 + kt];
                sum[j].x = sum[j].x + a.x * b.x;
                sum[j].y = sum[j].y + a.y * b.y;
                sum[j].z = sum[j].z + a.z * b.z;
                sum[j].w = sum[j].w + a.w * b.w;
            }
    }
    const float4 sc = *reinterpret_cast<const float4*>(scale + c), sh = *reinterpret_cast<const float4*>(shift + c);
#pragma unroll
    for (int j = 0; j < DW_TO; ++j) {
        const int to = to0 + j;
        if (to >= To) break;
        const float4 y = make_float4(silu_libm(sum[j].x * sc.x + sh.x), silu_libm(sum[j].y * sc.y + sh.y),
                                     silu_libm(sum[j].z * sc.z + sh.z), silu_libm(sum[j].w * sc.w + sh.w));
        *reinterpret_cast<float4*>(out + ((win * To + to) * Fo + fo) * C + c) = y;
    }
}

// ---------------------------------------------------------------------------------------------------- attention
// Frequency attention over the [125][20][192] image (frontend.cpp:222-231), one wave per time step: the 20 logits
// (an fma chain from +0 over the 192 channels, then + bias), their softmax (running max, exp(l - max), the sum in
// frequency order, division), and pooled[c] = sum over f of v * a_f from +0 in frequency order.
__global__ void __launch_bounds__(256) audio_freq_pool_kernel(const float* __restrict__ h, const float* __restrict__ w,
                                                              float bias, float* __restrict__ pooled, long long steps) {
    __shared__ float a[4][kAudioCnnFreq];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const long long step = (long long)blockIdx.x * 4 + wave;
    if (step >= steps) return;   // wave-uniform
    const float* v = h + step * (kAudioCnnFreq * kAudioCnnCh);
    float l = 0.0f;
    if (lane < kAudioCnnFreq) {
        const float* row = v + lane * kAudioCnnCh;
        for (int c = 0; c < kAudioCnnCh; ++c) l = __builtin_fmaf(row[c], w[c], l);
        l = l + bias;
        a[wave][lane] = l;
    }
    wave_lds_sync();
    float mx = -__builtin_inff();
    for (int f = 0; f < kAudioCnnFreq; ++f) mx = fmaxf(mx, a[wave][f]);
    wave_lds_sync();
    const float e = expf(l - mx);
    if (lane < kAudioCnnFreq) a[wave][lane] = e;
    wave_lds_sync();
    float sum = 0.0f;
    for (int f = 0; f < kAudioCnnFreq; ++f) sum = sum + a[wave][f];
    wave_lds_sync();
    if (lane < kAudioCnnFreq) a[wave][lane] = e / sum;
    wave_lds_sync();
    for (int c = lane; c < kAudioCnnCh; c += 64) {
        float p = 0.0f;
        for (int f = 0; f < kAudioCnnFreq; ++f) p = p + v[f * kAudioCnnCh + c] * a[wave][f];
        pooled[step * kAudioCnnCh + c] = p;
    }
}

}  // namespace

void launch_audio_mel(const float* pcm, long long stride, int n, const AudioMelTables& tb, float* mel, hipStream_t s) {
    if (n <= 0) return;
    if (!pcm || !mel || stride < kAudioWindowSamples) throw std::runtime_error("audio mel: bad PCM or window stride");
    hipLaunchKernelGGL(audio_mel_kernel, dim3(cdiv(kAudioMelFrames, MEL_WAVES), (unsigned)n), dim3(64 * MEL_WAVES), 0,
                       s, pcm, stride, tb, mel);
}

void launch_audio_stem(const float* mel, const float* w, const float* scale, const float* shift, float* out, int n,
                       hipStream_t s) {
    if (n <= 0) return;
    const long long pixels = (long long)n * kAudioMelFrames * kAudioMelBins;
    hipLaunchKernelGGL(audio_stem_kernel, dim3(cdiv(pixels * 4, 256)), dim3(256), 0, s, mel, w, scale, shift, out,
                       pixels);
}

void launch_audio_dw(const float* in, float* out, const float* w, const float* scale, const float* shift, int n,
                     int T, int F, int C, int st, int sf, hipStream_t s) {
    if (n <= 0) return;
    if (C % 4 || st < 1 || st > 2 || sf < 1 || sf > 2) throw std::runtime_error("audio depthwise: bad shape");
    const int To = (T + st - 1) / st, Fo = (F + sf - 1) / sf;
    const long long total = (long long)n * ((To + DW_TO - 1) / DW_TO) * Fo * (C / 4);
    if (st == 1)
        hipLaunchKernelGGL(audio_dw_kernel<1>, dim3(cdiv(total, 256)), dim3(256), 0, s, in, out, w, scale, shift, T,
                           F, C, sf, To, Fo, total);
    else
        hipLaunchKernelGGL(audio_dw_kernel<2>, dim3(cdiv(total, 256)), dim3(256), 0, s, in, out, w, scale, shift, T,
                           F, C, sf, To, Fo, total);
}

void launch_audio_freq_pool(const float* h, const float* w, float bias, float* pooled, int n, hipStream_t s) {
    if (n <= 0) return;
    const long long steps = (long long)n * kAudioTokensPerWindow;
    hipLaunchKernelGGL(audio_freq_pool_kernel, dim3(cdiv(steps, 4)), dim3(256), 0, s, h, w, bias, pooled, steps);
}

}  // namespace shv
