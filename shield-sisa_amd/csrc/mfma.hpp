// Split-operand MFMA for the fp16 / bf16 tiers on gfx950 (and its one-part fp32 form).
//
// Every fp32 operand value x is carried as a sum of T parts (fp16: hi + lo, bf16: hi + mid + lo, each part the
// rounding of what the previous parts leave).  The products whose magnitude can exceed ~2^-24 of hi*hi are issued
// as separate v_mfma_f32_16x16x32_{f16,bf16} into one fp32 accumulator, smallest first (fp16: 3 products,
// bf16: 6).  The matrix cores then deliver fp32-level operand precision: the random-init SHIELD-V encoder
// amplifies operand rounding ~100x, and plain fp16 operands moved logits by up to 1.1 on the seeded set.
//
// Fragment layout of v_mfma_f32_16x16x32 (64 lanes, lane l = 16 g + r):
//   A (16 x 32): lane holds row r, k = 8 g .. 8 g + 7
//   B (32 x 16): lane holds column r, k = 8 g .. 8 g + 7
//   C (16 x 16): lane holds column r, rows 4 g .. 4 g + 3 (element i of the f32x4)
#pragma once
#include "dev_common.hpp"

namespace shv {

template <typename T> struct Split;

template <> struct Split<f16> {
    typedef f16x8 V8;
    static constexpr int P = 2;     // hi, lo
    static constexpr int NPROD = 3; // (a part, w part) products, smallest first
    static __device__ __forceinline__ int ap(int i) { return i == 0 ? 1 : 0; }
    static __device__ __forceinline__ int wp(int i) { return i == 1 ? 1 : 0; }
    static __device__ __forceinline__ void split(float x, f16* part) {
        // x must be the fp32 value itself: without this the compiler may round a product a * b feeding x straight
        // to fp16 (v_fma_mixlo_f16, one rounding of the exact product) while lo is formed from the fp32-rounded
        // x, so that hi + lo is off by an fp16 ulp near ties
        asm("" : "+v"(x));
        const f16 h = f16(x);
        part[0] = h;
        part[1] = f16(x - float(h));
    }
    // two values at once, the same roundings as split: each part pair is one packed conversion, and hi goes back
    // to fp32 from the packed pair (as split one by one, the compiler converts x to fp16 twice: unpacked for the
    // remainder and again packed for the store)
    typedef f16x2 V2;
    static __device__ __forceinline__ void split2(float x0, float x1, V2* part) {
        asm("" : "+v"(x0), "+v"(x1));
        const V2 h = __builtin_convertvector(f32x2{x0, x1}, V2);
        part[0] = h;
        part[1] = __builtin_convertvector(f32x2{x0 - float(h[0]), x1 - float(h[1])}, V2);
    }
    static __device__ __forceinline__ f32x4 mfma(V8 a, V8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

template <> struct Split<bf16> {
    typedef bf16x8 V8;
    static constexpr int P = 3;     // hi, mid, lo
    static constexpr int NPROD = 6;
    // products (lo,hi) (hi,lo) (mid,mid) (mid,hi) (hi,mid) (hi,hi)
    static __device__ __forceinline__ int ap(int i) { const int t[6] = {2, 0, 1, 1, 0, 0}; return t[i]; }
    static __device__ __forceinline__ int wp(int i) { const int t[6] = {0, 2, 1, 0, 1, 0}; return t[i]; }
    static __device__ __forceinline__ void split(float x, bf16* part) {
        asm("" : "+v"(x));   // the fp32 value itself (as in Split<f16>::split)
        const bf16 h = bf16(x);
        const float r = x - float(h);
        const bf16 m = bf16(r);
        part[0] = h;
        part[1] = m;
        part[2] = bf16(r - float(m));
    }
    typedef bf16x2 V2;   // two values at once (as Split<f16>::split2)
    static __device__ __forceinline__ void split2(float x0, float x1, V2* part) {
        asm("" : "+v"(x0), "+v"(x1));
        const V2 h = __builtin_convertvector(f32x2{x0, x1}, V2);
        const float r0 = x0 - float(h[0]), r1 = x1 - float(h[1]);
        const V2 m = __builtin_convertvector(f32x2{r0, r1}, V2);
        part[0] = h;
        part[1] = m;
        part[2] = __builtin_convertvector(f32x2{r0 - float(m[0]), r1 - float(m[1])}, V2);
    }
    static __device__ __forceinline__ f32x4 mfma(V8 a, V8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};

// fp32 (the exact tier's chunked delta rule): one part, the value itself.  A 16 x 16 x 32 product in the fragment
// layout above is the sum of eight v_mfma_f32_16x16x4_f32 (fp32 operands and products): in step e lane (g, r)
// feeds its element e -- A[r][8 g + e] and B[8 g + e][r] -- into k slot g, so the eight steps cover k = e, 8 + e,
// 16 + e, 24 + e for e = 0..7, and the 16 x 16 x 4 accumulator layout (column r, rows 4 g .. 4 g + 3) is the same.
template <> struct Split<float> {
    typedef f32x8 V8;
    static constexpr int P = 1;
    static constexpr int NPROD = 1;
    static __device__ __forceinline__ int ap(int) { return 0; }
    static __device__ __forceinline__ int wp(int) { return 0; }
    static __device__ __forceinline__ void split(float x, float* part) { part[0] = x; }
    static __device__ __forceinline__ f32x4 mfma(V8 a, V8 b, f32x4 c) {
#pragma unroll
        for (int e = 0; e < 8; ++e) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[e], c, 0, 0, 0);
        return c;
    }
};

// 8 fp32 values -> the P part vectors of an MFMA A / B fragment
template <typename T>
__device__ __forceinline__ void split8(const float* x, typename Split<T>::V8* parts) {
    if constexpr (Split<T>::P == 1) {
#pragma unroll
        for (int e = 0; e < 8; ++e) parts[0][e] = x[e];
    } else {
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            typename Split<T>::V2 p[Split<T>::P];
            Split<T>::split2(x[e], x[e + 1], p);
#pragma unroll
            for (int q = 0; q < Split<T>::P; ++q) {
                parts[q][e] = p[q][0];
                parts[q][e + 1] = p[q][1];
            }
        }
    }
}

// 4 fp32 values -> each part's 4 elements packed in 8 bytes (the half types)
template <typename T>
__device__ __forceinline__ void split4_packed(const float (&x)[4], uint2* out) {
    static_assert(sizeof(T) == 2, "packed parts of the half types");
    typename Split<T>::V2 p01[Split<T>::P], p23[Split<T>::P];
    Split<T>::split2(x[0], x[1], p01);
    Split<T>::split2(x[2], x[3], p23);
#pragma unroll
    for (int q = 0; q < Split<T>::P; ++q)
        out[q] = make_uint2(__builtin_bit_cast(unsigned, p01[q]), __builtin_bit_cast(unsigned, p23[q]));
}

// 8 elements of one part (16 bytes for the half types, 32 for fp32; 16-byte aligned) -> V8
template <typename T>
__device__ __forceinline__ typename Split<T>::V8 load_part8(const T* p) {
    if constexpr (sizeof(T) == 4) {
        const float4 u = reinterpret_cast<const float4*>(p)[0], w = reinterpret_cast<const float4*>(p)[1];
        return f32x8{u.x, u.y, u.z, u.w, w.x, w.y, w.z, w.w};
    } else {
        const uint4 u = *reinterpret_cast<const uint4*>(p);
        return *reinterpret_cast<const typename Split<T>::V8*>(&u);
    }
}

// acc += A * B over all split products (fixed order, smallest first)
template <typename T>
__device__ __forceinline__ f32x4 mfma_split(const typename Split<T>::V8* a, const typename Split<T>::V8* b, f32x4 acc) {
#pragma unroll
    for (int i = 0; i < Split<T>::NPROD; ++i) acc = Split<T>::mfma(a[Split<T>::ap(i)], b[Split<T>::wp(i)], acc);
    return acc;
}

}  // namespace shv
