// Device helpers shared by the gfx950 kernels: storage types, conversions, activations.
// All code is compiled with -ffp-contract=off: every fused multiply-add below is written explicitly, so the
// fp32 tier performs the same IEEE operations per element as the reference CPU engine
// (engine/model/isa_impl.hpp:159-187).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace shv {

typedef _Float16 f16;
typedef __bf16 bf16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

enum Act { ACT_NONE = 0, ACT_RELU = 1, ACT_HS = 2, ACT_HSIG = 3, ACT_SILU = 4 };

template <typename T> __device__ __forceinline__ float to_f(T x) { return float(x); }
template <typename T> __device__ __forceinline__ T from_f(float x) { return T(x); }

// exp(x): Cephes expf polynomial with the reference's clamp and round-to-nearest trick (isa_impl.hpp:159-177).
// Used wherever the reference uses its vector exp (SiLU in the GEMM epilogues, short conv, gated norm, head).
__device__ __forceinline__ float cephes_exp(float x) {
    x = x > -87.33654f ? x : -87.33654f;
    x = x < 88.37626f ? x : 88.37626f;
    const float n = __builtin_fmaf(x, 1.44269504088896341f, 12582912.0f) - 12582912.0f;
    float r = __builtin_fmaf(n, -0.693359375f, x);
    r = __builtin_fmaf(n, 2.12194440e-4f, r);
    const float z = r * r;
    float p = 1.9875691500e-4f;
    p = __builtin_fmaf(p, r, 1.3981999507e-3f);
    p = __builtin_fmaf(p, r, 8.3334519073e-3f);
    p = __builtin_fmaf(p, r, 4.1665795894e-2f);
    p = __builtin_fmaf(p, r, 1.6666665459e-1f);
    p = __builtin_fmaf(p, r, 5.0000001201e-1f);
    p = __builtin_fmaf(p, z, r);
    p = p + 1.0f;
    const int ni = int(n);
    return p * __int_as_float((ni + 127) << 23);
}
__device__ __forceinline__ float silu(float x) { return x / (1.0f + cephes_exp(0.0f - x)); }
// SiLU of the fp16 / bf16 tiers: the hardware exp2 and reciprocal (each within 1 ulp), x * 1 / (1 + 2^(-x log2 e)).
// Five instructions instead of about twenty-five; a few fp32 ulp from silu(), well inside those tiers' bounds.
// Limits: x -> -inf gives -0, x -> +inf gives x, NaN stays NaN.
__device__ __forceinline__ float silu_fast(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504088896341f));
}
__device__ __forceinline__ float relu(float x) { return x > 0.0f ? x : 0.0f; }

// Element (row, col) of one part of a pre-split GEMM operand: 32-column groups kstride elements apart, rows ld
// elements apart inside a group.  kstride 32 with ld >= the column count is plain row-major; ld 32 with
// kstride >= rows * 32 is the group-major layout, where the 16 rows x 32 columns of an MFMA fragment block are
// 1 KB of contiguous memory.
__device__ __forceinline__ long long presplit_idx(long long row, int col, long long ld, long long kstride) {
    return (long long)(col >> 5) * kstride + row * ld + (col & 31);
}
// relu for the fp16 / bf16 tiers as one integer max on the bit pattern: every negative float (-0 included) is a
// negative int and becomes +0, every positive one stays.  Equal to relu() for all inputs but +NaN, which it passes
// on instead of mapping to 0 (the tiers' certification rejects non-finite output).  relu() costs a second op
// whenever the compiler cannot prove x canonical (MFMA results): it quiets x first so that its float max keeps the
// select's NaN semantics.
__device__ __forceinline__ float relu_nb(float x) { return __int_as_float(max(__float_as_int(x), 0)); }
__device__ __forceinline__ float clamp06(float x) {
    float t = x + 3.0f;
    t = t > 0.0f ? t : 0.0f;
    return t < 6.0f ? t : 6.0f;
}
// v / 6 correctly rounded: q = v * fp32(1/6) refined by one fma residual step.  Checked against the IEEE quotient
// for all 2^32 fp32 inputs: identical for every finite |v| >= 2.4e-38.  Zero is its own quotient (the step turns
// -0 into +0), a select; for the rest below 2.4e-38 (a subnormal quotient) the division itself runs, on an
// out-of-line path that is skipped when no lane needs it -- hardswish's zeros (x <= -3) no longer take it.
__device__ __forceinline__ float div6_step(float v) {   // the product and the residual step, zero kept
    const float r = 0.16666667163372039794921875f;
    const float q = v * r;
    const float s = __builtin_fmaf(__builtin_fmaf(-q, 6.0f, v), r, q);
    return v == 0.0f ? v : s;
}
__device__ __forceinline__ bool div6_tiny(float v) { return __builtin_fabsf(v) < 2.4e-38f && v != 0.0f; }
__device__ __forceinline__ float div6(float v) {
    float q = div6_step(v);
    if (__builtin_expect(div6_tiny(v), 0)) q = v / 6.0f;
    return q;
}
__device__ __forceinline__ float hswish(float x) { return div6(x * clamp06(x)); }
__device__ __forceinline__ float hsigmoid(float x) { return div6(clamp06(x)); }
// v / 6 for the fp16 / bf16 tiers: one product with fp32(1/6), within an ulp of the IEEE quotient that div6() gives
// the exact tier -- far below the rounding those tiers' split operands carry -- and two VALU ops cheaper, which
// counts in the depthwise kernels, where every expanded value goes through hardswish.
__device__ __forceinline__ float div6_nb(float v) { return v * 0.16666667163372039794921875f; }
__device__ __forceinline__ float hswish_nb(float x) { return div6_nb(x * clamp06(x)); }
__device__ __forceinline__ float apply_act_nb(float v, int act) {
    switch (act) {
    case ACT_RELU: return relu_nb(v);
    case ACT_HS: return div6_nb(v * clamp06(v));
    case ACT_HSIG: return div6_nb(clamp06(v));
    case ACT_SILU: return silu(v);
    default: return v;
    }
}
__device__ __forceinline__ float apply_act(float v, int act) {
    switch (act) {
    case ACT_RELU: return relu(v);
    case ACT_HS: return hswish(v);
    case ACT_HSIG: return hsigmoid(v);
    case ACT_SILU: return silu(v);
    default: return v;
    }
}
// apply_act on four values with the activation fixed, bitwise apply_act per value: hardswish / hardsigmoid run
// div6's product and residual step on all four and its division only when one of the four quotients is subnormal
// (one branch per four values instead of one per value)
template <int ACT> __device__ __forceinline__ void apply_act4(float (&x)[4]) {
    if constexpr (ACT == ACT_HS || ACT == ACT_HSIG) {
        float v[4];
        bool tiny = false;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = ACT == ACT_HS ? x[e] * clamp06(x[e]) : clamp06(x[e]);
            x[e] = div6_step(v[e]);
            tiny = tiny || div6_tiny(v[e]);
        }
        if (__builtin_expect(tiny, 0)) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (div6_tiny(v[e])) x[e] = v[e] / 6.0f;
        }
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = apply_act(x[e], ACT);
    }
}
// gate nonlinearities evaluated with the device libm (the reference uses glibc expf/log1pf here)
__device__ __forceinline__ float softplus_f(float x) { return x > 20.0f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float logsigmoid_f(float x) { return (x < 0.0f ? x : 0.0f) - log1pf(expf(-fabsf(x))); }

// Eight consecutive storage elements as eight floats, moved as one vector: 16 bytes for the half types, 32 for fp32
// (the pointer is 16-byte aligned; the vector type says so, so fp32 goes as two 16-byte accesses).  Widening is
// exact; narrowing rounds to nearest even, as from_f.
template <typename T> struct Row8 { typedef T type __attribute__((ext_vector_type(8), aligned(16))); };
typedef float f32x8 __attribute__((ext_vector_type(8)));
template <typename T> __device__ __forceinline__ void read8(const T* p, float* v) {
    const f32x8 x = __builtin_convertvector(*reinterpret_cast<const typename Row8<T>::type*>(p), f32x8);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = x[i];
}
template <typename T> __device__ __forceinline__ void write8(T* p, const float* v) {
    f32x8 x;
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = v[i];
    *reinterpret_cast<typename Row8<T>::type*>(p) = __builtin_convertvector(x, typename Row8<T>::type);
}

// Sums over a 16-lane row with the fixed tree ((l_i + l_i+8) + (.. +4)) + (.. +2) + (.. +1) of the reference vector
// code (isa_impl.hpp:45-53).
// Lane 0 of each 16-lane row: the row's sum as the xor butterfly (v + v^8, then ^4, ^2, ^1) brackets it, computed
// with DPP row rotations (8, 4, 2, 1).  At lane 0 the rotations pair the same partial sums as the butterfly, only
// with some operands of an addition swapped, which IEEE addition does not notice; other lanes hold other
// bracketings.
__device__ __forceinline__ float tree16_lane0(float v) {
    v = v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
    v = v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false));
    v = v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x122, 0xf, 0xf, false));
    v = v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x121, 0xf, 0xf, false));
    return v;
}
// The butterfly sum in every lane of the row (the butterfly gives all 16 lanes the same value): lane 0's, broadcast
// to its row (DPP row_newbcast)
__device__ __forceinline__ float tree16(float v) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, tree16_lane0(v)), 0x150, 0xf, 0xf, false));
}

}  // namespace shv
