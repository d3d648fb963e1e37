// GEMM kernels for gfx950.  C[m][n] = epilogue(sum_k A[m][k] W[n][k]); A, C, R fp32 in HBM.
//
// gemm_f32 (exact tier): 64x64 block tile, 256 threads, 4x4 outputs per thread, K staged through LDS in blocks
//   of 64.  Each output is one fma chain from +0 per K block, block totals added left to right -- the per-element
//   operation sequence of the reference CPU engine (engine/model/isa_impl.hpp:188-317), so results are bitwise
//   independent of the tile, of M and of the other rows, and equal to the reference's.
// gemm_mfma<T> (fp16 / bf16 tiers): v_mfma_f32_16x16x32_{f16,bf16} on split operands.  Every fp32 operand value x
//   is carried as a sum of T parts (fp16: hi + lo, bf16: hi + mid + lo, each part the rounding of what the previous
//   parts leave), and the products whose magnitude exceeds ~2^-24 of hi*hi are issued as separate MFMAs into one
//   fp32 accumulator (fp16: 3 products, bf16: 6).  This keeps the matrix cores while giving fp32-level operand
//   precision: the random-init SHIELD-V encoder amplifies operand rounding ~100x, and plain fp16 operands moved
//   logits by up to 1.1 on the seeded set.  Weights are split once at load (repack kernel); activations are split
//   in registers after their 32-byte fp32 loads.
//   A and W tiles are staged through LDS (A split once per workgroup), the next K step prefetched into registers;
//   K advances in steps of 32 in increasing order; a K tail is zero-filled, never split across waves.
#include "dev_common.hpp"
#include "kernels.hpp"
#include "mfma.hpp"

#include <cmath>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <type_traits>

namespace shv {
namespace {

// ------------------------------------------------------------------------------------------------ epilogue
// out = act(v * wscale + bias) (+ residual: res 1 R + v, res 2 R + v / sqrt(2), res 3 R + 0.70710678f * v).  wscale
// is a power of two (1 unless the weight was stored pre-scaled), so v * wscale is exact.
__device__ __forceinline__ float epi_value(const GemmArgs& p, float v, float b, float res) {
    v = v * p.wscale;
    if (p.bias) v = v + b;
    v = apply_act(v, p.act);
    if (p.res == 3) v = res + 0.7071067811865475244f * v;
    else if (p.res) v = p.res == 2 ? res + v / 1.41421356237309515f : res + v;
    return v;
}
// Epilogue of the 4 x J outputs one thread holds (rows row(i), columns col(j)).  Every bias and residual operand is
// loaded (at clamped, valid addresses) before the first store: C may alias R or the bias as far as the compiler
// knows, so a load written after a store would wait for it, one memory round trip per output.
template <int J, class Row, class Col, class Val>
__device__ __forceinline__ void epi_block(const GemmArgs& p, Row row, Col col, Val val) {
    float bv[J], rv[4][J];
#pragma unroll
    for (int j = 0; j < J; ++j) bv[j] = p.bias ? p.bias[min(col(j), p.N - 1)] : 0.0f;
    if (p.res) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < J; ++j)
                rv[i][j] = p.R[min(row(i), (long long)p.M - 1) * p.ldr + min(col(j), p.N - 1)];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const long long m = row(i);
        if (m >= p.M) continue;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int n = col(j);
            if (n < p.N) p.C[m * p.ldc + n] = epi_value(p, val(i, j), bv[j], p.res ? rv[i][j] : 0.0f);
        }
    }
}

// SwiGLU of the MFMA tiers from the gate and up sums
__device__ __forceinline__ float swiglu_value(const GemmArgs& p, float gate, float up) {
    return silu_fast(gate * p.wscale) * (up * p.wscale);
}
// A SwiGLU output: fp32, or its split parts when the consumer takes pre-split A
template <typename T>
__device__ __forceinline__ void swiglu_store(const GemmArgs& p, long long m, int col, float v) {
    if (p.Ch) {
        T part[Split<T>::P];
        Split<T>::split(v, part);
#pragma unroll
        for (int q = 0; q < Split<T>::P; ++q)
            static_cast<T*>(p.Ch)[q * p.cstride + presplit_idx(m, col, p.ldc, p.ckstride)] = part[q];
    } else {
        p.C[m * p.ldc + col] = v;
    }
}

// ------------------------------------------------------------------------------------------------ fp32 VALU
constexpr int F32_BM = 64, F32_BN = 64, F32_BK = 64;

template <bool SCALE>
__global__ void __launch_bounds__(256) gemm_f32_kernel(GemmArgs p) {
    __shared__ float As[F32_BM][F32_BK + 1];
    __shared__ float Ws[F32_BN][F32_BK + 1];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const long long m0 = (long long)blockIdx.x * F32_BM;
    const int n0 = blockIdx.y * F32_BN;
    const float* A = p.A;
    const float* W = static_cast<const float*>(p.W);
    float tot[4][4], blk[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) tot[i][j] = 0.0f;
    for (int k0 = 0; k0 < p.K; k0 += F32_BK) {
        const int kb = min(F32_BK, p.K - k0);
        // only the block's kb columns are staged (and read below): narrow layers (K 16..40) stage a quarter to
        // two thirds of the tile
        for (int i = tid; i < F32_BM * kb; i += 256) {
            const int r = i / kb, k = i - r * kb;
            const long long gm = m0 + r;
            const int gn = n0 + r, gk = k0 + k;
            float a = 0.0f, w = 0.0f;
            if (gm < p.M) {
                a = A[gm * p.lda + gk];
                if (SCALE) a = p.scale[(gm / p.scale_rows) * p.ld_scale + gk] * a;
            }
            if (gn < p.N) w = W[(long long)gn * p.ldw + gk];
            As[r][k] = a;
            Ws[r][k] = w;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) blk[i][j] = 0.0f;
        for (int kk = 0; kk < kb; ++kk) {
            float a[4], w[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = As[ty * 4 + i][kk];
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = Ws[tx * 4 + j][kk];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) blk[i][j] = __builtin_fmaf(a[i], w[j], blk[i][j]);
        }
        if (k0 == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) tot[i][j] = blk[i][j];
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) tot[i][j] = tot[i][j] + blk[i][j];
        }
        __syncthreads();
    }
    if (p.swiglu) {  // rows (2j, 2j+1) = (gate_j, up_j): this thread holds pairs j0, j0+1
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const long long m = m0 + ty * 4 + i;
            if (m >= p.M) continue;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int n = n0 + tx * 4 + 2 * q;
                if (n + 1 < p.N) p.C[m * p.ldc + (n >> 1)] = silu(tot[i][2 * q]) * tot[i][2 * q + 1];
            }
        }
        return;
    }
    epi_block<4>(p, [&](int i) { return m0 + ty * 4 + i; }, [&](int j) { return n0 + tx * 4 + j; },
                 [&](int i, int j) { return tot[i][j]; });
}

// Small M with few tiles (one clip's later CNN layers and sequence rows): the tiled kernel's per-output arithmetic is
// an fma chain from +0 over each 64-wide K block, then the block sums folded left to right (tot = b0, tot = tot +
// b1, ...).  The block chains are independent, so workgroup (M tile, N tile, K block) stages that block exactly as
// the tiled kernel does and writes its chains to the workspace [K block][M][N]; gemm_f32_fold_kernel folds them in
// order and applies the same epilogue.  The same operations, so bitwise the tiled kernel's results, from K / 64
// times the workgroups.
template <bool SCALE>
__global__ void __launch_bounds__(256) gemm_f32_kblock_kernel(GemmArgs p) {
    __shared__ float As[F32_BM][F32_BK + 1];
    __shared__ float Ws[F32_BN][F32_BK + 1];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const long long m0 = (long long)blockIdx.x * F32_BM;
    const int n0 = blockIdx.y * F32_BN;
    const int k0 = blockIdx.z * F32_BK, kb = min(F32_BK, p.K - k0);
    const float* A = p.A;
    const float* W = static_cast<const float*>(p.W);
    for (int i = tid; i < F32_BM * kb; i += 256) {   // the block's kb columns, as the tiled kernel
        const int r = i / kb, k = i - r * kb;
        const long long gm = m0 + r;
        const int gn = n0 + r, gk = k0 + k;
        float a = 0.0f, w = 0.0f;
        if (gm < p.M) {
            a = A[gm * p.lda + gk];
            if (SCALE) a = p.scale[(gm / p.scale_rows) * p.ld_scale + gk] * a;
        }
        if (gn < p.N) w = W[(long long)gn * p.ldw + gk];
        As[r][k] = a;
        Ws[r][k] = w;
    }
    __syncthreads();
    float blk[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) blk[i][j] = 0.0f;
    for (int kk = 0; kk < kb; ++kk) {
        float a[4], w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = As[ty * 4 + i][kk];
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = Ws[tx * 4 + j][kk];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) blk[i][j] = __builtin_fmaf(a[i], w[j], blk[i][j]);
    }
    float* out = p.ws + (long long)blockIdx.z * p.M * p.N;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const long long m = m0 + ty * 4 + i;
        if (m >= p.M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + tx * 4 + j;
            if (n < p.N) out[m * p.N + n] = blk[i][j];
        }
    }
}
// The tiled and K-block kernels' arithmetic with 16-byte operand traffic (K, lda, ldw, ld_scale multiples of 4, A, W,
// scale 16-byte aligned).  A K block is staged k-major -- As[k][m], Ws[k][n] -- from float4 global loads (lane i of a
// wave takes row i, so the transposing LDS stores are conflict-free), and each k step reads one float4 of A rows and
// one of W columns for its 16 fmas instead of eight scalars.  The next block's float4s are loaded into registers
// while the current one computes.  Per output the operations are the tiled kernel's (fma chain from +0 per 64-wide K
// block in increasing k, block sums added left to right, the same epilogue), so the results are bitwise equal.
// PART: one K block per workgroup (blockIdx.z), its chains written to the workspace for gemm_f32_fold_kernel.
template <bool SCALE, bool PART>
__global__ void __launch_bounds__(256) gemm_f32_v4_kernel(GemmArgs p) {
    __shared__ float4 As[F32_BK][F32_BM / 4];
    __shared__ float4 Ws[F32_BK][F32_BN / 4];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const long long m0 = (long long)blockIdx.x * F32_BM;
    const int n0 = blockIdx.y * F32_BN;
    const float* A = p.A;
    const float* W = static_cast<const float*>(p.W);
    const int kfirst = PART ? int(blockIdx.z) * F32_BK : 0;
    const int kend = PART ? min(p.K, kfirst + F32_BK) : p.K;
    // staging: float4 i of the tile is row (i & 63), k quad (i >> 6); four per thread
    float4 ra[4], rw[4];
    const int srow = tid & 63, sq = tid >> 6;
    const long long gm = m0 + srow;
    const int gn = n0 + srow;
    const float* arow = A + min(gm, (long long)p.M - 1) * p.lda;
    const float* wrow = W + (long long)min(gn, p.N - 1) * p.ldw;
    const float* srow_scale = SCALE ? p.scale + (min(gm, (long long)p.M - 1) / p.scale_rows) * p.ld_scale : nullptr;
    const auto load = [&](int k0, int kb) {
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int kq = sq + 4 * it;
            const bool kin = 4 * kq < kb;
            const int gk = k0 + 4 * min(kq, kb / 4 - 1);
            float4 a = *reinterpret_cast<const float4*>(arow + gk);
            if (SCALE) {
                const float4 sc = *reinterpret_cast<const float4*>(srow_scale + gk);
                a = make_float4(sc.x * a.x, sc.y * a.y, sc.z * a.z, sc.w * a.w);
            }
            const float4 w = *reinterpret_cast<const float4*>(wrow + gk);
            ra[it] = kin && gm < p.M ? a : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            rw[it] = kin && gn < p.N ? w : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    const auto store = [&](int kb) {
        float* as = reinterpret_cast<float*>(As);
        float* ws = reinterpret_cast<float*>(Ws);
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int kq = sq + 4 * it;
            if (4 * kq >= kb) continue;
            const float av[4] = {ra[it].x, ra[it].y, ra[it].z, ra[it].w};
            const float wv[4] = {rw[it].x, rw[it].y, rw[it].z, rw[it].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                as[(4 * kq + e) * F32_BM + srow] = av[e];
                ws[(4 * kq + e) * F32_BN + srow] = wv[e];
            }
        }
    };
    float tot[4][4], blk[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) tot[i][j] = 0.0f;
    load(kfirst, min(F32_BK, kend - kfirst));
    for (int k0 = kfirst; k0 < kend; k0 += F32_BK) {
        const int kb = min(F32_BK, kend - k0);
        store(kb);
        __syncthreads();
        if (k0 + F32_BK < kend) load(k0 + F32_BK, min(F32_BK, kend - k0 - F32_BK));
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) blk[i][j] = 0.0f;
#pragma unroll 4
        for (int kk = 0; kk < kb; ++kk) {
            const float4 a4 = As[kk][ty], w4 = Ws[kk][tx];
            const float a[4] = {a4.x, a4.y, a4.z, a4.w}, w[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) blk[i][j] = __builtin_fmaf(a[i], w[j], blk[i][j]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) tot[i][j] = k0 == kfirst ? blk[i][j] : tot[i][j] + blk[i][j];
        __syncthreads();
    }
    if constexpr (PART) {
        float* out = p.ws + (long long)blockIdx.z * p.M * p.N;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const long long m = m0 + ty * 4 + i;
            if (m >= p.M) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int n = n0 + tx * 4 + j;
                if (n < p.N) out[m * p.N + n] = tot[i][j];
            }
        }
        return;
    } else {
        if (p.swiglu) {  // rows (2j, 2j+1) = (gate_j, up_j): this thread holds pairs j0, j0+1
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const long long m = m0 + ty * 4 + i;
                if (m >= p.M) continue;
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const int n = n0 + tx * 4 + 2 * q;
                    if (n + 1 < p.N) p.C[m * p.ldc + (n >> 1)] = silu(tot[i][2 * q]) * tot[i][2 * q + 1];
                }
            }
            return;
        }
        epi_block<4>(p, [&](int i) { return m0 + ty * 4 + i; }, [&](int j) { return n0 + tx * 4 + j; },
                     [&](int i, int j) { return tot[i][j]; });
    }
}
// one thread per output: the K-block sums folded in order, then gemm_f32_kernel's epilogue (SwiGLU: weight rows
// 2j, 2j + 1 = gate, up of output j)
__global__ void __launch_bounds__(256) gemm_f32_fold_kernel(GemmArgs p, int nkb) {
    const int no = p.swiglu ? p.N / 2 : p.N;
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)p.M * no) return;
    const long long m = idx / no;
    const int j = int(idx % no);
    const long long plane = (long long)p.M * p.N;
    const auto fold = [&](int n) {
        const float* w = p.ws + m * p.N + n;
        float tot = w[0];
        for (int b = 1; b < nkb; ++b) tot = tot + w[b * plane];
        return tot;
    };
    if (p.swiglu) {
        p.C[m * p.ldc + j] = silu(fold(2 * j)) * fold(2 * j + 1);
        return;
    }
    const float b = p.bias ? p.bias[j] : 0.0f;
    const float r = p.res ? p.R[m * p.ldr + j] : 0.0f;
    p.C[m * p.ldc + j] = epi_value(p, fold(j), b, r);
}

// Exact tier, the narrow 1x1 layers of blocks 1-6 (K <= 128 inputs, N <= 120 outputs, many rows).  A workgroup of
// four waves takes 256 rows (one per lane) and NC of the N columns; K, N and NC are compile-time, so the row's
// K-block inputs, the block chains and the totals live in registers.  The workgroup stages its NC weight rows in
// LDS once (read back as broadcasts: every lane reads the same address); the per-output sequence is the
// reference's -- per K block of 64 an fma chain from +0 in increasing k, the second block's chain added to the
// first -- then the epilogue: bitwise gemm_f32_kernel's results.  Empty asm statements after every four k (the
// chains as operands, then a memory clobber) keep the compiler from hoisting all weight reads ahead of the chains
// (it did, and spilled).  Each wave
// stages its 64 x NC outputs in LDS and stores them as 16-byte pieces of consecutive row segments.
template <int K, int N, int NC, bool SCALE>
__global__ void __launch_bounds__(256) gemm_f32_narrow_kernel(GemmArgs p) {
    static_assert(K % 4 == 0 && NC % 4 == 0 && N % NC == 0 && K <= 2 * F32_BK, "narrow exact GEMM shape");
    constexpr int CS = NC + 4;   // LDS row stride of a wave's output tile (16-byte aligned rows)
    __shared__ float4 wsh[NC][K / 4];
    __shared__ float cs[4][64 * CS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const long long m0 = (long long)blockIdx.x * 256 + wave * 64, m = m0 + lane;
    const int n0 = blockIdx.y * NC;
    const bool live = m < p.M;
    const long long mc = live ? m : p.M - 1;
    const float* arow = p.A + mc * p.lda;
    const float* srow = SCALE ? p.scale + (mc / p.scale_rows) * p.ld_scale : nullptr;
    const float* W = static_cast<const float*>(p.W);
    for (int i = tid; i < NC * (K / 4); i += 256) {
        const int j = i / (K / 4), q = i % (K / 4);
        wsh[j][q] = *reinterpret_cast<const float4*>(W + (long long)(n0 + j) * p.ldw + 4 * q);
    }
    __syncthreads();
    float tot[NC];
    // one K block: the row's inputs k0 .. k0 + KB - 1 loaded, the chains run
    const auto block = [&](auto k0c, auto kbc, float (&out)[NC]) {
        constexpr int k0 = decltype(k0c)::value, KB = decltype(kbc)::value;
        float a[KB];
#pragma unroll
        for (int q = 0; q < KB / 4; ++q) {
            float4 v = *reinterpret_cast<const float4*>(arow + k0 + 4 * q);
            if (SCALE) {
                const float4 sc = *reinterpret_cast<const float4*>(srow + k0 + 4 * q);
                v = make_float4(sc.x * v.x, sc.y * v.y, sc.z * v.z, sc.w * v.w);
            }
            a[4 * q] = v.x; a[4 * q + 1] = v.y; a[4 * q + 2] = v.z; a[4 * q + 3] = v.w;
        }
#pragma unroll
        for (int j = 0; j < NC; ++j) out[j] = 0.0f;
#pragma unroll
        for (int q = 0; q < KB / 4; ++q) {
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                const float4 w = wsh[j][k0 / 4 + q];
                out[j] = __builtin_fmaf(a[4 * q], w.x, out[j]);
                out[j] = __builtin_fmaf(a[4 * q + 1], w.y, out[j]);
                out[j] = __builtin_fmaf(a[4 * q + 2], w.z, out[j]);
                out[j] = __builtin_fmaf(a[4 * q + 3], w.w, out[j]);
            }
            // the chains of these four k are complete before the next weights are read
#pragma unroll
            for (int j = 0; j < NC; ++j) asm volatile("" : "+v"(out[j]));
            asm volatile("" ::: "memory");
        }
    };
    constexpr int KB0 = K < F32_BK ? K : F32_BK;
    block(std::integral_constant<int, 0>(), std::integral_constant<int, KB0>(), tot);
    if constexpr (K > F32_BK) {
        float blk[NC];
        block(std::integral_constant<int, F32_BK>(), std::integral_constant<int, K - F32_BK>(), blk);
#pragma unroll
        for (int j = 0; j < NC; ++j) tot[j] = tot[j] + blk[j];
    }
    // epilogue: bias, activation, residual (all residual values of the tile read before its first store)
    float* ct = cs[wave];
#pragma unroll
    for (int q = 0; q < NC / 4; ++q) {
        float4 r = make_float4(0.0f, 0.0f, 0.0f, 0.0f), b = r;
        if (p.res) r = *reinterpret_cast<const float4*>(p.R + mc * p.ldr + n0 + 4 * q);
        if (p.bias) b = *reinterpret_cast<const float4*>(p.bias + n0 + 4 * q);
        float4 o;
        o.x = epi_value(p, tot[4 * q], b.x, r.x);
        o.y = epi_value(p, tot[4 * q + 1], b.y, r.y);
        o.z = epi_value(p, tot[4 * q + 2], b.z, r.z);
        o.w = epi_value(p, tot[4 * q + 3], b.w, r.w);
        *reinterpret_cast<float4*>(&ct[lane * CS + 4 * q]) = o;
    }
    __syncthreads();
#pragma unroll
    for (int i = lane; i < 64 * (NC / 4); i += 64) {
        const int row = i / (NC / 4), q = i % (NC / 4);
        if (m0 + row < p.M)
            *reinterpret_cast<float4*>(p.C + (m0 + row) * p.ldc + n0 + 4 * q) =
                *reinterpret_cast<const float4*>(&ct[row * CS + 4 * q]);
    }
}

// Exact tier, layers of at most 256 columns and up to 1024 inputs at 1k-20k rows (the later projects and SE
// projects of one clip, where the K-block kernel needs a fold pass): the narrow kernel's form with K at run time.
// A workgroup of four waves takes 256 rows (one per lane) and 8 columns; it stages those columns' weights (all K)
// in LDS once, and each lane runs the reference's per-output sequence over the K blocks of 64 -- its row's block
// inputs in registers, an fma chain from +0 per block, block sums added in order -- then the epilogue: bitwise
// gemm_f32_kernel's results.  Empty asm statements after every four k pin the chains (see the narrow kernel).
constexpr int COLS_NC = 8, COLS_KMAX = 1024;
template <bool SCALE>
__global__ void __launch_bounds__(256) gemm_f32_cols_kernel(GemmArgs p) {
    constexpr int NC = COLS_NC, CS = NC + 4;
    __shared__ float4 wsh[NC][COLS_KMAX / 4];
    __shared__ float cs[4][64 * CS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const long long m0 = (long long)blockIdx.x * 256 + wave * 64, m = m0 + lane;
    const int n0 = blockIdx.y * NC;
    const bool live = m < p.M;
    const long long mc = live ? m : p.M - 1;
    const float* arow = p.A + mc * p.lda;
    const float* srow = SCALE ? p.scale + (mc / p.scale_rows) * p.ld_scale : nullptr;
    const float* W = static_cast<const float*>(p.W);
    const int K4 = p.K / 4;
    for (int i = tid; i < NC * K4; i += 256) {
        const int j = i / K4, q = i % K4;
        wsh[j][q] = n0 + j < p.N ? *reinterpret_cast<const float4*>(W + (long long)(n0 + j) * p.ldw + 4 * q)
                                 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    __syncthreads();
    float tot[NC];
    for (int k0 = 0; k0 < p.K; k0 += F32_BK) {
        const int kb = min(F32_BK, p.K - k0);   // a multiple of 4
        float a[F32_BK];
#pragma unroll
        for (int q = 0; q < F32_BK / 4; ++q) {
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (4 * q < kb) {
                v = *reinterpret_cast<const float4*>(arow + k0 + 4 * q);
                if (SCALE) {
                    const float4 sc = *reinterpret_cast<const float4*>(srow + k0 + 4 * q);
                    v = make_float4(sc.x * v.x, sc.y * v.y, sc.z * v.z, sc.w * v.w);
                }
            }
            a[4 * q] = v.x; a[4 * q + 1] = v.y; a[4 * q + 2] = v.z; a[4 * q + 3] = v.w;
        }
        float blk[NC];
#pragma unroll
        for (int j = 0; j < NC; ++j) blk[j] = 0.0f;
#pragma unroll
        for (int q = 0; q < F32_BK / 4; ++q) {
            if (4 * q >= kb) break;
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                const float4 w = wsh[j][k0 / 4 + q];
                blk[j] = __builtin_fmaf(a[4 * q], w.x, blk[j]);
                blk[j] = __builtin_fmaf(a[4 * q + 1], w.y, blk[j]);
                blk[j] = __builtin_fmaf(a[4 * q + 2], w.z, blk[j]);
                blk[j] = __builtin_fmaf(a[4 * q + 3], w.w, blk[j]);
            }
#pragma unroll
            for (int j = 0; j < NC; ++j) asm volatile("" : "+v"(blk[j]));
            asm volatile("" ::: "memory");
        }
        if (k0 == 0) {
#pragma unroll
            for (int j = 0; j < NC; ++j) tot[j] = blk[j];
        } else {
#pragma unroll
            for (int j = 0; j < NC; ++j) tot[j] = tot[j] + blk[j];
        }
    }
    // epilogue (all residual values of the tile read before its first store), staged for row-segment stores
    float* ct = cs[wave];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int n = min(n0 + j, p.N - 1);
        const float b = p.bias ? p.bias[n] : 0.0f, r = p.res ? p.R[mc * p.ldr + n] : 0.0f;
        ct[lane * CS + j] = epi_value(p, tot[j], b, r);
    }
    __syncthreads();
    for (int i = lane; i < 64 * NC; i += 64) {
        const int row = i / NC, j = i % NC;
        if (m0 + row < p.M && n0 + j < p.N) p.C[(m0 + row) * p.ldc + n0 + j] = ct[row * CS + j];
    }
}

// ------------------------------------------------------------------------------------------------ fp32 MFMA
// The fp32 tier's all-row sequence GEMMs on the matrix cores: v_mfma_f32_16x16x4_f32 takes fp32 operands, forms
// fp32 products and accumulates in fp32 (no reduced-precision operand type).  Fragment layout, lane l = 16 g + r:
// A holds row r at k slot g, B column r at k slot g, C column r at rows 4 g .. 4 g + 3.
// A workgroup of four waves owns MT x NT blocks of 16 x 16 and splits K between its waves: K runs in steps of 16,
// and wave w takes steps w, w + 4, w + 8, ... in increasing order.  Per step, lane (g, r) loads A[row][k0 + 4 g ..
// + 3] and W[column][k0 + 4 g .. + 3] as one float4 each straight from memory (no LDS staging), and MFMA kk (0..3)
// takes k = k0 + 4 g + kk in slot g, into the wave's accumulator from +0.  The four partial sums are then added as
// (w0 + w1) + (w2 + w3) through LDS and wave 0 runs the epilogue.  Every output therefore receives the same
// operations whatever MT, NT, D, M or the other rows: results are bitwise independent of the tiling and of the
// batch.  Each wave keeps D of its steps' operands in flight (the 321-row GEMMs of one clip are bound by load
// latency, not by the matrix cores).  K, lda, ldw (and ld_scale) are multiples of 4; a K tail loads clamped
// addresses and zeros.
template <int MT, int NT, int D, bool SCALE>
__global__ void __launch_bounds__(256) gemm_f32_mfma_kernel(GemmArgs p) {
    __shared__ f32x4 part[3][MT][NT][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, r = lane & 15;
    const long long mbase = (long long)blockIdx.x * (MT * 16);
    const int nbase = blockIdx.y * (NT * 16);
    const float* W = static_cast<const float*>(p.W);
    const float* arow[MT];
    const float* srow[MT];
    bool alive[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const long long m = mbase + mt * 16 + r;
        alive[mt] = m < p.M;
        const long long mc = alive[mt] ? m : p.M - 1;
        arow[mt] = p.A + mc * p.lda + 4 * g;
        srow[mt] = SCALE ? p.scale + (mc / p.scale_rows) * p.ld_scale + 4 * g : nullptr;
    }
    const float* wrow[NT];
    bool wlive[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int n = nbase + nt * 16 + r;
        wlive[nt] = n < p.N;
        wrow[nt] = W + (long long)(wlive[nt] ? n : p.N - 1) * p.ldw + 4 * g;
    }
    const auto load = [&](int k0, float4 (&a)[MT], float4 (&w)[NT]) {
        const bool kin = k0 + 4 * g < p.K;
        const int kc = kin ? k0 : p.K - 4 - 4 * g;   // clamped so that the float4 stays inside the row
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            float4 v = *reinterpret_cast<const float4*>(arow[mt] + kc);
            if (SCALE) {
                const float4 sc = *reinterpret_cast<const float4*>(srow[mt] + kc);
                v = make_float4(sc.x * v.x, sc.y * v.y, sc.z * v.z, sc.w * v.w);
            }
            a[mt] = (kin && alive[mt]) ? v : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const float4 v = *reinterpret_cast<const float4*>(wrow[nt] + kc);
            w[nt] = (kin && wlive[nt]) ? v : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    f32x4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // this wave's steps wave + 4 i; step i sits in ring slot i % D and is reloaded with step i + D once consumed
    const int nsteps = (p.K + 15) / 16, mine = (nsteps - wave + 3) / 4;
    float4 a[D][MT], w[D][NT];
#pragma unroll
    for (int d = 0; d < D; ++d)
        if (d < mine) load(16 * (wave + 4 * d), a[d], w[d]);
    for (int i0 = 0; i0 < mine; i0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int i = i0 + d;
            if (i >= mine) break;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) {
                        const float av = kk == 0 ? a[d][mt].x : kk == 1 ? a[d][mt].y : kk == 2 ? a[d][mt].z : a[d][mt].w;
                        const float wv = kk == 0 ? w[d][nt].x : kk == 1 ? w[d][nt].y : kk == 2 ? w[d][nt].z : w[d][nt].w;
                        acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, wv, acc[mt][nt], 0, 0, 0);
                    }
            if (i + D < mine) load(16 * (wave + 4 * (i + D)), a[d], w[d]);
        }
    }
    if (wave) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) part[wave - 1][mt][nt][lane] = acc[mt][nt];
    }
    __syncthreads();
    if (wave) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
            acc[mt][nt] = (acc[mt][nt] + part[0][mt][nt][lane]) + (part[1][mt][nt][lane] + part[2][mt][nt][lane]);
    // lane holds C[mbase + mt * 16 + 4 g + i][nbase + nt * 16 + r]
    if (p.swiglu) {   // weight rows in 16-row panels alternating gate / up: NT even, nbase a multiple of 32
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const long long m = mbase + mt * 16 + 4 * g + i;
                if (m >= p.M) continue;
#pragma unroll
                for (int nt = 0; nt + 1 < NT; nt += 2) {
                    const int panel = nbase / 16 + nt;
                    if ((panel + 1) * 16 <= p.N)
                        p.C[m * p.ldc + (panel / 2) * 16 + r] = silu(acc[mt][nt][i]) * acc[mt][nt + 1][i];
                }
            }
        return;
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
        epi_block<NT>(p, [&](int i) { return mbase + mt * 16 + 4 * g + i; }, [&](int j) { return nbase + j * 16 + r; },
                      [&](int i, int j) { return acc[mt][j][i]; });
}

// Small M (<= 256 rows, e.g. the windows' last SISA rows): the same per-element arithmetic as gemm_f32_kernel -- K blocks
// of 64, fma chain from +0 inside a block, the first block's sum taken as is and the later ones added in order -- so
// results are bitwise those of the tiled kernel.  Only the chain inside a K block is serial, so a lane owns one
// (weight row, K block) pair: a wave covers GV_OPW = 64 / nkb weight rows (even for SwiGLU, whose gate and up rows
// are adjacent) with all their K blocks, and the block sums are added in order through LDS.  The lane's 64 weights
// stay in registers across the block's rows (blockIdx.y takes chunks of rpw <= GV_ROWS rows of M: fewer rows per
// workgroup at small M, where the chunks are the grid's only parallelism along M).
constexpr int GV_ROWS = 8;      // rows per workgroup at most
constexpr int GV_MAXM = 256;    // larger M goes to the tiled kernel
template <bool SCALE, bool VEC>
__device__ __forceinline__ void gv_load64(float* dst, const float* src, const float* sc, int n) {
    if (VEC && n == F32_BK) {
#pragma unroll
        for (int j = 0; j < F32_BK / 4; ++j) {
            const float4 v = reinterpret_cast<const float4*>(src)[j];
            dst[4 * j] = v.x; dst[4 * j + 1] = v.y; dst[4 * j + 2] = v.z; dst[4 * j + 3] = v.w;
        }
        if constexpr (SCALE) {
#pragma unroll
            for (int j = 0; j < F32_BK / 4; ++j) {
                const float4 c = reinterpret_cast<const float4*>(sc)[j];
                dst[4 * j] = c.x * dst[4 * j]; dst[4 * j + 1] = c.y * dst[4 * j + 1];
                dst[4 * j + 2] = c.z * dst[4 * j + 2]; dst[4 * j + 3] = c.w * dst[4 * j + 3];
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < F32_BK; ++k) {
            float v = k < n ? src[k] : 0.0f;
            if constexpr (SCALE) v = k < n ? sc[k] * v : 0.0f;
            dst[k] = v;
        }
    }
}
template <bool SCALE, bool VEC>
__global__ void __launch_bounds__(64) gemv_f32_kernel(GemmArgs p, int nkb, int opw, int rpw) {
    __shared__ float part[GV_ROWS][64];
    const int lane = threadIdx.x;
    const int mbase = blockIdx.y * rpw, mrows = min(rpw, p.M - mbase);
    const int o = lane / nkb, kb = lane - o * nkb;
    const int wn = blockIdx.x * opw + o;
    const bool live = o < opw && wn < p.N;
    const int k0 = kb * F32_BK, n = min(F32_BK, p.K - k0);
    const float* W = static_cast<const float*>(p.W);
    if (live) {
        float w[F32_BK];
        gv_load64<false, VEC>(w, W + (long long)wn * p.ldw + k0, nullptr, n);
        for (int i = 0; i < mrows; ++i) {
            const long long m = mbase + i;
            float a[F32_BK];
            gv_load64<SCALE, VEC>(a, p.A + m * p.lda + k0,
                                  SCALE ? p.scale + (m / p.scale_rows) * p.ld_scale + k0 : nullptr, n);
            float blk = 0.0f;
            if (n == F32_BK) {
#pragma unroll
                for (int k = 0; k < F32_BK; ++k) blk = __builtin_fmaf(a[k], w[k], blk);
            } else {
#pragma unroll
                for (int k = 0; k < F32_BK; ++k)
                    if (k < n) blk = __builtin_fmaf(a[k], w[k], blk);
            }
            part[i][lane] = blk;
        }
    }
    __syncthreads();
    if (!live || kb != 0 || (p.swiglu && (o & 1))) return;
    auto total = [&](int i, int l0) {
        float tot = part[i][l0];
        for (int j = 1; j < nkb; ++j) tot = tot + part[i][l0 + j];
        return tot;
    };
    const float b = p.bias && !p.swiglu ? p.bias[wn] : 0.0f;
    for (int i = 0; i < mrows; ++i) {
        const long long m = mbase + i;
        if (p.swiglu) {   // weight rows (wn, wn + 1) = (gate, up) of output wn / 2
            p.C[m * p.ldc + (wn >> 1)] = silu(total(i, lane)) * total(i, lane + nkb);
            continue;
        }
        const float r = p.res ? p.R[m * p.ldr + wn] : 0.0f;
        p.C[m * p.ldc + wn] = epi_value(p, total(i, lane), b, r);
    }
}

// ------------------------------------------------------------------------------------------------ MFMA
// Direct-fragment GEMM for N <= 160 (the SE-block projects, CNN 1x1 layers): the workgroup covers every output
// column in at most two column blocks, so A is read once or twice straight into MFMA fragments and staging it
// through LDS buys nothing.  A wave owns MFMA_MT x NT 16x16 tiles.
constexpr int MFMA_MT = 4;      // 16-row tiles per wave (64 rows)
constexpr int MFMA_WAVES = 4;   // waves per block, stacked along M (256 rows)

// Workgroup order: the 1-D grid is dealt round robin over the 8 XCDs (each with its own L2); workgroup id goes to
// XCD id % 8, and the column blocks of one row block take consecutive ids on the same XCD, so the second column
// block reads its rows of A from that L2 instead of HBM.
constexpr int XCDS = 8;

template <typename T, int NT, bool SCALE>
__global__ void __launch_bounds__(64 * MFMA_WAVES) gemm_direct_kernel(GemmArgs p, int mblocks, int nblocks) {
    typedef Split<T> S;
    typedef typename S::V8 V8;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane & 15, g = lane >> 4;
    const int xcd = blockIdx.x % XCDS, slot = blockIdx.x / XCDS;
    const int mb = (slot / nblocks) * XCDS + xcd, nb = slot % nblocks;
    if (mb >= mblocks) return;
    const long long mbase = ((long long)mb * MFMA_WAVES + wave) * (MFMA_MT * 16);
    const int nbase = nb * (NT * 16);
    if (mbase >= p.M) return;
    const T* W = static_cast<const T*>(p.W);
    f32x4 acc[MFMA_MT][NT];
#pragma unroll
    for (int i = 0; i < MFMA_MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < p.K; k0 += 32) {
        // all loads of the K step are issued unconditionally (rows, columns and K clamped into range) before any
        // is used, then out-of-range values are zeroed: one wait per step instead of one per tile
        const int kk = k0 + g * 8;
        const bool kin = kk < p.K;
        const int kc = kin ? kk : p.K - 8;
        V8 a[MFMA_MT][S::P], b[NT][S::P];
        float x[MFMA_MT][8], sc[SCALE ? MFMA_MT : 1][8];
        uint4 wv[NT][S::P];
#pragma unroll
        for (int mt = 0; mt < MFMA_MT; ++mt) {
            const long long row = mbase + mt * 16 + r;
            const long long rc = row < p.M ? row : p.M - 1;
            read8(p.A + rc * p.lda + kc, x[mt]);
        }
        if constexpr (SCALE) {
#pragma unroll
            for (int mt = 0; mt < MFMA_MT; ++mt) {
                const long long row = mbase + mt * 16 + r;
                const long long rc = row < p.M ? row : p.M - 1;
                read8(p.scale + (rc / p.scale_rows) * p.ld_scale + kc, sc[mt]);
            }
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int col = nbase + nt * 16 + r;
            const int cc = col < p.N ? col : p.N - 1;
#pragma unroll
            for (int q = 0; q < S::P; ++q)
                wv[nt][q] = *reinterpret_cast<const uint4*>(W + q * p.wstride + (long long)cc * p.ldw + kc);
        }
#pragma unroll
        for (int mt = 0; mt < MFMA_MT; ++mt) {
            const bool live = kin && mbase + mt * 16 + r < p.M;
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float t = x[mt][e];
                if constexpr (SCALE) t = sc[mt][e] * t;
                v[e] = live ? t : 0.0f;
            }
            split8<T>(v, a[mt]);
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const bool live = kin && nbase + nt * 16 + r < p.N;
#pragma unroll
            for (int q = 0; q < S::P; ++q) {
                const uint4 u = live ? wv[nt][q] : make_uint4(0u, 0u, 0u, 0u);
                b[nt][q] = *reinterpret_cast<const V8*>(&u);
            }
        }
#pragma unroll
        for (int i = 0; i < S::NPROD; ++i)
#pragma unroll
            for (int mt = 0; mt < MFMA_MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = S::mfma(a[mt][S::ap(i)], b[nt][S::wp(i)], acc[mt][nt]);
    }
    // lane holds C[mbase + mt*16 + g*4 + i][nbase + nt*16 + r]
    if (p.swiglu) {  // 16-row panels alternate gate / up; NT is even and nbase is a multiple of 32
#pragma unroll
        for (int mt = 0; mt < MFMA_MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const long long m = mbase + mt * 16 + g * 4 + i;
                if (m >= p.M) continue;
#pragma unroll
                for (int nt = 0; nt + 1 < NT; nt += 2) {
                    const int panel = nbase / 16 + nt;
                    if ((panel + 1) * 16 <= p.N)
                        swiglu_store<T>(p, m, (panel / 2) * 16 + r, swiglu_value(p, acc[mt][nt][i], acc[mt][nt + 1][i]));
                }
            }
        return;
    }
#pragma unroll
    for (int mt = 0; mt < MFMA_MT; ++mt)
        epi_block<NT>(p, [&](int i) { return mbase + mt * 16 + g * 4 + i; }, [&](int j) { return nbase + j * 16 + r; },
                      [&](int i, int j) { return acc[mt][j][i]; });
}

// Workgroup barrier that waits for LDS traffic only (the next K step's global loads stay in flight across it).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// waits for the wave's own LDS accesses (one wave's LDS instructions execute in order)
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// LDS-staged split-operand GEMM.  A workgroup (4 waves, WGM x WGN) owns a BM x BN tile of C; per K step of 32 it
// stages A[BM][32] (fp32 from HBM, SE-scaled, split into the T parts once per workgroup) and the pre-split W parts
// [BN][32] in LDS, while the next step's global loads are already in flight; each wave multiplies WM x WN 16x16
// tiles from LDS fragments.  Every accumulator receives, per K step, the same NPROD MFMAs in the same order as
// before staging existed, so results do not depend on the tiling.
constexpr int LG_KT = 64;          // K per staged step: two MFMA K steps
constexpr int LG_LD = LG_KT + 8;   // staged row stride in T elements (144 B): 16-lane fragment reads hit 64 banks once

template <typename T, int WM, int WN, int WGM, int WGN, bool SCALE, bool AH>
__global__ void __launch_bounds__(256) gemm_lds_kernel(GemmArgs p, int mblocks, int nblocks) {
    static_assert(!(SCALE && AH), "pre-split A carries no SE scale");
    static_assert(WGM * WGN == 4, "4 waves");
    typedef Split<T> S;
    typedef typename S::V8 V8;
    constexpr int P = S::P;
    constexpr int BM = 16 * WM * WGM, BN = 16 * WN * WGN;
    __shared__ __attribute__((aligned(16))) T As[P][BM][LG_LD];
    __shared__ __attribute__((aligned(16))) T Ws[P][BN][LG_LD];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r = lane & 15, g = lane >> 4;
    const int wm = wave / WGN, wn = wave % WGN;
    // XCD-aware order (as in gemm_direct_kernel): the column blocks of a row block take consecutive ids on one XCD
    const int xcd = blockIdx.x % XCDS, slot = blockIdx.x / XCDS;
    const int mb = (slot / nblocks) * XCDS + xcd, nb = slot % nblocks;
    if (mb >= mblocks) return;
    const long long m0 = (long long)mb * BM;
    const int n0 = nb * BN;
    const T* W = static_cast<const T*>(p.W);

    constexpr int A4 = BM * (LG_KT / 4);      // float4s of an A tile
    constexpr int AR = AH ? 1 : (A4 + 255) / 256;
    constexpr int A8 = BM * (LG_KT / 8);      // 8-element groups of a pre-split A part tile
    constexpr int AHR = AH ? (A8 + 255) / 256 : 1;
    constexpr int W8 = BN * (LG_KT / 8);      // 8-element groups of a W part tile
    constexpr int WR = (W8 + 255) / 256;
    float4 ra[AR];
    uint4 rah[AHR][AH ? P : 1];
    uint4 rw[WR][P];
    const T* Ah = static_cast<const T*>(p.Ah);
    auto load = [&](int k0) {
        if constexpr (AH) {
#pragma unroll
            for (int k = 0; k < AHR; ++k) {
                const int i = tid + 256 * k;
                const int row = i / (LG_KT / 8), c = i % (LG_KT / 8);
                const long long gm = m0 + row;
                const int kk = k0 + c * 8;
                const bool in = i < A8 && gm < p.M && kk < p.K;
#pragma unroll
                for (int q = 0; q < P; ++q)
                    rah[k][q] = in ? *reinterpret_cast<const uint4*>(Ah + q * p.astride + presplit_idx(gm, kk, p.lda, p.akstride))
                                   : make_uint4(0u, 0u, 0u, 0u);
            }
        }
#pragma unroll
        for (int k = 0; k < (AH ? 0 : AR); ++k) {
            const int i = tid + 256 * k;
            const int row = i / (LG_KT / 4), c = i % (LG_KT / 4);
            const long long gm = m0 + row;
            const int kk = k0 + c * 4;
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (i < A4 && gm < p.M && kk < p.K) {
                v = *reinterpret_cast<const float4*>(p.A + gm * p.lda + kk);
                if constexpr (SCALE) {
                    const float4 sc = *reinterpret_cast<const float4*>(p.scale + (gm / p.scale_rows) * p.ld_scale + kk);
                    v.x = sc.x * v.x; v.y = sc.y * v.y; v.z = sc.z * v.z; v.w = sc.w * v.w;
                }
            }
            ra[k] = v;
        }
#pragma unroll
        for (int k = 0; k < WR; ++k) {
            const int i = tid + 256 * k;
            const int row = i / (LG_KT / 8), c = i % (LG_KT / 8);
            const int gn = n0 + row, kk = k0 + c * 8;
            const bool in = i < W8 && gn < p.N && kk < p.K;
#pragma unroll
            for (int q = 0; q < P; ++q)
                rw[k][q] = in ? *reinterpret_cast<const uint4*>(
                                    W + q * p.wstride +
                                    (AH ? presplit_idx(gn, kk, p.ldw, p.wkstride) : (long long)gn * p.ldw + kk))
                              : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    auto store = [&]() {
        if constexpr (AH) {
#pragma unroll
            for (int k = 0; k < AHR; ++k) {
                const int i = tid + 256 * k;
                if (i >= A8) continue;
                const int row = i / (LG_KT / 8), c = i % (LG_KT / 8);
#pragma unroll
                for (int q = 0; q < P; ++q) *reinterpret_cast<uint4*>(&As[q][row][c * 8]) = rah[k][q];
            }
        }
#pragma unroll
        for (int k = 0; k < (AH ? 0 : AR); ++k) {
            const int i = tid + 256 * k;
            if (i >= A4) continue;
            const int row = i / (LG_KT / 4), c = i % (LG_KT / 4);
            const float x[4] = {ra[k].x, ra[k].y, ra[k].z, ra[k].w};
            uint2 four[P];
            split4_packed<T>(x, four);
#pragma unroll
            for (int q = 0; q < P; ++q) *reinterpret_cast<uint2*>(&As[q][row][c * 4]) = four[q];
        }
#pragma unroll
        for (int k = 0; k < WR; ++k) {
            const int i = tid + 256 * k;
            if (i >= W8) continue;
            const int row = i / (LG_KT / 8), c = i % (LG_KT / 8);
#pragma unroll
            for (int q = 0; q < P; ++q) *reinterpret_cast<uint4*>(&Ws[q][row][c * 8]) = rw[k][q];
        }
    };

    f32x4 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    load(0);
    for (int k0 = 0; k0 < p.K; k0 += LG_KT) {
        store();
        lds_barrier();
        if (k0 + LG_KT < p.K) load(k0 + LG_KT);
#pragma unroll 1
        for (int ks = 0; ks < LG_KT / 32; ++ks) {   // MFMA K steps of the staged step, in increasing K
            if (k0 + ks * 32 >= p.K) break;          // uniform
            V8 a[WM][P], b[WN][P];
#pragma unroll
            for (int mt = 0; mt < WM; ++mt)
#pragma unroll
                for (int q = 0; q < P; ++q)
                    a[mt][q] = *reinterpret_cast<const V8*>(&As[q][(wm * WM + mt) * 16 + r][ks * 32 + g * 8]);
#pragma unroll
            for (int nt = 0; nt < WN; ++nt)
#pragma unroll
                for (int q = 0; q < P; ++q)
                    b[nt][q] = *reinterpret_cast<const V8*>(&Ws[q][(wn * WN + nt) * 16 + r][ks * 32 + g * 8]);
#pragma unroll
            for (int i = 0; i < S::NPROD; ++i)
#pragma unroll
                for (int mt = 0; mt < WM; ++mt)
#pragma unroll
                    for (int nt = 0; nt < WN; ++nt)
                        acc[mt][nt] = S::mfma(a[mt][S::ap(i)], b[nt][S::wp(i)], acc[mt][nt]);
        }
        lds_barrier();
    }
    // lane holds C[m0 + (wm*WM + mt)*16 + g*4 + i][n0 + (wn*WN + nt)*16 + r]
    const int nbase = n0 + wn * WN * 16;
    if (p.swiglu) {  // 16-row panels alternate gate / up; WN is even and nbase a multiple of 32
#pragma unroll
        for (int mt = 0; mt < WM; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const long long m = m0 + (wm * WM + mt) * 16 + g * 4 + i;
                if (m >= p.M) continue;
#pragma unroll
                for (int nt = 0; nt + 1 < WN; nt += 2) {
                    const int panel = nbase / 16 + nt;
                    if ((panel + 1) * 16 <= p.N)
                        swiglu_store<T>(p, m, (panel / 2) * 16 + r, swiglu_value(p, acc[mt][nt][i], acc[mt][nt + 1][i]));
                }
            }
        return;
    }
#pragma unroll
    for (int mt = 0; mt < WM; ++mt)
        epi_block<WN>(p, [&](int i) { return m0 + (wm * WM + mt) * 16 + g * 4 + i; },
                      [&](int j) { return nbase + j * 16 + r; }, [&](int i, int j) { return acc[mt][j][i]; });
}

inline unsigned int cdiv(long long a, long long b) { return (unsigned int)((a + b - 1) / b); }

// Pre-split A GEMM with direct global -> LDS loads (the sequence GEMMs of the half tiers, whose A arrives already
// split into the tier's parts).  Workgroup tile 64 WGM x 32 WN, 2 WGM waves of 64 x 16 WN, K steps of 32.
// The operand tiles of a K step are sixteen-row fragment blocks of 1 KB each (A: 8 blocks per part, W: 8 per part),
// written by global_load_lds_dwordx4 (16 bytes per lane, lane l to byte 16 l of its block) with no register staging,
// and read back as MFMA fragments.  DMA lane l carries row l / 4 and 16-byte K chunk (l % 4) ^ dma_swz(l / 4) of the
// block (a per-row chunk permutation), so that a fragment read's lanes hit distinct banks.  NS K steps
// share an LDS ring (fp16: 2 x 32 KB for 128 x 128 tiles, two 4-wave workgroups per CU; bf16: 2 x 72 KB for
// 256 x 128 tiles, one 8-wave workgroup per CU): a step waits for its own loads (s_waitcnt on the wave's count of younger loads) and one barrier, then issues
// the loads of step k + NS - 1 into the slot step k - 1 used.  Per output the MFMA sequence is that of every other MFMA GEMM kernel (K steps in order,
// the split products in order), so results are bitwise equal to theirs.
template <typename T, int NS_, int WN_, int WGM_> struct DmaCfg {
    static constexpr int P = Split<T>::P;
    static constexpr int NS = NS_;                            // K steps in flight
    static constexpr int WN = WN_;                            // 16-column tiles per wave (2 x WN per workgroup)
    static constexpr int WGM = WGM_, WAVES = 2 * WGM_;        // wave rows (64 rows each) x 2 wave columns
    static constexpr int BM = 64 * WGM;
    static constexpr int AB = BM / 16, WB = 2 * WN;           // fragment blocks per part: A, W
    static constexpr int BLK = 1024;                          // bytes of one 16 x 32 fragment block
    static constexpr int TB = P * (AB + WB);                  // blocks per K step: [A part][block], [W part][block]
    static constexpr int STAGE = TB * BLK;
    static constexpr int DPW = TB / WAVES;                    // loads per wave per K step
    static_assert(TB % WAVES == 0, "the step's blocks are dealt evenly over the waves");
};

// Chunk permutation of a fragment block's row r (16-byte K chunk c stored at slot 4 r + (c ^ dma_swz(r))): the 16
// lanes of a fragment read (one chunk of rows 0..15) then fall on 16 distinct 16-byte bank groups, and so do the
// 8-lane halves on 8 distinct groups of a 128-byte bank row.
__device__ __forceinline__ int dma_swz(int r) { return ((r >> 2) ^ (r >> 1)) & 3; }
constexpr int DMA_GM = 8;   // local M blocks per tile-order group (see gemm_dma_kernel)

// the wave's loads of one K step are issued; wait until at most N younger ones are outstanding
template <int N> __device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }
__device__ __forceinline__ void dma16(const void* src, void* lds_block) {
    __builtin_amdgcn_global_load_lds(src, lds_block, 16, 0, 0);
}

template <typename T, int NS_, int WN_, int WGM_>
__global__ void __launch_bounds__(128 * WGM_) gemm_dma_kernel(GemmArgs p, int mblocks, int nblocks, int vec_c) {
    typedef Split<T> S;
    typedef typename S::V8 V8;
    typedef DmaCfg<T, NS_, WN_, WGM_> D;
    constexpr int P = S::P, NS = D::NS, DPW = D::DPW, AB = D::AB, WB = D::WB;
    constexpr int WM = 4, WN = D::WN, WGN = 2, BN = 16 * WN * WGN;
    __shared__ __attribute__((aligned(1024))) unsigned char ring[NS * D::STAGE];
    const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: the LDS destinations are scalar
    const int wm = wave / WGN, wn = wave % WGN;
    // Tile order: workgroups go round-robin over the XCDs, so XCD x runs slots 0, 1, ... of its own M blocks
    // (mb = 8 mbl + x).  Its slots walk groups of DMA_GM local M blocks column block by column block, so the ~64
    // workgroups resident on an XCD share DMA_GM A blocks and a few W column blocks: both stay in the XCD's L2
    // (4 MB) instead of the whole W being cycled through it once per M block.
    const int xcd = blockIdx.x % XCDS, slot = blockIdx.x / XCDS;
    const int mloc = (mblocks + XCDS - 1) / XCDS;                // local M blocks per XCD
    const int grp = slot / (DMA_GM * nblocks), within = slot % (DMA_GM * nblocks);
    const int gsize = min(DMA_GM, mloc - grp * DMA_GM);
    const int mb = (grp * DMA_GM + within % gsize) * XCDS + xcd, nb = within / gsize;
    if (mb >= mblocks) return;   // uniform over the workgroup
    const long long m0 = (long long)mb * D::BM;
    const int n0 = nb * BN;
    const T* Ah = static_cast<const T*>(p.Ah);
    const T* W = static_cast<const T*>(p.W);
    const int nk = p.K / 32;

    // this lane's source rows of the wave's DPW loads (rows clamped into range; K chunk swizzled), at the first K
    // step; each K step advances a load by its operand's 32-column group stride
    const int drow = lane >> 2, dchunk = (lane & 3) ^ dma_swz(drow);
    const T* src[DPW];
    long long kst[DPW];
    int boff[DPW];
#pragma unroll
    for (int j = 0; j < DPW; ++j) {
        const int jj = wave * DPW + j;                 // 0 .. TB - 1
        boff[j] = jj * D::BLK;
        if (jj < P * AB) {
            const int q = jj / AB, blk = jj % AB;
            const long long row = min(m0 + blk * 16 + drow, (long long)p.M - 1);
            src[j] = Ah + q * p.astride + row * p.lda + dchunk * 8;
            kst[j] = p.akstride;
        } else {
            const int q = (jj - P * AB) / WB, blk = (jj - P * AB) % WB;
            const int n = min(n0 + blk * 16 + drow, p.N - 1);
            src[j] = W + q * p.wstride + (long long)n * p.ldw + dchunk * 8;
            kst[j] = p.wkstride;
        }
    }
    auto issue = [&](int ks) {
        unsigned char* st = ring + (ks % NS) * D::STAGE;
#pragma unroll
        for (int j = 0; j < DPW; ++j) dma16(src[j] + ks * kst[j], st + boff[j]);
    };
    // fragment reads: lane (r, g) takes chunk g of row r of a block, stored at lane slot 4 r + (g ^ dma_swz(r))
    const int foff = 16 * (4 * r + (g ^ dma_swz(r)));

    f32x4 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < NS - 1; ++ks)
        if (ks < nk) issue(ks);
    static_assert(NS >= 2 && NS - 2 <= 2, "wait counts cover at most two younger steps");
    for (int ks = 0; ks < nk; ++ks) {
        // this step's loads are the oldest of the wave's outstanding ones: younger = min(NS - 2, nk - 1 - ks) steps
        const int younger = min(NS - 2, nk - 1 - ks);
        if (younger >= 2) wait_vm<2 * DPW>();
        else if (younger == 1) wait_vm<DPW>();
        else wait_vm<0>();
        __builtin_amdgcn_s_barrier();   // every wave's loads of step ks are in LDS; step ks - 1's slot is free
        if (ks + NS - 1 < nk) issue(ks + NS - 1);
        const unsigned char* st = ring + (ks % NS) * D::STAGE;
        V8 a[WM][P], b[WN][P];
#pragma unroll
        for (int mt = 0; mt < WM; ++mt)
#pragma unroll
            for (int q = 0; q < P; ++q)
                a[mt][q] = *reinterpret_cast<const V8*>(st + (q * AB + wm * WM + mt) * D::BLK + foff);
#pragma unroll
        for (int nt = 0; nt < WN; ++nt)
#pragma unroll
            for (int q = 0; q < P; ++q)
                b[nt][q] = *reinterpret_cast<const V8*>(st + (P * AB + q * WB + wn * WN + nt) * D::BLK + foff);
#pragma unroll
        for (int i = 0; i < S::NPROD; ++i)
#pragma unroll
            for (int mt = 0; mt < WM; ++mt)
#pragma unroll
                for (int nt = 0; nt < WN; ++nt) acc[mt][nt] = S::mfma(a[mt][S::ap(i)], b[nt][S::wp(i)], acc[mt][nt]);
    }
    // lane holds C[m0 + (wm*WM + mt)*16 + g*4 + i][n0 + (wn*WN + nt)*16 + r]
    const int nbase = n0 + wn * WN * 16;
    if (p.swiglu) {  // 16-row panels alternate gate / up; WN is even and nbase a multiple of 32
#pragma unroll
        for (int mt = 0; mt < WM; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const long long m = m0 + (wm * WM + mt) * 16 + g * 4 + i;
                if (m >= p.M) continue;
#pragma unroll
                for (int nt = 0; nt + 1 < WN; nt += 2) {
                    const int panel = nbase / 16 + nt;
                    if ((panel + 1) * 16 <= p.N)
                        swiglu_store<T>(p, m, (panel / 2) * 16 + r, swiglu_value(p, acc[mt][nt][i], acc[mt][nt + 1][i]));
                }
            }
        return;
    }
    constexpr int TW = 16 * WN, GPR = TW / 4;   // tile columns, float4 groups per row
    if constexpr ((TW & (TW - 1)) == 0 && TW >= 32) {
        // fp32 C in 16-byte column groups (vec_c: the host checked alignment and strides): the wave's 64 x TW tile
        // goes through its own LDS region of the (now idle) ring, then each store instruction writes 64 / GPR whole
        // rows of the tile (TW x 4 bytes each) instead of 64-byte pieces of 16.  The region is [64][TW] floats with
        // the 16-column group index XOR-ed by the row's (row / 4) % 4 (modulo the width), so the fragment writes
        // (rows 4g + i, 16 columns per lane group g) and the row reads spread over the banks.
        if (vec_c) {
            static_assert(D::WAVES * 64 * TW * 4 <= NS * D::STAGE, "the ring holds every wave's C tile");
            __syncthreads();   // every wave has read its last operands from the ring
            float* wt = reinterpret_cast<float*>(ring) + wave * 64 * TW;
#pragma unroll
            for (int mt = 0; mt < WM; ++mt)
#pragma unroll
                for (int nt = 0; nt < WN; ++nt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int row = mt * 16 + g * 4 + i;
                        wt[row * TW + ((nt * 16 + r) ^ ((g * 16) & (TW - 1)))] = acc[mt][nt][i];
                    }
            __syncthreads();
            constexpr int PASSES = 64 * GPR / 64;
            const int c4 = lane % GPR, rsub = lane / GPR;   // this lane's column group; row within a pass
            const int n = nbase + c4 * 4;
            const bool ncol = n < p.N;                      // N % 4 == 0: a group is wholly in or out
            float4 bv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (p.bias && ncol) bv = *reinterpret_cast<const float4*>(p.bias + n);
            float4 v[PASSES], rv[PASSES];
            const long long mw = m0 + wm * WM * 16;
#pragma unroll
            for (int q = 0; q < PASSES; ++q) {
                const int row = q * (64 / GPR) + rsub;
                v[q] = *reinterpret_cast<const float4*>(wt + row * TW + ((c4 * 4) ^ ((((row >> 2) & 3) * 16) & (TW - 1))));
                const long long m = min(mw + row, (long long)p.M - 1);
                rv[q] = p.res ? *reinterpret_cast<const float4*>(p.R + m * p.ldr + min(n, p.N - 4))
                              : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
            for (int q = 0; q < PASSES; ++q) {
                const long long m = mw + q * (64 / GPR) + rsub;
                if (m >= p.M || !ncol) continue;
                float4 o;
                o.x = epi_value(p, v[q].x, bv.x, rv[q].x);
                o.y = epi_value(p, v[q].y, bv.y, rv[q].y);
                o.z = epi_value(p, v[q].z, bv.z, rv[q].z);
                o.w = epi_value(p, v[q].w, bv.w, rv[q].w);
                // non-temporal: C (up to 381 MB per launch) would otherwise evict the A group and W blocks the
                // tile order keeps in L2 (sequence GEMMs 2.09 -> 2.05 ms, step -0.5% per 128 clips)
                __builtin_nontemporal_store(f32x4{o.x, o.y, o.z, o.w}, reinterpret_cast<f32x4*>(p.C + m * p.ldc + n));
            }
            return;
        }
    }
#pragma unroll
    for (int mt = 0; mt < WM; ++mt)
        epi_block<WN>(p, [&](int i) { return m0 + (wm * WM + mt) * 16 + g * 4 + i; },
                      [&](int j) { return nbase + j * 16 + r; }, [&](int i, int j) { return acc[mt][j][i]; });
}



// Small M (one clip's frames or window): one wave per 16 rows x SM_NT*16 columns, the operands of SM_D K steps in
// flight (a ring of registers refilled as each step is consumed), so a wave waits on memory once per SM_D steps
// instead of once per step.  The MFMA sequence of every output (K steps in order, the split products in order) is
// the direct kernel's, so results are bitwise those of the large-M kernels: the kernel choice by M keeps rows
// independent of the batch.
constexpr int SM_NT = 2, SM_D = 4;

template <typename T, bool SCALE, bool AH>
__global__ void __launch_bounds__(64) gemm_small_kernel(GemmArgs p) {
    static_assert(!(SCALE && AH), "pre-split A carries no SE scale");
    typedef Split<T> S;
    typedef typename S::V8 V8;
    constexpr int P = S::P;
    const int lane = threadIdx.x, r = lane & 15, g = lane >> 4;
    const long long mbase = (long long)blockIdx.x * 16;
    const int nbase = blockIdx.y * (SM_NT * 16);
    const T* W = static_cast<const T*>(p.W);
    const long long row = mbase + r, rc = row < p.M ? row : p.M - 1;
    const bool row_live = row < p.M;
    const int ksteps = (p.K + 31) / 32;
    float xa[AH ? 1 : SM_D][8], xs[SCALE ? SM_D : 1][8];
    uint4 xh[AH ? SM_D : 1][P];
    uint4 wv[SM_D][SM_NT][P];
    const T* Ah = static_cast<const T*>(p.Ah);
    // The K chunk kc of step st lies st * kstride + (kc - 32 st) past an operand row: kc - 32 st is the lane's chunk
    // g * 8 in the group, or (row-major, last step of a K not a multiple of 32) the clamp back to K - 8, where
    // kstride is 32.  Pre-split A comes with the sequence GEMMs' layouts; otherwise W is row-major.
    auto load = [&](int slot, int st) {
        const int kc = min(st * 32 + g * 8, p.K - 8);
        const long long wk = AH ? (long long)st * p.wkstride + (kc - st * 32) : kc;
        if constexpr (AH) {
            const T* a = Ah + rc * p.lda + (long long)st * p.akstride + (kc - st * 32);
#pragma unroll
            for (int q = 0; q < P; ++q) xh[slot][q] = *reinterpret_cast<const uint4*>(a + q * p.astride);
        } else {
            read8(p.A + rc * p.lda + kc, xa[slot]);
        }
        if constexpr (SCALE) read8(p.scale + (rc / p.scale_rows) * p.ld_scale + kc, xs[slot]);
#pragma unroll
        for (int nt = 0; nt < SM_NT; ++nt) {
            const int col = min(nbase + nt * 16 + r, p.N - 1);
#pragma unroll
            for (int q = 0; q < P; ++q)
                wv[slot][nt][q] = *reinterpret_cast<const uint4*>(W + q * p.wstride + (long long)col * p.ldw + wk);
        }
    };
#pragma unroll
    for (int d = 0; d < SM_D; ++d)
        if (d < ksteps) load(d, d);
    f32x4 acc[SM_NT];
#pragma unroll
    for (int nt = 0; nt < SM_NT; ++nt) acc[nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < ksteps; s0 += SM_D) {
#pragma unroll
        for (int d = 0; d < SM_D; ++d) {
            const int st = s0 + d;
            if (st >= ksteps) break;   // uniform
            const bool kin = st * 32 + g * 8 < p.K;
            V8 a[P], b[SM_NT][P];
            if constexpr (AH) {
#pragma unroll
                for (int q = 0; q < P; ++q) {
                    const uint4 u = kin && row_live ? xh[d][q] : make_uint4(0u, 0u, 0u, 0u);
                    a[q] = *reinterpret_cast<const V8*>(&u);
                }
            } else {
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    float t = xa[d][e];
                    if constexpr (SCALE) t = xs[d][e] * t;
                    v[e] = kin && row_live ? t : 0.0f;
                }
                split8<T>(v, a);
            }
#pragma unroll
            for (int nt = 0; nt < SM_NT; ++nt) {
                const bool live = kin && nbase + nt * 16 + r < p.N;
#pragma unroll
                for (int q = 0; q < P; ++q) {
                    const uint4 u = live ? wv[d][nt][q] : make_uint4(0u, 0u, 0u, 0u);
                    b[nt][q] = *reinterpret_cast<const V8*>(&u);
                }
            }
            if (st + SM_D < ksteps) load(d, st + SM_D);
#pragma unroll
            for (int i = 0; i < S::NPROD; ++i)
#pragma unroll
                for (int nt = 0; nt < SM_NT; ++nt) acc[nt] = S::mfma(a[S::ap(i)], b[nt][S::wp(i)], acc[nt]);
        }
    }
    // lane holds C[mbase + g*4 + i][nbase + nt*16 + r]
    if (p.swiglu) {  // 16-row panels alternate gate / up; SM_NT is 2 and nbase a multiple of 32
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const long long m = mbase + g * 4 + i;
            if (m >= p.M) continue;
            const int panel = nbase / 16;
            if ((panel + 1) * 16 <= p.N) swiglu_store<T>(p, m, (panel / 2) * 16 + r, swiglu_value(p, acc[0][i], acc[1][i]));
        }
        return;
    }
    epi_block<SM_NT>(p, [&](int i) { return mbase + g * 4 + i; }, [&](int j) { return nbase + j * 16 + r; },
                     [&](int i, int j) { return acc[j][i]; });
}

template <typename T> void launch_small(const GemmArgs& p, hipStream_t s) {
    if (!p.Ah && p.wkstride != 32) throw std::runtime_error("gemm_small: group-major W comes with pre-split A");
    const dim3 grid(cdiv(p.M, 16), cdiv(p.N, SM_NT * 16));
    if (p.Ah) hipLaunchKernelGGL((gemm_small_kernel<T, false, true>), grid, dim3(64), 0, s, p);
    else if (p.scale) hipLaunchKernelGGL((gemm_small_kernel<T, true, false>), grid, dim3(64), 0, s, p);
    else hipLaunchKernelGGL((gemm_small_kernel<T, false, false>), grid, dim3(64), 0, s, p);
}

// Streaming GEMM for narrow N (<= 160 columns, every column in one workgroup) and large M: the SE-block projects,
// whose A (the depthwise output, fp32) is the only large operand and is read exactly once.  A workgroup (4 waves)
// takes 128 rows; a wave owns 32 rows x all NT column tiles.  Each wave keeps the A rows of the next ST_D K steps in
// flight in a register ring (issued as soon as a ring slot has been split), so it waits on HBM once per ST_D steps;
// the K step's pre-split weight tile [NT*16][32] is staged in a double-buffered LDS tile by the whole workgroup (one
// LDS barrier per step) and the SE scale rows of the frames the workgroup's rows span are staged once.  Same
// fragments, split products and K order per output as the direct kernel: results are bitwise those of every other
// MFMA GEMM kernel.
constexpr int ST_D = 2;                         // K steps of A in flight ahead of the one being multiplied
constexpr int ST_WLD = 32 + 8;                  // staged W row stride in T elements

template <typename T, int NT, bool SCALE, int WPF, int ST_MT>
__global__ void __launch_bounds__(64 * MFMA_WAVES, 2) gemm_stream_kernel(GemmArgs p) {
    constexpr int ST_ROWS = MFMA_WAVES * ST_MT * 16;   // rows per workgroup
    typedef Split<T> S;
    typedef typename S::V8 V8;
    constexpr int P = S::P, BN = NT * 16;
    constexpr int WV = P * BN * 4;                          // 16-byte vectors of one staged W tile
    constexpr int WR = (WV + 64 * MFMA_WAVES - 1) / (64 * MFMA_WAVES);
    __shared__ __attribute__((aligned(16))) T Ws[2][P][BN][ST_WLD];
    extern __shared__ __attribute__((aligned(16))) float Sc[];   // SCALE: [nf][K]
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r = lane & 15, g = lane >> 4;
    const long long m0 = (long long)blockIdx.x * ST_ROWS;
    const long long mbase = m0 + wave * ST_MT * 16;
    const T* W = static_cast<const T*>(p.W);
    const int nks = (p.K + 31) / 32;
    long long f0 = 0;
    if constexpr (SCALE) {
        f0 = m0 / p.scale_rows;
        const int nf = int((min(m0 + ST_ROWS, (long long)p.M) - 1) / p.scale_rows - f0) + 1;
        for (int i = tid; i < nf * (p.K / 4); i += 64 * MFMA_WAVES) {
            const int fi = i / (p.K / 4), k4 = i - fi * (p.K / 4);
            *reinterpret_cast<float4*>(Sc + fi * p.K + k4 * 4) =
                *reinterpret_cast<const float4*>(p.scale + (f0 + fi) * p.ld_scale + k4 * 4);
        }
    }
    // this lane's A rows (clamped into range: every load is unconditional) and their frames' scale rows in LDS
    const float* arow[ST_MT];
    int srow[ST_MT];
    bool rlive[ST_MT];
#pragma unroll
    for (int mt = 0; mt < ST_MT; ++mt) {
        const long long row = mbase + mt * 16 + r;
        const long long rc = row < p.M ? row : p.M - 1;
        rlive[mt] = row < p.M;
        arow[mt] = p.A + rc * p.lda;
        srow[mt] = SCALE ? int(rc / p.scale_rows - f0) * p.K : 0;
    }
    // pre-split W tiles: K step ks + WPF is loaded into a register slot while step ks multiplies and stored into the
    // other LDS buffer at the end of step ks + WPF - 1 (WPF = 2 hides the weights' L2 latency behind two steps, at
    // the cost of a second slot of registers)
    static_assert(WPF == 1 || WPF == 2, "one or two steps of weight prefetch");
    uint4 wr[WPF][WR];
    auto load_w = [&](int ks, uint4 (&dst)[WR]) {
#pragma unroll
        for (int k = 0; k < WR; ++k) {
            const int i = min(tid + k * 64 * MFMA_WAVES, WV - 1);
            const int c8 = i & 3, n = (i >> 2) % BN, q = (i >> 2) / BN;
            const int kk = ks * 32 + c8 * 8;
            const bool in = n < p.N && kk < p.K;
            const uint4 v = *reinterpret_cast<const uint4*>(W + q * p.wstride + (long long)min(n, p.N - 1) * p.ldw +
                                                          min(kk, p.K - 8));
            dst[k] = in ? v : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    auto store_w = [&](int buf, const uint4 (&src)[WR]) {
#pragma unroll
        for (int k = 0; k < WR; ++k) {
            const int i = tid + k * 64 * MFMA_WAVES;
            if (i >= WV) continue;
            const int c8 = i & 3, n = (i >> 2) % BN, q = (i >> 2) / BN;
            *reinterpret_cast<uint4*>(&Ws[buf][q][n][c8 * 8]) = src[k];
        }
    };
    float ring[ST_D][ST_MT][8];
    auto load_a = [&](int ks, float (&dst)[ST_MT][8]) {
        const int kc = min(ks * 32 + g * 8, p.K - 8);
#pragma unroll
        for (int mt = 0; mt < ST_MT; ++mt) read8(arow[mt] + kc, dst[mt]);
    };
    load_w(0, wr[0]);
#pragma unroll
    for (int d = 0; d < ST_D; ++d)
        if (d < nks) load_a(d, ring[d]);
    store_w(0, wr[0]);
    if (WPF == 2 && nks > 1) load_w(1, wr[WPF - 1]);
    lds_barrier();

    f32x4 acc[ST_MT][NT];
#pragma unroll
    for (int i = 0; i < ST_MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // one K step: W of step ks + WPF into register slot wload, split the A ring slot's rows (scaled), refill that
    // slot ST_D steps ahead, multiply, stage W of step ks + 1 (register slot wstore) in the other LDS buffer
    auto step = [&](int ks, float (&slot)[ST_MT][8], uint4 (&wload)[WR], const uint4 (&wstore)[WR]) {
        if (ks + WPF < nks) load_w(ks + WPF, wload);
        const int kk = ks * 32 + g * 8;
        const bool kin = kk < p.K;
        const int kc = kin ? kk : p.K - 8;
        V8 a[ST_MT][P];
#pragma unroll
        for (int mt = 0; mt < ST_MT; ++mt) {
            const bool live = kin && rlive[mt];
            float sc[8];
            if constexpr (SCALE) read8(Sc + srow[mt] + kc, sc);
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float t = slot[mt][e];
                if constexpr (SCALE) t = sc[e] * t;
                v[e] = live ? t : 0.0f;
            }
            split8<T>(v, a[mt]);
        }
        if (ks + ST_D < nks) load_a(ks + ST_D, slot);
        const int buf = ks & 1;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            V8 b[P];
#pragma unroll
            for (int q = 0; q < P; ++q) b[q] = *reinterpret_cast<const V8*>(&Ws[buf][q][nt * 16 + r][g * 8]);
#pragma unroll
            for (int i = 0; i < S::NPROD; ++i)
#pragma unroll
                for (int mt = 0; mt < ST_MT; ++mt) acc[mt][nt] = S::mfma(a[mt][S::ap(i)], b[S::wp(i)], acc[mt][nt]);
        }
        if (ks + 1 < nks) store_w(buf ^ 1, wstore);
        lds_barrier();
    };
    static_assert(ST_D == 2, "the A ring and the W register slots alternate with the step parity");
    for (int ks = 0; ks < nks; ks += 2) {
        step(ks, ring[0], wr[0], wr[WPF - 1]);
        if (ks + 1 < nks) step(ks + 1, ring[1], wr[WPF - 1], wr[0]);
    }
    if (mbase >= p.M) return;
#pragma unroll
    for (int mt = 0; mt < ST_MT; ++mt)
        epi_block<NT>(p, [&](int i) { return mbase + mt * 16 + g * 4 + i; }, [&](int j) { return j * 16 + r; },
                      [&](int i, int j) { return acc[mt][j][i]; });
}

// Wide GEMM: large M, short K (<= 256), many columns (the config-2 expand M x 160 -> 960, the audio frontend's
// 1x1 layers).  A workgroup (4 waves) takes 64 rows: their K values are loaded once (16-byte loads), split into the
// operand parts and staged in LDS, where every wave reads them; wave w then walks the 16-column tiles w, w + 4, ...
// of N, each a 64 x 16 output block of 4 accumulators.  A tile's weight fragments for all KS K steps are loaded in
// one go one tile ahead (two register sets alternating with the tile parity), so a wave waits on L2 once per tile,
// not once per K step.  Results go through the wave's LDS region and leave as whole 64-byte row pieces,
// non-temporal.  A is read from HBM exactly once (the direct and LDS-tiled kernels re-read it once per column block:
// 7-12 times at N = 960).  Per output: K steps of 32 in increasing order, the split products in mfma_split's order,
// the accumulator from +0, epi_value's epilogue -- bitwise the other MFMA kernels' results.
constexpr int WD_ROWS = 64, WD_KMAX = 256, WD_PAD = 8, WD_SLD = 64 + 4;
template <typename T, int KS, int GR>
__global__ void __launch_bounds__(256, 2) gemm_wide_kernel(GemmArgs p) {
    typedef Split<T> S;
    typedef typename S::V8 V8;
    constexpr int P = S::P;
    extern __shared__ __attribute__((aligned(16))) unsigned char wd_lds[];
    constexpr int kp = KS * 32, ld = kp + WD_PAD;
    T* As = reinterpret_cast<T*>(wd_lds);   // [P][64][ld], then the waves' C staging regions [4][16][WD_SLD]
    float* Cs = reinterpret_cast<float*>(wd_lds + (size_t)P * WD_ROWS * ld * sizeof(T));
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, r = lane & 15;
    const long long m0 = (long long)blockIdx.x * WD_ROWS;
    // stage: row i / (kp / 4), k quad i % (kp / 4); zero outside [M) x [K)
    constexpr int q4 = kp / 4;
#pragma unroll 2
    for (int i = tid; i < WD_ROWS * q4; i += 256) {
        const int row = i / q4, kq = i - row * q4, k = kq * 4;
        const long long m = m0 + row;
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (m < p.M && k < p.K) v = *reinterpret_cast<const float4*>(p.A + m * p.lda + k);
        const float x[4] = {v.x, v.y, v.z, v.w};
        uint2 four[P];
        split4_packed<T>(x, four);
#pragma unroll
        for (int q = 0; q < P; ++q) *reinterpret_cast<uint2*>(As + (q * WD_ROWS + row) * ld + k) = four[q];
    }
    lds_barrier();
    const T* W = static_cast<const T*>(p.W);
    const int tiles = (p.N + 15) / 16;
    // tile t's fragments for every K step: lane chunk k = 32 ks + 8 g (zero past K, read at a valid address)
    const auto load_tile = [&](V8 (&dst)[KS][P], int t) {
        const T* wrow = W + (long long)min(t * 16 + r, p.N - 1) * p.ldw + g * 8;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const bool kin = ks * 32 + g * 8 < p.K;
#pragma unroll
            for (int q = 0; q < P; ++q) {
                const V8 v = load_part8<T>(wrow + q * p.wstride + (kin ? ks * 32 : 0));
                dst[ks][q] = kin ? v : V8{};
            }
        }
    };
    float* wt = Cs + wave * 16 * WD_SLD;
    // one 16-column tile's 64 x 16 outputs into acc (4 row tiles), from its prefetched weight fragments
    const auto tile = [&](f32x4 (&acc)[4], const V8 (&wf)[KS][P]) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) acc[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                V8 a[P];
#pragma unroll
                for (int q = 0; q < P; ++q)
                    a[q] = *reinterpret_cast<const V8*>(As + (q * WD_ROWS + mt * 16 + r) * ld + ks * 32 + g * 8);
                acc[mt] = mfma_split<T>(a, wf[ks], acc[mt]);
            }
            // keeps the compiler from hoisting every K step's A fragment reads ahead of the products
            asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3])::"memory");
        }
    };
    // a group's 64 x 16 GR outputs (tiles j < GR of columns nbase + 16 j ..): per 16-row block through the wave's
    // LDS region [16][WD_SLD] (a lane group's fragment writes land 16 banks apart), then lane l stores row
    // l / (4 GR) + (16 / GR) k, columns 4 (l % 4 GR) .. + 3: each store instruction writes whole 64 GR-byte row
    // pieces, non-temporal
    constexpr int C4 = 4 * GR, RPS = 64 / C4;   // float4 groups per row, rows per store instruction
    const auto store_group = [&](const f32x4 (&acc)[GR][4], int nbase) {
        const int c4 = lane % C4, rsub = lane / C4;
        const int n = min(nbase + c4 * 4, p.N - 4);
        const float4 bv = p.bias ? *reinterpret_cast<const float4*>(p.bias + n) : make_float4(0.f, 0.f, 0.f, 0.f);
        // PLAIN (bias, no residual: the expand layers): the flags leave the per-element code
        const auto go = [&](auto act, auto plain) {
            constexpr int ACT = decltype(act)::value;
            constexpr bool PLAIN = decltype(plain)::value;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
                for (int j = 0; j < GR; ++j)
#pragma unroll
                    for (int i = 0; i < 4; ++i) wt[(4 * g + i) * WD_SLD + j * 16 + r] = acc[j][mt][i];
                wave_lds_sync();
                float4 v[16 / RPS], rv[16 / RPS];
#pragma unroll
                for (int k = 0; k < 16 / RPS; ++k) {
                    const int row = RPS * k + rsub;
                    const long long m = min(m0 + mt * 16 + row, (long long)p.M - 1);
                    v[k] = *reinterpret_cast<const float4*>(wt + row * WD_SLD + c4 * 4);
                    rv[k] = p.res ? *reinterpret_cast<const float4*>(p.R + m * p.ldr + n) : make_float4(0.f, 0.f, 0.f, 0.f);
                }
                wave_lds_sync();   // the region is rewritten by the next block
#pragma unroll
                for (int k = 0; k < 16 / RPS; ++k) {
                    const long long m = m0 + mt * 16 + RPS * k + rsub;
                    if (m >= p.M || nbase + c4 * 4 >= p.N) continue;
                    const float in[4] = {v[k].x, v[k].y, v[k].z, v[k].w}, bb[4] = {bv.x, bv.y, bv.z, bv.w},
                                rr[4] = {rv[k].x, rv[k].y, rv[k].z, rv[k].w};
                    f32x4 o;
                    if constexpr (PLAIN) {   // epi_value's operations with bias, activation fixed, no residual
                        float x[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) x[e] = in[e] * p.wscale + bb[e];
                        apply_act4<ACT>(x);
                        o = f32x4{x[0], x[1], x[2], x[3]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {   // epi_value's operations with the activation fixed
                            float x = in[e] * p.wscale;
                            if (p.bias) x = x + bb[e];
                            x = apply_act(x, ACT);
                            if (p.res == 3) x = rr[e] + 0.7071067811865475244f * x;
                            else if (p.res) x = p.res == 2 ? rr[e] + x / 1.41421356237309515f : rr[e] + x;
                            o[e] = x;
                        }
                    }
                    __builtin_nontemporal_store(o, reinterpret_cast<f32x4*>(p.C + m * p.ldc + nbase + c4 * 4));
                }
            }
        };
        const auto go_act = [&](auto act) {
            if (p.bias && !p.res) go(act, std::true_type{});
            else go(act, std::false_type{});
        };
        // the activation is uniform: one branch per group, straight-line code per element
        switch (p.act) {
        case ACT_RELU: go_act(std::integral_constant<int, ACT_RELU>{}); break;
        case ACT_HS: go_act(std::integral_constant<int, ACT_HS>{}); break;
        case ACT_HSIG: go_act(std::integral_constant<int, ACT_HSIG>{}); break;
        case ACT_SILU: go_act(std::integral_constant<int, ACT_SILU>{}); break;
        default: go_act(std::integral_constant<int, ACT_NONE>{}); break;
        }
    };
    // wave w takes the GR-tile groups w, w + 4, ...; its tiles' weights alternate between two register sets, the
    // next tile's loads in flight while one computes
    static_assert(GR == 2 || GR == 4, "groups of 2 or 4 tiles");
    const int groups = (tiles + GR - 1) / GR;
    V8 w0[KS][P], w1[KS][P];
    const auto tile_of = [&](int gi, int j) { return min(gi * GR + j, tiles - 1); };   // past N: recomputes the last
    if (wave < groups) load_tile(w0, tile_of(wave, 0));
    for (int gi = wave; gi < groups; gi += 4) {
        f32x4 acc[GR][4];
        load_tile(w1, tile_of(gi, 1));
        tile(acc[0], w0);
        if constexpr (GR == 4) {
            load_tile(w0, tile_of(gi, 2));
            tile(acc[1], w1);
            load_tile(w1, tile_of(gi, 3));
            tile(acc[2], w0);
            if (gi + 4 < groups) load_tile(w0, tile_of(gi + 4, 0));
            tile(acc[3], w1);
        } else {
            if (gi + 4 < groups) load_tile(w0, tile_of(gi + 4, 0));
            tile(acc[1], w1);
        }
        store_group(acc, gi * GR * 16);
    }
}
// groups of four tiles (256-byte row pieces) where the registers allow, else two (fp16 K <= 192, bf16 K <= 128)
template <typename T, int KS> void launch_wide_ks(const GemmArgs& p, hipStream_t s) {
    constexpr int GR = (Split<T>::P == 2 ? KS <= 6 : KS <= 4) ? 4 : 2;
    const size_t lds = size_t(Split<T>::P) * WD_ROWS * (KS * 32 + WD_PAD) * sizeof(T) +
                       size_t(4) * 16 * WD_SLD * sizeof(float);
    hipLaunchKernelGGL((gemm_wide_kernel<T, KS, GR>), dim3(cdiv(p.M, WD_ROWS)), dim3(256), lds, s, p);
}
bool wide_ok(const GemmArgs& p) {
    const auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    return !p.Ah && !p.Ch && !p.swiglu && !p.scale && p.wkstride == 32 && p.K <= WD_KMAX && p.K % 8 == 0 &&
           p.lda % 4 == 0 && al16(p.A) && p.ldc % 4 == 0 && p.N % 4 == 0 && al16(p.C) && (!p.bias || al16(p.bias)) &&
           (!p.res || (p.ldr % 4 == 0 && al16(p.R)));
}
template <typename T> void launch_wide(const GemmArgs& p, hipStream_t s) {
    if (!wide_ok(p))
        throw std::runtime_error("gemm_wide: fp32 A and C (16-byte rows), N % 4 == 0, K <= 256 (multiple of 8), "
                                 "row-major W, no SE scale or SwiGLU");
    if (Split<T>::P == 3 && p.K > 192) throw std::runtime_error("gemm_wide: bf16 takes K <= 192");   // registers
    switch ((p.K + 31) / 32) {
    case 1: launch_wide_ks<T, 1>(p, s); return;
    case 2: launch_wide_ks<T, 2>(p, s); return;
    case 3: launch_wide_ks<T, 3>(p, s); return;
    case 4: launch_wide_ks<T, 4>(p, s); return;
    case 5: launch_wide_ks<T, 5>(p, s); return;
    case 6: launch_wide_ks<T, 6>(p, s); return;
    default:
        if constexpr (Split<T>::P == 2) {
            if (p.K <= 224) launch_wide_ks<T, 7>(p, s);
            else launch_wide_ks<T, 8>(p, s);
        }
        return;
    }
}

template <typename T, int NT, int ST_MT>
void launch_stream_mt(const GemmArgs& p, hipStream_t s) {
    constexpr int ST_ROWS = MFMA_WAVES * ST_MT * 16;
    if (p.K % 8 || p.N > NT * 16) throw std::runtime_error("gemm_stream: K must be a multiple of 8 and N fit the tiles");
    size_t lds = 0;
    if (p.scale) {
        if (p.scale_rows < 1) throw std::runtime_error("gemm_stream: bad scale row count");
        const size_t nf = size_t((ST_ROWS - 1) / p.scale_rows + 2);   // frames a workgroup's rows can span
        lds = nf * size_t(p.K) * sizeof(float);
        if (lds > 64 * 1024) throw std::runtime_error("gemm_stream: SE scale rows exceed the LDS budget");
    }
    const unsigned blocks = cdiv(p.M, ST_ROWS);
    // measured: the second weight slot pays only for the widest fp16 tiles; bf16's three-part weight tile is better
    // single-slotted (N 160, K 960, 38,400 rows: 180 vs 195 us; fp16 82.5 vs 83.8)
    constexpr int WPF = (NT >= 8 && Split<T>::P == 2) ? 2 : 1;
    if (p.scale)
        hipLaunchKernelGGL((gemm_stream_kernel<T, NT, true, WPF, ST_MT>), dim3(blocks), dim3(64 * MFMA_WAVES), lds, s, p);
    else
        hipLaunchKernelGGL((gemm_stream_kernel<T, NT, false, WPF, ST_MT>), dim3(blocks), dim3(64 * MFMA_WAVES), 0, s, p);
}
// rows per wave: 32, or 16 for N <= 48 (blocks 4-6 on a 640-frame branch, 588,800 rows, N 40: fp16 62.6 vs 71.5 us
// at K 72 and 112 vs 122.5 at K 120, bf16 78 vs 93 and 127-131 vs 139-140; 64 rows slower, and they spill at the
// widest tiles)
template <typename T, int NT>
void launch_stream_nt(const GemmArgs& p, hipStream_t s) { launch_stream_mt<T, NT, (NT <= 3 ? 1 : 2)>(p, s); }

template <typename T> void launch_stream(const GemmArgs& p, hipStream_t s) {
    if (p.Ah || p.Ch || p.swiglu) throw std::runtime_error("gemm_stream: fp32 A and C only, no SwiGLU");
    switch ((p.N + 15) / 16) {
    case 1: launch_stream_nt<T, 1>(p, s); return;
    case 2: launch_stream_nt<T, 2>(p, s); return;
    case 3: launch_stream_nt<T, 3>(p, s); return;
    case 4: launch_stream_nt<T, 4>(p, s); return;
    case 5: launch_stream_nt<T, 5>(p, s); return;
    case 6: launch_stream_nt<T, 6>(p, s); return;
    case 7: launch_stream_nt<T, 7>(p, s); return;
    case 8: launch_stream_nt<T, 8>(p, s); return;
    case 9: launch_stream_nt<T, 9>(p, s); return;
    case 10: launch_stream_nt<T, 10>(p, s); return;
    }
    throw std::runtime_error("gemm_stream: N must be at most 160");
}

template <typename T, int NT>
void launch_direct(const GemmArgs& p, hipStream_t s) {
    const int mblocks = (int)cdiv(p.M, 16LL * MFMA_MT * MFMA_WAVES), nblocks = (int)cdiv(p.N, NT * 16);
    const long long blocks = (long long)cdiv(mblocks, XCDS) * XCDS * nblocks;
    if (blocks >= (1ll << 31)) throw std::runtime_error("gemm_direct: grid too large");
    const dim3 grid((unsigned)blocks);
    if (p.scale)
        hipLaunchKernelGGL((gemm_direct_kernel<T, NT, true>), grid, dim3(64 * MFMA_WAVES), 0, s, p, mblocks, nblocks);
    else
        hipLaunchKernelGGL((gemm_direct_kernel<T, NT, false>), grid, dim3(64 * MFMA_WAVES), 0, s, p, mblocks, nblocks);
}

template <typename T, int NS, int WN, int WGM> void launch_dma_cfg(const GemmArgs& p, hipStream_t s) {
    const int mblocks = (int)cdiv(p.M, 64 * WGM), nblocks = (int)cdiv(p.N, 32 * WN);
    const long long blocks = (long long)cdiv(mblocks, XCDS) * XCDS * nblocks;
    if (blocks >= (1ll << 31)) throw std::runtime_error("gemm_dma: grid too large");
    // fp32 C stored in 16-byte column groups when N, the strides and the pointers allow it
    const auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    const int vec_c = !p.swiglu && p.ldc % 4 == 0 && p.N % 4 == 0 && al16(p.C) && (!p.bias || al16(p.bias)) &&
                      (!p.res || (p.ldr % 4 == 0 && al16(p.R)));
    hipLaunchKernelGGL((gemm_dma_kernel<T, NS, WN, WGM>), dim3((unsigned)blocks), dim3(128 * WGM), 0, s, p, mblocks,
                       nblocks, vec_c);
}

// fp16 sequence GEMMs that take 256 x 64 workgroup tiles: fp32 C wider than 1024 columns
inline bool dma_narrow_tiles(const GemmArgs& p) { return !p.swiglu && p.N > 1024; }

template <typename T> void launch_dma(const GemmArgs& p, hipStream_t s) {
    if (!p.Ah || p.K % 32 || p.astride % 8 || p.wstride % 8 || p.lda % 8 || p.ldw % 8)
        throw std::runtime_error("gemm_dma: needs pre-split A, K % 32 == 0 and 16-byte aligned rows");
    // Configurations are (ring depth NS, column tiles per wave WN, wave rows WGM): 2 WGM waves per workgroup on a
    // (64 WGM) x (32 WN) tile.  Deeper rings lose everywhere (fp16 in-projection: ring 3 +19-52%, ring 4
    // +96%): the occupancy their LDS costs is worth more than the latency they hide.  Per shape (64-window launches,
    // 20,544 rows, timed alone on one box): fp16 -- the wide fp32-C GEMMs (in-projection N 2316, SISA N 1068) run
    // 12% faster on 256 x 64 tiles (2,2,4) with the staged 16-byte C stores (in-projection 153-165 vs 176-187 us,
    // SISA 71 vs 81-83 us); the N = 384 and SwiGLU shapes stay on 128 x 128 (2,4,2) (o_proj 47 vs 58 us, FFN down 55
    // vs 69 us).  bf16 -- 128 x 64 tiles (2,2,2) on every shape (against 256 x 128 (2,4,4): o_proj 78 vs 123 us, FFN
    // down 95 vs 146, SISA 125 vs 158, in-projection 278 vs 291-295, FFN up 200 vs 198-210).  A workgroup that
    // computes several column tiles and stores the previous tile's C during the next one's K steps was bitwise
    // equal and 35-50% slower: the registers that hold the pending outputs cost a resident workgroup per CU.
    if constexpr (Split<T>::P == 2) {
        if (dma_narrow_tiles(p)) launch_dma_cfg<T, 2, 2, 4>(p, s);
        else launch_dma_cfg<T, 2, 4, 2>(p, s);
    } else {
        launch_dma_cfg<T, 2, 2, 2>(p, s);
    }
}

// the direct-to-LDS kernel for pre-split A unless SHV_HIP_NO_GEMM_DMA is set (read per launch: the bitwise
// cross-check against the register-staged kernel switches it within one process)
static bool gemm_dma_enabled() { return std::getenv("SHV_HIP_NO_GEMM_DMA") == nullptr; }

template <typename T, int WM, int WN, int WGM, int WGN>
void launch_lds(const GemmArgs& p, hipStream_t s) {
    if (!p.Ah && p.wkstride != 32) throw std::runtime_error("gemm_lds: group-major W comes with pre-split A");
    const int mblocks = (int)cdiv(p.M, 16LL * WM * WGM), nblocks = (int)cdiv(p.N, 16 * WN * WGN);
    const long long blocks = (long long)cdiv(mblocks, XCDS) * XCDS * nblocks;
    if (blocks >= (1ll << 31)) throw std::runtime_error("gemm_lds: grid too large");
    const dim3 grid((unsigned)blocks);
    if (p.Ah)
        hipLaunchKernelGGL((gemm_lds_kernel<T, WM, WN, WGM, WGN, false, true>), grid, dim3(256), 0, s, p, mblocks,
                           nblocks);
    else if (p.scale)
        hipLaunchKernelGGL((gemm_lds_kernel<T, WM, WN, WGM, WGN, true, false>), grid, dim3(256), 0, s, p, mblocks,
                           nblocks);
    else
        hipLaunchKernelGGL((gemm_lds_kernel<T, WM, WN, WGM, WGN, false, false>), grid, dim3(256), 0, s, p, mblocks,
                           nblocks);
}

// The kernel a GEMM of the MFMA tiers runs: one decision, used to launch and to name the launch.
// N up to 160 (CNN projects and 1x1 layers): direct fragments, 16-column tiles per wave chosen to minimise
// padded columns (at most 5 per wave); wider N (last 1x1, sequence): LDS-staged 128 x 128 workgroup tiles.
struct GemmPlan {
    enum Kind { Small, Dma, Lds, Stream, Direct, Wide } kind;
    int nt;   // column tiles (Stream, Direct)
};
template <typename T> GemmPlan plan_gemm(const GemmArgs& p) {
    if (p.M <= 2048) return {GemmPlan::Small, 0};   // latency: one clip's shapes
    // SE excitation layers (fp32 A, M = frames): one wave per 16 x 32 tile spreads them over the device (measured
    // at 2560 frames: 124 vs 282 us for the ten fc shapes with the tiled kernels)
    if (!p.Ah && !p.scale && !p.swiglu && p.M <= 8192) return {GemmPlan::Small, 0};
    const int tiles = (p.N + 15) / 16;
    if (p.Ah && p.K % 32 == 0 && gemm_dma_enabled()) return {GemmPlan::Dma, 0};
    // fp32 A, no SE scale, K >= 64, large M (the GEMM tool's shapes, the layer path, the audio frontend), measured
    // per shape: N > 160 on the wide kernel (M x 160 -> 960: fp16 268 vs 459 us, bf16 364 vs 906; 614,400 x 112 ->
    // 672: 906 vs 1,400, bf16 1,112 vs 2,817), N <= 160 on the streaming kernel (153,600 x 960 -> 160: 298 vs 409;
    // 614,400 x 672 -> 112: 605 vs 795; 2,355,200 x 120 -> 40: 378 vs 465); K 40 stays on the direct kernel
    // (2,007,040 x 40 -> 120: stream 702 vs 534, wide 860)
    if (!p.Ah && !p.scale && !p.swiglu && p.K >= 64) {
        if (tiles > 10 && wide_ok(p) && (Split<T>::P == 2 || p.K <= 192)) return {GemmPlan::Wide, 0};
        if (tiles <= 10 && p.K % 8 == 0 && p.wkstride == 32) return {GemmPlan::Stream, tiles};
    }
    // K < 64, large M, measured per shape: up to 5 column tiles the streaming kernel (9,216,000 x 24 -> 72: 859 vs
    // 980 us; the SHIELD-A frontend's 1,276,160 x 32 -> 64: 156 vs 168); 6 tiles the direct kernel at 2 per wave
    // (319,360 x 48 -> 96: 66 vs 79 at 3 per wave, streaming 77); more than 10 the wide kernel (2,355,200 x 40 ->
    // 240: fp16 1,176 vs 1,553 LDS-tiled, bf16 1,247 vs 3,005); 7 to 10 the direct choice below (2,007,040 x 40 ->
    // 120: fp16 531 vs 548 wide and 699 streaming; bf16 723 vs 933 wide)
    if (!p.Ah && !p.scale && !p.swiglu && p.K < 64 && p.K % 8 == 0 && p.wkstride == 32) {
        if (tiles <= 5) return {GemmPlan::Stream, tiles};
        if (tiles == 6) return {GemmPlan::Direct, 2};
        if (tiles > 10 && wide_ok(p)) return {GemmPlan::Wide, 0};
    }
    if (p.swiglu || tiles > 10) return {GemmPlan::Lds, 0};
    if (p.Ah) throw std::runtime_error("gemm: pre-split A needs N > 160 or M <= 2048");
    if (p.scale) {   // SE projects: A read once, all columns per workgroup -- unless that leaves the device idle
        // measured per shape (one to four clips' blocks 4-15): the small-M kernel wins while the streaming grid
        // (128 rows per workgroup) is under 128 workgroups (4,800 rows N 112: 15 vs 34 us; 9,600: 27 vs 34; 4,800
        // rows N 160: 40 vs 63) or, for N <= 48, under 256 (18,400 rows N 40: 8.4 vs 10.5 us); above, streaming
        // (19,200 rows N 112: 37 vs 45 us; 36,800 rows N 40: 13.7 vs 16.7)
        const long long wgs = cdiv(p.M, 128);
        if (wgs < 128 || (tiles <= 3 && wgs < 256)) return {GemmPlan::Small, 0};
        return {GemmPlan::Stream, tiles};
    }
    int nt = tiles;
    if (tiles > 5) {
        int best_cols = 1 << 30;
        for (int c = 5; c >= 3; --c) {
            const int cols = (tiles + c - 1) / c * c;
            if (cols < best_cols) { best_cols = cols; nt = c; }
        }
    }
    return {GemmPlan::Direct, nt};
}

template <typename T> void launch_gemm(const GemmArgs& p, hipStream_t s) {
    const GemmPlan pl = plan_gemm<T>(p);
    if ((pl.kind == GemmPlan::Stream || pl.kind == GemmPlan::Direct) && p.wkstride != 32)
        throw std::runtime_error("gemm: the streaming and direct kernels take a row-major W");
    switch (pl.kind) {
    case GemmPlan::Small: launch_small<T>(p, s); return;
    case GemmPlan::Dma: launch_dma<T>(p, s); return;
    case GemmPlan::Lds: launch_lds<T, 4, 4, 2, 2>(p, s); return;
    case GemmPlan::Wide: launch_wide<T>(p, s); return;
    case GemmPlan::Stream: launch_stream<T>(p, s); return;
    case GemmPlan::Direct:
        switch (pl.nt) {
        case 1: launch_direct<T, 1>(p, s); return;
        case 2: launch_direct<T, 2>(p, s); return;
        case 3: launch_direct<T, 3>(p, s); return;
        case 4: launch_direct<T, 4>(p, s); return;
        default: launch_direct<T, 5>(p, s); return;
        }
    }
}

// Last 1x1 (160 -> 960, + bias, hardswish) fused with the 4x4 adaptive pool of the 6x10 map, half tiers.  One
// workgroup per frame: the frame's 60 x 160 input is staged in LDS (split into the operand parts, rows 60..63
// zero), each wave takes output-channel tiles nt = wave, wave + 4, ... and computes C[64 px][16 ch] with the same
// split products in the same K order as the GEMM kernels, applies the same epilogue, writes the tile to its own LDS
// rows and pools it exactly as the pool kernel does (bin = rows {0,1,3,4}[r] + [0,2) x cols {0,2,5,7}[c] + [0,3),
// sum from +0 row by row, then (sum / 2) / 3).  The pooled tokens are therefore bitwise those of the unfused path,
// and the 60 x 960 map never reaches HBM.
constexpr int TAIL_K = 160, TAIL_N = 960, TAIL_XLD = TAIL_K + 8, TAIL_ELD = 16 + 1;

template <typename T>
__global__ void __launch_bounds__(256) tail_pool_kernel(const float* __restrict__ X, const T* __restrict__ W,
                                                        long long wstride, float wscale, const float* __restrict__ bias,
                                                        float* __restrict__ out, int F, int ns) {
    typedef Split<T> S;
    typedef typename S::V8 V8;
    constexpr int P = S::P;
    __shared__ __attribute__((aligned(16))) T Xs[P][64][TAIL_XLD];
    __shared__ float Es[4][64][TAIL_ELD];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r = lane & 15, g = lane >> 4;
    // ns workgroups per frame (few frames): workgroup `part` takes output tiles part * 4 + wave + 4 ns j
    const long long f = blockIdx.x / ns;
    const int part = int(blockIdx.x % ns), nt0 = part * 4 + wave, ntstep = 4 * ns;
    const float* Xf = X + f * 60 * TAIL_K;
    // stage: 64 rows x 40 float4 (rows 60..63 zero), split into the parts
    for (int i = tid; i < 64 * (TAIL_K / 4); i += 256) {
        const int row = i / (TAIL_K / 4), c4 = i - row * (TAIL_K / 4);
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (row < 60) v = *reinterpret_cast<const float4*>(Xf + row * TAIL_K + c4 * 4);
        const float x[4] = {v.x, v.y, v.z, v.w};
        uint2 four[P];
        split4_packed<T>(x, four);
#pragma unroll
        for (int q = 0; q < P; ++q) *reinterpret_cast<uint2*>(&Xs[q][row][c4 * 4]) = four[q];
    }
    __syncthreads();
    float(*E)[TAIL_ELD] = Es[wave];
    // weight fragments of the wave's next output tile load while the current one computes
    V8 w[TAIL_K / 32][P], wn[TAIL_K / 32][P];
    auto load_w = [&](int nt, V8 (&dst)[TAIL_K / 32][P]) {
#pragma unroll
        for (int ks = 0; ks < TAIL_K / 32; ++ks)
#pragma unroll
            for (int q = 0; q < P; ++q)
                dst[ks][q] = load_part8<T>(W + q * wstride + (long long)(nt * 16 + r) * TAIL_K + ks * 32 + g * 8);
    };
    load_w(nt0, w);
    for (int nt = nt0; nt < TAIL_N / 16; nt += ntstep) {
        if (nt + ntstep < TAIL_N / 16) load_w(nt + ntstep, wn);
        const float b = bias[nt * 16 + r];
        f32x4 acc[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) acc[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < TAIL_K / 32; ++ks) {
            V8 a[4][P];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int q = 0; q < P; ++q) a[mt][q] = *reinterpret_cast<const V8*>(&Xs[q][mt * 16 + r][ks * 32 + g * 8]);
#pragma unroll
            for (int i = 0; i < S::NPROD; ++i)
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) acc[mt] = S::mfma(a[mt][S::ap(i)], w[ks][S::wp(i)], acc[mt]);
        }
        // lane holds C[mt*16 + 4g + i][nt*16 + r]: * wscale, + bias, hardswish (the GEMM epilogue), into this
        // wave's rows
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) E[mt * 16 + 4 * g + i][r] = apply_act(acc[mt][i] * wscale + b, ACT_HS);
        asm volatile("" ::: "memory");   // one wave's LDS accesses execute in issue order
        // pool: lane (channel r, bins g, g + 4, g + 8, g + 12)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int tok = g + 4 * j;
            const int r0 = ((tok >> 2) * 3) >> 1, c0 = ((tok & 3) * 5) >> 1;
            float sum = 0.0f;
#pragma unroll
            for (int y = 0; y < 2; ++y)
#pragma unroll
                for (int x = 0; x < 3; ++x) sum = sum + E[(r0 + y) * 10 + c0 + x][r];
            out[(f * 16 + tok) * TAIL_N + nt * 16 + r] = (sum / 2.0f) / 3.0f;
        }
        asm volatile("" ::: "memory");
#pragma unroll
        for (int ks = 0; ks < TAIL_K / 32; ++ks)
#pragma unroll
            for (int q = 0; q < P; ++q) w[ks][q] = wn[ks][q];
    }
}

// One past the last element of a rows x cols part in GemmArgs' operand layout (row stride ld, 32-column group
// stride kstride).
long long presplit_span(long long rows, int cols, long long ld, long long kstride) {
    return (long long)((cols - 1) >> 5) * kstride + (rows - 1) * ld + ((cols - 1) & 31) + 1;
}
// 16-byte aligned rows and groups, and no two elements at one address: row-major (kstride 32, ld >= cols) or
// group-major (cols % 32 == 0, ld >= 32, a group's rows before the next group)
bool presplit_layout_ok(long long rows, int cols, long long ld, long long kstride) {
    if (ld % 8 || kstride % 8) return false;
    if (kstride == 32) return ld >= cols;
    return cols % 32 == 0 && ld >= 32 && kstride >= (rows - 1) * ld + 32;
}
bool row_major_operands(const GemmArgs& p) { return p.wkstride == 32 && p.akstride == 32 && p.ckstride == 32; }

void check_args(const GemmArgs& p, bool mfma) {
    if (p.M <= 0 || p.N <= 0 || p.K <= 0) throw std::runtime_error("gemm: empty shape");
    if (!(p.A || p.Ah) || !p.W || !(p.C || p.Ch)) throw std::runtime_error("gemm: null operand");
    if ((p.Ah || p.Ch) && !mfma) throw std::runtime_error("gemm_f32: pre-split operands are for the MFMA tiers");
    if (!mfma && !row_major_operands(p)) throw std::runtime_error("gemm_f32: row-major operands only");
    if ((!p.Ah && p.akstride != 32) || (!p.Ch && p.ckstride != 32))
        throw std::runtime_error("gemm: fp32 A and C are row-major");
    if (p.Ah && (p.A || p.scale || !presplit_layout_ok(p.M, p.K, p.lda, p.akstride) ||
                 p.astride < presplit_span(p.M, p.K, p.lda, p.akstride)))
        throw std::runtime_error("gemm: pre-split A takes no fp32 A or SE scale and needs a valid layout and part stride");
    if (p.Ch && (p.C || !p.swiglu || !presplit_layout_ok(p.M, p.N / 2, p.ldc, p.ckstride) ||
                 p.cstride < presplit_span(p.M, p.N / 2, p.ldc, p.ckstride)))
        throw std::runtime_error("gemm: a pre-split output is a SwiGLU output with a valid layout and part stride");
    if (p.res && !p.R) throw std::runtime_error("gemm: residual without R");
    if (p.res < 0 || p.res > 3) throw std::runtime_error("gemm: unknown residual mode");
    if (p.scale && (p.scale_rows <= 0 || p.ld_scale < p.K)) throw std::runtime_error("gemm: bad SE scale");
    int wexp = 0;
    if (!(p.wscale > 0.0f) || std::frexp(p.wscale, &wexp) != 0.5f)
        throw std::runtime_error("gemm: the weight scale must be a power of two");
    if (!mfma && p.wscale != 1.0f) throw std::runtime_error("gemm_f32: fp32 weights are not pre-scaled");
    if (mfma) {
        // 32-byte A and 16-byte W fragments: K, lda, ldw, ld_scale multiples of 8 elements
        if (p.K % 8 || p.lda % 8 || p.ldw % 8 || (!p.Ah && p.lda < p.K) || (p.scale && p.ld_scale % 8) ||
            !presplit_layout_ok(p.N, p.K, p.ldw, p.wkstride))
            throw std::runtime_error("gemm_mfma: K/lda/ldw must be multiples of 8 (K=" + std::to_string(p.K) + ")");
        if (p.swiglu && (p.N % 32)) throw std::runtime_error("gemm_mfma: swiglu needs N % 32 == 0");
        if (p.wstride < presplit_span(p.N, p.K, p.ldw, p.wkstride))
            throw std::runtime_error("gemm_mfma: bad weight part stride");
    } else {
        if (p.lda < p.K || p.ldw < p.K) throw std::runtime_error("gemm_f32: bad leading dimension");
        if (p.swiglu && (p.N % 2)) throw std::runtime_error("gemm_f32: swiglu needs even N");
    }
}

}  // namespace

namespace {
void launch_gemv_f32(const GemmArgs& p, hipStream_t s) {
    const int nkb = cdiv(p.K, F32_BK);
    if (nkb > 32) throw std::runtime_error("gemm_f32: the GEMV kernel takes K <= 2048");
    const int opw = p.swiglu ? (64 / nkb) & ~1 : 64 / nkb;
    const auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    const bool vec = al16(p.A) && al16(p.W) && p.lda % 4 == 0 && p.ldw % 4 == 0 &&
                     (!p.scale || (al16(p.scale) && p.ld_scale % 4 == 0));
    // rows per workgroup: one clip's SE excitation (20 rows) ran 18.5 us per layer in 8-row chunks
    const int rpw = p.M <= 32 ? 1 : p.M <= 64 ? 2 : p.M <= 128 ? 4 : GV_ROWS;
    const long long yblocks = cdiv(p.M, rpw);
    if (yblocks > 65535) throw std::runtime_error("gemm_f32: M too large for the GEMV kernel");
    const dim3 grid(cdiv(p.N, opw), (unsigned)yblocks);
    if (p.scale) {
        if (vec) hipLaunchKernelGGL((gemv_f32_kernel<true, true>), grid, dim3(64), 0, s, p, nkb, opw, rpw);
        else hipLaunchKernelGGL((gemv_f32_kernel<true, false>), grid, dim3(64), 0, s, p, nkb, opw, rpw);
    } else {
        if (vec) hipLaunchKernelGGL((gemv_f32_kernel<false, true>), grid, dim3(64), 0, s, p, nkb, opw, rpw);
        else hipLaunchKernelGGL((gemv_f32_kernel<false, false>), grid, dim3(64), 0, s, p, nkb, opw, rpw);
    }
}
// the 16-byte staging of gemm_f32_v4_kernel applies
bool v4_f32_ok(const GemmArgs& p) {
    const auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    return p.K % 4 == 0 && p.lda % 4 == 0 && p.ldw % 4 == 0 && p.lda >= p.K && p.ldw >= p.K && al16(p.A) &&
           al16(p.W) && (!p.scale || (p.ld_scale % 4 == 0 && al16(p.scale)));
}
void launch_tiled_f32(const GemmArgs& p, hipStream_t s) {
    const dim3 grid(cdiv(p.M, F32_BM), cdiv(p.N, F32_BN));
    if (v4_f32_ok(p)) {
        if (p.scale) hipLaunchKernelGGL((gemm_f32_v4_kernel<true, false>), grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((gemm_f32_v4_kernel<false, false>), grid, dim3(256), 0, s, p);
        return;
    }
    if (p.scale) hipLaunchKernelGGL(gemm_f32_kernel<true>, grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL(gemm_f32_kernel<false>, grid, dim3(256), 0, s, p);
}
void launch_kblock_f32(const GemmArgs& p, hipStream_t s) {
    const int nkb = cdiv(p.K, F32_BK);
    if (!p.ws || (long long)nkb * p.M * p.N > p.ws_floats)
        throw std::runtime_error("gemm_f32: the K-block kernel needs a workspace of ceil(K / 64) * M * N floats");
    const dim3 grid(cdiv(p.M, F32_BM), cdiv(p.N, F32_BN), (unsigned)nkb);
    if (v4_f32_ok(p)) {
        if (p.scale) hipLaunchKernelGGL((gemm_f32_v4_kernel<true, true>), grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((gemm_f32_v4_kernel<false, true>), grid, dim3(256), 0, s, p);
    } else if (p.scale) {
        hipLaunchKernelGGL(gemm_f32_kblock_kernel<true>, grid, dim3(256), 0, s, p);
    } else {
        hipLaunchKernelGGL(gemm_f32_kblock_kernel<false>, grid, dim3(256), 0, s, p);
    }
    const long long outs = (long long)p.M * (p.swiglu ? p.N / 2 : p.N);
    hipLaunchKernelGGL(gemm_f32_fold_kernel, dim3(cdiv(outs, 256)), dim3(256), 0, s, p, nkb);
}
// The narrow exact kernel's shapes (K, N) and column chunks NC: the 1x1 layers of blocks 1-6, at 4096 rows or more
// (a workgroup per 256 rows and NC columns)
template <int K, int N, int NC> void launch_narrow_f32_shape(const GemmArgs& p, hipStream_t s) {
    const dim3 grid(cdiv(p.M, 256), N / NC);
    if (p.scale) hipLaunchKernelGGL((gemm_f32_narrow_kernel<K, N, NC, true>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((gemm_f32_narrow_kernel<K, N, NC, false>), grid, dim3(256), 0, s, p);
}
bool narrow_f32_shape(const GemmArgs& p, bool launch, hipStream_t s) {
    const auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    if (p.swiglu || p.lda % 4 || p.ldw % 4 || p.ldc % 4 || (p.res && p.ldr % 4) || !al16(p.A) || !al16(p.W) ||
        !al16(p.C) || (p.bias && !al16(p.bias)) || (p.res && !al16(p.R)) || p.lda < p.K || p.ldw < p.K ||
        (p.scale && (p.ld_scale % 4 || !al16(p.scale))))
        return false;
    struct Shape { int K, N; void (*go)(const GemmArgs&, hipStream_t); };
    static const Shape shapes[] = {{16, 16, launch_narrow_f32_shape<16, 16, 16>},
                                   {16, 64, launch_narrow_f32_shape<16, 64, 16>},
                                   {64, 24, launch_narrow_f32_shape<64, 24, 8>},
                                   {24, 72, launch_narrow_f32_shape<24, 72, 24>},
                                   {72, 24, launch_narrow_f32_shape<72, 24, 8>},
                                   {72, 40, launch_narrow_f32_shape<72, 40, 8>},
                                   {40, 120, launch_narrow_f32_shape<40, 120, 24>},
                                   {120, 40, launch_narrow_f32_shape<120, 40, 8>}};
    for (const Shape& sh : shapes)
        if (sh.K == p.K && sh.N == p.N) {
            if (launch) sh.go(p, s);
            return true;
        }
    return false;
}
bool use_narrow_f32(const GemmArgs& p) { return p.M >= 4096 && narrow_f32_shape(p, false, nullptr); }
bool cols_f32_ok(const GemmArgs& p) {
    const auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    return !p.swiglu && p.K % 4 == 0 && p.K <= COLS_KMAX && p.lda % 4 == 0 && p.ldw % 4 == 0 && p.lda >= p.K &&
           p.ldw >= p.K && al16(p.A) && al16(p.W) && (!p.scale || (p.ld_scale % 4 == 0 && al16(p.scale)));
}
// Column chunks are not chosen automatically: at one clip's shapes the 16-byte tiled kernel beats them (blocks 8-10's
// expands, 4,800 rows, K 80, N 184-200: 10.3-11.5 vs 13.6-13.8 us; N 480-960: 15-23 vs 26-42 us), and K blocks +
// fold beat them on the long-K projects.  Kept as an explicit variant.
void launch_cols_f32(const GemmArgs& p, hipStream_t s) {
    if (!cols_f32_ok(p))
        throw std::runtime_error("gemm_f32: the column-chunk kernel needs K <= 1024, K / lda / ldw % 4 == 0, aligned "
                                 "operands and no SwiGLU");
    const dim3 grid(cdiv(p.M, 256), cdiv(p.N, COLS_NC));
    if (p.scale) hipLaunchKernelGGL(gemm_f32_cols_kernel<true>, grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL(gemm_f32_cols_kernel<false>, grid, dim3(256), 0, s, p);
}
void launch_narrow_f32(const GemmArgs& p, hipStream_t s) {
    if (!narrow_f32_shape(p, true, s))
        throw std::runtime_error("gemm_f32: no narrow kernel for K=" + std::to_string(p.K) + " N=" + std::to_string(p.N) +
                                 " with these leading dimensions / alignments");
}
// The exact-tier kernel for M above the GEMV range: K blocks in parallel when the tiled grid would not give every
// CU a workgroup and the workspace holds the block sums (measured with one clip: blocks 13-15 SE projects, 57
// tiles, and the 321-row sequence GEMMs ran 45-200 us on the tiled kernel)
bool use_kblock_f32(const GemmArgs& p) {
    const long long nkb = cdiv(p.K, F32_BK), tiles = (long long)cdiv(p.M, F32_BM) * cdiv(p.N, F32_BN);
    return p.ws && nkb >= 2 && tiles < 256 && nkb * p.M * p.N <= p.ws_floats;
}
}  // namespace

namespace {
struct F32MfmaTile {
    int mt, nt;
};
// Tiles of the fp32 matrix-core GEMM by shape (every choice gives the same per-output operations): 32 x 64 per
// workgroup while that grid gives every CU eight workgroups, 16 x 32 below (one clip's 321-row GEMMs: 252 to 1,533
// workgroups instead of 66 to 407).
F32MfmaTile plan_f32_mfma(const GemmArgs& p) {
    if ((long long)cdiv(p.M, 32) * cdiv(p.N, 64) >= 2048) return {2, 4};
    return {1, 2};
}
template <int MT, int NT> void launch_f32_mfma(const GemmArgs& p, hipStream_t s) {
    constexpr int D = MT * NT >= 8 ? 2 : 4;   // K steps in flight per wave: deeper for the small tiles
    const dim3 grid(cdiv(p.M, MT * 16), cdiv(p.N, NT * 16));
    if (p.scale) hipLaunchKernelGGL((gemm_f32_mfma_kernel<MT, NT, D, true>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((gemm_f32_mfma_kernel<MT, NT, D, false>), grid, dim3(256), 0, s, p);
}
}  // namespace

void gemm_f32_mfma(const GemmArgs& p, hipStream_t s) {
    check_args(p, false);
    const auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    if (p.K % 4 || p.lda % 4 || p.ldw % 4 || !al16(p.A) || !al16(p.W) ||
        (p.scale && (p.ld_scale % 4 || !al16(p.scale))))
        throw std::runtime_error("gemm_f32_mfma: K, lda, ldw, ld_scale must be multiples of 4 and A, W, scale "
                                 "16-byte aligned (K=" + std::to_string(p.K) + ")");
    if (p.swiglu && p.N % 32) throw std::runtime_error("gemm_f32_mfma: swiglu needs N % 32 == 0");
    const F32MfmaTile t = plan_f32_mfma(p);
    if (t.mt == 2) launch_f32_mfma<2, 4>(p, s);
    else launch_f32_mfma<1, 2>(p, s);
}

std::string gemm_f32_mfma_kernel_name(const GemmArgs& p) {
    const F32MfmaTile t = plan_f32_mfma(p);
    return "gemm_f32_mfma_kernel<" + std::to_string(t.mt) + "," + std::to_string(t.nt) + ">";
}

void gemm_f32(const GemmArgs& p, hipStream_t s) { gemm_f32_variant(p, s, 0); }

void gemm_f32_variant(const GemmArgs& p, hipStream_t s, int variant) {
    check_args(p, false);
    switch (variant) {
    case 0:
        if (p.M <= GV_MAXM && cdiv(p.K, F32_BK) <= 32) launch_gemv_f32(p, s);
        else if (use_narrow_f32(p)) launch_narrow_f32(p, s);
        else if (use_kblock_f32(p)) launch_kblock_f32(p, s);
        else launch_tiled_f32(p, s);
        return;
    case 1: launch_gemv_f32(p, s); return;
    case 2: launch_tiled_f32(p, s); return;
    case 3: launch_kblock_f32(p, s); return;
    case 5: launch_narrow_f32(p, s); return;
    case 6: launch_cols_f32(p, s); return;
    }
    throw std::runtime_error("gemm_f32: unknown kernel variant " + std::to_string(variant));
}

std::string gemm_f32_kernel(const GemmArgs& p) {
    if (p.M <= GV_MAXM && cdiv(p.K, F32_BK) <= 32) return "gemv_f32_kernel";
    if (use_narrow_f32(p)) return "gemm_f32_narrow_kernel<" + std::to_string(p.K) + "," + std::to_string(p.N) + ">";
    if (v4_f32_ok(p)) return use_kblock_f32(p) ? "gemm_f32_v4_kernel<part>" : "gemm_f32_v4_kernel";
    return use_kblock_f32(p) ? "gemm_f32_kblock_kernel" : "gemm_f32_kernel";
}

template <typename T> std::string gemm_mfma_kernel(const GemmArgs& p) {
    const std::string t = std::is_same<T, bf16>::value ? "bf16" : "f16";
    const GemmPlan pl = plan_gemm<T>(p);
    switch (pl.kind) {
    case GemmPlan::Small: return "gemm_small_kernel<" + t + ">";
    case GemmPlan::Dma:
        if (Split<T>::P != 2) return "gemm_dma_kernel<" + t + ",2,2,2>";
        return dma_narrow_tiles(p) ? "gemm_dma_kernel<" + t + ",2,2,4>" : "gemm_dma_kernel<" + t + ",2,4,2>";
    case GemmPlan::Lds: return "gemm_lds_kernel<" + t + ",4,4,2,2>";
    case GemmPlan::Stream: return "gemm_stream_kernel<" + t + "," + std::to_string(pl.nt) + ">";
    case GemmPlan::Wide: return "gemm_wide_kernel<" + t + ">";
    case GemmPlan::Direct: return "gemm_direct_kernel<" + t + "," + std::to_string(std::min(pl.nt, 5)) + ">";
    }
    return "gemm";
}
template std::string gemm_mfma_kernel<f16>(const GemmArgs&);
template std::string gemm_mfma_kernel<bf16>(const GemmArgs&);

template <typename T> void gemm_mfma(const GemmArgs& p, hipStream_t s) {
    check_args(p, true);
    launch_gemm<T>(p, s);
}

template <typename T> void gemm_mfma_variant(const GemmArgs& p, hipStream_t s, int variant) {
    check_args(p, true);
    if (variant >= 2 && variant <= 6 && (p.Ah || p.Ch || p.swiglu))
        throw std::runtime_error("gemm: the direct kernel takes fp32 A and C and no SwiGLU");
    if (((variant >= 2 && variant <= 6) || variant == 8) && p.wkstride != 32)
        throw std::runtime_error("gemm: the streaming and direct kernels take a row-major W");
    switch (variant) {
    case 0: launch_gemm<T>(p, s); return;
    case 1: launch_small<T>(p, s); return;
    case 2: launch_direct<T, 1>(p, s); return;
    case 3: launch_direct<T, 2>(p, s); return;
    case 4: launch_direct<T, 3>(p, s); return;
    case 5: launch_direct<T, 4>(p, s); return;
    case 6: launch_direct<T, 5>(p, s); return;
    case 7: launch_lds<T, 4, 4, 2, 2>(p, s); return;
    case 8: launch_stream<T>(p, s); return;
    case 9: launch_wide<T>(p, s); return;
    }
    throw std::runtime_error("gemm: unknown kernel variant " + std::to_string(variant));
}
template void gemm_mfma_variant<f16>(const GemmArgs&, hipStream_t, int);
template void gemm_mfma_variant<bf16>(const GemmArgs&, hipStream_t, int);
template void gemm_mfma<f16>(const GemmArgs&, hipStream_t);
template void gemm_mfma<bf16>(const GemmArgs&, hipStream_t);

template <typename T>
void launch_tail_pool(const float* x, const void* w, long long wstride, float wscale, const float* bias,
                      float* pooled, int F, hipStream_t s) {
    if (F <= 0) return;
    if (wstride < (long long)TAIL_N * TAIL_K) throw std::runtime_error("tail_pool: bad weight part stride");
    // workgroups per frame: a divisor of the 15 rounds of 4 tiles, so every wave gets whole tiles; one clip's 20
    // frames ran 50 us in 20 workgroups, and three per frame also balance the batch-128 branches (640 frames: fp16
    // 83 vs 86 us, bf16 110 vs 115; 320 frames: 43 vs 48, 57 vs 65; five per frame slower)
    const int ns = F >= 1024 ? 1 : F >= 86 ? 3 : F >= 52 ? 5 : 15;
    hipLaunchKernelGGL(tail_pool_kernel<T>, dim3((unsigned)(F * ns)), dim3(256), 0, s, x, static_cast<const T*>(w),
                       wstride, wscale, bias, pooled, F, ns);
}
template void launch_tail_pool<f16>(const float*, const void*, long long, float, const float*, float*, int,
                                   hipStream_t);
template void launch_tail_pool<bf16>(const float*, const void*, long long, float, const float*, float*, int,
                                    hipStream_t);

}  // namespace shv
