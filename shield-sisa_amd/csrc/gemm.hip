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
//   A wave owns MT x NT 16x16 output tiles (64 rows x NT*16 columns); operand fragments come straight from the
//   row-major A [M][K] and W [N][K] arrays (lane l: row l%16, k = k0 + (l/16)*8 .. +8); no LDS.  K advances in
//   steps of 32 in increasing order; a K tail is zero-filled, never split across waves.
#include "dev_common.hpp"
#include "kernels.hpp"
#include "mfma.hpp"

#include <stdexcept>
#include <string>

namespace shv {
namespace {

// ------------------------------------------------------------------------------------------------ epilogue
__device__ __forceinline__ void epi_store(const GemmArgs& p, long long m, int n, float v) {
    if (p.bias) v = v + p.bias[n];
    v = apply_act(v, p.act);
    if (p.res) {
        const float r = p.R[m * p.ldr + n];
        v = p.res == 2 ? r + v / 1.41421356237309515f : r + v;
    }
    p.C[m * p.ldc + n] = v;
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
        for (int i = tid; i < F32_BM * F32_BK; i += 256) {
            const int r = i / F32_BK, k = i % F32_BK;
            const long long gm = m0 + r;
            const int gn = n0 + r, gk = k0 + k;
            float a = 0.0f, w = 0.0f;
            if (k < kb) {
                if (gm < p.M) {
                    a = A[gm * p.lda + gk];
                    if (SCALE) a = p.scale[(gm / p.scale_rows) * p.ld_scale + gk] * a;
                }
                if (gn < p.N) w = W[(long long)gn * p.ldw + gk];
            }
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
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const long long m = m0 + ty * 4 + i;
        if (m >= p.M) continue;
        if (p.swiglu) {  // rows (2j, 2j+1) = (gate_j, up_j): this thread holds pairs j0, j0+1
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int n = n0 + tx * 4 + 2 * q;
                if (n + 1 < p.N) p.C[m * p.ldc + (n >> 1)] = silu(tot[i][2 * q]) * tot[i][2 * q + 1];
            }
            continue;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + tx * 4 + j;
            if (n < p.N) epi_store(p, m, n, tot[i][j]);
        }
    }
}

// ------------------------------------------------------------------------------------------------ MFMA
constexpr int MFMA_MT = 4;      // 16-row tiles per wave (64 rows)
constexpr int MFMA_WAVES = 4;   // waves per block, stacked along M (256 rows)

template <typename T, int NT, bool SCALE>
__global__ void __launch_bounds__(64 * MFMA_WAVES) gemm_mfma_kernel(GemmArgs p) {
    typedef Split<T> S;
    typedef typename S::V8 V8;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane & 15, g = lane >> 4;
    const long long mbase = ((long long)blockIdx.x * MFMA_WAVES + wave) * (MFMA_MT * 16);
    const int nbase = blockIdx.y * (NT * 16);
    if (mbase >= p.M) return;
    const T* W = static_cast<const T*>(p.W);
    f32x4 acc[MFMA_MT][NT];
#pragma unroll
    for (int i = 0; i < MFMA_MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < p.K; k0 += 32) {
        const int kk = k0 + g * 8;
        const bool kin = kk < p.K;
        V8 a[MFMA_MT][S::P], b[NT][S::P];
#pragma unroll
        for (int mt = 0; mt < MFMA_MT; ++mt) {
            const long long row = mbase + mt * 16 + r;
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = 0.0f;
            if (kin && row < p.M) {
                load8(p.A + row * p.lda + kk, x);
                if (SCALE) {
                    float sc[8];
                    load8(p.scale + (row / p.scale_rows) * p.ld_scale + kk, sc);
#pragma unroll
                    for (int e = 0; e < 8; ++e) x[e] = sc[e] * x[e];
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                T part[S::P];
                S::split(x[e], part);
#pragma unroll
                for (int q = 0; q < S::P; ++q) a[mt][q][e] = part[q];
            }
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int col = nbase + nt * 16 + r;
#pragma unroll
            for (int q = 0; q < S::P; ++q) {
                V8 v = {};
                if (kin && col < p.N) {
                    const uint4 u = *reinterpret_cast<const uint4*>(W + q * p.wstride + (long long)col * p.ldw + kk);
                    v = *reinterpret_cast<const V8*>(&u);
                }
                b[nt][q] = v;
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
#pragma unroll
    for (int mt = 0; mt < MFMA_MT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const long long m = mbase + mt * 16 + g * 4 + i;
            if (m >= p.M) continue;
            if (p.swiglu) {  // 16-row panels alternate gate / up; NT is even and nbase is a multiple of 32
#pragma unroll
                for (int nt = 0; nt + 1 < NT; nt += 2) {
                    const int panel = nbase / 16 + nt;
                    if ((panel + 1) * 16 <= p.N)
                        p.C[m * p.ldc + (panel / 2) * 16 + r] = silu(acc[mt][nt][i]) * acc[mt][nt + 1][i];
                }
                continue;
            }
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int n = nbase + nt * 16 + r;
                if (n < p.N) epi_store(p, m, n, acc[mt][nt][i]);
            }
        }
    }
}

inline unsigned int cdiv(long long a, long long b) { return (unsigned int)((a + b - 1) / b); }

template <typename T, int NT>
void launch_mfma_nt(const GemmArgs& p, hipStream_t s) {
    const dim3 grid(cdiv(p.M, 16LL * MFMA_MT * MFMA_WAVES), cdiv(p.N, NT * 16));
    if (p.scale) hipLaunchKernelGGL((gemm_mfma_kernel<T, NT, true>), grid, dim3(64 * MFMA_WAVES), 0, s, p);
    else hipLaunchKernelGGL((gemm_mfma_kernel<T, NT, false>), grid, dim3(64 * MFMA_WAVES), 0, s, p);
}

// N tiles per wave: minimise padded columns, at most 5 tiles
int pick_nt(int N, bool swiglu) {
    if (swiglu) return 4;
    const int tiles = (N + 15) / 16;
    if (tiles <= 5) return tiles;
    int best = 5, best_cols = 1 << 30;
    for (int nt = 5; nt >= 3; --nt) {
        const int cols = (tiles + nt - 1) / nt * nt;
        if (cols < best_cols) { best_cols = cols; best = nt; }
    }
    return best;
}

void check_args(const GemmArgs& p, bool mfma) {
    if (p.M <= 0 || p.N <= 0 || p.K <= 0) throw std::runtime_error("gemm: empty shape");
    if (!p.A || !p.W || !p.C) throw std::runtime_error("gemm: null operand");
    if (p.res && !p.R) throw std::runtime_error("gemm: residual without R");
    if (p.scale && (p.scale_rows <= 0 || p.ld_scale < p.K)) throw std::runtime_error("gemm: bad SE scale");
    if (mfma) {
        // 32-byte A and 16-byte W fragments: K, lda, ldw, ld_scale multiples of 8 elements
        if (p.K % 8 || p.lda % 8 || p.ldw % 8 || p.lda < p.K || p.ldw < p.K || (p.scale && p.ld_scale % 8))
            throw std::runtime_error("gemm_mfma: K/lda/ldw must be multiples of 8 (K=" + std::to_string(p.K) + ")");
        if (p.swiglu && (p.N % 32)) throw std::runtime_error("gemm_mfma: swiglu needs N % 32 == 0");
        if (p.wstride < (long long)p.N * p.ldw) throw std::runtime_error("gemm_mfma: bad weight part stride");
    } else {
        if (p.lda < p.K || p.ldw < p.K) throw std::runtime_error("gemm_f32: bad leading dimension");
        if (p.swiglu && (p.N % 2)) throw std::runtime_error("gemm_f32: swiglu needs even N");
    }
}

}  // namespace

void gemm_f32(const GemmArgs& p, hipStream_t s) {
    check_args(p, false);
    const dim3 grid(cdiv(p.M, F32_BM), cdiv(p.N, F32_BN));
    if (p.scale) hipLaunchKernelGGL(gemm_f32_kernel<true>, grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL(gemm_f32_kernel<false>, grid, dim3(256), 0, s, p);
}

template <typename T> void gemm_mfma(const GemmArgs& p, hipStream_t s) {
    check_args(p, true);
    switch (pick_nt(p.N, p.swiglu != 0)) {
    case 1: launch_mfma_nt<T, 1>(p, s); break;
    case 2: launch_mfma_nt<T, 2>(p, s); break;
    case 3: launch_mfma_nt<T, 3>(p, s); break;
    case 4: launch_mfma_nt<T, 4>(p, s); break;
    default: launch_mfma_nt<T, 5>(p, s); break;
    }
}
template void gemm_mfma<f16>(const GemmArgs&, hipStream_t);
template void gemm_mfma<bf16>(const GemmArgs&, hipStream_t);

}  // namespace shv
