// Sequence-stage kernels (GDN-A, GDN-B, SISA last row, head).  Residual stream and all non-GEMM arithmetic in
// fp32, SISA prefix sums in double.  Reductions reproduce the reference CPU engine's order: 16 lane partial sums
// (element i into lane i % 16, first product unfused, then fmas) and the fixed 16-lane tree
// (engine/model/isa_impl.hpp:45-53, 854-863, 866-962, 996-1069, 1127-1133).
#include "dev_common.hpp"
#include "engine.hpp"
#include "host_model.hpp"
#include "kernels.hpp"
#include "mfma.hpp"

#include <algorithm>
#include <mutex>
#include <stdexcept>
#include <string>
#include <type_traits>

namespace shv {
namespace {

inline unsigned int cdiv(long long a, long long b) { return (unsigned int)((a + b - 1) / b); }

// A normalised value for the next GEMM: fp32, or (MFMA tiers) its split parts, part q at base[q * pstride + idx]
template <typename T>
__device__ __forceinline__ void put_value(T* base, long long pstride, long long idx, float y) {
    if constexpr (std::is_same<T, float>::value) {
        base[idx] = y;
    } else {
        T part[Split<T>::P];
        Split<T>::split(y, part);
#pragma unroll
        for (int q = 0; q < Split<T>::P; ++q) base[q * pstride + idx] = part[q];
    }
}

// ------------------------------------------------------------------------------------------------ window input
// A window's residual stream and the A operand of GDN-A's first in-projection in one pass (no separate assembly
// pass over h).  Row t of window b is token t % 16 of the frame at window position t / 16 -- found through a table
// of frame token blocks (TABLE) or at tokens + b * ldw + t * 384 (a window's 20 frames' tokens back to back, or a
// SHIELD-A window's 125 tokens) -- plus position row t when there is a position table (SHIELD-V); the last row is
// the readout vector.  The row is written to h, then normalised exactly as rmsnorm_kernel does it (16 lanes per
// row, lane l owns columns l + 16 i).
template <typename T, int TT, bool TABLE, bool POS>
__global__ void __launch_bounds__(256)
window_input_kernel(WindowInput in, const float* __restrict__ w, float* __restrict__ h, T* __restrict__ out,
                    long long ldo, long long pstride, long long kstride, int rows) {
    const long long row = ((long long)blockIdx.x * blockDim.x + threadIdx.x) >> 4;
    const int l = threadIdx.x & 15;
    const bool live = row < rows;
    const long long r = live ? row : 0;   // dead rows recompute row 0: the 16-lane tree needs every lane
    const int t = int(r % TT);
    const long long b = r / TT;
    float v[24];
    if (t == TT - 1) {
#pragma unroll
        for (int i = 0; i < 24; ++i) v[i] = in.readout[i * 16 + l];
    } else {
        const float* tok = TABLE ? in.frame_tokens[b * kFrames + t / 16] + (t % 16) * kD
                                 : in.tokens + b * in.ldw + (long long)t * kD;
        if constexpr (POS) {
            const float* pos = in.pos + (long long)t * kD;
#pragma unroll
            for (int i = 0; i < 24; ++i) v[i] = tok[i * 16 + l] + pos[i * 16 + l];
        } else {
#pragma unroll
            for (int i = 0; i < 24; ++i) v[i] = tok[i * 16 + l];
        }
    }
    float acc = v[0] * v[0];
#pragma unroll
    for (int i = 1; i < 24; ++i) acc = __builtin_fmaf(v[i], v[i], acc);
    const float ss = tree16(acc);
    if (!live) return;
    float* hr = h + row * kD;
#pragma unroll
    for (int i = 0; i < 24; ++i) hr[i * 16 + l] = v[i];
    const float inv = 1.0f / sqrtf(ss / 384.0f + 1e-6f);
#pragma unroll
    for (int i = 0; i < 24; ++i)
        put_value(out, pstride, presplit_idx(row, i * 16 + l, ldo, kstride), (v[i] * inv) * w[i * 16 + l]);
}

// ------------------------------------------------------------------------------------------------ RMSNorm
// 16 lanes per row (4 rows per wave): lane l accumulates x[l + 16 i]^2, tree16, then (x * inv) * w
template <typename T>
__global__ void __launch_bounds__(256)
rmsnorm_kernel(const float* __restrict__ x, long long ldx, const float* __restrict__ w, T* __restrict__ out,
               long long ldo, long long pstride, long long kstride, int rows) {
    const long long row = ((long long)blockIdx.x * blockDim.x + threadIdx.x) >> 4;
    const int l = threadIdx.x & 15;
    const bool live = row < rows;
    const float* xr = x + (live ? row : 0) * ldx;
    float v[24];
#pragma unroll
    for (int i = 0; i < 24; ++i) v[i] = xr[i * 16 + l];
    float acc = v[0] * v[0];
#pragma unroll
    for (int i = 1; i < 24; ++i) acc = __builtin_fmaf(v[i], v[i], acc);
    const float s = tree16(acc);
    if (!live) return;
    const float inv = 1.0f / sqrtf(s / 384.0f + 1e-6f);
#pragma unroll
    for (int i = 0; i < 24; ++i)
        put_value(out, pstride, presplit_idx(row, i * 16 + l, ldo, kstride), (v[i] * inv) * w[i * 16 + l]);
}

// Row 3 (lanes 48 + l): the values of lanes l, l + 16, l + 32 (rows 0, 1, 2), moved up by row swaps.  Only the
// first result of the swap builtins is used (the first operand after the swap): with this compiler the second
// result is not reliably the second operand's.
__device__ __forceinline__ void row3_gather(float v, float (&out)[3]) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const unsigned up2 = __builtin_amdgcn_permlane32_swap(0u, u, false, false)[0];   // rows 2, 3 <- rows 0, 1
    out[0] = __builtin_bit_cast(float, __builtin_amdgcn_permlane16_swap(0u, up2, false, false)[0]);  // row 3 <- row 0
    out[1] = __builtin_bit_cast(float, up2);                                                           // row 3 <- row 1
    out[2] = __builtin_bit_cast(float, __builtin_amdgcn_permlane16_swap(0u, u, false, false)[0]);    // row 3 <- row 2
}

// ------------------------------------------------------------------------------------------------ GDN prep
// One block per (window, run of GP_T tokens), wave h = head h.  Lane l owns q channel h*64+l, k channel h*64+l and
// v channels h*128+l, h*128+64+l, and keeps those columns of the last 4 rows of P in registers while it walks the
// run, so each element of P is read once (plus a 3-row halo per run).  Per row: short conv acc from +0, taps t-3..t
// in order, + bias, SiLU (isa_impl.hpp:871-889); L2 norms with the 16-lane structure over 64 elements
// (isa_impl.hpp:893-906); gates with device libm (expf, log1pf).  TT tokens per window; AUDIO selects SHIELD-A's
// L2 norm (no q scale here: its output is scaled after the recurrence).
constexpr int GP_T = 4;
template <int TT, bool AUDIO, bool FAST>
__global__ void __launch_bounds__(384)
gdn_prep_kernel(const float* __restrict__ P, const float* __restrict__ cw, const float* __restrict__ cb,
                const float* __restrict__ neg_rate, const float* __restrict__ dt_bias, float* __restrict__ Q,
                float* __restrict__ K, float* __restrict__ V, float* __restrict__ dec, float* __restrict__ beta) {
    constexpr int RUNS = (TT + GP_T - 1) / GP_T;
    const int b = blockIdx.x / RUNS, t0 = (blockIdx.x % RUNS) * GP_T, t1 = min(TT, t0 + GP_T);
    const int h = threadIdx.x >> 6, l = threadIdx.x & 63;
    const long long row0 = (long long)b * TT;
    const int cq = kGq + h * 64 + l, ck = kGk + h * 64 + l, cv0 = kGv + h * 128 + l, cv1 = cv0 + 64;
    const int wq = h * 64 + l, wk = 384 + h * 64 + l, wv0 = 768 + h * 128 + l, wv1 = wv0 + 64;
    float w[4][4], bias[4];   // [column][tap]
    const int wc[4] = {wq, wk, wv0, wv1}, pc[4] = {cq, ck, cv0, cv1};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int j = 0; j < 4; ++j) w[c][j] = cw[j * 1536 + wc[c]];
        bias[c] = cb[wc[c]];
    }
    // hist[c][j]: column c of row t - 3 + j (rows before the window's first token are 0 and never used)
    float hist[4][4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int t = t0 - 3 + j;
            hist[c][j] = t >= 0 ? P[(row0 + t) * kGld + pc[c]] : 0.0f;
        }
    float na = 0.0f, nb = 0.0f;
    if (l == 0) {
        na = P[(row0 + t0) * kGld + kGa + h];
        nb = P[(row0 + t0) * kGld + kGb + h];
    }
    // rows t + 1 and t + 2 are in flight while row t is worked on (row index clamped into the run)
    float nxt[4], nxt2[4], na2 = 0.0f, nb2 = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        nxt[c] = P[(row0 + t0) * kGld + pc[c]];
        nxt2[c] = P[(row0 + min(t0 + 1, t1 - 1)) * kGld + pc[c]];
    }
    if (l == 0) {
        na2 = P[(row0 + min(t0 + 1, t1 - 1)) * kGld + kGa + h];
        nb2 = P[(row0 + min(t0 + 1, t1 - 1)) * kGld + kGb + h];
    }
    for (int t = t0; t < t1; ++t) {
        const long long row = row0 + t;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            hist[c][3] = nxt[c];
            nxt[c] = nxt2[c];
        }
        const float ga = na, gb = nb;
        na = na2;
        nb = nb2;
        {
            const long long r2 = row0 + min(t + 2, t1 - 1);
#pragma unroll
            for (int c = 0; c < 4; ++c) nxt2[c] = P[r2 * kGld + pc[c]];
            if (l == 0) {
                na2 = P[r2 * kGld + kGa + h];
                nb2 = P[r2 * kGld + kGb + h];
            }
        }
        float y[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float acc = 0.0f;
            if (t >= 3) acc = __builtin_fmaf(hist[c][0], w[c][0], acc);
            if (t >= 2) acc = __builtin_fmaf(hist[c][1], w[c][1], acc);
            if (t >= 1) acc = __builtin_fmaf(hist[c][2], w[c][2], acc);
            acc = __builtin_fmaf(hist[c][3], w[c][3], acc);
            y[c] = FAST ? silu_fast(acc + bias[c]) : silu(acc + bias[c]);
        }
        const float q = y[0], k = y[1];
        V[row * kVD + h * 128 + l] = y[2];
        V[row * kVD + h * 128 + 64 + l] = y[3];
        // lanes 48 + l (row 3) gather elements l, l+16, l+32, l+48 (row swaps), then the 16-lane tree; lane 48's
        // total is the head's
        float aq, ak;
        {
            float g[2][3];
            row3_gather(q, g[0]);
            row3_gather(k, g[1]);
            aq = g[0][0] * g[0][0];
            ak = g[1][0] * g[1][0];
#pragma unroll
            for (int s = 1; s < 3; ++s) {
                aq = __builtin_fmaf(g[0][s], g[0][s], aq);
                ak = __builtin_fmaf(g[1][s], g[1][s], ak);
            }
            aq = __builtin_fmaf(q, q, aq);
            ak = __builtin_fmaf(k, k, ak);
        }
        aq = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, tree16_lane0(aq)), 48));
        ak = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, tree16_lane0(ak)), 48));
        // FAST (fp16 / bf16 tiers): the hardware reciprocal square root, exp2 and log2 (each within 1 ulp) in place
        // of the correctly rounded division and device libm
        if constexpr (AUDIO) {   // SHIELD-A: x / max(|x|, 1e-12); q unscaled (engine/audio/sequence.cpp:136-143)
            const float iq = FAST ? __builtin_amdgcn_rsqf(fmaxf(aq, 1e-24f)) : 1.0f / fmaxf(sqrtf(aq), 1e-12f);
            const float ik = FAST ? __builtin_amdgcn_rsqf(fmaxf(ak, 1e-24f)) : 1.0f / fmaxf(sqrtf(ak), 1e-12f);
            Q[row * kD + h * 64 + l] = q * iq;
            K[row * kD + h * 64 + l] = k * ik;
        } else {
            const float iq = FAST ? __builtin_amdgcn_rsqf(aq + 1e-6f) : 1.0f / sqrtf(aq + 1e-6f);
            const float ik = FAST ? __builtin_amdgcn_rsqf(ak + 1e-6f) : 1.0f / sqrtf(ak + 1e-6f);
            Q[row * kD + h * 64 + l] = (q * iq) * 0.125f;
            K[row * kD + h * 64 + l] = k * ik;
        }
        if (l == 0) {
            if constexpr (FAST) {
                constexpr float kLog2e = 1.44269504088896341f, kLn2 = 0.693147180559945309f;
                const float x = ga + dt_bias[h];
                const float sp = x > 20.0f ? x : __builtin_amdgcn_logf(1.0f + __builtin_amdgcn_exp2f(x * kLog2e)) * kLn2;
                dec[row * 8 + h] = __builtin_amdgcn_exp2f((neg_rate[h] * sp) * kLog2e);
                beta[row * 8 + h] = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gb * -kLog2e));
            } else {
                dec[row * 8 + h] = expf(neg_rate[h] * softplus_f(ga + dt_bias[h]));
                beta[row * 8 + h] = 1.0f / (1.0f + expf(-gb));
            }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int j = 0; j < 3; ++j) hist[c][j] = hist[c][j + 1];
    }
}

// ------------------------------------------------------------------------------------------------ delta rule
// One workgroup per (window, head, half of the value columns); one thread per value column c (64).  The recurrence
// of a value column needs only that column (S[:, c], v_c), so the halves are independent.  The thread keeps
// S[0..63][c] in registers.  Per token (isa_impl.hpp:911-947): u = (v - a * pred) * beta; S[j] = fma(k_j, u, S[j] * a);
// o = fma chain over j of S[j] * q_j; pred = fma chain over j of S[j] * k_{t+1, j}.  q, k, v, decay and beta of
// 32-token chunks are staged in LDS (q and k read as broadcasts), so no global load sits on the serial chain.
constexpr int DCH = 32;
constexpr int DCOLS = 64;   // value columns per workgroup
template <int TT>
__global__ void __launch_bounds__(DCOLS)
delta_kernel(const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
             const float* __restrict__ dec, const float* __restrict__ beta, float* __restrict__ O) {
    const int half = blockIdx.x & 1, wh = blockIdx.x >> 1;
    const int b = wh / kHeads, h = wh % kHeads, c = threadIdx.x;
    const int col = h * 128 + half * DCOLS + c;   // value column in [0, 768)
    __shared__ __attribute__((aligned(16))) float sq[DCH][64];
    __shared__ __attribute__((aligned(16))) float sk[DCH + 1][64];
    __shared__ float sv[DCH][DCOLS];
    __shared__ float sa[DCH], sb[DCH];
    const long long row0 = (long long)b * TT;
    float S[64];
#pragma unroll
    for (int j = 0; j < 64; ++j) S[j] = 0.0f;
    float pred = 0.0f;
    for (int t0 = 0; t0 < TT; t0 += DCH) {
        const int nt = min(DCH, TT - t0);
        // staging loads are unconditional (token index clamped) so that all of them are in flight together;
        // slots past the last token are then zeroed (q, v) or repeat the last k (the next-k slot of the last
        // token, unused downstream)
        constexpr int QK4 = (DCH + 1) * 16;                       // float4s of q (DCH rows) and k (DCH+1 rows)
        constexpr int QKR = (QK4 + DCOLS - 1) / DCOLS;
        float4 rq[QKR], rk[QKR];
        float rv[DCH];
#pragma unroll
        for (int k = 0; k < QKR; ++k) {
            const int i = threadIdx.x + k * DCOLS;
            const int tt = i >> 4, j4 = (i & 15) * 4;
            const int t = min(t0 + tt, TT - 1);
            rq[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            rk[k] = rq[k];
            if (i < QK4) {
                rq[k] = *reinterpret_cast<const float4*>(Q + (row0 + t) * kD + h * 64 + j4);
                rk[k] = *reinterpret_cast<const float4*>(K + (row0 + t) * kD + h * 64 + j4);
            }
        }
#pragma unroll
        for (int tt = 0; tt < DCH; ++tt) rv[tt] = V[(row0 + min(t0 + tt, TT - 1)) * kVD + col];
#pragma unroll
        for (int k = 0; k < QKR; ++k) {
            const int i = threadIdx.x + k * DCOLS;
            const int tt = i >> 4, j4 = (i & 15) * 4;
            if (i < QK4) {
                if (tt < DCH)
                    *reinterpret_cast<float4*>(&sq[tt][j4]) = t0 + tt < TT ? rq[k] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                *reinterpret_cast<float4*>(&sk[tt][j4]) = rk[k];
            }
        }
#pragma unroll
        for (int tt = 0; tt < DCH; ++tt) sv[tt][c] = t0 + tt < TT ? rv[tt] : 0.0f;
        if (threadIdx.x < DCH) {
            const int t = t0 + threadIdx.x;
            sa[threadIdx.x] = t < TT ? dec[(row0 + t) * 8 + h] : 0.0f;
            sb[threadIdx.x] = t < TT ? beta[(row0 + t) * 8 + h] : 0.0f;
        }
        __syncthreads();
        for (int i = 0; i < nt; ++i) {
            const long long row = row0 + t0 + i;
            const float a = sa[i], bt = sb[i];
            const float u = (sv[i][c] - a * pred) * bt;
            float o = 0.0f, pn = 0.0f;
            // q, k and next-k as float4 broadcasts (48 LDS reads per token); j still runs 0..63 in order
#pragma unroll
            for (int j4 = 0; j4 < 64; j4 += 4) {
                const float4 kk = *reinterpret_cast<const float4*>(&sk[i][j4]);
                const float4 qq = *reinterpret_cast<const float4*>(&sq[i][j4]);
                const float4 kn = *reinterpret_cast<const float4*>(&sk[i + 1][j4]);
                const float kv[4] = {kk.x, kk.y, kk.z, kk.w}, qv[4] = {qq.x, qq.y, qq.z, qq.w},
                            nv[4] = {kn.x, kn.y, kn.z, kn.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float x = __builtin_fmaf(kv[e], u, S[j4 + e] * a);
                    S[j4 + e] = x;
                    o = __builtin_fmaf(x, qv[e], o);
                    pn = __builtin_fmaf(x, nv[e], pn);
                }
            }
            pred = pn;
            O[row * kVD + col] = o;
        }
        __syncthreads();
    }
}

// Half tiers: the same recurrence with each value column's 64 keys split over KQ lane groups of a wave (group kq
// holds keys (64/KQ) kq .. of S[:, c]; 64/KQ columns per wave).  Per token a lane updates its state entries and
// forms the partial dots of the output and of the next prediction.  Every split sums in ONE canonical order: eight
// fma chains from +0 over keys 8m .. 8m+7 (m = 0..7), combined as ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7)).
// A lane adds the chains it holds in that bracketing and the lane groups add the rest by cross-lane exchanges
// (KQ = 8: DPP row rotation by 8, then row swaps; KQ = 4: row swaps; KQ = 2: half swap), and IEEE addition is
// commutative, so o and pred are bitwise the same for KQ = 2, 4 and 8 and in every lane of a column.  That lets the
// launch pick the split from the batch size without breaking row independence: small batches take KQ = 8 (the
// dependent chain per token is 8 fmas + 3 exchanges), large ones KQ = 2 (fewest instructions per token overall).
// The sums are rounded in another (fixed) order than the reference's 64-key chain.
__device__ __forceinline__ float row_pair_sum(float v, int g) {   // rows (0,1) and (2,3): v + partner row
    const auto s = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                    false, false);
    return v + __builtin_bit_cast(float, (g & 1) ? s[0] : s[1]);
}
__device__ __forceinline__ float half_sum(float v, int g) {       // rows (0,1) + (2,3)
    const auto s = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                    false, false);
    const float other = __builtin_bit_cast(float, g < 2 ? s[1] : s[0]);
    return g < 2 ? v + other : other + v;
}
__device__ __forceinline__ float ror8_sum(float v) {               // lanes l, l ^ 8 of a 16-lane row
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf,
                                                                     false));
}
// One token's operands for a lane's KEYS keys: k, q and the next token's k (for the prediction), decay, beta, v.
template <int KEYS>
struct DTok {
    float4 k[KEYS / 4], q[KEYS / 4], n[KEYS / 4];
    float a, b, v;
    __device__ __forceinline__ void load_k(const float* sk) {
#pragma unroll
        for (int j = 0; j < KEYS / 4; ++j) k[j] = reinterpret_cast<const float4*>(sk)[j];
    }
    __device__ __forceinline__ void take_k(const DTok& prev) {
#pragma unroll
        for (int j = 0; j < KEYS / 4; ++j) k[j] = prev.n[j];
    }
    __device__ __forceinline__ void load_rest(const float* sq, const float* skn, float a_, float b_, float v_) {
#pragma unroll
        for (int j = 0; j < KEYS / 4; ++j) {
            q[j] = reinterpret_cast<const float4*>(sq)[j];
            n[j] = reinterpret_cast<const float4*>(skn)[j];
        }
        a = a_;
        b = b_;
        v = v_;
    }
};
// Sum of a lane's 8-key chains in the canonical bracketing, then across the KQ lane groups.
template <int KQ>
__device__ __forceinline__ float delta_combine(const float* c, int g) {
    constexpr int NC = 8 / KQ;
    float v = c[0];
    if constexpr (NC == 2) v = c[0] + c[1];
    if constexpr (NC == 4) v = (c[0] + c[1]) + (c[2] + c[3]);
    if constexpr (KQ == 8) v = ror8_sum(v);
    if constexpr (KQ >= 4) v = row_pair_sum(v, g);
    return half_sum(v, g);
}
// One token of the split recurrence: updates S and pred, returns o.  Per key j (in order): S_j = fma(k_j, u, S_j a).
template <int KQ, int KEYS>
__device__ __forceinline__ float delta_token(const DTok<KEYS>& t, float* S, float& pred, int g) {
    constexpr int NC = KEYS / 8;
    const float u = (t.v - t.a * pred) * t.b;
    float o[NC], pn[NC];
#pragma unroll
    for (int m = 0; m < NC; ++m) {
        o[m] = 0.0f;
        pn[m] = 0.0f;
    }
#pragma unroll
    for (int j4 = 0; j4 < KEYS / 4; ++j4) {
        const float kv[4] = {t.k[j4].x, t.k[j4].y, t.k[j4].z, t.k[j4].w};
        const float qv[4] = {t.q[j4].x, t.q[j4].y, t.q[j4].z, t.q[j4].w};
        const float nv[4] = {t.n[j4].x, t.n[j4].y, t.n[j4].z, t.n[j4].w};
        const int m = j4 / 2;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float x = __builtin_fmaf(kv[e], u, S[4 * j4 + e] * t.a);
            S[4 * j4 + e] = x;
            o[m] = __builtin_fmaf(x, qv[e], o[m]);
            pn[m] = __builtin_fmaf(x, nv[e], pn[m]);
        }
    }
    pred = delta_combine<KQ>(pn, g);
    return delta_combine<KQ>(o, g);
}
constexpr int kDeltaPipeWaves = 1024;   // one wave per SIMD (256 CUs x 4)
// PIPE: full 32-token chunks run unrolled with token i+1's operands read from LDS ahead of token i's chain (for
// grids of at most one wave per SIMD, where nothing else hides the LDS latency), and the outputs of a chunk are
// kept in registers (lane group kq keeps tokens i = kq mod KQ) and stored after the next chunk's operands have been
// staged: one vmcnt counter retires loads and stores in order, so a store issued just before the wait for the
// prefetched operands would put a full memory round trip on the serial path.  The next chunk's operands are loaded
// into registers while the current chunk runs (the rolled form, for grids of several waves per SIMD, loads them at
// the start of the chunk and keeps its registers for occupancy).  Both forms issue the same arithmetic per token, so their results
// are bitwise equal.
template <int KQ, bool PIPE, int TT>   // KQ: key groups per column: 2 (halves), 4 (rows) or 8 (half rows)
__global__ void __launch_bounds__(64)
delta_split_kernel(const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
                   const float* __restrict__ dec, const float* __restrict__ beta, float* __restrict__ O) {
    constexpr int DS_COLS = 64 / KQ, KEYS = 64 / KQ;
    constexpr int NB = 128 / DS_COLS;   // column blocks per head
    const int cb = blockIdx.x % NB, wh = blockIdx.x / NB;
    const int b = wh / kHeads, h = wh % kHeads;
    const int lane = threadIdx.x, c16 = lane % DS_COLS, kq = lane / DS_COLS, g = lane >> 4;
    const int col = h * 128 + cb * DS_COLS + c16;
    __shared__ __attribute__((aligned(16))) float sq[DCH][64];
    __shared__ __attribute__((aligned(16))) float sk[DCH + 1][64];
    __shared__ float sv[DCH][DS_COLS];
    __shared__ float sa[DCH], sb[DCH];
    const long long row0 = (long long)b * TT;
    // chunk operands in registers: loads are unconditional (token index clamped) so all of them are in flight
    // together; slots past the last token are then zeroed (q, v, decay, beta) or repeat the last k (the next-k slot
    // of the last token, unused downstream)
    constexpr int QK4 = (DCH + 1) * 16;   // float4s of q (DCH rows) and k (DCH + 1 rows)
    constexpr int QKR = (QK4 + 63) / 64;
    constexpr int VR = DCH * DS_COLS / 64;
    float4 rq[QKR], rk[QKR];
    float rv[VR], ra = 0.0f, rb = 0.0f;
    auto fetch = [&](int t0) {
#pragma unroll
        for (int k = 0; k < QKR; ++k) {
            const int i = lane + k * 64;
            const int tt = i >> 4, j4 = (i & 15) * 4;
            const int t = min(t0 + tt, TT - 1);
            rq[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            rk[k] = rq[k];
            if (i < QK4) {
                rq[k] = *reinterpret_cast<const float4*>(Q + (row0 + t) * kD + h * 64 + j4);
                rk[k] = *reinterpret_cast<const float4*>(K + (row0 + t) * kD + h * 64 + j4);
            }
        }
#pragma unroll
        for (int k = 0; k < VR; ++k) rv[k] = V[(row0 + min(t0 + kq + KQ * k, TT - 1)) * kVD + col];
        if (lane < DCH) {
            const int t = min(t0 + lane, TT - 1);
            ra = dec[(row0 + t) * 8 + h];
            rb = beta[(row0 + t) * 8 + h];
        }
    };
    auto stage = [&](int t0) {
#pragma unroll
        for (int k = 0; k < QKR; ++k) {
            const int i = lane + k * 64;
            const int tt = i >> 4, j4 = (i & 15) * 4;
            if (i < QK4) {
                if (tt < DCH)
                    *reinterpret_cast<float4*>(&sq[tt][j4]) = t0 + tt < TT ? rq[k] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                *reinterpret_cast<float4*>(&sk[tt][j4]) = rk[k];
            }
        }
#pragma unroll
        for (int k = 0; k < VR; ++k) {
            const int tt = kq + KQ * k;
            sv[tt][c16] = t0 + tt < TT ? rv[k] : 0.0f;
        }
        if (lane < DCH) {
            const bool in = t0 + lane < TT;
            sa[lane] = in ? ra : 0.0f;
            sb[lane] = in ? rb : 0.0f;
        }
    };
    float S[KEYS];
#pragma unroll
    for (int j = 0; j < KEYS; ++j) S[j] = 0.0f;
    float pred = 0.0f;
    float ob[DCH / KQ] = {};   // PIPE: this lane's outputs of the last full chunk, tokens kq + KQ m
    int ob_t0 = -1;            // first token of that chunk (-1: none pending)
    if (PIPE) fetch(0);
    for (int t0 = 0; t0 < TT; t0 += DCH) {
        const int nt = min(DCH, TT - t0);
        if (!PIPE) fetch(t0);   // PIPE: fetched while the previous chunk ran
        stage(t0);
        __syncthreads();
        if (PIPE && ob_t0 >= 0) {
#pragma unroll
            for (int m = 0; m < DCH / KQ; ++m) O[(row0 + ob_t0 + kq + KQ * m) * kVD + col] = ob[m];
            ob_t0 = -1;
        }
        if (PIPE && t0 + DCH < TT) fetch(t0 + DCH);
        // all lane groups of a column hold the same o; in the rolled form every lane stores it (same value, same
        // address), so the token step has no branch
        if (PIPE && nt == DCH) {
            DTok<KEYS> cur;
            cur.load_k(&sk[0][kq * KEYS]);
            cur.load_rest(&sq[0][kq * KEYS], &sk[1][kq * KEYS], sa[0], sb[0], sv[0][c16]);
#pragma unroll
            for (int i = 0; i < DCH; ++i) {
                DTok<KEYS> nxt;
                if (i + 1 < DCH) {
                    nxt.take_k(cur);
                    nxt.load_rest(&sq[i + 1][kq * KEYS], &sk[i + 2][kq * KEYS], sa[i + 1], sb[i + 1],
                                  sv[i + 1][c16]);
                }
                const float o = delta_token<KQ, KEYS>(cur, S, pred, g);
                if (kq == i % KQ) ob[i / KQ] = o;
                if (i + 1 < DCH) cur = nxt;
            }
            ob_t0 = t0;
        } else {
            for (int i = 0; i < nt; ++i) {
                DTok<KEYS> cur;
                cur.load_k(&sk[i][kq * KEYS]);
                cur.load_rest(&sq[i][kq * KEYS], &sk[i + 1][kq * KEYS], sa[i], sb[i], sv[i][c16]);
                O[(row0 + t0 + i) * kVD + col] = delta_token<KQ, KEYS>(cur, S, pred, g);
            }
        }
        __syncthreads();
    }
    if (PIPE && ob_t0 >= 0) {
#pragma unroll
        for (int m = 0; m < DCH / KQ; ++m) O[(row0 + ob_t0 + kq + KQ * m) * kVD + col] = ob[m];
    }
}

// ------------------------------------------------------------------------------------------------ chunked delta rule
// Half tiers.  Per (window, head) the recurrence S_t = a_t S_{t-1} + k_t u_t^T, u_t = b_t (v_t - a_t S_{t-1}^T k_t),
// o_t = S_t^T q_t (S: 64 keys x 128 values; isa_impl.hpp:911-947) runs over chunks of DC = 32 tokens.  Inside a
// chunk, with g_i = a_0 ... a_i (inclusive cumulative decay) and G_ij = a_{j+1} ... a_i (j <= i, 1 on the diagonal),
// unrolling the recurrence gives (I + L) U = diag(b) (V - diag(g) K S_0), L_ij = b_i G_ij (k_i . k_j) for j < i.
// With T = (I + L)^-1:
//   U   = A1V - B1 S_0,              A1V = T diag(b) V,   B1 = T diag(b g) K,
//   O   = diag(g) Q S_0 + P U,       P_ij = G_ij (q_i . k_j) for j <= i, else 0,
//   S_C = g_31 S_0 + Kd^T U,         Kd_j = G_31,j k_j.
// Tokens past the window's end pad the last chunk with a = 1, b = 0, k = q = v = 0, which leaves every real
// quantity unchanged.  delta_chunk_prep_kernel forms every state-independent operand of every chunk in parallel
// (A1V, B1, P, g, G_31,j); delta_chunk_scan_kernel walks the chunks of one (window, head) in order, the state's fp32
// value in MFMA accumulators and its split parts in LDS.  Every product runs on the split-operand matrix cores (fp32-level
// operand precision); T comes from forward substitution in fp32, the decay products from running products of a.
// The results equal the token-by-token recurrence up to rounding (tested against it on the GPU).
constexpr int DC = 32;                      // tokens per chunk
constexpr int DNC = (kT + DC - 1) / DC;     // chunks per window
// floats per chunk in the prep buffer: A1V [32][128], B1 [32][64], P [32][32], g [32], G_31,j [32]
constexpr int DCO_B1 = DC * 128, DCO_P = DCO_B1 + DC * 64, DCO_G = DCO_P + DC * DC, DCO_GD = DCO_G + DC;
constexpr int DCF = DCO_GD + DC;

// 8 fp32 values (two float4 in LDS) -> the P split-part fragments
template <typename T>
__device__ __forceinline__ void frag_lds(const float* p, typename Split<T>::V8* parts) {
    const float4 u = reinterpret_cast<const float4*>(p)[0], w = reinterpret_cast<const float4*>(p)[1];
    const float x[8] = {u.x, u.y, u.z, u.w, w.x, w.y, w.z, w.w};
    split8<T>(x, parts);
}
// 8 pre-split elements of each part (16 bytes per part) -> fragments
template <typename T>
__device__ __forceinline__ void frag_parts(const T* p, long long part_stride, typename Split<T>::V8* parts) {
#pragma unroll
    for (int q = 0; q < Split<T>::P; ++q) parts[q] = load_part8<T>(p + q * part_stride);
}
// 4 consecutive elements of each part <- split(v[0..3]) (8-byte stores; fp32: one 16-byte store)
template <typename T>
__device__ __forceinline__ void put4(T* p, long long part_stride, float v0, float v1, float v2, float v3) {
    if constexpr (sizeof(T) == 4) {
        *reinterpret_cast<float4*>(p) = make_float4(v0, v1, v2, v3);
    } else {
        const float v[4] = {v0, v1, v2, v3};
        uint2 four[Split<T>::P];
        split4_packed<T>(v, four);
#pragma unroll
        for (int q = 0; q < Split<T>::P; ++q) *reinterpret_cast<uint2*>(p + q * part_stride) = four[q];
    }
}
template <typename T>
__device__ __forceinline__ void put1(T* p, long long part_stride, float v) {
    T part[Split<T>::P];
    Split<T>::split(v, part);
#pragma unroll
    for (int q = 0; q < Split<T>::P; ++q) p[q * part_stride] = part[q];
}

// Decay products of one chunk (one wave; lane i < 32 holds a_i in `ai`, read by every lane with readlane, so no
// memory carries it between lanes): lane j < 32 writes column j of G, lane 32 writes g.
__device__ __forceinline__ void chunk_decays(float ai, float (*Gs)[DC + 1], float* gs, int lane) {
    float p = 1.0f, q = 1.0f;
#pragma unroll
    for (int i = 0; i < DC; ++i) {
        const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ai), i));
        if (i > lane) p = p * a;
        q = q * a;
        if (lane < DC) Gs[i][lane] = i >= lane ? p : 0.0f;
        if (lane == DC) gs[i] = q;
    }
}

// One wave per (window, head, chunk): A1V and B1 into CH [window][head][chunk][DCF].  Only K (read as both operands
// of K K^T and by B1), L, T and the decay products live in LDS (22 KB: seven waves per CU); Q fragments and the V
// columns of A1V are read straight from global memory, issued early so that they land during the products and the
// forward substitution.
template <typename T, int TT>
__global__ void __launch_bounds__(64)
delta_chunk_prep_kernel(const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
                        const float* __restrict__ dec, const float* __restrict__ beta, float* __restrict__ CH) {
    constexpr int NC = (TT + DC - 1) / DC;   // chunks per window
    typedef Split<T> S;
    typedef typename S::V8 V8;
    constexpr int P = S::P;
    const int c = blockIdx.x % NC, wh = blockIdx.x / NC;
    const int b = wh / kHeads, h = wh % kHeads;
    const int lane = threadIdx.x, r = lane & 15, g = lane >> 4;
    const int t0 = c * DC, n = min(DC, TT - t0);
    const long long row0 = (long long)b * TT + t0;
    __shared__ __attribute__((aligned(16))) float Ks[DC][64 + 4];
    __shared__ __attribute__((aligned(16))) float Ls[DC][DC + 4];
    __shared__ __attribute__((aligned(16))) float Ts[DC][DC + 4];
    __shared__ float Gs[DC][DC + 1];
    __shared__ float bs[DC], gs[DC];
    // Q fragments (rows ti*16 + r, keys ks*32 + 8g..): clamped rows, zero past the window's end
    float qf[2][2][8];
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
            read8(Q + (row0 + min(ti * 16 + r, n - 1)) * kD + h * 64 + ks * 32 + 8 * g, qf[ti][ks]);
    {   // stage K (loads at clamped rows, all in flight together; zero / a = 1 past the window's end)
        float av = 1.0f, bv = 0.0f;
        if (lane < DC) {
            av = dec[(row0 + min(lane, n - 1)) * 8 + h];
            bv = beta[(row0 + min(lane, n - 1)) * 8 + h];
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int i = lane + 64 * k, row = i >> 4, c4 = (i & 15) * 4;
            const float4 v = *reinterpret_cast<const float4*>(K + (row0 + min(row, n - 1)) * kD + h * 64 + c4);
            const bool in = row < n;   // per component: a select of whole float4s went through scratch memory
            *reinterpret_cast<float4*>(&Ks[row][c4]) =
                make_float4(in ? v.x : 0.0f, in ? v.y : 0.0f, in ? v.z : 0.0f, in ? v.w : 0.0f);
        }
        if (lane < DC) bs[lane] = lane < n ? bv : 0.0f;
        chunk_decays(lane < n ? av : 1.0f, Gs, gs, lane);
    }
    // V column values of A1V: lane (r, g) takes rows 8g..8g+7 of value columns tc*16 + r (issued now, used last)
    float vcol[8][8];
#pragma unroll
    for (int tc = 0; tc < 8; ++tc)
#pragma unroll
        for (int e = 0; e < 8; ++e)
            vcol[tc][e] = V[(row0 + min(8 * g + e, n - 1)) * kVD + h * 128 + tc * 16 + r];
    __syncthreads();
    // L = b_i G_ij (k_i . k_j) for j < i and P = G_ij (q_i . k_j) for j <= i: tiles (ti, tj) of K K^T and Q K^T,
    // keys in two K steps; tile (0, 1) of both is all zero
    float* out = CH + ((long long)wh * NC + c) * DCF;
#pragma unroll
    for (int tile = 0; tile < 4; ++tile) {
        const int ti = tile >> 1, tj = tile & 1;
        f32x4 kk = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, qk = kk;
        if (ti >= tj) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                V8 ap[P], qp[P], bp[P];
                frag_lds<T>(&Ks[ti * 16 + r][ks * 32 + 8 * g], ap);
                float qx[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) qx[e] = ti * 16 + r < n ? qf[ti][ks][e] : 0.0f;
                split8<T>(qx, qp);
                frag_lds<T>(&Ks[tj * 16 + r][ks * 32 + 8 * g], bp);
                kk = mfma_split<T>(ap, bp, kk);
                qk = mfma_split<T>(qp, bp, qk);
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = ti * 16 + 4 * g + e, j = tj * 16 + r;
            Ls[i][j] = j < i ? bs[i] * (Gs[i][j] * kk[e]) : 0.0f;
            out[DCO_P + i * DC + j] = j <= i ? Gs[i][j] * qk[e] : 0.0f;
        }
    }
    if (lane < DC) {
        out[DCO_G + lane] = gs[lane];
        out[DCO_GD + lane] = Gs[DC - 1][lane];
    }
    __syncthreads();
    // T = (I + L)^-1: lane j solves column j, t_i = [i == j] - sum_{m < i} L_im t_m (fma chain over m in order)
    if (lane < DC) {
        float t[DC];
#pragma unroll
        for (int i = 0; i < DC; ++i) {
            float acc = i == lane ? 1.0f : 0.0f;
#pragma unroll
            for (int m4 = 0; m4 < (i + 3) / 4; ++m4) {
                const float4 l4 = *reinterpret_cast<const float4*>(&Ls[i][4 * m4]);
                const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (4 * m4 + e < i) acc = __builtin_fmaf(-lv[e], t[4 * m4 + e], acc);
            }
            t[i] = acc;
        }
#pragma unroll
        for (int i = 0; i < DC; ++i) Ts[i][lane] = t[i];
    }
    __syncthreads();
    // A1V = T diag(b) V (32 x 128) and B1 = T diag(b g) K (32 x 64): one K step over the chunk's 32 tokens
    V8 tp[2][P];
#pragma unroll
    for (int ti = 0; ti < 2; ++ti) frag_lds<T>(&Ts[ti * 16 + r][8 * g], tp[ti]);
#pragma unroll
    for (int tc = 0; tc < 8; ++tc) {
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = bs[8 * g + e] * (8 * g + e < n ? vcol[tc][e] : 0.0f);
        V8 bp[P];
        split8<T>(y, bp);
#pragma unroll
        for (int ti = 0; ti < 2; ++ti) {
            const f32x4 acc = mfma_split<T>(tp[ti], bp, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
            for (int e = 0; e < 4; ++e) out[(ti * 16 + 4 * g + e) * 128 + tc * 16 + r] = acc[e];
        }
    }
#pragma unroll
    for (int tk = 0; tk < 4; ++tk) {
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = (bs[8 * g + e] * gs[8 * g + e]) * Ks[8 * g + e][tk * 16 + r];
        V8 bp[P];
        split8<T>(y, bp);
#pragma unroll
        for (int ti = 0; ti < 2; ++ti) {
            const f32x4 acc = mfma_split<T>(tp[ti], bp, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
            for (int e = 0; e < 4; ++e) out[DCO_B1 + (ti * 16 + 4 * g + e) * 64 + tk * 16 + r] = acc[e];
        }
    }
}

// One workgroup (4 waves) per (window, head, block of VS value columns), the chunks in order.  Value columns are
// independent in every product below, so VS = 32 or 64 splits a head over 4 or 2 workgroups with every output
// computed by the same fragments in the same order (bitwise equal for every VS).  Tiles: U / Q S_0 / O
// [token tile 0..1][value tile] as u = wave + 4 j (ti = u % 2, vt = u / 2), state S[key tile][value tile] as
// s = wave + 4 j (kt = s % 4, vt = s / 4).  Per chunk: stage Q, -B1, P, Kd^T parts and g from registers / barrier /
// U = A1V - B1 S_0 and Q S_0 / barrier / O = g Q S_0 + P U, S = g_31 S + Kd^T U (state parts rewritten).  A chunk's
// operands are loaded two chunks ahead (two register sets, the chunk loop unrolled by two), and its outputs are
// stored after the next chunk's staging: one vmcnt counter retires loads and stores in order.
template <int UT>
struct DChunkRegs {   // one chunk's operands as a thread loads them
    float4 q[2], k[2], b1[2], p;
    float gd[2], g, a1v[UT][4];
};
template <typename T, int VS, int TT>
__global__ void __launch_bounds__(256)
delta_chunk_scan_kernel(const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ CH,
                        float* __restrict__ O) {
    constexpr int NC = (TT + DC - 1) / DC;   // chunks per window
    typedef Split<T> S;
    typedef typename S::V8 V8;
    constexpr int P = S::P;
    constexpr int NVT = VS / 16, UT = NVT / 2, ST = NVT;   // value tiles; U and state tiles per wave
    constexpr int NB = 128 / VS;                           // value blocks per head
    constexpr int KL = 64 + 8, TL = DC + 8;   // element strides of key-major and token-major part rows
    __shared__ __attribute__((aligned(16))) T Sp[P][VS][KL];    // state [value][key]
    __shared__ __attribute__((aligned(16))) T Qp[P][DC][KL];    // q [token][key]
    __shared__ __attribute__((aligned(16))) T Bp[P][DC][KL];    // -B1 [token][key]
    __shared__ __attribute__((aligned(16))) T KdT[P][64][TL];   // Kd^T [key][token]
    __shared__ __attribute__((aligned(16))) T Pp[P][DC][TL];    // P [token i][token j]
    __shared__ __attribute__((aligned(16))) T Up[P][VS][TL];    // U [value][token]
    __shared__ float gs[DC];
    const int vb = blockIdx.x % NB, wh = blockIdx.x / NB, b = wh / kHeads, h = wh % kHeads;
    const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const long long rowb = (long long)b * TT;
    const int vcol0 = h * 128 + vb * VS;   // first value column of this block in the [rows][768] layout
    const float* chb = CH + (long long)wh * NC * DCF;
    for (int i = tid; i < P * VS * KL; i += 256) (&Sp[0][0][0])[i] = T(0.0f);

    auto fetch = [&](DChunkRegs<UT>& F, int c) {   // loads at clamped rows; rows past the end are zeroed when staged
        const int t0 = c * DC, n = min(DC, TT - t0);
        const float* cc = chb + (long long)c * DCF;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int i = tid + 256 * k, row = i >> 4, c4 = (i & 15) * 4;
            const long long gr = rowb + t0 + min(row, n - 1);
            F.q[k] = *reinterpret_cast<const float4*>(Q + gr * kD + h * 64 + c4);
            F.k[k] = *reinterpret_cast<const float4*>(K + gr * kD + h * 64 + c4);
            F.b1[k] = *reinterpret_cast<const float4*>(cc + DCO_B1 + row * 64 + c4);
            F.gd[k] = cc[DCO_GD + row];
        }
        F.p = *reinterpret_cast<const float4*>(cc + DCO_P + tid * 4);
        F.g = cc[DCO_G + (tid & (DC - 1))];
#pragma unroll
        for (int j = 0; j < UT; ++j) {
            const int u = wave + 4 * j, ti = u % 2, vt = u / 2;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                F.a1v[j][e] = cc[(ti * 16 + 4 * g + e) * 128 + vb * VS + vt * 16 + r];
        }
    };
    f32x4 Sacc[ST];
#pragma unroll
    for (int j = 0; j < ST; ++j) Sacc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float ob[UT][4];   // this lane's outputs of the previous chunk (U-tile order, rows 4 g + e)
    int ob_t0 = -1;
    auto store_out = [&]() {
#pragma unroll
        for (int j = 0; j < UT; ++j) {
            const int u = wave + 4 * j, ti = u % 2, vt = u / 2;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = ob_t0 + ti * 16 + 4 * g + e;
                if (i < TT) O[(rowb + i) * kVD + vcol0 + vt * 16 + r] = ob[j][e];
            }
        }
    };
    auto chunk = [&](int c, DChunkRegs<UT>& F) {
        const int t0 = c * DC, n = min(DC, TT - t0);
        __syncthreads();   // the previous chunk is done with every LDS operand
        // ---- stage: q, -B1, P, Kd^T parts and g
        float av[UT][4];
        {
            const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int i = tid + 256 * k, row = i >> 4, c4 = (i & 15) * 4;
                const bool in = row < n;
                const float4 q = in ? F.q[k] : z, kk = in ? F.k[k] : z;
                put4<T>(&Qp[0][row][c4], (long long)DC * KL, q.x, q.y, q.z, q.w);
                put4<T>(&Bp[0][row][c4], (long long)DC * KL, -F.b1[k].x, -F.b1[k].y, -F.b1[k].z, -F.b1[k].w);
                const float gd = F.gd[k];
                put1<T>(&KdT[0][c4 + 0][row], 64LL * TL, gd * kk.x);
                put1<T>(&KdT[0][c4 + 1][row], 64LL * TL, gd * kk.y);
                put1<T>(&KdT[0][c4 + 2][row], 64LL * TL, gd * kk.z);
                put1<T>(&KdT[0][c4 + 3][row], 64LL * TL, gd * kk.w);
            }
            put4<T>(&Pp[0][tid >> 3][(tid & 7) * 4], (long long)DC * TL, F.p.x, F.p.y, F.p.z, F.p.w);
            if (tid < DC) gs[tid] = F.g;
#pragma unroll
            for (int j = 0; j < UT; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) av[j][e] = F.a1v[j][e];
        }
        // the previous chunk's outputs, now that this chunk's operands have arrived; then the registers take the
        // chunk after next
        if (ob_t0 >= 0) {
            store_out();
            ob_t0 = -1;
        }
        if (c + 2 < NC) fetch(F, c + 2);
        __syncthreads();
        // ---- phase 1: U = A1V - B1 S_0 and Q S_0
        f32x4 qs[UT];
#pragma unroll
        for (int j = 0; j < UT; ++j) {
            const int u = wave + 4 * j, ti = u % 2, vt = u / 2;
            f32x4 uu = f32x4{av[j][0], av[j][1], av[j][2], av[j][3]};
            f32x4 x = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                V8 sf[P], bf[P], qf[P];
                frag_parts<T>(&Sp[0][vt * 16 + r][ks * 32 + 8 * g], (long long)VS * KL, sf);
                frag_parts<T>(&Bp[0][ti * 16 + r][ks * 32 + 8 * g], (long long)DC * KL, bf);
                frag_parts<T>(&Qp[0][ti * 16 + r][ks * 32 + 8 * g], (long long)DC * KL, qf);
                uu = mfma_split<T>(bf, sf, uu);
                x = mfma_split<T>(qf, sf, x);
            }
            qs[j] = x;
            put4<T>(&Up[0][vt * 16 + r][ti * 16 + 4 * g], (long long)VS * TL, uu[0], uu[1], uu[2], uu[3]);
        }
        __syncthreads();
        // ---- phase 2: O = g Q S_0 + P U; S = g_31 S + Kd^T U
#pragma unroll
        for (int j = 0; j < UT; ++j) {
            const int u = wave + 4 * j, ti = u % 2, vt = u / 2;
            V8 uf[P], pf[P];
            frag_parts<T>(&Up[0][vt * 16 + r][8 * g], (long long)VS * TL, uf);
            frag_parts<T>(&Pp[0][ti * 16 + r][8 * g], (long long)DC * TL, pf);
            f32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = gs[ti * 16 + 4 * g + e] * qs[j][e];
            o = mfma_split<T>(pf, uf, o);
#pragma unroll
            for (int e = 0; e < 4; ++e) ob[j][e] = o[e];
        }
        const float g31 = gs[DC - 1];
#pragma unroll
        for (int j = 0; j < ST; ++j) {
            const int sidx = wave + 4 * j, kt = sidx % 4, vt = sidx / 4;
            V8 uf[P], kf[P];
            frag_parts<T>(&Up[0][vt * 16 + r][8 * g], (long long)VS * TL, uf);
            frag_parts<T>(&KdT[0][kt * 16 + r][8 * g], 64LL * TL, kf);
            f32x4 sacc;
#pragma unroll
            for (int e = 0; e < 4; ++e) sacc[e] = g31 * Sacc[j][e];
            sacc = mfma_split<T>(kf, uf, sacc);
            Sacc[j] = sacc;
            put4<T>(&Sp[0][vt * 16 + r][kt * 16 + 4 * g], (long long)VS * KL, sacc[0], sacc[1], sacc[2], sacc[3]);
        }
        ob_t0 = t0;
    };
    DChunkRegs<UT> F0, F1;
    fetch(F0, 0);
    fetch(F1, 1);
    for (int c = 0; c < NC; c += 2) {
        chunk(c, F0);
        if (c + 1 < NC) chunk(c + 1, F1);
    }
    store_out();
}

// ------------------------------------------------------------------------------------------------ gated norm
// 16 lanes per (row, head): lane l accumulates o[l + 16 z]^2 (z = 0..7), tree16, then ((o * rstd) * w) * silu(g).
// A wave takes one head of four consecutive rows, so that its stores of a group-major output fill whole 64-byte
// row pieces of four adjacent rows.
// AUDIO: SHIELD-A scales o by 0.125 first and uses eps 1e-5 (engine/audio/sequence.cpp:196-201).
template <typename T, bool AUDIO>
__global__ void __launch_bounds__(256)
gated_norm_kernel(const float* __restrict__ O, const float* __restrict__ P, const float* __restrict__ w,
                  T* __restrict__ out, long long pstride, long long ld, long long kstride, int rows) {
    const long long grp = ((long long)blockIdx.x * blockDim.x + threadIdx.x) >> 4;
    const int l = threadIdx.x & 15;
    const long long quad = grp >> 2;   // (four-row block, head)
    const int h = int(quad % kHeads);
    const long long r = (quad / kHeads) * 4 + (grp & 3);
    const bool live = r < rows;
    const long long row = live ? r : 0;
    const float* o = O + row * kVD + h * 128;
    float v[8];
#pragma unroll
    for (int z = 0; z < 8; ++z) v[z] = AUDIO ? o[z * 16 + l] * 0.125f : o[z * 16 + l];
    float acc = v[0] * v[0];
#pragma unroll
    for (int z = 1; z < 8; ++z) acc = __builtin_fmaf(v[z], v[z], acc);
    const float s = tree16(acc);
    if (!live) return;
    const float rstd = 1.0f / sqrtf(s / 128.0f + (AUDIO ? 1e-5f : 1e-6f));
    const float* g = P + row * kGld + kGg + h * 128;
#pragma unroll
    for (int z = 0; z < 8; ++z) {
        const int i = z * 16 + l;
        const float sg = std::is_same<T, float>::value ? silu(g[i]) : silu_fast(g[i]);
        put_value(out, pstride, presplit_idx(row, h * 128 + i, ld, kstride), ((v[z] * rstd) * w[i]) * sg);
    }
}

// ------------------------------------------------------------------------------------------------ SISA
// One block per (window, head), 512 threads (isa_impl.hpp:996-1069): the per-token work of a 321-token window in one
// pass, the six 64-token output blocks on six waves at once.
// 1. per token: -softplus(alpha), logsigmoid(forget), theta (device libm)
// 2. prefix sums in double, one thread per series, rounded to float per element
// 3. rotate c (last token's angles) and each b_t; scores with the 16-lane dot structure
// 4. softmax: max, expf, sum in double in token order (one thread); y_j = sum over 64-token blocks of fma chains
// The order of every rounded operation is the reference's; only order-free work (the maximum, the exponentials,
// the independent block chains, loads) runs in parallel.
constexpr int SA_THREADS = 512;
template <int TT>
__global__ void __launch_bounds__(SA_THREADS)
sisa_kernel(float* __restrict__ S, const float* __restrict__ QC, const float* __restrict__ lam_h,
            float* __restrict__ Y) {
    const int b = blockIdx.x / kHeads, h = blockIdx.x % kHeads, tid = threadIdx.x;
    float* S0 = S + (long long)b * TT * kSld;
    __shared__ float gt[TT], ft[TT], sco[TT];
    __shared__ float phi[TT][kPairs + 1];
    constexpr int SA_NB = (TT + 63) / 64;   // 64-token blocks of the output sums
    __shared__ float sq[64], crot[32];
    __shared__ float s_inv;
    __shared__ float yblk[SA_NB][64];
    for (int t = tid; t < TT; t += SA_THREADS) {
        const float* row = S0 + (long long)t * kSld;
        gt[t] = -softplus_f(row[kSal + h]);
        ft[t] = logsigmoid_f(row[kSfg + h]);
#pragma unroll
        for (int p = 0; p < kPairs; ++p) phi[t][p] = row[kSth + h * kPairs + p];
    }
    if (tid < 64) sq[tid] = QC[(long long)b * 576 + h * 64 + tid];
    __syncthreads();
    if (tid < 2 + kPairs) {
        // one series per thread, in token order; 32 tokens at a time go through registers so that the LDS loads
        // of a block are in flight together and only the additions chain
        float* series = tid == 0 ? gt : tid == 1 ? ft : &phi[0][tid - 2];
        const int stride = tid < 2 ? 1 : kPairs + 1;
        double acc = 0.0;
        for (int t0 = 0; t0 < TT; t0 += 32) {
            float x[32];
#pragma unroll
            for (int i = 0; i < 32; ++i)
                if (t0 + i < TT) x[i] = series[(t0 + i) * stride];
#pragma unroll
            for (int i = 0; i < 32; ++i)
                if (t0 + i < TT) {
                    acc += double(x[i]);
                    x[i] = float(acc);
                }
#pragma unroll
            for (int i = 0; i < 32; ++i)
                if (t0 + i < TT) series[(t0 + i) * stride] = x[i];
        }
    }
    __syncthreads();
    if (tid < kPairs) {
        float sn, cs;
        sincosf(phi[TT - 1][tid], &sn, &cs);
        const float* c = QC + (long long)b * 576 + 384 + h * 32;
        const float ce = c[2 * tid], co = c[2 * tid + 1];
        crot[2 * tid] = ce * cs - co * sn;
        crot[2 * tid + 1] = ce * sn + co * cs;
    }
    __syncthreads();
    const float lam = lam_h[h], gl = gt[TT - 1], fl = ft[TT - 1];
    for (int t = tid; t < TT; t += SA_THREADS) {
        const float* row = S0 + (long long)t * kSld;
        const float* k = row + kSk + h * 64;
        const float* bb = row + kSb + h * 32;
        float br[32];
#pragma unroll
        for (int p = 0; p < kPairs; ++p) {
            float sn, cs;
            sincosf(phi[t][p], &sn, &cs);
            const float e = bb[2 * p], o = bb[2 * p + 1];
            br[2 * p] = e * cs - o * sn;
            br[2 * p + 1] = e * sn + o * cs;
        }
        float la[16], ls[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            la[i] = sq[i] * k[i];
            la[i] = __builtin_fmaf(sq[16 + i], k[16 + i], la[i]);
            la[i] = __builtin_fmaf(sq[32 + i], k[32 + i], la[i]);
            la[i] = __builtin_fmaf(sq[48 + i], k[48 + i], la[i]);
            ls[i] = crot[i] * br[i];
            ls[i] = __builtin_fmaf(crot[16 + i], br[16 + i], ls[i]);
        }
        float a8[8], s8[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) { a8[i] = la[i] + la[i + 8]; s8[i] = ls[i] + ls[i + 8]; }
        const float content = ((a8[0] + a8[4]) + (a8[2] + a8[6])) + ((a8[1] + a8[5]) + (a8[3] + a8[7]));
        const float ssm = ((s8[0] + s8[4]) + (s8[2] + s8[6])) + ((s8[1] + s8[5]) + (s8[3] + s8[7]));
        float score = content * 0.125f;
        score = score + (lam * expf(gl - gt[t])) * ssm;
        score = score + (fl - ft[t]);
        sco[t] = score;
    }
    __syncthreads();
    // softmax: the maximum (exact in any order; a NaN score is never selected, as in the sequential scan), the
    // exponentials in parallel, their sum in double in token order by one thread
    {
        float mx = -INFINITY;
        for (int t = tid; t < TT; t += SA_THREADS) mx = sco[t] > mx ? sco[t] : mx;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float o = __shfl_xor(mx, off);
            mx = o > mx ? o : mx;
        }
        if ((tid & 63) == 0) sq[tid >> 6] = mx;   // sq is free again: the scores are done
        __syncthreads();
        mx = sq[0];
#pragma unroll
        for (int w = 1; w < SA_THREADS / 64; ++w) mx = sq[w] > mx ? sq[w] : mx;
        for (int t = tid; t < TT; t += SA_THREADS) sco[t] = expf(sco[t] - mx);
    }
    __syncthreads();
    if (tid == 0) {
        double sum = 0.0;
        for (int t0 = 0; t0 < TT; t0 += 32) {
            float x[32];
#pragma unroll
            for (int i = 0; i < 32; ++i) x[i] = t0 + i < TT ? sco[t0 + i] : 0.0f;
#pragma unroll
            for (int i = 0; i < 32; ++i)
                if (t0 + i < TT) sum += double(x[i]);
        }
        s_inv = 1.0f / float(sum);
    }
    __syncthreads();
    // y_j: the 64-token blocks' fma chains on the waves (block x on wave x % 8, its 64 values loaded together),
    // then added in block order
    {
        const float inv = s_inv;
        const int j = tid & 63;
        const float* col = S0 + kSv + h * 64 + j;
        for (int x = tid >> 6; x < SA_NB; x += SA_THREADS / 64) {
            const int t0 = x * 64;
            float v[64];
#pragma unroll
            for (int i = 0; i < 64; ++i) v[i] = t0 + i < TT ? col[(long long)(t0 + i) * kSld] : 0.0f;
            float blk = 0.0f;
#pragma unroll
            for (int i = 0; i < 64; ++i)
                if (t0 + i < TT) blk = __builtin_fmaf(sco[t0 + i] * inv, v[i], blk);
            yblk[x][j] = blk;
        }
    }
    __syncthreads();
    if (tid < 64) {
        float tot = yblk[0][tid];
        for (int x = 1; x < SA_NB; ++x) tot = tot + yblk[x][tid];
        Y[(long long)b * kD + h * 64 + tid] = tot;
    }
}

// ------------------------------------------------------------------------------------------------ head
// final RMSNorm (16-lane tree), Linear(384,128) as K blocks of 64 (one thread per output), SiLU (AUDIO: GELU), then
// the 128-long dot with the 16-lane structure + bias.  w0 row-major [128][384].
template <bool AUDIO>
__global__ void __launch_bounds__(128)
head_kernel(const float* __restrict__ X, const float* __restrict__ nw, const float* __restrict__ w0,
            const float* __restrict__ b0, const float* __restrict__ w2, float b2, float* __restrict__ logits) {
    const int b = blockIdx.x, tid = threadIdx.x;
    __shared__ float xn[kD];
    __shared__ float hid[128];
    const float* x = X + (long long)b * kD;
    if (tid < 16) {
        float acc = x[tid] * x[tid];
        for (int i = 1; i < 24; ++i) acc = __builtin_fmaf(x[i * 16 + tid], x[i * 16 + tid], acc);
        const float s = tree16(acc);
        const float inv = 1.0f / sqrtf(s / 384.0f + 1e-6f);
        for (int i = 0; i < 24; ++i) xn[i * 16 + tid] = (x[i * 16 + tid] * inv) * nw[i * 16 + tid];
    }
    __syncthreads();
    {
        const float* wr = w0 + (long long)tid * kD;
        float tot = 0.0f;
        for (int k0 = 0; k0 < kD; k0 += 64) {
            float blk = 0.0f;
            for (int k = k0; k < k0 + 64; ++k) blk = __builtin_fmaf(xn[k], wr[k], blk);
            tot = k0 == 0 ? blk : tot + blk;
        }
        const float z = tot + b0[tid];
        // SHIELD-A: exact GELU 0.5 z (1 + erf(z / sqrt 2)) (engine/audio/sequence.cpp:333-334); SHIELD-V: SiLU
        hid[tid] = AUDIO ? 0.5f * z * (1.0f + erff(z * 0.7071067811865475244f)) : silu(z);
    }
    __syncthreads();
    if (tid < 16) {
        float acc = hid[tid] * w2[tid];
        for (int i = 1; i < 8; ++i) acc = __builtin_fmaf(hid[i * 16 + tid], w2[i * 16 + tid], acc);
        const float s = tree16(acc);
        if (tid == 0) logits[b] = s + b2;
    }
}

// Token-slot stores of one batch.  The host lists only the frames that store, as (batch frame, pool slot) pairs,
// so the grid covers exactly the rows to move: thread i copies 16-byte piece i % 1536 of pair i / 1536, striding by
// the grid.
constexpr int kRowPieces = int(kTokenFloats / 4);
__global__ void __launch_bounds__(256)
slot_store_kernel(const float4* __restrict__ tokens, const int2* __restrict__ pairs, long long pieces,
                  float4* __restrict__ pool) {
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < pieces; i += (long long)gridDim.x * blockDim.x) {
        const int2 fs = pairs[i / kRowPieces];
        const int c = int(i % kRowPieces);
        pool[(long long)fs.y * kRowPieces + c] = tokens[(long long)fs.x * kRowPieces + c];
    }
}

}  // namespace

template <typename T>
void launch_rmsnorm(const float* x, long long ldx, const float* w, T* out, long long ldo, int rows, hipStream_t s,
                    long long pstride, long long kstride) {
    hipLaunchKernelGGL(rmsnorm_kernel<T>, dim3(cdiv((long long)rows * 16, 256)), dim3(256), 0, s, x, ldx, w, out, ldo,
                       pstride, kstride, rows);
}
// The kernels are instantiated for SHIELD-V's windows (321 tokens) and SHIELD-A's (126): f(integral_constant<TT>).
template <class F> void for_window(int T, F&& f) {
    if (T == kT) f(std::integral_constant<int, kT>());
    else if (T == kTAudio) f(std::integral_constant<int, kTAudio>());
    else throw std::runtime_error("sequence kernels: unsupported window length " + std::to_string(T));
}

template <typename T>
void launch_window_input(const WindowInput& in, const float* w, float* h, T* out, long long ldo, int B, int TT,
                         hipStream_t s, long long pstride, long long kstride) {
    const bool table = in.frame_tokens != nullptr;
    if (!in.readout || (TT == kT && !in.pos) || (!table && (!in.tokens || in.ldw < (long long)(TT - 1) * kD)))
        throw std::runtime_error("window input: missing token source or position table, or a window stride below "
                                 "its tokens");
    const int rows = B * TT;
    const dim3 grid(cdiv((long long)rows * 16, 256));
    for_window(TT, [&](auto tt) {
        constexpr int W = decltype(tt)::value;
        const auto go = [&](auto kern) {
            hipLaunchKernelGGL(kern, grid, dim3(256), 0, s, in, w, h, out, ldo, pstride, kstride, rows);
        };
        if (table) go(window_input_kernel<T, W, true, W == kT>);
        else if (in.pos) go(window_input_kernel<T, W, false, true>);
        else go(window_input_kernel<T, W, false, false>);
    });
}
void launch_gdn_prep(const float* P, const float* conv_w, const float* conv_b, const float* neg_rate,
                     const float* dt_bias, float* Q, float* K, float* V, float* dec, float* beta, int B,
                     hipStream_t s, int T, bool audio, bool fast) {
    for_window(T, [&](auto tt) {
        constexpr int TT = decltype(tt)::value;
        const dim3 grid(B * ((TT + GP_T - 1) / GP_T));
        const auto go = [&](auto kern) {
            hipLaunchKernelGGL(kern, grid, dim3(384), 0, s, P, conv_w, conv_b, neg_rate, dt_bias, Q, K, V, dec, beta);
        };
        if (audio) {
            if (fast) go(gdn_prep_kernel<TT, true, true>);
            else go(gdn_prep_kernel<TT, true, false>);
        } else {
            if (fast) go(gdn_prep_kernel<TT, false, true>);
            else go(gdn_prep_kernel<TT, false, false>);
        }
    });
}
void launch_delta(const float* Q, const float* K, const float* V, const float* dec, const float* beta, float* O,
                  int B, bool exact, hipStream_t s, int T) {
    for_window(T, [&](auto tt) {
        constexpr int TT = decltype(tt)::value;
        if (exact) {
            hipLaunchKernelGGL((delta_kernel<TT>), dim3(B * kHeads * 2), dim3(DCOLS), 0, s, Q, K, V, dec, beta, O);
            return;
        }
        // the split follows the batch (results are bitwise the same for every split): the most lane groups per
        // column that still fit one wave per SIMD; KQ = 2 past that
        if (B * kHeads * 16 <= kDeltaPipeWaves)
            hipLaunchKernelGGL((delta_split_kernel<8, true, TT>), dim3(B * kHeads * 16), dim3(64), 0, s, Q, K, V, dec,
                               beta, O);
        else if (B * kHeads * 8 <= kDeltaPipeWaves)
            hipLaunchKernelGGL((delta_split_kernel<4, true, TT>), dim3(B * kHeads * 8), dim3(64), 0, s, Q, K, V, dec,
                               beta, O);
        else if (B * kHeads * 4 <= kDeltaPipeWaves)
            hipLaunchKernelGGL((delta_split_kernel<2, true, TT>), dim3(B * kHeads * 4), dim3(64), 0, s, Q, K, V, dec,
                               beta, O);
        else
            hipLaunchKernelGGL((delta_split_kernel<2, false, TT>), dim3(B * kHeads * 4), dim3(64), 0, s, Q, K, V, dec,
                               beta, O);
    });
}
size_t delta_chunk_floats(int B, int T) { return size_t(B) * kHeads * size_t((T + DC - 1) / DC) * DCF; }
template <typename T>
void launch_delta_chunked(const float* Q, const float* K, const float* V, const float* dec, const float* beta,
                          float* O, float* work, int B, hipStream_t s, int Tw) {
    if (!work) throw std::runtime_error("delta: the chunked scan needs its work buffer");
    for_window(Tw, [&](auto tt) {
        constexpr int TT = decltype(tt)::value;
        constexpr int NC = (TT + DC - 1) / DC;
        hipLaunchKernelGGL((delta_chunk_prep_kernel<T, TT>), dim3(B * kHeads * NC), dim3(64), 0, s, Q, K, V, dec, beta,
                           work);
        // value blocks per head by batch (bitwise the same results for every split): small batches spread a
        // head's state over more workgroups
        if (B <= 16)
            hipLaunchKernelGGL((delta_chunk_scan_kernel<T, 32, TT>), dim3(B * kHeads * 4), dim3(256), 0, s, Q, K, work,
                               O);
        else
            hipLaunchKernelGGL((delta_chunk_scan_kernel<T, 64, TT>), dim3(B * kHeads * 2), dim3(256), 0, s, Q, K, work,
                               O);
    });
}
template void launch_delta_chunked<f16>(const float*, const float*, const float*, const float*, const float*, float*,
                                        float*, int, hipStream_t, int);
template void launch_delta_chunked<float>(const float*, const float*, const float*, const float*, const float*,
                                          float*, float*, int, hipStream_t, int);
template void launch_delta_chunked<bf16>(const float*, const float*, const float*, const float*, const float*,
                                         float*, float*, int, hipStream_t, int);
template <typename T>
void launch_gated_norm(const float* O, const float* P, const float* w, T* out, int rows, hipStream_t s,
                       long long pstride, bool audio, long long ld, long long kstride) {
    const dim3 grid(cdiv((long long)cdiv(rows, 4) * 4 * kHeads * 16, 256));
    if (audio)
        hipLaunchKernelGGL((gated_norm_kernel<T, true>), grid, dim3(256), 0, s, O, P, w, out, pstride, ld, kstride,
                           rows);
    else
        hipLaunchKernelGGL((gated_norm_kernel<T, false>), grid, dim3(256), 0, s, O, P, w, out, pstride, ld, kstride,
                           rows);
}
void launch_sisa(float* S, const float* QC, const float* lam, float* Y, int B, hipStream_t s, int T) {
    for_window(T, [&](auto tt) {
        constexpr int TT = decltype(tt)::value;
        hipLaunchKernelGGL((sisa_kernel<TT>), dim3(B * kHeads), dim3(SA_THREADS), 0, s, S, QC, lam, Y);
    });
}
void launch_head(const float* X, const float* norm_w, const float* w0, const float* b0, const float* w2, float b2,
                 float* logits, int B, hipStream_t s, bool audio) {
    if (audio) hipLaunchKernelGGL((head_kernel<true>), dim3(B), dim3(128), 0, s, X, norm_w, w0, b0, w2, b2, logits);
    else hipLaunchKernelGGL((head_kernel<false>), dim3(B), dim3(128), 0, s, X, norm_w, w0, b0, w2, b2, logits);
}
void launch_slot_store(const float* tokens, const int32_t* pairs, int n_pairs, float* pool, hipStream_t s) {
    if (n_pairs <= 0) return;
    const long long pieces = (long long)n_pairs * kRowPieces;
    const unsigned grid = unsigned(std::min<long long>(cdiv(pieces, 256), 2048));
    hipLaunchKernelGGL(slot_store_kernel, dim3(grid), dim3(256), 0, s, reinterpret_cast<const float4*>(tokens),
                       reinterpret_cast<const int2*>(pairs), pieces, reinterpret_cast<float4*>(pool));
}

// ------------------------------------------------------------------------------------------------ no allocation
// Work memory of the chunked scan for callers that cannot allocate (code under graph capture, serving loops): a
// file-scope device array for kDeltaNoAllocWindows windows (6 heads x 11 chunks x 7232 floats each, 30.5 MB), one
// copy per GPU for the life of the process.  The prep kernel writes every float of a chunk's area before the scan
// reads it, so nothing has to be cleared between calls.  In host code `scratch` names a host-side stand-in, never
// the device memory: kernels get the address hipGetSymbolAddress returns, kept per device.
static __device__ __align__(256) float scratch[size_t(kDeltaNoAllocWindows) * kHeads * DNC * DCF];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_addr[kMaxDevices] = {};

// The device address of `scratch` on the current device, looked up once per device (no allocation).
float* scratch_on_current_device() {
    int dev = -1;
    SHV_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) throw std::runtime_error("delta rule (no allocation): device ordinal out of range");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            throw std::runtime_error(std::string("delta rule (no allocation): hipGetSymbolAddress failed: ") +
                                     hipGetErrorString(e));
        g_scratch_addr[dev] = static_cast<float*>(p);
    }
    return g_scratch_addr[dev];
}
}  // namespace

void run_delta_rule_noalloc(Precision p, const float* Q, const float* K, const float* V, const float* dec,
                            const float* beta, int n_windows, float* O, int variant, hipStream_t s) {
    const DeltaKernel kern = delta_rule_kernel(p, Q, K, V, dec, beta, n_windows, O, variant);
    if (kern != DeltaKernel::Chunked) {
        launch_delta(Q, K, V, dec, beta, O, n_windows, kern == DeltaKernel::Reference, s, kT);
        SHV_HIP_CHECK(hipGetLastError());
        return;
    }
    if (n_windows > kDeltaNoAllocWindows)
        throw std::runtime_error("delta rule (no allocation): " + std::to_string(n_windows) +
                                 " windows exceed the static work area of " + std::to_string(kDeltaNoAllocWindows));
    float* work = scratch_on_current_device();
    if (p == Precision::BF16) launch_delta_chunked<bf16>(Q, K, V, dec, beta, O, work, n_windows, s, kT);
    else if (p == Precision::FP16) launch_delta_chunked<f16>(Q, K, V, dec, beta, O, work, n_windows, s, kT);
    else launch_delta_chunked<float>(Q, K, V, dec, beta, O, work, n_windows, s, kT);
    SHV_HIP_CHECK(hipGetLastError());
}

#define SHV_NORMS(T)                                                                                             \
    template void launch_rmsnorm<T>(const float*, long long, const float*, T*, long long, int, hipStream_t,      \
                                    long long, long long);                                                       \
    template void launch_gated_norm<T>(const float*, const float*, const float*, T*, int, hipStream_t, long long,  \
                                       bool, long long, long long);                                               \
    template void launch_window_input<T>(const WindowInput&, const float*, float*, T*, long long, int, int,       \
                                         hipStream_t, long long, long long);
SHV_NORMS(float)
SHV_NORMS(f16)
SHV_NORMS(bf16)
#undef SHV_NORMS

}  // namespace shv
