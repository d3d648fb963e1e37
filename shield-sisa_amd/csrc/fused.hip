// Fused MobileNetV3 inverted-residual blocks for the fp16 / bf16 tiers (gfx950).
//
// One workgroup (256 threads, 4 waves) owns a TH x TW tile of output pixels of one frame.  It stages the input
// tile with its halo in LDS (zero outside the map) -- already split into the MFMA operand parts when the tile is
// expanded, so each value is split once, not once per chunk -- then walks the expanded channels in chunks of 32:
//   expand    E[p][c] = act(X[p] . Wexp[c] + b) for every input-tile pixel (split-operand MFMA, K = cin)
//   depthwise D[q][c] = act(sum over taps of E * w + b), fma chain over (dy, dx) from +0 (VALU, LDS reads)
//   project   Y[q] += D[q][chunk] . Wproj[:, chunk]   (split-operand MFMA, accumulators stay in registers)
// so the expanded tensors never leave the CU: per block only the narrow input and output maps touch HBM.  The
// project's K runs chunk by chunk in increasing order, one MFMA K step per chunk, exactly as the layer GEMM does.
// Blocks with squeeze-excite need the spatial mean of D before the project, so their kernel writes D and per-tile
// channel sums instead; the engine reduces the sums, runs the SE fc layers and the project GEMM with the SE scale.
//
// The reference runs these stages as separate kernels with half-precision storage between them
// (engine/cuda/engine.cu:348-382; engine/cuda/fused.cu:16-114 fuses expand + depthwise for two blocks only); here
// all activations stay fp32 and every block is fused.
#include "dev_common.hpp"
#include "kernels.hpp"
#include "mfma.hpp"

#include <algorithm>
#include <cstdlib>
#include <stdexcept>

namespace shv {
namespace {

constexpr int IR_THREADS = 256;
constexpr int CW = 32;           // expanded channels per chunk: one MFMA K step of the project
constexpr int CS_LD = CW + 4;    // fp32 row stride of the chunk buffers: 16-lane fragment reads hit 64 banks once
constexpr int LDS_BUDGET = 80 * 1024;   // two workgroups per CU

// Workgroup barrier that waits for LDS traffic only.  A full workgroup barrier also drains every outstanding global
// load, which would stall the weight prefetches issued one chunk ahead; LDS is the only memory shared across the
// workgroup here (global stores are never read back by it).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int CIN_, int CEXP_, int COUT_, int KS_, int S_, int HS_, int SE_, int TH_, int TW_, int R_, int MODE_>
struct IrCfg {
    static constexpr int CIN = CIN_, CEXP = CEXP_, COUT = COUT_, KS = KS_, S = S_, TH = TH_, TW = TW_, R = R_;
    // Launch and pipeline style, chosen per block by measurement (they trade registers against latency hiding):
    //   PERSIST  (MODE bit 0) workgroups loop over (frame, tile) items, loading the next item's input tile into
    //            registers while computing (else one workgroup per item);
    //   RELOAD   (MODE bit 1) expand / project fragments re-issued right after their last use (one register set,
    //            live across the chunk) instead of expand fragments double-buffered a chunk ahead and project
    //            fragments issued at the top of their own chunk;
    //   NOSPLIT  (MODE bit 2) input tile kept as fp32 in LDS and split per chunk instead of split once.
    static constexpr bool PERSIST = (MODE_ & 1) != 0;
    static constexpr bool RELOAD = (MODE_ & 2) != 0;
    static constexpr bool NOSPLIT = (MODE_ & 4) != 0;
    //   ROLLED   (MODE bit 3) the tile is staged by a rolled copy loop (one float4 in flight per thread at a time)
    //            instead of grouped loads -- fewer live registers where the grouped form costs a wave per SIMD.
    static constexpr bool ROLLED = (MODE_ & 8) != 0;
    //   WHOLE    (MODE bit 4) a non-persistent workgroup issues the loads of its whole tile before storing any
    //            (else 4 float4s per thread at a time).
    static constexpr bool WHOLE = (MODE_ & 16) != 0;
    static constexpr int ACT = HS_ ? ACT_HS : ACT_RELU;
    static constexpr bool SE = SE_ != 0;
    static constexpr bool EXPAND = CEXP != CIN;
    static constexpr bool RES = !SE && S == 1 && CIN == COUT;   // SE blocks add the residual in the project GEMM
    static constexpr int PAD = (KS - 1) / 2;
    static constexpr int IH = (TH - 1) * S + KS, IW = (TW - 1) * S + KS;
    static constexpr int PIN = IH * IW, POUT = TH * TW;
    static constexpr int CINP = (CIN + 31) / 32 * 32;
    static constexpr int CEXPP = (CEXP + CW - 1) / CW * CW;
    static constexpr int COUTP = (COUT + 15) / 16 * 16;
    static constexpr int XS_LD = CIN + 4;                       // fp32 tile row stride
    static constexpr int MT_IN = (PIN + 15) / 16, MT_OUT = (POUT + 15) / 16;
    static constexpr int MPW_IN = (MT_IN + 3) / 4, MPW_OUT = (MT_OUT + 3) / 4;
    static constexpr int NT_OUT = COUTP / 16;
    static constexpr int NCH = CEXPP / CW;
    static constexpr int ES_FLOATS = EXPAND ? MT_IN * 16 * CS_LD : 0;
    static constexpr int DS_FLOATS = MT_OUT * 16 * CS_LD;
    static constexpr int WD_FLOATS = (KS * KS + 1) * CW;        // chunk's depthwise taps + bias
    static constexpr int RED_FLOATS = SE ? 4 * CW : 0;          // SE: per-wave channel sums
    // depthwise work units: (4-channel group, tile column, strip of R output rows)
    static constexpr int NCG = (CEXP < CW ? CEXP : CW) / 4;
    static constexpr int NSTRIP = (TH + R - 1) / R;
    static constexpr int DW_UNITS = NCG * TW * NSTRIP;
    static_assert(CIN % 8 == 0 && CEXP % 8 == 0, "channel counts must be multiples of 8");
    static_assert(TH % R == 0, "depthwise strips must tile the output rows");
};

// LDS layout for storage type T.  Expanded blocks keep the input tile pre-split ([part][row][CINP + 8] of T, the
// K padding zero; a row stride of CINP + 8 elements makes the 16-lane 16-byte fragment reads conflict-free) when
// that fits the budget, else as fp32 and split per chunk.
template <typename T, class C> struct IrLayout {
    static constexpr int P = Split<T>::P;
    static constexpr int XH_LD = C::CINP + 8;
    static constexpr int XH_ROWS = C::MT_IN * 16;
    static constexpr int XS_SPLIT_BYTES = P * XH_ROWS * XH_LD * 2;
    static constexpr int XS_F32_BYTES = C::PIN * C::XS_LD * 4;
    static constexpr int REST_BYTES = (C::ES_FLOATS + C::DS_FLOATS + C::WD_FLOATS + C::RED_FLOATS) * 4;
    static constexpr bool PRESPLIT = C::EXPAND && !C::NOSPLIT && XS_SPLIT_BYTES + REST_BYTES <= LDS_BUDGET;
    static constexpr int XS_BYTES = PRESPLIT ? XS_SPLIT_BYTES : XS_F32_BYTES;
    static constexpr int BYTES = XS_BYTES + REST_BYTES;
    static_assert(BYTES <= LDS_BUDGET, "tile exceeds the LDS budget (two workgroups per CU)");
};

// The 15 blocks of MobileNetV3-Large (engine/cuda/model.hpp:23-29) with their output tiles, depthwise strips and
// launch / pipeline mode (bit 0 persistent, bit 1 reload-after-use, bit 2 fp32 tile, bit 3 rolled staging, bit 4
// whole-tile staging; see IrCfg).
//                  cin cexp cout k  s hs se TH TW R  mode
typedef IrCfg<16, 16, 16, 3, 1, 0, 0, 10, 16, 5, 1> B1;    // 90x160
typedef IrCfg<16, 64, 24, 3, 2, 0, 0, 5, 8, 1, 4> B2;      // 90x160 -> 45x80
typedef IrCfg<24, 72, 24, 3, 1, 0, 0, 9, 16, 3, 8> B3;     // 45x80
typedef IrCfg<24, 72, 40, 5, 2, 0, 1, 4, 8, 1, 3> B4;      // 45x80 -> 23x40
typedef IrCfg<40, 120, 40, 5, 1, 0, 1, 8, 8, 2, 2> B5;     // 23x40 (b5, b6)
typedef IrCfg<40, 240, 80, 3, 2, 1, 0, 4, 10, 1, 18> B7;    // 23x40 -> 12x20
typedef IrCfg<80, 200, 80, 3, 1, 1, 0, 6, 10, 2, 2> B8;    // 12x20
typedef IrCfg<80, 184, 80, 3, 1, 1, 0, 6, 10, 2, 2> B9;    // 12x20 (b9, b10)
typedef IrCfg<80, 480, 112, 3, 1, 1, 1, 6, 10, 2, 3> B11;  // 12x20
typedef IrCfg<112, 672, 112, 3, 1, 1, 1, 6, 10, 2, 0> B12; // 12x20
typedef IrCfg<112, 672, 160, 5, 2, 1, 1, 3, 5, 1, 8> B13;  // 12x20 -> 6x10
typedef IrCfg<160, 960, 160, 5, 1, 1, 1, 3, 5, 1, 4> B14;  // 6x10 (b14, b15)

template <typename T, class C>
__global__ void __launch_bounds__(IR_THREADS) ir_block_kernel(IrArgs a) {
    typedef Split<T> S;
    typedef typename S::V8 V8;
    typedef IrLayout<T, C> L;
    __shared__ __attribute__((aligned(16))) unsigned char lds_raw[L::BYTES];
    float* Xs = reinterpret_cast<float*>(lds_raw);     // fp32 input tile [PIN][XS_LD]         (!PRESPLIT)
    T* Xh = reinterpret_cast<T*>(lds_raw);             // split input tile [P][XH_ROWS][XH_LD] (PRESPLIT)
    float* Es = reinterpret_cast<float*>(lds_raw + L::XS_BYTES);
    float* Ds = Es + C::ES_FLOATS;
    float* Wd = Ds + C::DS_FLOATS;
    float* red = Wd + C::WD_FLOATS;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r = lane & 15, g = lane >> 4;
    const int items = a.ntiles * a.frames;
    const T* wexp = static_cast<const T*>(a.wexp);
    const T* wproj = static_cast<const T*>(a.wproj);

    // ---- weight pipeline.  The chunk index runs on across items (after the last chunk comes chunk 0 of the next
    // item).  Depthwise taps and expand bias of the next chunk are always fetched one chunk ahead.  Expand / project
    // fragments either (RELOAD) are re-issued right after their last use, or are double-buffered a chunk ahead
    // (expand, when 64 VGPRs hold them) / issued at the top of their own chunk.  All stay in flight across the
    // LDS-only barriers.
    constexpr int KST = C::CINP / 32;
    constexpr bool PROJ = !C::SE;
    constexpr bool PF_EXP = !C::RELOAD && C::EXPAND && KST * 2 * S::P * 4 <= 64;
    constexpr int WD4 = (C::KS * C::KS + 1) * (CW / 4);   // float4s of a chunk's depthwise table
    static_assert(WD4 <= IR_THREADS, "one float4 of depthwise taps per thread");
    float4 wd_n = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float eb_n[2] = {0.0f, 0.0f};
    V8 ew[C::EXPAND ? KST : 1][2][S::P];        // fragments used by the expand of the current chunk
    V8 ew_n[PF_EXP ? KST : 1][2][S::P];         // double buffer (PF_EXP)
    V8 pw[PROJ ? C::NT_OUT : 1][S::P];
    auto fetch_wd = [&](int c0) {
        if (tid < WD4) {
            const int t = tid / (CW / 4), q = tid - t * (CW / 4);
            const float* src = t < C::KS * C::KS ? a.wdw + t * C::CEXPP + c0 + q * 4 : a.bdw + c0 + q * 4;
            wd_n = *reinterpret_cast<const float4*>(src);
        }
        if constexpr (C::EXPAND) {
            eb_n[0] = a.bexp[c0 + r];
            eb_n[1] = a.bexp[c0 + 16 + r];
        }
    };
    auto load_ew_into = [&](V8 (&dst)[C::EXPAND ? KST : 1][2][S::P], int c0) {
        if constexpr (C::EXPAND) {
#pragma unroll
            for (int ks = 0; ks < KST; ++ks)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                    for (int q = 0; q < S::P; ++q)
                        dst[ks][nt][q] = load_part8<T>(wexp + q * a.wexp_stride +
                                                       (long long)(c0 + nt * 16 + r) * C::CINP + ks * 32 + g * 8);
        }
    };
    auto load_pw = [&](int c0) {
        if constexpr (PROJ) {
#pragma unroll
            for (int nt = 0; nt < C::NT_OUT; ++nt)
#pragma unroll
                for (int q = 0; q < S::P; ++q)
                    pw[nt][q] = load_part8<T>(wproj + q * a.wproj_stride + (long long)(nt * 16 + r) * C::CEXPP +
                                              c0 + g * 8);
        }
    };

    // ---- input pipeline: the next item's tile (with halo, zero outside the map and in the K padding) is loaded
    // into registers while the current item computes, then written to LDS -- split into the operand parts when
    // the block expands.  Tile rows are contiguous NHWC runs.
    constexpr int XQ = L::PRESPLIT ? C::CINP / 4 : C::CIN / 4;   // float4 columns per tile row
    constexpr int XROWS = L::PRESPLIT ? L::XH_ROWS : C::PIN;
    constexpr int XN = XROWS * XQ;
    constexpr int XR = (XN + IR_THREADS - 1) / IR_THREADS;
    float4 xr[(C::PERSIST || C::WHOLE) ? XR : (XR < 4 ? XR : 4)];
    // staging of one tile in groups of float4s per thread: within a group every load is issued (at a clamped,
    // always valid address) before any is used; positions outside the map or the channel count take zero.
    // Persistent workgroups hold the whole next tile in registers; the others stage 4 float4s at a time.
    constexpr int XG = (C::PERSIST || C::WHOLE) ? XR : (XR < 4 ? XR : 4);
    auto load_x = [&](int item, int k0) {
        const int tile = item % a.ntiles;
        const long long f = item / a.ntiles;
        const int iy0 = (tile / a.tiles_x) * C::TH * C::S - C::PAD, ix0 = (tile % a.tiles_x) * C::TW * C::S - C::PAD;
        const float* Xf = a.X + f * a.H * a.W * C::CIN;
#pragma unroll
        for (int k = 0; k < XG; ++k) {
            const int i = tid + (k0 + k) * IR_THREADS;
            const int row = i / XQ, q = i - row * XQ;
            const int ly = row / C::IW, lx = row - ly * C::IW;
            const int iy = iy0 + ly, ix = ix0 + lx;
            const bool in = i < XN && row < C::PIN && q * 4 < C::CIN && iy >= 0 && iy < a.H && ix >= 0 && ix < a.W;
            const int cy = min(max(iy, 0), a.H - 1), cx = min(max(ix, 0), a.W - 1), cq = min(q, C::CIN / 4 - 1);
            const float4 v = *reinterpret_cast<const float4*>(Xf + ((long long)cy * a.W + cx) * C::CIN + cq * 4);
            xr[k] = in ? v : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    auto store_x = [&](int k0) {
#pragma unroll
        for (int k = 0; k < XG; ++k) {
            const int i = tid + (k0 + k) * IR_THREADS;
            if (i >= XN) continue;
            const int row = i / XQ, q = i - row * XQ;
            if constexpr (L::PRESPLIT) {
                const float x[4] = {xr[k].x, xr[k].y, xr[k].z, xr[k].w};
                uint2 four[S::P];
                split4_packed<T>(x, four);
#pragma unroll
                for (int pq = 0; pq < S::P; ++pq)
                    *reinterpret_cast<uint2*>(Xh + (pq * L::XH_ROWS + row) * L::XH_LD + q * 4) = four[pq];
            } else {
                *reinterpret_cast<float4*>(Xs + row * C::XS_LD + q * 4) = xr[k];
            }
        }
    };

    fetch_wd(0);
    if constexpr (PF_EXP) load_ew_into(ew_n, 0);
    if constexpr (C::RELOAD) {
        load_ew_into(ew, 0);
        load_pw(0);
    }
    if constexpr (C::PERSIST) {
        if ((int)blockIdx.x < items) load_x(blockIdx.x, 0);
    }

    for (int item = blockIdx.x; item < items; item += gridDim.x) {
        const int tile = item % a.ntiles;
        const long long f = item / a.ntiles;
        const int ty0 = (tile / a.tiles_x) * C::TH, tx0 = (tile % a.tiles_x) * C::TW;
        const int iy0 = ty0 * C::S - C::PAD, ix0 = tx0 * C::S - C::PAD;
        const float* Xf = a.X + f * a.H * a.W * C::CIN;

        if constexpr (C::PERSIST) {
            store_x(0);
            if (item + (int)gridDim.x < items) load_x(item + gridDim.x, 0);
        } else if constexpr (C::ROLLED) {
            for (int i = tid; i < XN; i += IR_THREADS) {
                const int row = i / XQ, q = i - row * XQ;
                const int ly = row / C::IW, lx = row - ly * C::IW;
                const int iy = iy0 + ly, ix = ix0 + lx;
                float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (row < C::PIN && q * 4 < C::CIN && iy >= 0 && iy < a.H && ix >= 0 && ix < a.W)
                    v = *reinterpret_cast<const float4*>(Xf + ((long long)iy * a.W + ix) * C::CIN + q * 4);
                if constexpr (L::PRESPLIT) {
                    const float x[4] = {v.x, v.y, v.z, v.w};
                    uint2 four[S::P];
                    split4_packed<T>(x, four);
#pragma unroll
                    for (int pq = 0; pq < S::P; ++pq)
                        *reinterpret_cast<uint2*>(Xh + (pq * L::XH_ROWS + row) * L::XH_LD + q * 4) = four[pq];
                } else {
                    *reinterpret_cast<float4*>(Xs + row * C::XS_LD + q * 4) = v;
                }
            }
        } else {
            for (int k0 = 0; k0 < XR; k0 += XG) {
                load_x(item, k0);
                store_x(k0);
            }
        }
        // Ds entries the depthwise never writes (channels past cexp of a narrow block, rows past the tile) stay 0
        for (int i = tid; i < C::DS_FLOATS; i += IR_THREADS) Ds[i] = 0.0f;
        // expand epilogue rows of this lane that are inside the map (bit 4 j + i)
        unsigned inside = 0;
        if constexpr (C::EXPAND) {
#pragma unroll
            for (int j = 0; j < C::MPW_IN; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = (wave + 4 * j) * 16 + g * 4 + i;
                    const int ly = row / C::IW, lx = row - ly * C::IW;
                    const int iy = iy0 + ly, ix = ix0 + lx;
                    if (row < C::PIN && iy >= 0 && iy < a.H && ix >= 0 && ix < a.W) inside |= 1u << (4 * j + i);
                }
        }
        lds_barrier();

        f32x4 yacc[C::MPW_OUT][C::NT_OUT];
#pragma unroll
        for (int j = 0; j < C::MPW_OUT; ++j)
#pragma unroll
            for (int nt = 0; nt < C::NT_OUT; ++nt) yacc[j][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

        for (int ch = 0; ch < C::NCH; ++ch) {
            const int c0 = ch * CW;
            const int cn = ch + 1 < C::NCH ? c0 + CW : 0;   // next chunk (wraps to the next item's first)
            // this chunk's depthwise table -> Wd (visible after the next barrier); fetch the next chunk's
            if (tid < WD4) *reinterpret_cast<float4*>(Wd + tid * 4) = wd_n;
            const float eb_c[2] = {eb_n[0], eb_n[1]};
            if constexpr (!C::RELOAD) {
                if constexpr (PF_EXP) {
#pragma unroll
                    for (int ks = 0; ks < KST; ++ks)
#pragma unroll
                        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                            for (int q = 0; q < S::P; ++q) ew[ks][nt][q] = ew_n[ks][nt][q];
                } else {
                    load_ew_into(ew, c0);
                }
                load_pw(c0);   // consumed after the depthwise
                if constexpr (PF_EXP) load_ew_into(ew_n, cn);
            }
            fetch_wd(cn);

            if constexpr (C::EXPAND) {
                // ---- expand: E[rows][32] = act(X . Wexp[c0 .. c0+32) + b), waves take 16-row tiles round robin
                f32x4 eacc[C::MPW_IN][2];
#pragma unroll
                for (int j = 0; j < C::MPW_IN; ++j) eacc[j][0] = eacc[j][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int ks = 0; ks < KST; ++ks) {
                    const int kk = ks * 32 + g * 8;
#pragma unroll
                    for (int j = 0; j < C::MPW_IN; ++j) {
                        const int mt = wave + 4 * j;
                        if (mt < C::MT_IN) {
                            const int row = mt * 16 + r;
                            V8 ap[S::P];
                            if constexpr (L::PRESPLIT) {
#pragma unroll
                                for (int q = 0; q < S::P; ++q)
                                    ap[q] = *reinterpret_cast<const V8*>(Xh + (q * L::XH_ROWS + row) * L::XH_LD + kk);
                            } else {
                                float x[8];
                                if (row < C::PIN && kk < C::CIN) {
                                    const float4 lo = *reinterpret_cast<const float4*>(Xs + row * C::XS_LD + kk);
                                    const float4 hi = *reinterpret_cast<const float4*>(Xs + row * C::XS_LD + kk + 4);
                                    x[0] = lo.x; x[1] = lo.y; x[2] = lo.z; x[3] = lo.w;
                                    x[4] = hi.x; x[5] = hi.y; x[6] = hi.z; x[7] = hi.w;
                                } else {
#pragma unroll
                                    for (int e = 0; e < 8; ++e) x[e] = 0.0f;
                                }
                                split8<T>(x, ap);
                            }
                            eacc[j][0] = mfma_split<T>(ap, ew[ks][0], eacc[j][0]);
                            eacc[j][1] = mfma_split<T>(ap, ew[ks][1], eacc[j][1]);
                        }
                    }
                }
                if constexpr (C::RELOAD) load_ew_into(ew, cn);
#pragma unroll
                for (int j = 0; j < C::MPW_IN; ++j) {
                    const int mt = wave + 4 * j;
                    if (mt >= C::MT_IN) continue;
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) {
                        const int col = nt * 16 + r;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int row = mt * 16 + g * 4 + i;
                            float v = 0.0f;
                            if (inside & (1u << (4 * j + i))) v = apply_act_nb(eacc[j][nt][i] * a.sexp + eb_c[nt], C::ACT);
                            Es[row * CS_LD + col] = v;
                        }
                    }
                }
            }
            lds_barrier();   // E (or, without expand, Wd) complete; the previous chunk's project has read Ds

            // ---- depthwise over the chunk.  Unit = (4 channels, tile column ox, rows oy0 .. oy0+R-1); each output
            // is one fma chain over (dy, dx) from +0.  Taps outside the map read the zeros staged there: a product
            // with an exact zero added to a chain that starts at +0 leaves every value (and the sign of zero)
            // unchanged, so this equals skipping them.
            for (int u = tid; u < C::DW_UNITS; u += IR_THREADS) {
                const int cgi = u % C::NCG, rest = u / C::NCG;
                const int ox = rest % C::TW, oy0 = (rest / C::TW) * C::R;
                const float* src = C::EXPAND ? Es + (oy0 * C::S * C::IW + ox * C::S) * CS_LD + cgi * 4
                                             : Xs + (oy0 * C::S * C::IW + ox * C::S) * C::XS_LD + c0 + cgi * 4;
                constexpr int LD = C::EXPAND ? CS_LD : C::XS_LD;
                float4 acc[C::R];
#pragma unroll
                for (int rr = 0; rr < C::R; ++rr) acc[rr] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 1
                for (int dy = 0; dy < C::KS; ++dy) {   // rolled: keeps one kernel row of taps and inputs live
#pragma unroll
                    for (int dx = 0; dx < C::KS; ++dx) {
                        const float4 w = *reinterpret_cast<const float4*>(Wd + (dy * C::KS + dx) * CW + cgi * 4);
#pragma unroll
                        for (int rr = 0; rr < C::R; ++rr) {
                            const float4 x =
                                *reinterpret_cast<const float4*>(src + ((rr * C::S + dy) * C::IW + dx) * LD);
                            acc[rr].x = __builtin_fmaf(x.x, w.x, acc[rr].x);
                            acc[rr].y = __builtin_fmaf(x.y, w.y, acc[rr].y);
                            acc[rr].z = __builtin_fmaf(x.z, w.z, acc[rr].z);
                            acc[rr].w = __builtin_fmaf(x.w, w.w, acc[rr].w);
                        }
                    }
                }
                const float4 bb = *reinterpret_cast<const float4*>(Wd + C::KS * C::KS * CW + cgi * 4);
#pragma unroll
                for (int rr = 0; rr < C::R; ++rr) {
                    const int oy = oy0 + rr;
                    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    if (ty0 + oy < a.Ho && tx0 + ox < a.Wo) {
                        v.x = apply_act_nb(acc[rr].x + bb.x, C::ACT);
                        v.y = apply_act_nb(acc[rr].y + bb.y, C::ACT);
                        v.z = apply_act_nb(acc[rr].z + bb.z, C::ACT);
                        v.w = apply_act_nb(acc[rr].w + bb.w, C::ACT);
                    }
                    *reinterpret_cast<float4*>(Ds + (oy * C::TW + ox) * CS_LD + cgi * 4) = v;
                }
            }
            lds_barrier();

            if constexpr (PROJ) {
                // ---- project: Y[POUT][COUT] += D[POUT][chunk] . Wproj[:, chunk]
                V8 af[C::MPW_OUT][S::P];
#pragma unroll
                for (int j = 0; j < C::MPW_OUT; ++j) {
                    const int mt = wave + 4 * j;
                    float x[8];
                    if (mt < C::MT_OUT) {
                        const float* src = Ds + (mt * 16 + r) * CS_LD + g * 8;
                        const float4 lo = *reinterpret_cast<const float4*>(src);
                        const float4 hi = *reinterpret_cast<const float4*>(src + 4);
                        x[0] = lo.x; x[1] = lo.y; x[2] = lo.z; x[3] = lo.w;
                        x[4] = hi.x; x[5] = hi.y; x[6] = hi.z; x[7] = hi.w;
                    } else {
#pragma unroll
                        for (int e = 0; e < 8; ++e) x[e] = 0.0f;
                    }
                    split8<T>(x, af[j]);
                }
#pragma unroll
                for (int nt = 0; nt < C::NT_OUT; ++nt)
#pragma unroll
                    for (int j = 0; j < C::MPW_OUT; ++j)
                        if (wave + 4 * j < C::MT_OUT) yacc[j][nt] = mfma_split<T>(af[j], pw[nt], yacc[j][nt]);
                if constexpr (C::RELOAD) load_pw(cn);
            } else {
                // ---- SE blocks: D chunk -> HBM, and the tile's channel sums: thread (pixel group pg, 4 channels
                // q) sums pixels pg, pg + 32 in order, lanes with equal q are combined by an xor tree inside the
                // wave, the 4 wave totals in wave order after a barrier (a fixed order that never involves other
                // frames)
                const int q = tid & 7, pg = tid >> 3;
                float4 sum = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                for (int p = pg; p < C::POUT; p += IR_THREADS / 8) {
                    const int oy = p / C::TW, ox = p - oy * C::TW;
                    const int gy = ty0 + oy, gx = tx0 + ox;
                    if (gy < a.Ho && gx < a.Wo) {
                        const float4 v = *reinterpret_cast<const float4*>(Ds + p * CS_LD + q * 4);
                        if (c0 + q * 4 < C::CEXP)
                            *reinterpret_cast<float4*>(a.D + ((f * a.Ho + gy) * a.Wo + gx) * C::CEXP + c0 + q * 4) = v;
                        sum.x = sum.x + v.x; sum.y = sum.y + v.y; sum.z = sum.z + v.z; sum.w = sum.w + v.w;
                    }
                }
#pragma unroll
                for (int m = 8; m < 64; m <<= 1) {
                    sum.x = sum.x + __shfl_xor(sum.x, m);
                    sum.y = sum.y + __shfl_xor(sum.y, m);
                    sum.z = sum.z + __shfl_xor(sum.z, m);
                    sum.w = sum.w + __shfl_xor(sum.w, m);
                }
                if (lane < 8) *reinterpret_cast<float4*>(red + wave * CW + lane * 4) = sum;
                lds_barrier();
                if (tid < CW)
                    a.part[(f * a.ntiles + tile) * C::CEXPP + c0 + tid] =
                        ((red[tid] + red[CW + tid]) + red[2 * CW + tid]) + red[3 * CW + tid];
            }
        }

        if constexpr (PROJ) {
            // ---- epilogue: + bias (+ residual: the block input at the same pixel), fp32 NHWC store.  Per 16-row
            // tile, the bias and residual operands are loaded (clamped) before its first store: the memory counter
            // retires in order, so a load issued after a store would wait for that store.
            float bias[C::NT_OUT];
#pragma unroll
            for (int nt = 0; nt < C::NT_OUT; ++nt) bias[nt] = a.bproj[nt * 16 + r];   // padded to COUTP
#pragma unroll
            for (int j = 0; j < C::MPW_OUT; ++j) {
                const int mt = wave + 4 * j;
                if (mt >= C::MT_OUT) continue;
                float res[C::RES && L::PRESPLIT ? C::NT_OUT : 1][4];
                if constexpr (C::RES && L::PRESPLIT) {
#pragma unroll
                    for (int nt = 0; nt < C::NT_OUT; ++nt)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int p = min(mt * 16 + g * 4 + i, C::POUT - 1);
                            const int oy = p / C::TW, ox = p - oy * C::TW;
                            const int gy = min(ty0 + oy, a.Ho - 1), gx = min(tx0 + ox, a.Wo - 1);
                            res[nt][i] = Xf[((long long)gy * a.W + gx) * C::CIN + min(nt * 16 + r, C::CIN - 1)];
                        }
                }
#pragma unroll
                for (int nt = 0; nt < C::NT_OUT; ++nt) {
                    const int n = nt * 16 + r;
                    if (n >= C::COUT) continue;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int p = mt * 16 + g * 4 + i;
                        if (p >= C::POUT) continue;
                        const int oy = p / C::TW, ox = p - oy * C::TW;
                        const int gy = ty0 + oy, gx = tx0 + ox;
                        if (gy >= a.Ho || gx >= a.Wo) continue;
                        float v = yacc[j][nt][i] * a.sproj + bias[nt];
                        if constexpr (C::RES) {
                            if constexpr (L::PRESPLIT) v = res[nt][i] + v;
                            else v = Xs[((oy + C::PAD) * C::IW + ox + C::PAD) * C::XS_LD + n] + v;
                        }
                        a.Y[((f * a.Ho + gy) * a.Wo + gx) * C::COUT + n] = v;
                    }
                }
            }
        }
        lds_barrier();   // LDS of this item fully consumed before the next item's tile is written
    }
}

// ------------------------------------------------------------------------------------------------------------
// Squeeze-excite blocks, barrier-free: the workgroup stages the split input tile once; then each of its 4 waves
// owns chunks of 16 expanded channels (chunk c = wave, wave + 4, ...) and runs expand -> depthwise -> D store and
// channel sums for them in its own LDS region.  A wave's LDS traffic is ordered by the hardware (one wave's LDS
// instructions execute in issue order), so no workgroup barrier is needed inside the chunk loop and the 4 waves
// never wait for each other.
constexpr int WCW = 16;            // channels per wave chunk (one MFMA n-tile)
constexpr int WCS_LD = WCW + 4;    // fp32 row stride of the per-wave chunk buffers

template <int CIN_, int CEXP_, int KS_, int S_, int HS_, int TH_, int TW_, int R_>
struct SeCfg {
    static constexpr int CIN = CIN_, CEXP = CEXP_, KS = KS_, S = S_, TH = TH_, TW = TW_, R = R_;
    static constexpr int ACT = HS_ ? ACT_HS : ACT_RELU;
    static constexpr int PAD = (KS - 1) / 2;
    static constexpr int IH = (TH - 1) * S + KS, IW = (TW - 1) * S + KS;
    static constexpr int PIN = IH * IW, POUT = TH * TW;
    static constexpr int CINP = (CIN + 31) / 32 * 32;
    static constexpr int CEXPP = (CEXP + WCW - 1) / WCW * WCW;
    static constexpr int MT_IN = (PIN + 15) / 16, MT_OUT = (POUT + 15) / 16;
    static constexpr int NCH = CEXPP / WCW;
    static constexpr int KST = CINP / 32;
    static constexpr int XH_LD = CINP + 8;
    static constexpr int XH_ROWS = MT_IN * 16;
    static constexpr int ES_W = MT_IN * 16 * WCS_LD;
    static constexpr int DS_W = MT_OUT * 16 * WCS_LD;
    static constexpr int WD_W = (KS * KS + 1) * WCW;
    static constexpr int NSTRIP = TH / R;
    static constexpr int DW_UNITS = (WCW / 4) * TW * NSTRIP;
    static_assert(TH % R == 0, "depthwise strips must tile the output rows");
    static_assert(MT_IN <= 8, "inside mask holds 8 m-tiles");
};
template <typename T, class C> struct SeLayout {
    static constexpr int P = Split<T>::P;
    static constexpr int XS_BYTES = P * C::XH_ROWS * C::XH_LD * 2;
    static constexpr int WAVE_FLOATS = C::ES_W + C::DS_W + C::WD_W;
    static constexpr int BYTES = XS_BYTES + 4 * WAVE_FLOATS * 4;
    static constexpr bool FITS = BYTES <= LDS_BUDGET;
};

__device__ __forceinline__ void wave_lds_fence() { asm volatile("" ::: "memory"); }

template <typename T, class C>
__global__ void __launch_bounds__(IR_THREADS) ir_se_wave_kernel(IrArgs a) {
    typedef Split<T> S;
    typedef typename S::V8 V8;
    typedef SeLayout<T, C> L;
    static_assert(L::FITS, "tile exceeds the LDS budget");
    __shared__ __attribute__((aligned(16))) unsigned char lds_raw[L::BYTES];
    T* Xh = reinterpret_cast<T*>(lds_raw);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r = lane & 15, g = lane >> 4;
    float* Es = reinterpret_cast<float*>(lds_raw + L::XS_BYTES) + wave * L::WAVE_FLOATS;
    float* Ds = Es + C::ES_W;
    float* Wd = Ds + C::DS_W;
    const int tile = blockIdx.x % a.ntiles;
    const long long f = blockIdx.x / a.ntiles;
    const int ty0 = (tile / a.tiles_x) * C::TH, tx0 = (tile % a.tiles_x) * C::TW;
    const int iy0 = ty0 * C::S - C::PAD, ix0 = tx0 * C::S - C::PAD;
    const T* wexp = static_cast<const T*>(a.wexp);
    const float* Xf = a.X + f * a.H * a.W * C::CIN;

    // weights of this wave's next chunk (expand fragments, expand bias, depthwise taps + bias) are fetched into
    // registers one chunk ahead, the first ones while the tile is staged
    constexpr int WD4 = (C::KS * C::KS + 1) * (WCW / 4);   // float4s of a chunk's depthwise table
    constexpr int WDR = (WD4 + 63) / 64;                   // per lane
    V8 ew_n[C::KST][S::P];
    float eb_n = 0.0f;
    float4 wd_n[WDR];
    auto fetch = [&](int c0) {
#pragma unroll
        for (int ks = 0; ks < C::KST; ++ks)
#pragma unroll
            for (int q = 0; q < S::P; ++q)
                ew_n[ks][q] = load_part8<T>(wexp + q * a.wexp_stride + (long long)(c0 + r) * C::CINP + ks * 32 + g * 8);
        eb_n = a.bexp[c0 + r];
#pragma unroll
        for (int k = 0; k < WDR; ++k) {
            const int i = lane + 64 * k;
            const int t = i / (WCW / 4), q = i - t * (WCW / 4);
            wd_n[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (i < WD4) {
                const float* src = t < C::KS * C::KS ? a.wdw + t * C::CEXPP + c0 + q * 4 : a.bdw + c0 + q * 4;
                wd_n[k] = *reinterpret_cast<const float4*>(src);
            }
        }
    };
    if (wave < C::NCH) fetch(wave * WCW);

    // ---- input tile (+halo, zero outside the map and in the K padding) -> LDS, split into the operand parts.
    // All loads are issued (at clamped, always valid addresses) before any is used: the tile is in flight at once.
    {
        constexpr int XQ = C::CINP / 4;
        constexpr int XN = C::XH_ROWS * XQ;
        constexpr int XR = (XN + IR_THREADS - 1) / IR_THREADS;
        float4 xr[XR];
#pragma unroll
        for (int k = 0; k < XR; ++k) {
            const int i = tid + k * IR_THREADS;
            const int row = i / XQ, q = i - row * XQ;
            const int ly = row / C::IW, lx = row - ly * C::IW;
            const int iy = iy0 + ly, ix = ix0 + lx;
            const bool in = i < XN && row < C::PIN && q * 4 < C::CIN && iy >= 0 && iy < a.H && ix >= 0 && ix < a.W;
            const int cy = min(max(iy, 0), a.H - 1), cx = min(max(ix, 0), a.W - 1), cq = min(q, C::CIN / 4 - 1);
            const float4 v = *reinterpret_cast<const float4*>(Xf + ((long long)cy * a.W + cx) * C::CIN + cq * 4);
            xr[k] = in ? v : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int k = 0; k < XR; ++k) {
            const int i = tid + k * IR_THREADS;
            if (i >= XN) continue;
            const int row = i / XQ, q = i - row * XQ;
            const float x[4] = {xr[k].x, xr[k].y, xr[k].z, xr[k].w};
            uint2 four[S::P];
            split4_packed<T>(x, four);
#pragma unroll
            for (int pq = 0; pq < S::P; ++pq)
                *reinterpret_cast<uint2*>(Xh + (pq * C::XH_ROWS + row) * C::XH_LD + q * 4) = four[pq];
        }
    }
    // expand rows of this lane inside the map: bit 4 mt + i
    unsigned inside = 0;
#pragma unroll
    for (int mt = 0; mt < C::MT_IN; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = mt * 16 + g * 4 + i;
            const int ly = row / C::IW, lx = row - ly * C::IW;
            const int iy = iy0 + ly, ix = ix0 + lx;
            if (row < C::PIN && iy >= 0 && iy < a.H && ix >= 0 && ix < a.W) inside |= 1u << (4 * mt + i);
        }
    lds_barrier();   // the only workgroup barrier: the staged tile is read-only from here on

    for (int ch = wave; ch < C::NCH; ch += 4) {
        const int c0 = ch * WCW;
        V8 ew[C::KST][S::P];
#pragma unroll
        for (int ks = 0; ks < C::KST; ++ks)
#pragma unroll
            for (int q = 0; q < S::P; ++q) ew[ks][q] = ew_n[ks][q];
        const float bias = eb_n;
        // depthwise taps and bias of the chunk -> this wave's Wd (layout [t][16] = float4 index i)
#pragma unroll
        for (int k = 0; k < WDR; ++k) {
            const int i = lane + 64 * k;
            if (i < WD4) *reinterpret_cast<float4*>(Wd + i * 4) = wd_n[k];
        }
        if (ch + 4 < C::NCH) fetch(c0 + 4 * WCW);
        // ---- expand: E[rows][16] = act(X . Wexp[c0 .. c0+16) + b) over all input-tile rows
#pragma unroll
        for (int mt = 0; mt < C::MT_IN; ++mt) {
            f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < C::KST; ++ks) {
                V8 ap[S::P];
#pragma unroll
                for (int q = 0; q < S::P; ++q)
                    ap[q] = *reinterpret_cast<const V8*>(Xh + (q * C::XH_ROWS + mt * 16 + r) * C::XH_LD + ks * 32 + g * 8);
                acc = mfma_split<T>(ap, ew[ks], acc);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float v = 0.0f;
                if (inside & (1u << (4 * mt + i))) v = apply_act_nb(acc[i] * a.sexp + bias, C::ACT);
                Es[(mt * 16 + g * 4 + i) * WCS_LD + r] = v;
            }
        }
        wave_lds_fence();
        // ---- depthwise: unit = (4 channels, tile column, R rows); fma chain over (dy, dx) from +0, padding taps
        // read the staged zeros (the same values as skipping them)
        for (int u = lane; u < C::DW_UNITS; u += 64) {
            const int cgi = u % (WCW / 4), rest = u / (WCW / 4);
            const int ox = rest % C::TW, oy0 = (rest / C::TW) * C::R;
            const float* src = Es + (oy0 * C::S * C::IW + ox * C::S) * WCS_LD + cgi * 4;
            float4 acc[C::R];
#pragma unroll
            for (int rr = 0; rr < C::R; ++rr) acc[rr] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 1
            for (int dy = 0; dy < C::KS; ++dy) {
#pragma unroll
                for (int dx = 0; dx < C::KS; ++dx) {
                    const float4 w = *reinterpret_cast<const float4*>(Wd + (dy * C::KS + dx) * WCW + cgi * 4);
#pragma unroll
                    for (int rr = 0; rr < C::R; ++rr) {
                        const float4 x =
                            *reinterpret_cast<const float4*>(src + ((rr * C::S + dy) * C::IW + dx) * WCS_LD);
                        acc[rr].x = __builtin_fmaf(x.x, w.x, acc[rr].x);
                        acc[rr].y = __builtin_fmaf(x.y, w.y, acc[rr].y);
                        acc[rr].z = __builtin_fmaf(x.z, w.z, acc[rr].z);
                        acc[rr].w = __builtin_fmaf(x.w, w.w, acc[rr].w);
                    }
                }
            }
            const float4 bb = *reinterpret_cast<const float4*>(Wd + C::KS * C::KS * WCW + cgi * 4);
#pragma unroll
            for (int rr = 0; rr < C::R; ++rr) {
                const int oy = oy0 + rr;
                float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (ty0 + oy < a.Ho && tx0 + ox < a.Wo) {
                    v.x = apply_act_nb(acc[rr].x + bb.x, C::ACT);
                    v.y = apply_act_nb(acc[rr].y + bb.y, C::ACT);
                    v.z = apply_act_nb(acc[rr].z + bb.z, C::ACT);
                    v.w = apply_act_nb(acc[rr].w + bb.w, C::ACT);
                }
                *reinterpret_cast<float4*>(Ds + (oy * C::TW + ox) * WCS_LD + cgi * 4) = v;
            }
        }
        wave_lds_fence();
        // ---- D chunk -> HBM and the tile's channel sums: lane (pixel group pg, 4 channels q) sums pixels
        // pg, pg + 16, ... in order; lanes with equal q are combined by an xor tree (a fixed, frame-local order)
        {
            const int q = lane & 3, pg = lane >> 2;
            float4 sum = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            for (int p = pg; p < C::POUT; p += 16) {
                const int oy = p / C::TW, ox = p - oy * C::TW;
                const int gy = ty0 + oy, gx = tx0 + ox;
                if (gy < a.Ho && gx < a.Wo) {
                    const float4 v = *reinterpret_cast<const float4*>(Ds + p * WCS_LD + q * 4);
                    if (c0 + q * 4 < C::CEXP)
                        *reinterpret_cast<float4*>(a.D + ((f * a.Ho + gy) * a.Wo + gx) * C::CEXP + c0 + q * 4) = v;
                    sum.x = sum.x + v.x; sum.y = sum.y + v.y; sum.z = sum.z + v.z; sum.w = sum.w + v.w;
                }
            }
#pragma unroll
            for (int m = 4; m < 64; m <<= 1) {
                sum.x = sum.x + __shfl_xor(sum.x, m);
                sum.y = sum.y + __shfl_xor(sum.y, m);
                sum.z = sum.z + __shfl_xor(sum.z, m);
                sum.w = sum.w + __shfl_xor(sum.w, m);
            }
            if (lane < 4)
                *reinterpret_cast<float4*>(a.part + (f * a.ntiles + tile) * C::CEXPP + c0 + lane * 4) = sum;
        }
        wave_lds_fence();
    }
}

// SE blocks that take the barrier-free kernel (fp16 tier; a type whose staged tile does not fit keeps the
// chunk-synchronous kernel)
//                 cin cexp k  s hs TH TW R
typedef SeCfg<40, 120, 5, 1, 0, 4, 8, 2> W5;       // 23x40 (b5, b6)
typedef SeCfg<80, 480, 3, 1, 1, 3, 10, 1> W11;     // 12x20
typedef SeCfg<112, 672, 3, 1, 1, 3, 10, 1> W12;    // 12x20
typedef SeCfg<160, 960, 5, 1, 1, 3, 5, 1> W14;     // 6x10 (b14, b15)

// pooled[f][c] = (sum over tiles t in order of part[f][t][c]) / (float)hw
__global__ void __launch_bounds__(256)
se_reduce_kernel(const float* __restrict__ part, int ntiles, int cexpp, int cexp, float hw, float* __restrict__ pooled,
                 int F) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)F * cexp) return;
    const int c = int(idx % cexp);
    const long long f = idx / cexp;
    const float* p = part + f * ntiles * cexpp + c;
    float s = p[0];
    for (int t = 1; t < ntiles; ++t) s = s + p[(long long)t * cexpp];
    pooled[idx] = s / hw;
}

template <class C> IrShape shape_of() {
    IrShape s;
    s.cin = C::CIN; s.cexp = C::CEXP; s.cout = C::COUT; s.k = C::KS; s.stride = C::S; s.se = C::SE;
    s.hs = C::ACT == ACT_HS; s.th = C::TH; s.tw = C::TW; s.cinp = C::CINP; s.cexpp = C::CEXPP; s.coutp = C::COUTP;
    return s;
}
// the barrier-free kernel's shape, with the block's cout / padding taken from its chunk-synchronous twin
template <class W, class C> IrShape shape_of_wave() {
    IrShape s = shape_of<C>();
    s.th = W::TH; s.tw = W::TW; s.cexpp = W::CEXPP;
    return s;
}

template <typename T, class W> void launch_wave(const IrArgs& a, int F, hipStream_t s) {
    const int ty = (a.Ho + W::TH - 1) / W::TH, tx = (a.Wo + W::TW - 1) / W::TW;
    if (tx != a.tiles_x || ty * tx != a.ntiles || a.frames != F) throw std::runtime_error("ir_se_wave: tile grid mismatch");
    hipLaunchKernelGGL((ir_se_wave_kernel<T, W>), dim3((unsigned)((long long)a.ntiles * F)), dim3(IR_THREADS), 0, s, a);
}

template <typename T, class C> void launch_cfg(const IrArgs& a, int F, hipStream_t s) {
    const int ty = (a.Ho + C::TH - 1) / C::TH, tx = (a.Wo + C::TW - 1) / C::TW;
    if (tx != a.tiles_x || ty * tx != a.ntiles || a.frames != F) throw std::runtime_error("ir_block: tile grid mismatch");
    // persistent workgroups: as many as the device holds at once (per-instantiation occupancy, cached)
    const long long items = (long long)a.ntiles * F;
    if (!C::PERSIST) {   // one workgroup per item
        hipLaunchKernelGGL((ir_block_kernel<T, C>), dim3((unsigned)items), dim3(IR_THREADS), 0, s, a);
        return;
    }
    static const int resident = [] {
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, ir_block_kernel<T, C>, IR_THREADS, 0) != hipSuccess)
            throw std::runtime_error("ir_block: cannot query the device occupancy");
        return std::max(1, cus) * std::max(1, per_cu);
    }();
    const int grid = (int)std::min<long long>(items, resident);
    hipLaunchKernelGGL((ir_block_kernel<T, C>), dim3(grid), dim3(IR_THREADS), 0, s, a);
}

}  // namespace

template <typename T> IrShape ir_shape_t(int block) {
    switch (block) {
    case 0: return shape_of<B1>();
    case 1: return shape_of<B2>();
    case 2: return shape_of<B3>();
    case 3: return shape_of<B4>();
    case 4: case 5: return SeLayout<T, W5>::FITS ? shape_of_wave<W5, B5>() : shape_of<B5>();
    case 6: return shape_of<B7>();
    case 7: return shape_of<B8>();
    case 8: case 9: return shape_of<B9>();
    case 10: return SeLayout<T, W11>::FITS ? shape_of_wave<W11, B11>() : shape_of<B11>();
    case 11: return SeLayout<T, W12>::FITS ? shape_of_wave<W12, B12>() : shape_of<B12>();
    case 12: return shape_of<B13>();
    case 13: case 14: return SeLayout<T, W14>::FITS ? shape_of_wave<W14, B14>() : shape_of<B14>();
    }
    throw std::runtime_error("ir_shape: block index out of range");
}
IrShape ir_shape(int block, bool bf16_tier) {
    IrShape s;
    if (strip_kernels_enabled() && ir_strip_shape(block, bf16_tier, &s)) return s;
    return bf16_tier ? ir_shape_t<bf16>(block) : ir_shape_t<f16>(block);
}

template <typename T, class W, class C> void launch_se(const IrArgs& a, int F, hipStream_t s) {
    if constexpr (SeLayout<T, W>::FITS) launch_wave<T, W>(a, F, s);
    else launch_cfg<T, C>(a, F, s);
}

template <typename T> void launch_ir_block(int block, const IrArgs& a, int F, hipStream_t s) {
    if (F <= 0) return;
    if (strip_kernels_enabled() && launch_ir_strip<T>(block, a, F, s)) return;
    switch (block) {
    case 0: launch_cfg<T, B1>(a, F, s); break;
    case 1: launch_cfg<T, B2>(a, F, s); break;
    case 2: launch_cfg<T, B3>(a, F, s); break;
    case 3: launch_cfg<T, B4>(a, F, s); break;
    case 4: case 5: launch_se<T, W5, B5>(a, F, s); break;
    case 6: launch_cfg<T, B7>(a, F, s); break;
    case 7: launch_cfg<T, B8>(a, F, s); break;
    case 8: case 9: launch_cfg<T, B9>(a, F, s); break;
    case 10: launch_se<T, W11, B11>(a, F, s); break;
    case 11: launch_se<T, W12, B12>(a, F, s); break;
    case 12: launch_cfg<T, B13>(a, F, s); break;
    case 13: case 14: launch_se<T, W14, B14>(a, F, s); break;
    default: throw std::runtime_error("launch_ir_block: block index out of range");
    }
}
template void launch_ir_block<f16>(int, const IrArgs&, int, hipStream_t);
template void launch_ir_block<bf16>(int, const IrArgs&, int, hipStream_t);

void launch_se_reduce(const float* part, int ntiles, int cexpp, int cexp, int hw, float* pooled, int F,
                      hipStream_t s) {
    const long long n = (long long)F * cexp;
    hipLaunchKernelGGL(se_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, part, ntiles, cexpp, cexp,
                       float(hw), pooled, F);
}

}  // namespace shv
