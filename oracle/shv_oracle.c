/* TEST INFRASTRUCTURE ONLY (see shv_oracle.h).  Scalar restatement of the reference CPU engine, exact tier.
 *
 * Parity status of every function is pinned by tests/test_oracle.py:
 *   - whole forward (orc_encode_frame, orc_classify) and every dumped stage: bitwise against the reference CPU
 *     engine compiled from /root/reference (oracle/_ref), through committed golden fixtures;
 *   - orc_gemm: brute-force float64 bound + the K-block order (a dropped block or a transposed operand fails);
 *   - orc_exp / orc_silu: against float64 exp within 2 ulp;
 *   - orc_delta_rule: against a float64 recurrence and closed forms (beta = 0 gives o = 0; one token gives
 *     o = beta (q.k) v).
 * Arithmetic order follows engine/model/isa_impl.hpp (cited per function); weight folding follows
 * engine/model/runtime.cpp. */
#define _GNU_SOURCE
#include "shv_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static __thread char g_err[512];
static void set_err(const char* m) { snprintf(g_err, sizeof g_err, "%s", m); }
const char* orc_last_error(void) { return g_err; }

#define T_TOK 321
#define DM 384
#define GP 2316   /* fused GDN projection width (q 384 | k 384 | v 768 | g 768 | a 6 | b 6) */
#define SP 1068   /* fused SISA projection width (K 384 | V 384 | B 192 | theta 96 | alpha 6 | forget 6) */

/* ------------------------------------------------------------------------------------------ scalar math */
/* exp with the Cephes expf polynomial and the reference's range clamp / rounding trick (isa_impl.hpp:159-177) */
float orc_exp(float x) {
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
    const int ni = (int)n;
    const unsigned int bits = (unsigned int)(ni + 127) << 23;
    float two;
    memcpy(&two, &bits, 4);
    return p * two;
}
float orc_silu(float x) { return x / (1.0f + orc_exp(0.0f - x)); }
static float clamp06(float x) {
    float t = x + 3.0f;
    t = t > 0.0f ? t : 0.0f;
    return t < 6.0f ? t : 6.0f;
}
float orc_hswish(float x) { return (x * clamp06(x)) / 6.0f; }
static float hsig(float x) { return clamp06(x) / 6.0f; }
static float relu(float x) { return x > 0.0f ? x : 0.0f; }
static float softplus_f(float x) { return x > 20.0f ? x : log1pf(expf(x)); }
static float logsigmoid_f(float x) { return (x < 0.0f ? x : 0.0f) - log1pf(expf(-fabsf(x))); }

/* 16-lane reduction tree of the reference vector code (vsum, isa_impl.hpp:45-53 / 109-115) */
static float tree16(const float* l) {
    float s8[8], s4[4];
    for (int i = 0; i < 8; ++i) s8[i] = l[i] + l[i + 8];
    for (int i = 0; i < 4; ++i) s4[i] = s8[i] + s8[i + 4];
    return (s4[0] + s4[2]) + (s4[1] + s4[3]);
}
/* sum_i x[i]*y[i], n % 16 == 0, lane l accumulates i = l, l+16, ... (first product unfused), then tree16 */
static float lanes_dot(const float* x, const float* y, int n) {
    float acc[16];
    for (int l = 0; l < 16; ++l) acc[l] = x[l] * y[l];
    for (int i = 16; i < n; i += 16)
        for (int l = 0; l < 16; ++l) acc[l] = __builtin_fmaf(x[i + l], y[i + l], acc[l]);
    return tree16(acc);
}

/* ------------------------------------------------------------------------------------------ GEMM */
typedef struct {
    int K, N;
    float* wt;    /* [K][N] (transposed PyTorch weight) */
    float* bias;  /* [N] or NULL */
} Lin;

/* One row of sum_k a[k] W[n][k] for all n: K blocks of 64, fma chain from +0 inside a block, block sums added
 * left to right (isa_impl.hpp:188-198, 289-317). */
static void row_dot(const float* a, const Lin* L, float* tot, float* blk) {
    const int K = L->K, N = L->N;
    for (int k0 = 0; k0 < K; k0 += 64) {
        const int k1 = k0 + 64 < K ? k0 + 64 : K;
        for (int n = 0; n < N; ++n) blk[n] = 0.0f;
        for (int k = k0; k < k1; ++k) {
            const float av = a[k];
            const float* w = L->wt + (size_t)k * N;
            for (int n = 0; n < N; ++n) blk[n] = __builtin_fmaf(av, w[n], blk[n]);
        }
        if (k0 == 0) memcpy(tot, blk, sizeof(float) * (size_t)N);
        else
            for (int n = 0; n < N; ++n) tot[n] = tot[n] + blk[n];
    }
}

/* epilogue of one value (isa_impl.hpp:318-345) */
static float epi_apply(int epi, float v, float b, float c_old, float r) {
    switch (epi) {
    case ORC_STORE: return v + b;
    case ORC_RELU: return relu(v + b);
    case ORC_HS: return orc_hswish(v + b);
    case ORC_HSIG: return hsig(v + b);
    case ORC_SILU: return orc_silu(v + b);
    case ORC_RES: return (v + b) + r;
    case ORC_ACC: return c_old + v;
    case ORC_ACC_DIV2: return c_old + v / 1.41421356237309515f;
    default: return v;
    }
}

static void lin_gemm(const float* A, int lda, int M, const Lin* L, float* C, int ldc, int epi, const float* R,
                     int ldr) {
    float* tot = (float*)malloc(sizeof(float) * (size_t)L->N * 2);
    float* blk = tot + L->N;
    for (int m = 0; m < M; ++m) {
        row_dot(A + (size_t)m * lda, L, tot, blk);
        float* c = C + (size_t)m * ldc;
        for (int n = 0; n < L->N; ++n) {
            const int has_b = L->bias != NULL && epi != ORC_ACC && epi != ORC_ACC_DIV2;
            const float b = has_b ? L->bias[n] : 0.0f;
            if (epi == ORC_STORE && !has_b) { c[n] = tot[n]; continue; }
            c[n] = epi_apply(epi, tot[n], b, c[n], R ? R[(size_t)m * ldr + n] : 0.0f);
        }
    }
    free(tot);
}
/* SwiGLU pair: out[m][j] = silu(gate_j) * up_j (isa_impl.hpp:309-317) */
static void swiglu_gemm(const float* A, int lda, int M, const Lin* G, const Lin* U, float* C, int ldc) {
    const int N = G->N;
    float* g = (float*)malloc(sizeof(float) * (size_t)N * 3);
    float* u = g + N;
    float* blk = u + N;
    for (int m = 0; m < M; ++m) {
        row_dot(A + (size_t)m * lda, G, g, blk);
        row_dot(A + (size_t)m * lda, U, u, blk);
        for (int n = 0; n < N; ++n) C[(size_t)m * ldc + n] = orc_silu(g[n]) * u[n];
    }
    free(g);
}

static void lin_from(Lin* L, const float* W, int N, int K, const float* bias) {
    L->K = K;
    L->N = N;
    L->wt = (float*)malloc(sizeof(float) * (size_t)K * N);
    for (int n = 0; n < N; ++n)
        for (int k = 0; k < K; ++k) L->wt[(size_t)k * N + n] = W[(size_t)n * K + k];
    L->bias = NULL;
    if (bias) {
        L->bias = (float*)malloc(sizeof(float) * (size_t)N);
        memcpy(L->bias, bias, sizeof(float) * (size_t)N);
    }
}
static void lin_free(Lin* L) { free(L->wt); free(L->bias); L->wt = L->bias = NULL; }

void orc_gemm(const float* A, int lda, int M, const float* W, const float* bias, int N, int K, float* C, int ldc,
              int epi, const float* R, int ldr) {
    if (epi == ORC_SWIGLU) {
        const int F = N / 2;
        float* gw = (float*)malloc(sizeof(float) * (size_t)F * K);
        float* uw = (float*)malloc(sizeof(float) * (size_t)F * K);
        for (int j = 0; j < F; ++j) {
            memcpy(gw + (size_t)j * K, W + (size_t)(2 * j) * K, sizeof(float) * (size_t)K);
            memcpy(uw + (size_t)j * K, W + (size_t)(2 * j + 1) * K, sizeof(float) * (size_t)K);
        }
        Lin G, U;
        lin_from(&G, gw, F, K, NULL);
        lin_from(&U, uw, F, K, NULL);
        swiglu_gemm(A, lda, M, &G, &U, C, ldc);
        lin_free(&G);
        lin_free(&U);
        free(gw);
        free(uw);
        return;
    }
    Lin L;
    lin_from(&L, W, N, K, bias);
    lin_gemm(A, lda, M, &L, C, ldc, epi, R, ldr);
    lin_free(&L);
}

/* ------------------------------------------------------------------------------------------ model */
typedef struct {
    int H, W, Ho, Wo, cin, cexp, cout, k, s, p, hs, has_expand, has_se, residual, csq;
    Lin expand, se1, se2, project;
    float* dw_w;  /* [k*k][cexp] */
    float* dw_b;  /* [cexp] */
} Blk;

typedef struct {
    float norm_w[DM], ffn_norm_w[DM];
    Lin in;                     /* N = 2316 */
    float conv_w[4][1536], conv_b[1536];
    float neg_rate[6], dt_bias[6];
    float o_norm_w[128];
    Lin out, gate, up, down;
    int repeats;
} Gdn;

struct orc_model {
    float lut[3][256];
    float stem_w[27][16], stem_b[16];
    Blk blk[15];
    Lin last, proj;
    float* pos;  /* [320][384] */
    float readout[DM];
    Gdn gdn[2];
    float s_attn_norm_w[DM], s_ffn_norm_w[DM];
    Lin s_in, s_q, s_c, s_o, s_gate, s_up, s_down;
    float lam[6];
    float final_norm_w[DM];
    Lin head0;
    float head2_w[128], head2_b;
};

typedef struct {
    char* name;
    int rank, dims[8];
    size_t n;
    float* data;
} Tns;
typedef struct {
    Tns* t;
    int n;
} File;

static void file_free(File* f) {
    for (int i = 0; i < f->n; ++i) { free(f->t[i].name); free(f->t[i].data); }
    free(f->t);
}
static int file_read(const char* path, File* f) {
    FILE* fp = fopen(path, "rb");
    memset(f, 0, sizeof *f);
    if (!fp) { set_err("cannot open weights"); return -1; }
    char magic[8];
    uint32_t count = 0;
    if (fread(magic, 1, 8, fp) != 8 || memcmp(magic, "SHLDV001", 8) || fread(&count, 4, 1, fp) != 1 || !count ||
        count > 10000) {
        fclose(fp);
        set_err("not a SHLDV001 file");
        return -1;
    }
    f->t = (Tns*)calloc(count, sizeof(Tns));
    for (uint32_t i = 0; i < count; ++i) {
        Tns* t = &f->t[i];
        uint32_t nl = 0, rank = 0;
        uint64_t e = 0;
        if (fread(&nl, 4, 1, fp) != 1 || nl == 0 || nl > 4096) goto bad;
        t->name = (char*)calloc(nl + 1, 1);
        f->n = (int)i + 1;
        if (fread(t->name, 1, nl, fp) != nl || fread(&rank, 4, 1, fp) != 1 || rank > 8) goto bad;
        t->rank = (int)rank;
        for (uint32_t d = 0; d < rank; ++d) {
            uint32_t dim;
            if (fread(&dim, 4, 1, fp) != 1) goto bad;
            t->dims[d] = (int)dim;
        }
        if (fread(&e, 8, 1, fp) != 1 || e > 100000000u) goto bad;
        t->n = (size_t)e;
        t->data = (float*)malloc(sizeof(float) * (t->n ? t->n : 1));
        if (fread(t->data, 4, t->n, fp) != t->n) goto bad;
    }
    fclose(fp);
    return 0;
bad:
    fclose(fp);
    file_free(f);
    set_err("truncated or invalid weight file");
    return -1;
}
static const float* need(const File* f, const char* name, size_t n) {
    for (int i = 0; i < f->n; ++i)
        if (!strcmp(f->t[i].name, name)) {
            if (f->t[i].n != n) return NULL;
            return f->t[i].data;
        }
    return NULL;
}

/* BatchNorm (eps 1e-3) folded in double (runtime.cpp:188-203): w' = w*s, b' = beta - mean*s, s = g/sqrt(var+eps) */
static int fold(const File* f, const char* conv, const char* bn, int out, int per, float* wf, float* bf) {
    char n[128];
    const float* w = need(f, conv, (size_t)out * per);
    snprintf(n, sizeof n, "%s.weight", bn);
    const float* g = need(f, n, (size_t)out);
    snprintf(n, sizeof n, "%s.bias", bn);
    const float* b = need(f, n, (size_t)out);
    snprintf(n, sizeof n, "%s.running_mean", bn);
    const float* mu = need(f, n, (size_t)out);
    snprintf(n, sizeof n, "%s.running_var", bn);
    const float* var = need(f, n, (size_t)out);
    if (!w || !g || !b || !mu || !var) return -1;
    for (int o = 0; o < out; ++o) {
        const double s = (double)g[o] / sqrt((double)var[o] + 1e-3);
        for (int e = 0; e < per; ++e) wf[(size_t)o * per + e] = (float)((double)w[(size_t)o * per + e] * s);
        bf[o] = (float)((double)b[o] - (double)mu[o] * s);
    }
    return 0;
}

static const int kB[15][6] = { /* in, k, exp, out, se, hardswish; stride below */
    {16, 3, 16, 16, 0, 0},   {16, 3, 64, 24, 0, 0},   {24, 3, 72, 24, 0, 0},   {24, 5, 72, 40, 1, 0},
    {40, 5, 120, 40, 1, 0},  {40, 5, 120, 40, 1, 0},  {40, 3, 240, 80, 0, 1},  {80, 3, 200, 80, 0, 1},
    {80, 3, 184, 80, 0, 1},  {80, 3, 184, 80, 0, 1},  {80, 3, 480, 112, 1, 1}, {112, 3, 672, 112, 1, 1},
    {112, 5, 672, 160, 1, 1}, {160, 5, 960, 160, 1, 1}, {160, 5, 960, 160, 1, 1}};
static const int kStride[15] = {1, 2, 1, 2, 1, 1, 2, 1, 1, 1, 1, 1, 2, 1, 1};

#define NEED(var, name, count)                                 \
    const float* var = need(&f, name, (size_t)(count));        \
    if (!var) { set_err("missing or misshapen tensor " name); goto fail; }

static int need_lin(const File* f, Lin* L, const char* name, int N, int K, const float* bias) {
    const float* w = need(f, name, (size_t)N * K);
    if (!w) return -1;
    lin_from(L, w, N, K, bias);
    return 0;
}

orc_model* orc_load(const char* path) {
    File f;
    if (file_read(path, &f)) return NULL;
    orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
    char n[128], n2[128];
    float* wf = (float*)malloc(sizeof(float) * 960 * 960);
    float* bf = (float*)malloc(sizeof(float) * 960);
    /* normalisation LUT (runtime.cpp:224-230): ((v / 255) - mean) / std in float32 */
    {
        const float mean[3] = {0.485f, 0.456f, 0.406f}, stdv[3] = {0.229f, 0.224f, 0.225f};
        for (int c = 0; c < 3; ++c)
            for (int v = 0; v < 256; ++v) {
                volatile float x = (float)v / 255.0f;
                volatile float y = x - mean[c];
                m->lut[c][v] = y / stdv[c];
            }
    }
    if (fold(&f, "cnn.0.0.weight", "cnn.0.1", 16, 27, wf, bf)) { set_err("stem"); goto fail; }
    for (int o = 0; o < 16; ++o) {
        for (int c = 0; c < 3; ++c)
            for (int dy = 0; dy < 3; ++dy)
                for (int dx = 0; dx < 3; ++dx) m->stem_w[(dy * 3 + dx) * 3 + c][o] = wf[o * 27 + c * 9 + dy * 3 + dx];
        m->stem_b[o] = bf[o];
    }
    {
        int H = 90, W = 160;
        for (int i = 0; i < 15; ++i) {
            Blk* B = &m->blk[i];
            B->cin = kB[i][0]; B->k = kB[i][1]; B->cexp = kB[i][2]; B->cout = kB[i][3];
            B->has_se = kB[i][4]; B->hs = kB[i][5]; B->s = kStride[i]; B->p = (B->k - 1) / 2;
            B->H = H; B->W = W;
            B->Ho = (H + 2 * B->p - B->k) / B->s + 1;
            B->Wo = (W + 2 * B->p - B->k) / B->s + 1;
            B->has_expand = B->cexp != B->cin;
            B->residual = B->s == 1 && B->cin == B->cout;
            int j = 0;
            if (B->has_expand) {
                snprintf(n, sizeof n, "cnn.%d.block.%d.0.weight", i + 1, j);
                snprintf(n2, sizeof n2, "cnn.%d.block.%d.1", i + 1, j);
                if (fold(&f, n, n2, B->cexp, B->cin, wf, bf)) { set_err("expand"); goto fail; }
                lin_from(&B->expand, wf, B->cexp, B->cin, bf);
                ++j;
            }
            snprintf(n, sizeof n, "cnn.%d.block.%d.0.weight", i + 1, j);
            snprintf(n2, sizeof n2, "cnn.%d.block.%d.1", i + 1, j);
            if (fold(&f, n, n2, B->cexp, B->k * B->k, wf, bf)) { set_err("depthwise"); goto fail; }
            B->dw_w = (float*)malloc(sizeof(float) * (size_t)B->k * B->k * B->cexp);
            B->dw_b = (float*)malloc(sizeof(float) * (size_t)B->cexp);
            for (int c = 0; c < B->cexp; ++c) {
                for (int t = 0; t < B->k * B->k; ++t) B->dw_w[(size_t)t * B->cexp + c] = wf[(size_t)c * B->k * B->k + t];
                B->dw_b[c] = bf[c];
            }
            ++j;
            if (B->has_se) {
                int sq = (B->cexp / 4 + 4) / 8 * 8;
                if (sq < 8) sq = 8;
                if (10 * sq < 9 * (B->cexp / 4)) sq += 8;
                B->csq = sq;
                snprintf(n, sizeof n, "cnn.%d.block.%d.fc1.bias", i + 1, j);
                const float* b1 = need(&f, n, (size_t)sq);
                snprintf(n, sizeof n, "cnn.%d.block.%d.fc2.bias", i + 1, j);
                const float* b2 = need(&f, n, (size_t)B->cexp);
                snprintf(n, sizeof n, "cnn.%d.block.%d.fc1.weight", i + 1, j);
                snprintf(n2, sizeof n2, "cnn.%d.block.%d.fc2.weight", i + 1, j);
                if (!b1 || !b2 || need_lin(&f, &B->se1, n, sq, B->cexp, b1) ||
                    need_lin(&f, &B->se2, n2, B->cexp, sq, b2)) { set_err("SE"); goto fail; }
                ++j;
            }
            snprintf(n, sizeof n, "cnn.%d.block.%d.0.weight", i + 1, j);
            snprintf(n2, sizeof n2, "cnn.%d.block.%d.1", i + 1, j);
            if (fold(&f, n, n2, B->cout, B->cexp, wf, bf)) { set_err("project"); goto fail; }
            lin_from(&B->project, wf, B->cout, B->cexp, bf);
            H = B->Ho;
            W = B->Wo;
        }
    }
    if (fold(&f, "cnn.16.0.weight", "cnn.16.1", 960, 160, wf, bf)) { set_err("last conv"); goto fail; }
    lin_from(&m->last, wf, 960, 160, bf);
    if (need_lin(&f, &m->proj, "projection.weight", DM, 960, NULL)) { set_err("projection"); goto fail; }
    {
        NEED(te, "time_embedding", 20 * DM);
        NEED(re, "row_embedding", 4 * DM);
        NEED(ce, "col_embedding", 4 * DM);
        NEED(ro, "readout", DM);
        /* position table (runtime.cpp:332-340): (time + row) + col, float32, no contraction */
        m->pos = (float*)malloc(sizeof(float) * 320 * DM);
        for (int t = 0; t < 20; ++t)
            for (int r = 0; r < 4; ++r)
                for (int c = 0; c < 4; ++c)
                    for (int d = 0; d < DM; ++d) {
                        volatile float a = te[t * DM + d] + re[r * DM + d];
                        m->pos[((size_t)t * 16 + r * 4 + c) * DM + d] = a + ce[c * DM + d];
                    }
        memcpy(m->readout, ro, sizeof(float) * DM);
    }
    for (int g = 0; g < 2; ++g) {
        Gdn* G = &m->gdn[g];
        const char* p = g == 0 ? "gdn_a" : "gdn_b";
        G->repeats = g == 0 ? 1 : 2;
        const float* v;
        snprintf(n, sizeof n, "%s.norm.weight", p);
        if (!(v = need(&f, n, DM))) goto fail_t;
        memcpy(G->norm_w, v, sizeof(float) * DM);
        snprintf(n, sizeof n, "%s.ffn_norm.weight", p);
        if (!(v = need(&f, n, DM))) goto fail_t;
        memcpy(G->ffn_norm_w, v, sizeof(float) * DM);
        float* w = (float*)calloc((size_t)GP * DM, sizeof(float));
        const char* parts[6] = {"q_proj", "k_proj", "v_proj", "g_proj", "a_proj", "b_proj"};
        const int rows[6] = {384, 384, 768, 768, 6, 6}, at[6] = {0, 384, 768, 1536, 2304, 2310};
        for (int i = 0; i < 6; ++i) {
            snprintf(n, sizeof n, "%s.mixer.%s.weight", p, parts[i]);
            if (!(v = need(&f, n, (size_t)rows[i] * DM))) { free(w); goto fail_t; }
            memcpy(w + (size_t)at[i] * DM, v, sizeof(float) * rows[i] * DM);
        }
        lin_from(&G->in, w, GP, DM, NULL);
        free(w);
        const char* convs[3] = {"q_conv1d", "k_conv1d", "v_conv1d"};
        const int widths[3] = {384, 384, 768}, offs[3] = {0, 384, 768};
        for (int i = 0; i < 3; ++i) {
            snprintf(n, sizeof n, "%s.mixer.%s.weight", p, convs[i]);
            const float* cw = need(&f, n, (size_t)widths[i] * 4);
            snprintf(n, sizeof n, "%s.mixer.%s.bias", p, convs[i]);
            const float* cb = need(&f, n, (size_t)widths[i]);
            if (!cw || !cb) goto fail_t;
            for (int c = 0; c < widths[i]; ++c) {
                for (int j = 0; j < 4; ++j) G->conv_w[j][offs[i] + c] = cw[c * 4 + j];
                G->conv_b[offs[i] + c] = cb[c];
            }
        }
        snprintf(n, sizeof n, "%s.mixer.A_log", p);
        const float* al = need(&f, n, 6);
        snprintf(n, sizeof n, "%s.mixer.dt_bias", p);
        const float* dt = need(&f, n, 6);
        if (!al || !dt) goto fail_t;
        for (int h = 0; h < 6; ++h) { G->neg_rate[h] = -expf(al[h]); G->dt_bias[h] = dt[h]; }
        snprintf(n, sizeof n, "%s.mixer.o_norm.weight", p);
        if (!(v = need(&f, n, 128))) goto fail_t;
        memcpy(G->o_norm_w, v, sizeof(float) * 128);
        snprintf(n, sizeof n, "%s.mixer.o_proj.weight", p);
        if (need_lin(&f, &G->out, n, DM, 768, NULL)) goto fail_t;
        snprintf(n, sizeof n, "%s.ffn.gate.weight", p);
        if (need_lin(&f, &G->gate, n, 960, DM, NULL)) goto fail_t;
        snprintf(n, sizeof n, "%s.ffn.up.weight", p);
        if (need_lin(&f, &G->up, n, 960, DM, NULL)) goto fail_t;
        snprintf(n, sizeof n, "%s.ffn.down.weight", p);
        if (need_lin(&f, &G->down, n, DM, 960, NULL)) goto fail_t;
    }
    {
        NEED(an, "sisa.attn_norm.weight", DM);
        NEED(fn, "sisa.ffn_norm.weight", DM);
        memcpy(m->s_attn_norm_w, an, sizeof(float) * DM);
        memcpy(m->s_ffn_norm_w, fn, sizeof(float) * DM);
        float* w = (float*)calloc((size_t)SP * DM, sizeof(float));
        float b[SP];
        memset(b, 0, sizeof b);
        const char* parts[6] = {"W_K", "W_V", "W_B", "theta_proj", "alpha_proj", "forget_proj"};
        const int rows[6] = {384, 384, 192, 96, 6, 6}, at[6] = {0, 384, 768, 960, 1056, 1062};
        for (int i = 0; i < 6; ++i) {
            snprintf(n, sizeof n, "sisa.attn.%s.weight", parts[i]);
            const float* v = need(&f, n, (size_t)rows[i] * DM);
            if (!v) { free(w); goto fail_t; }
            memcpy(w + (size_t)at[i] * DM, v, sizeof(float) * rows[i] * DM);
        }
        NEED(ab, "sisa.attn.alpha_proj.bias", 6);
        NEED(fb, "sisa.attn.forget_proj.bias", 6);
        memcpy(b + 1056, ab, sizeof(float) * 6);
        memcpy(b + 1062, fb, sizeof(float) * 6);
        lin_from(&m->s_in, w, SP, DM, b);
        free(w);
        if (need_lin(&f, &m->s_q, "sisa.attn.W_Q.weight", DM, DM, NULL) ||
            need_lin(&f, &m->s_c, "sisa.attn.W_C.weight", 192, DM, NULL) ||
            need_lin(&f, &m->s_o, "sisa.attn.W_O.weight", DM, DM, NULL) ||
            need_lin(&f, &m->s_gate, "sisa.ffn.w_gate.weight", 960, DM, NULL) ||
            need_lin(&f, &m->s_up, "sisa.ffn.w_up.weight", 960, DM, NULL) ||
            need_lin(&f, &m->s_down, "sisa.ffn.w_down.weight", DM, 960, NULL))
            goto fail_t;
        NEED(lr, "sisa.attn.lambda_raw", 6);
        for (int h = 0; h < 6; ++h) m->lam[h] = softplus_f(lr[h]);
        NEED(fw, "final_norm.weight", DM);
        memcpy(m->final_norm_w, fw, sizeof(float) * DM);
        NEED(h0b, "head.0.bias", 128);
        if (need_lin(&f, &m->head0, "head.0.weight", 128, DM, h0b)) goto fail_t;
        NEED(h2w, "head.2.weight", 128);
        NEED(h2b, "head.2.bias", 1);
        memcpy(m->head2_w, h2w, sizeof(float) * 128);
        m->head2_b = h2b[0];
    }
    free(wf);
    free(bf);
    file_free(&f);
    return m;
fail_t:
    set_err("missing or misshapen tensor");
fail:
    free(wf);
    free(bf);
    file_free(&f);
    orc_free(m);
    return NULL;
}

void orc_free(orc_model* m) {
    if (!m) return;
    for (int i = 0; i < 15; ++i) {
        Blk* B = &m->blk[i];
        lin_free(&B->expand); lin_free(&B->se1); lin_free(&B->se2); lin_free(&B->project);
        free(B->dw_w); free(B->dw_b);
    }
    lin_free(&m->last); lin_free(&m->proj);
    free(m->pos);
    for (int g = 0; g < 2; ++g) {
        lin_free(&m->gdn[g].in); lin_free(&m->gdn[g].out); lin_free(&m->gdn[g].gate);
        lin_free(&m->gdn[g].up); lin_free(&m->gdn[g].down);
    }
    lin_free(&m->s_in); lin_free(&m->s_q); lin_free(&m->s_c); lin_free(&m->s_o);
    lin_free(&m->s_gate); lin_free(&m->s_up); lin_free(&m->s_down); lin_free(&m->head0);
    free(m);
}

/* ------------------------------------------------------------------------------------------ CNN */
/* stem (isa_impl.hpp:558-600): fma chain over (dy, dx, c) from +0, zero padding taps included, + bias, hswish */
static void stem(const orc_model* m, const uint8_t* rgb, float* out) {
    for (int y = 0; y < 90; ++y)
        for (int x = 0; x < 160; ++x) {
            float acc[16];
            for (int o = 0; o < 16; ++o) acc[o] = 0.0f;
            for (int dy = 0; dy < 3; ++dy) {
                const int iy = 2 * y - 1 + dy;
                for (int dx = 0; dx < 3; ++dx) {
                    const int ix = 2 * x - 1 + dx;
                    const int in = iy >= 0 && iy < 180 && ix >= 0 && ix < 320;
                    for (int c = 0; c < 3; ++c) {
                        const float v = in ? m->lut[c][rgb[((size_t)iy * 320 + ix) * 3 + c]] : 0.0f;
                        const float* w = m->stem_w[(dy * 3 + dx) * 3 + c];
                        for (int o = 0; o < 16; ++o) acc[o] = __builtin_fmaf(v, w[o], acc[o]);
                    }
                }
            }
            float* o = out + ((size_t)y * 160 + x) * 16;
            for (int c = 0; c < 16; ++c) o[c] = orc_hswish(acc[c] + m->stem_b[c]);
        }
}

/* depthwise KxK (isa_impl.hpp:603-643): fma chain over (dy, dx) from +0 with zero padding, + bias, act */
static void dwconv(const Blk* B, const float* in, float* out) {
    const int C = B->cexp;
    float* acc = (float*)malloc(sizeof(float) * (size_t)C);
    for (int y = 0; y < B->Ho; ++y)
        for (int x = 0; x < B->Wo; ++x) {
            for (int c = 0; c < C; ++c) acc[c] = 0.0f;
            for (int dy = 0; dy < B->k; ++dy) {
                const int iy = y * B->s - B->p + dy;
                for (int dx = 0; dx < B->k; ++dx) {
                    const int ix = x * B->s - B->p + dx;
                    const int inside = iy >= 0 && iy < B->H && ix >= 0 && ix < B->W;
                    const float* w = B->dw_w + (size_t)(dy * B->k + dx) * C;
                    const float* src = in + ((size_t)iy * B->W + ix) * C;
                    for (int c = 0; c < C; ++c) acc[c] = __builtin_fmaf(inside ? src[c] : 0.0f, w[c], acc[c]);
                }
            }
            float* o = out + ((size_t)y * B->Wo + x) * C;
            for (int c = 0; c < C; ++c) {
                const float v = acc[c] + B->dw_b[c];
                o[c] = B->hs ? orc_hswish(v) : relu(v);
            }
        }
    free(acc);
}

/* one inverted-residual block (isa_impl.hpp:731-791) */
static void block(const Blk* B, const float* in, float* out) {
    const float* e = in;
    float* ebuf = NULL;
    if (B->has_expand) {
        ebuf = (float*)malloc(sizeof(float) * (size_t)B->H * B->W * B->cexp);
        lin_gemm(in, B->cin, B->H * B->W, &B->expand, ebuf, B->cexp, B->hs ? ORC_HS : ORC_RELU, NULL, 0);
        e = ebuf;
    }
    const int n = B->Ho * B->Wo, C = B->cexp;
    float* d = (float*)malloc(sizeof(float) * (size_t)n * C);
    dwconv(B, e, d);
    free(ebuf);
    if (B->has_se) {
        /* mean over the map: per row left-to-right sums, then rows in order, / (float)(H*W) */
        float* pooled = (float*)malloc(sizeof(float) * (size_t)C * 3);
        float* sq = pooled + C;
        float* scale = sq + C;
        for (int c = 0; c < C; ++c) {
            float tot = 0.0f;
            for (int y = 0; y < B->Ho; ++y) {
                const float* row = d + (size_t)y * B->Wo * C + c;
                float acc = row[0];
                for (int x = 1; x < B->Wo; ++x) acc = acc + row[(size_t)x * C];
                tot = y == 0 ? acc : tot + acc;
            }
            pooled[c] = tot / (float)n;
        }
        lin_gemm(pooled, C, 1, &B->se1, sq, B->csq, ORC_RELU, NULL, 0);
        lin_gemm(sq, B->csq, 1, &B->se2, scale, C, ORC_HSIG, NULL, 0);
        for (int p = 0; p < n; ++p)
            for (int c = 0; c < C; ++c) d[(size_t)p * C + c] = scale[c] * d[(size_t)p * C + c];
        free(pooled);
    }
    lin_gemm(d, C, n, &B->project, out, B->cout, B->residual ? ORC_RES : ORC_STORE, B->residual ? in : NULL,
             B->cin);
    free(d);
}

int orc_encode_frame(const orc_model* m, const uint8_t* rgb, float* tokens, orc_dump_fn dump, void* ctx) {
    float* a = (float*)malloc(sizeof(float) * 90 * 160 * 24);
    float* b = (float*)malloc(sizeof(float) * 90 * 160 * 24);
    stem(m, rgb, a);
    if (dump) dump(ctx, "cnn00", a, (size_t)90 * 160 * 16);
    for (int i = 0; i < 15; ++i) {
        const Blk* B = &m->blk[i];
        block(B, a, b);
        float* t = a; a = b; b = t;
        if (dump) {
            char name[8];
            snprintf(name, sizeof name, "cnn%02d", i + 1);
            dump(ctx, name, a, (size_t)B->Ho * B->Wo * B->cout);
        }
    }
    float* map = (float*)malloc(sizeof(float) * 60 * 960);
    lin_gemm(a, 160, 60, &m->last, map, 960, ORC_HS, NULL, 0);
    if (dump) dump(ctx, "cnn16", map, (size_t)60 * 960);
    /* 4x4 adaptive pool (isa_impl.hpp:827-842): bins rows {0,1,3,4}+2, cols {0,2,5,7}+3, left-to-right sum
     * from +0, then (acc / 2) / 3 */
    static const int r0[4] = {0, 1, 3, 4}, c0[4] = {0, 2, 5, 7};
    float* pooled = (float*)malloc(sizeof(float) * 16 * 960);
    for (int t = 0; t < 16; ++t)
        for (int c = 0; c < 960; ++c) {
            float acc = 0.0f;
            for (int yy = r0[t / 4]; yy < r0[t / 4] + 2; ++yy)
                for (int xx = c0[t % 4]; xx < c0[t % 4] + 3; ++xx) acc = acc + map[(size_t)(yy * 10 + xx) * 960 + c];
            pooled[(size_t)t * 960 + c] = (acc / 2.0f) / 3.0f;
        }
    lin_gemm(pooled, 960, 16, &m->proj, tokens, DM, ORC_STORE, NULL, 0);
    if (dump) dump(ctx, "tokens", tokens, (size_t)16 * DM);
    free(pooled); free(map); free(a); free(b);
    return 0;
}

/* ------------------------------------------------------------------------------------------ sequence */
/* RMSNorm over 384 (isa_impl.hpp:854-860): x * (1/sqrt(sum(x^2)/n + 1e-6)) * w */
static void rms_row(const float* x, float* y, const float* w, int n) {
    const float inv = 1.0f / sqrtf(lanes_dot(x, x, n) / (float)n + 1e-6f);
    for (int i = 0; i < n; ++i) y[i] = (x[i] * inv) * w[i];
}

/* gated delta rule (isa_impl.hpp:911-947): pred for token t is S_{t-1}^T k_t, accumulated while S_{t-1} is
 * written; u = (v - a pred) b; S_t[j] = k_j u + a S_{t-1}[j]; o = S_t^T q (fma chains over j = 0..63). */
void orc_delta_rule(const float* q, const float* k, const float* v, const float* decay, const float* beta, int T,
                    int ldq, int ldv, float* o, int ldo) {
    float* S = (float*)calloc(64 * 128, sizeof(float));
    float pred[128], u[128], oo[128];
    for (int c = 0; c < 128; ++c) pred[c] = 0.0f;
    for (int t = 0; t < T; ++t) {
        const float* qt = q + (size_t)t * ldq;
        const float* kt = k + (size_t)t * ldq;
        const float* vt = v + (size_t)t * ldv;
        const float* kn = t + 1 < T ? k + (size_t)(t + 1) * ldq : kt;
        const float a = decay[t], b = beta[t];
        for (int c = 0; c < 128; ++c) {
            u[c] = (vt[c] - a * pred[c]) * b;
            oo[c] = 0.0f;
            pred[c] = 0.0f;
        }
        for (int j = 0; j < 64; ++j) {
            float* s = S + j * 128;
            for (int c = 0; c < 128; ++c) {
                const float x = __builtin_fmaf(kt[j], u[c], s[c] * a);
                s[c] = x;
                oo[c] = __builtin_fmaf(x, qt[j], oo[c]);
                pred[c] = __builtin_fmaf(x, kn[j], pred[c]);
            }
        }
        memcpy(o + (size_t)t * ldo, oo, sizeof oo);
    }
    free(S);
}

/* per-head GDN core (isa_impl.hpp:866-962) on P [321][2316] in place; output O [321][768] columns h*128.. */
static void gdn_head(const Gdn* G, int h, float* P, float* O) {
    const int cols[3] = {h * 64, 384 + h * 64, 768 + h * 128}, widths[3] = {64, 64, 128};
    const int wofs[3] = {h * 64, 384 + h * 64, 768 + h * 128};
    for (int g = 0; g < 3; ++g)
        for (int c = 0; c < widths[g]; ++c) {
            const int col = cols[g] + c, wc = wofs[g] + c;
            for (int t = T_TOK - 1; t >= 0; --t) {
                float acc = 0.0f;
                if (t >= 3) acc = __builtin_fmaf(P[(size_t)(t - 3) * GP + col], G->conv_w[0][wc], acc);
                if (t >= 2) acc = __builtin_fmaf(P[(size_t)(t - 2) * GP + col], G->conv_w[1][wc], acc);
                if (t >= 1) acc = __builtin_fmaf(P[(size_t)(t - 1) * GP + col], G->conv_w[2][wc], acc);
                acc = __builtin_fmaf(P[(size_t)t * GP + col], G->conv_w[3][wc], acc);
                P[(size_t)t * GP + col] = orc_silu(acc + G->conv_b[wc]);
            }
        }
    float decay[T_TOK], beta[T_TOK];
    for (int t = 0; t < T_TOK; ++t) {
        float* row = P + (size_t)t * GP;
        float* q = row + h * 64;
        float* k = row + 384 + h * 64;
        const float iq = 1.0f / sqrtf(lanes_dot(q, q, 64) + 1e-6f);
        const float ik = 1.0f / sqrtf(lanes_dot(k, k, 64) + 1e-6f);
        for (int i = 0; i < 64; ++i) {
            q[i] = (q[i] * iq) * 0.125f;
            k[i] = k[i] * ik;
        }
        decay[t] = expf(G->neg_rate[h] * softplus_f(row[2304 + h] + G->dt_bias[h]));
        beta[t] = 1.0f / (1.0f + expf(-row[2310 + h]));
    }
    orc_delta_rule(P + h * 64, P + 384 + h * 64, P + 768 + h * 128, decay, beta, T_TOK, GP, GP, O + h * 128, 768);
    for (int t = 0; t < T_TOK; ++t) {
        float* o = O + (size_t)t * 768 + h * 128;
        const float* gate = P + (size_t)t * GP + 1536 + h * 128;
        const float rstd = 1.0f / sqrtf(lanes_dot(o, o, 128) / 128.0f + 1e-6f);
        for (int i = 0; i < 128; ++i) o[i] = ((o[i] * rstd) * G->o_norm_w[i]) * orc_silu(gate[i]);
    }
}

static void gdn_stage(const Gdn* G, float* h, float* hn, float* P, float* O, float* F) {
    for (int rep = 0; rep < G->repeats; ++rep) {
        for (int t = 0; t < T_TOK; ++t) rms_row(h + (size_t)t * DM, hn + (size_t)t * DM, G->norm_w, DM);
        lin_gemm(hn, DM, T_TOK, &G->in, P, GP, ORC_STORE, NULL, 0);
        for (int hd = 0; hd < 6; ++hd) gdn_head(G, hd, P, O);
        lin_gemm(O, 768, T_TOK, &G->out, h, DM, G->repeats == 2 ? ORC_ACC_DIV2 : ORC_ACC, NULL, 0);
    }
    for (int t = 0; t < T_TOK; ++t) rms_row(h + (size_t)t * DM, hn + (size_t)t * DM, G->ffn_norm_w, DM);
    swiglu_gemm(hn, DM, T_TOK, &G->gate, &G->up, F, 960);
    lin_gemm(F, 960, T_TOK, &G->down, h, DM, ORC_ACC, NULL, 0);
}

/* SISA head for the last query row (isa_impl.hpp:996-1069) on S [321][1068]; rotates B in place */
static void sisa_head(const orc_model* m, int h, float* S, const float* q320, float* c320, float* y) {
    float gt[T_TOK], ft[T_TOK], sco[T_TOK];
    double g = 0.0, f = 0.0, phi[16];
    for (int i = 0; i < 16; ++i) phi[i] = 0.0;
    for (int t = 0; t < T_TOK; ++t) {
        float* row = S + (size_t)t * SP;
        g += (double)(-softplus_f(row[1056 + h]));
        f += (double)logsigmoid_f(row[1062 + h]);
        gt[t] = (float)g;
        ft[t] = (float)f;
        float* b = row + 768 + h * 32;
        const float* th = row + 960 + h * 16;
        for (int pr = 0; pr < 16; ++pr) {
            phi[pr] += (double)th[pr];
            float sn, cs;
            sincosf((float)phi[pr], &sn, &cs);
            const float e = b[2 * pr], o = b[2 * pr + 1];
            b[2 * pr] = e * cs - o * sn;
            b[2 * pr + 1] = e * sn + o * cs;
            if (t == T_TOK - 1) {
                float* c = c320 + h * 32;
                const float ce = c[2 * pr], co = c[2 * pr + 1];
                c[2 * pr] = ce * cs - co * sn;
                c[2 * pr + 1] = ce * sn + co * cs;
            }
        }
    }
    const float* q = q320 + h * 64;
    const float* c = c320 + h * 32;
    const float lam = m->lam[h], gl = gt[T_TOK - 1], fl = ft[T_TOK - 1];
    float mx = -INFINITY;
    for (int t = 0; t < T_TOK; ++t) {
        const float* row = S + (size_t)t * SP;
        float score = lanes_dot(q, row + h * 64, 64) * 0.125f;
        score = score + (lam * expf(gl - gt[t])) * lanes_dot(c, row + 768 + h * 32, 32);
        score = score + (fl - ft[t]);
        sco[t] = score;
        if (score > mx) mx = score;
    }
    double sum = 0.0;
    for (int t = 0; t < T_TOK; ++t) {
        sco[t] = expf(sco[t] - mx);
        sum += (double)sco[t];
    }
    const float inv = 1.0f / (float)sum;
    float tot[64], blk[64];
    for (int t0 = 0; t0 < T_TOK; t0 += 64) {
        for (int j = 0; j < 64; ++j) blk[j] = 0.0f;
        for (int t = t0; t < t0 + 64 && t < T_TOK; ++t) {
            const float p = sco[t] * inv;
            const float* vv = S + (size_t)t * SP + 384 + h * 64;
            for (int j = 0; j < 64; ++j) blk[j] = __builtin_fmaf(p, vv[j], blk[j]);
        }
        for (int j = 0; j < 64; ++j) tot[j] = t0 == 0 ? blk[j] : tot[j] + blk[j];
    }
    memcpy(y + h * 64, tot, sizeof tot);
}

int orc_classify(const orc_model* m, const float* const* tok, float* logit, orc_dump_fn dump, void* ctx) {
    float* h = (float*)malloc(sizeof(float) * T_TOK * DM);
    float* hn = (float*)malloc(sizeof(float) * T_TOK * DM);
    float* P = (float*)malloc(sizeof(float) * T_TOK * GP);
    float* O = (float*)malloc(sizeof(float) * T_TOK * 768);
    float* F = (float*)malloc(sizeof(float) * T_TOK * 960);
    for (int i = 0; i < 320; ++i)
        for (int d = 0; d < DM; ++d)
            h[(size_t)i * DM + d] = tok[i / 16][(size_t)(i % 16) * DM + d] + m->pos[(size_t)i * DM + d];
    memcpy(h + (size_t)320 * DM, m->readout, sizeof(float) * DM);
    if (dump) dump(ctx, "h0", h, (size_t)T_TOK * DM);
    gdn_stage(&m->gdn[0], h, hn, P, O, F);
    if (dump) dump(ctx, "after_gdn_a", h, (size_t)T_TOK * DM);
    gdn_stage(&m->gdn[1], h, hn, P, O, F);
    if (dump) dump(ctx, "after_gdn_b", h, (size_t)T_TOK * DM);
    /* SISA block, last row only (isa_impl.hpp:1092-1126) */
    for (int t = 0; t < T_TOK; ++t) rms_row(h + (size_t)t * DM, hn + (size_t)t * DM, m->s_attn_norm_w, DM);
    lin_gemm(hn, DM, T_TOK, &m->s_in, P, SP, ORC_STORE, NULL, 0);
    float q320[DM], c320[192], y[DM], x[DM], xn[DM], mid[960], hid[128];
    const float* last = hn + (size_t)320 * DM;
    lin_gemm(last, DM, 1, &m->s_q, q320, DM, ORC_STORE, NULL, 0);
    lin_gemm(last, DM, 1, &m->s_c, c320, 192, ORC_STORE, NULL, 0);
    for (int hd = 0; hd < 6; ++hd) sisa_head(m, hd, P, q320, c320, y);
    memcpy(x, h + (size_t)320 * DM, sizeof x);
    lin_gemm(y, DM, 1, &m->s_o, x, DM, ORC_ACC, NULL, 0);
    rms_row(x, xn, m->s_ffn_norm_w, DM);
    swiglu_gemm(xn, DM, 1, &m->s_gate, &m->s_up, mid, 960);
    lin_gemm(mid, 960, 1, &m->s_down, x, DM, ORC_ACC, NULL, 0);
    if (dump) dump(ctx, "after_sisa_last", x, DM);
    rms_row(x, xn, m->final_norm_w, DM);
    lin_gemm(xn, DM, 1, &m->head0, hid, 128, ORC_SILU, NULL, 0);
    *logit = lanes_dot(hid, m->head2_w, 128) + m->head2_b;
    if (dump) {
        dump(ctx, "final_norm_row", xn, DM);
        dump(ctx, "head_hidden", hid, 128);
        dump(ctx, "logit", logit, 1);
    }
    free(h); free(hn); free(P); free(O); free(F);
    return 0;
}
