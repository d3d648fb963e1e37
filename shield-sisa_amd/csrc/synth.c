/* Seeded synthetic inputs: SHIELD-V SHLDV001 weights (+ "<file>.json" sidecar), uint8 crops, and the sequence-stage
 * weights of the SHIELD-A audio model (SHLDA001, engine/audio/weights.cpp container).
 *
 * The real checkpoint is not available offline, so every test and benchmark runs on weights drawn here from a
 * seed.  Only IEEE add/mul/div/sqrt on doubles are used (no libm transcendentals), so the same seed yields the
 * same bytes, hence the same SHA-256, on every x86-64 host.
 *
 * Tensor names and shapes are those of the reference export (tools/export_v.py:52-71, which writes every
 * parameter and buffer of ShieldV; the architecture is fixed by engine/model/runtime.cpp:212-330 and
 * oracle/shieldv_ref.py:359-375).  Distributions:
 *   convolutions (stem, expand, depthwise, project, SE fc1/fc2, last 1x1): He-normal, std sqrt(2 / fan_in)
 *   BatchNorm: weight 1, bias 0, running_mean 0, running_var 1
 *   linears: Xavier-uniform, bound sqrt(6 / (fan_in + fan_out)); all biases 0
 *   RMSNorm / gated-norm weights 1; time/row/col embeddings and readout N(0, 0.02^2)
 *   GDN: A_log = ln U[1,16], dt_bias 0, short convs He-normal (fan_in 4), conv biases 0; SISA lambda_raw 0
 * Normal deviates are Irwin-Hall sums of 12 uniforms minus 6.
 * SHIELD-A: the tensors its sequence stages read, names and shapes as engine/audio/sequence.cpp:304-331 validates
 * them; the same distributions, head biases 0.  The whole-model file adds the frontend's tensors (BatchNorm
 * statistics drawn away from the identity, a polynomial analysis window and a triangular filterbank). */
#include "sha256.h"

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define SHV_SYNTH_API __attribute__((visibility("default")))

/* ---------------------------------------------------------------------------------------------- generator */
typedef struct { uint64_t s[4]; } Rng;

static uint64_t splitmix(uint64_t* x) {
    uint64_t z = (*x += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
static void rng_seed(Rng* r, uint64_t seed) {
    uint64_t x = seed;
    for (int i = 0; i < 4; ++i) r->s[i] = splitmix(&x);
}
static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
static uint64_t rng_next(Rng* r) { /* xoshiro256** */
    const uint64_t out = rotl(r->s[1] * 5, 7) * 9;
    const uint64_t t = r->s[1] << 17;
    r->s[2] ^= r->s[0];
    r->s[3] ^= r->s[1];
    r->s[1] ^= r->s[2];
    r->s[0] ^= r->s[3];
    r->s[2] ^= t;
    r->s[3] = rotl(r->s[3], 45);
    return out;
}
static double rng_unit(Rng* r) { return (double)(rng_next(r) >> 11) * (1.0 / 9007199254740992.0); } /* [0,1) */
static double rng_normal(Rng* r) {
    double s = 0.0;
    for (int i = 0; i < 12; ++i) s += rng_unit(r);
    return s - 6.0;
}
/* ln(x) for x in [1, 16]: 2 atanh(z), z = (x-1)/(x+1), by its power series (converges for z < 1) */
static double ln_series(double x) {
    const double z = (x - 1.0) / (x + 1.0), z2 = z * z;
    double term = z, sum = 0.0;
    for (int k = 0; k < 400; ++k) {
        sum += term / (double)(2 * k + 1);
        term *= z2;
    }
    return 2.0 * sum;
}

/* ---------------------------------------------------------------------------------------------- tensor table */
enum { D_HE = 0, D_XAVIER, D_ONE, D_ZERO, D_EMB, D_ALOG,
       /* SHIELD-A frontend: BatchNorm statistics drawn away from the identity, log-mel normalisation, a smooth
        * analysis window and a triangular filterbank (position-dependent, no random draws) */
       D_BN_W, D_BN_B, D_BN_VAR, D_MEL_MEAN, D_MEL_STD, D_WINDOW, D_MELFB };

typedef struct {
    char name[96];
    int rank, dims[4];
    int dist, fan_in, fan_out;
    int param;  /* 1 = parameter (counts towards the model's parameter total), 0 = buffer */
} Spec;

typedef struct {
    Spec* v;
    int n, cap;
} Table;

static void add(Table* t, const char* name, int rank, const int* dims, int dist, int fan_in, int fan_out, int param) {
    if (t->n == t->cap) {
        t->cap = t->cap ? 2 * t->cap : 64;
        t->v = (Spec*)realloc(t->v, sizeof(Spec) * (size_t)t->cap);
    }
    Spec* s = &t->v[t->n++];
    memset(s, 0, sizeof *s);
    snprintf(s->name, sizeof s->name, "%s", name);
    s->rank = rank;
    for (int i = 0; i < rank; ++i) s->dims[i] = dims[i];
    s->dist = dist;
    s->fan_in = fan_in;
    s->fan_out = fan_out;
    s->param = param;
}
static void t1(Table* t, const char* n, int a, int dist) { int d[1] = {a}; add(t, n, 1, d, dist, 0, 0, 1); }
static void lin(Table* t, const char* n, int out, int in) { int d[2] = {out, in}; add(t, n, 2, d, D_XAVIER, in, out, 1); }
static void conv(Table* t, const char* n, int out, int per_in, int k) {
    int d[4] = {out, per_in, k, k};
    add(t, n, 4, d, D_HE, per_in * k * k, 0, 1);
}
static void bn(Table* t, const char* prefix, int c) {
    char n[96];
    int d[1] = {c};
    snprintf(n, sizeof n, "%s.weight", prefix); add(t, n, 1, d, D_ONE, 0, 0, 1);
    snprintf(n, sizeof n, "%s.bias", prefix); add(t, n, 1, d, D_ZERO, 0, 0, 1);
    snprintf(n, sizeof n, "%s.running_mean", prefix); add(t, n, 1, d, D_ZERO, 0, 0, 0);
    snprintf(n, sizeof n, "%s.running_var", prefix); add(t, n, 1, d, D_ONE, 0, 0, 0);
}
static int make_div8(int v) { /* torchvision _make_divisible(v, 8) for integer v */
    int nv = (v + 4) / 8 * 8;
    if (nv < 8) nv = 8;
    if (10 * nv < 9 * v) nv += 8;
    return nv;
}

/* MobileNetV3-Large features[1..15]: in, kernel, expanded, out, SE, stride (torchvision inverted-residual table) */
static const int kBlk[15][6] = {
    {16, 3, 16, 16, 0, 1},   {16, 3, 64, 24, 0, 2},   {24, 3, 72, 24, 0, 1},   {24, 5, 72, 40, 1, 2},
    {40, 5, 120, 40, 1, 1},  {40, 5, 120, 40, 1, 1},  {40, 3, 240, 80, 0, 2},  {80, 3, 200, 80, 0, 1},
    {80, 3, 184, 80, 0, 1},  {80, 3, 184, 80, 0, 1},  {80, 3, 480, 112, 1, 1}, {112, 3, 672, 112, 1, 1},
    {112, 5, 672, 160, 1, 2}, {160, 5, 960, 160, 1, 1}, {160, 5, 960, 160, 1, 1}};

static void build_table(Table* t) {
    char n[96];
    conv(t, "cnn.0.0.weight", 16, 3, 3);
    bn(t, "cnn.0.1", 16);
    for (int i = 0; i < 15; ++i) {
        const int in = kBlk[i][0], k = kBlk[i][1], ex = kBlk[i][2], out = kBlk[i][3], se = kBlk[i][4];
        int j = 0;
        if (ex != in) {
            snprintf(n, sizeof n, "cnn.%d.block.%d.0.weight", i + 1, j); conv(t, n, ex, in, 1);
            snprintf(n, sizeof n, "cnn.%d.block.%d.1", i + 1, j); bn(t, n, ex);
            ++j;
        }
        snprintf(n, sizeof n, "cnn.%d.block.%d.0.weight", i + 1, j); conv(t, n, ex, 1, k);
        snprintf(n, sizeof n, "cnn.%d.block.%d.1", i + 1, j); bn(t, n, ex);
        ++j;
        if (se) {
            const int sq = make_div8(ex / 4);
            snprintf(n, sizeof n, "cnn.%d.block.%d.fc1.weight", i + 1, j); conv(t, n, sq, ex, 1);
            snprintf(n, sizeof n, "cnn.%d.block.%d.fc1.bias", i + 1, j); t1(t, n, sq, D_ZERO);
            snprintf(n, sizeof n, "cnn.%d.block.%d.fc2.weight", i + 1, j); conv(t, n, ex, sq, 1);
            snprintf(n, sizeof n, "cnn.%d.block.%d.fc2.bias", i + 1, j); t1(t, n, ex, D_ZERO);
            ++j;
        }
        snprintf(n, sizeof n, "cnn.%d.block.%d.0.weight", i + 1, j); conv(t, n, out, ex, 1);
        snprintf(n, sizeof n, "cnn.%d.block.%d.1", i + 1, j); bn(t, n, out);
    }
    conv(t, "cnn.16.0.weight", 960, 160, 1);
    bn(t, "cnn.16.1", 960);
    lin(t, "projection.weight", 384, 960);
    { int d[2] = {20, 384}; add(t, "time_embedding", 2, d, D_EMB, 0, 0, 1); }
    { int d[2] = {4, 384}; add(t, "row_embedding", 2, d, D_EMB, 0, 0, 1); }
    { int d[2] = {4, 384}; add(t, "col_embedding", 2, d, D_EMB, 0, 0, 1); }
    { int d[3] = {1, 1, 384}; add(t, "readout", 3, d, D_EMB, 0, 0, 1); }
    const char* stages[2] = {"gdn_a", "gdn_b"};
    for (int s = 0; s < 2; ++s) {
        const char* p = stages[s];
        snprintf(n, sizeof n, "%s.norm.weight", p); t1(t, n, 384, D_ONE);
        snprintf(n, sizeof n, "%s.ffn_norm.weight", p); t1(t, n, 384, D_ONE);
        snprintf(n, sizeof n, "%s.mixer.q_proj.weight", p); lin(t, n, 384, 384);
        snprintf(n, sizeof n, "%s.mixer.k_proj.weight", p); lin(t, n, 384, 384);
        snprintf(n, sizeof n, "%s.mixer.v_proj.weight", p); lin(t, n, 768, 384);
        snprintf(n, sizeof n, "%s.mixer.a_proj.weight", p); lin(t, n, 6, 384);
        snprintf(n, sizeof n, "%s.mixer.b_proj.weight", p); lin(t, n, 6, 384);
        snprintf(n, sizeof n, "%s.mixer.A_log", p); t1(t, n, 6, D_ALOG);
        snprintf(n, sizeof n, "%s.mixer.dt_bias", p); t1(t, n, 6, D_ZERO);
        const char* cv[3] = {"q_conv1d", "k_conv1d", "v_conv1d"};
        const int cw[3] = {384, 384, 768};
        for (int c = 0; c < 3; ++c) {
            int d[3] = {cw[c], 1, 4};
            snprintf(n, sizeof n, "%s.mixer.%s.weight", p, cv[c]); add(t, n, 3, d, D_HE, 4, 0, 1);
            snprintf(n, sizeof n, "%s.mixer.%s.bias", p, cv[c]); t1(t, n, cw[c], D_ZERO);
        }
        snprintf(n, sizeof n, "%s.mixer.g_proj.weight", p); lin(t, n, 768, 384);
        snprintf(n, sizeof n, "%s.mixer.o_norm.weight", p); t1(t, n, 128, D_ONE);
        snprintf(n, sizeof n, "%s.mixer.o_proj.weight", p); lin(t, n, 384, 768);
        snprintf(n, sizeof n, "%s.ffn.gate.weight", p); lin(t, n, 960, 384);
        snprintf(n, sizeof n, "%s.ffn.up.weight", p); lin(t, n, 960, 384);
        snprintf(n, sizeof n, "%s.ffn.down.weight", p); lin(t, n, 384, 960);
    }
    t1(t, "sisa.attn_norm.weight", 384, D_ONE);
    lin(t, "sisa.attn.W_Q.weight", 384, 384);
    lin(t, "sisa.attn.W_K.weight", 384, 384);
    lin(t, "sisa.attn.W_V.weight", 384, 384);
    lin(t, "sisa.attn.W_O.weight", 384, 384);
    lin(t, "sisa.attn.W_B.weight", 192, 384);
    lin(t, "sisa.attn.W_C.weight", 192, 384);
    lin(t, "sisa.attn.alpha_proj.weight", 6, 384);
    t1(t, "sisa.attn.alpha_proj.bias", 6, D_ZERO);
    lin(t, "sisa.attn.theta_proj.weight", 96, 384);
    lin(t, "sisa.attn.forget_proj.weight", 6, 384);
    t1(t, "sisa.attn.forget_proj.bias", 6, D_ZERO);
    t1(t, "sisa.attn.lambda_raw", 6, D_ZERO);
    t1(t, "sisa.ffn_norm.weight", 384, D_ONE);
    lin(t, "sisa.ffn.w_gate.weight", 960, 384);
    lin(t, "sisa.ffn.w_up.weight", 960, 384);
    lin(t, "sisa.ffn.w_down.weight", 384, 960);
    t1(t, "final_norm.weight", 384, D_ONE);
    lin(t, "head.0.weight", 128, 384);
    t1(t, "head.0.bias", 128, D_ZERO);
    lin(t, "head.2.weight", 1, 128);
    t1(t, "head.2.bias", 1, D_ZERO);
}

static size_t numel(const Spec* s) {
    size_t e = 1;
    for (int i = 0; i < s->rank; ++i) e *= (size_t)s->dims[i];
    return e;
}

static void fill(const Spec* s, float* out, Rng* r) {
    const size_t e = numel(s);
    double scale = 0.0;
    if (s->dist == D_HE) scale = __builtin_sqrt(2.0 / (double)s->fan_in);
    if (s->dist == D_XAVIER) scale = __builtin_sqrt(6.0 / (double)(s->fan_in + s->fan_out));
    for (size_t i = 0; i < e; ++i) {
        double v = 0.0;
        switch (s->dist) {
        case D_HE: v = rng_normal(r) * scale; break;
        case D_XAVIER: v = (2.0 * rng_unit(r) - 1.0) * scale; break;
        case D_ONE: v = 1.0; break;
        case D_ZERO: v = 0.0; break;
        case D_EMB: v = rng_normal(r) * 0.02; break;
        case D_ALOG: v = ln_series(1.0 + 15.0 * rng_unit(r)); break;
        case D_BN_W: v = 1.0 + 0.1 * rng_normal(r); break;
        case D_BN_B: v = 0.1 * rng_normal(r); break;
        case D_BN_VAR: { const double g = rng_normal(r); v = 1.0 + 0.2 * (g < 0.0 ? -g : g); break; }
        case D_MEL_MEAN: v = 1.0 + 0.5 * rng_normal(r); break;
        case D_MEL_STD: { const double g = rng_normal(r); v = 1.0 + 0.25 * (g < 0.0 ? -g : g); break; }
        case D_WINDOW: {   /* 16 x^2 (1 - x)^2, x = i / 400: zero at the ends, 1 in the middle */
            const double x = (double)i / 400.0;
            v = 16.0 * x * x * (1.0 - x) * (1.0 - x);
            break;
        }
        case D_MELFB: {    /* filter m over FFT bin k: a triangle on the points 1 + 254 (0.3 u + 0.7 u^2), u = j / 81 */
            const int m = (int)(i / 257), k = (int)(i % 257);
            double pt[3];
            for (int q = 0; q < 3; ++q) {
                const double u = (double)(m + q) / 81.0;
                pt[q] = 1.0 + 254.0 * (0.3 * u + 0.7 * u * u);
            }
            const double up = ((double)k - pt[0]) / (pt[1] - pt[0]), down = (pt[2] - (double)k) / (pt[2] - pt[1]);
            v = up < down ? up : down;
            if (v < 0.0) v = 0.0;
            break;
        }
        default: break;
        }
        out[i] = (float)v;
    }
}

/* ---------------------------------------------------------------------------------------------- C API */
static void build_audio_table(Table* t) {
    char n[96];
    { int d[3] = {1, 1, 384}; add(t, "readout", 3, d, D_EMB, 0, 0, 1); }
    const char* stages[2] = {"gdn_a", "gdn_b"};
    for (int s = 0; s < 2; ++s) {
        const char* p = stages[s];
        snprintf(n, sizeof n, "%s.mixer_norm.weight", p); t1(t, n, 384, D_ONE);
        snprintf(n, sizeof n, "%s.ffn_norm.weight", p); t1(t, n, 384, D_ONE);
        snprintf(n, sizeof n, "%s.mixer.q_proj.weight", p); lin(t, n, 384, 384);
        snprintf(n, sizeof n, "%s.mixer.k_proj.weight", p); lin(t, n, 384, 384);
        snprintf(n, sizeof n, "%s.mixer.v_proj.weight", p); lin(t, n, 768, 384);
        snprintf(n, sizeof n, "%s.mixer.a_proj.weight", p); lin(t, n, 6, 384);
        snprintf(n, sizeof n, "%s.mixer.b_proj.weight", p); lin(t, n, 6, 384);
        snprintf(n, sizeof n, "%s.mixer.g_proj.weight", p); lin(t, n, 768, 384);
        snprintf(n, sizeof n, "%s.mixer.o_proj.weight", p); lin(t, n, 384, 768);
        snprintf(n, sizeof n, "%s.mixer.A_log", p); t1(t, n, 6, D_ALOG);
        snprintf(n, sizeof n, "%s.mixer.dt_bias", p); t1(t, n, 6, D_ZERO);
        snprintf(n, sizeof n, "%s.mixer.o_norm.weight", p); t1(t, n, 128, D_ONE);
        const char* cv[3] = {"q_conv1d", "k_conv1d", "v_conv1d"};
        const int cw[3] = {384, 384, 768};
        for (int c = 0; c < 3; ++c) {
            int d[3] = {cw[c], 1, 4};
            snprintf(n, sizeof n, "%s.mixer.%s.weight", p, cv[c]); add(t, n, 3, d, D_HE, 4, 0, 1);
            snprintf(n, sizeof n, "%s.mixer.%s.bias", p, cv[c]); t1(t, n, cw[c], D_ZERO);
        }
        snprintf(n, sizeof n, "%s.ffn.w_gate.weight", p); lin(t, n, 960, 384);
        snprintf(n, sizeof n, "%s.ffn.w_up.weight", p); lin(t, n, 960, 384);
        snprintf(n, sizeof n, "%s.ffn.w_down.weight", p); lin(t, n, 384, 960);
    }
    t1(t, "sisa.attn_norm.weight", 384, D_ONE);
    t1(t, "sisa.ffn_norm.weight", 384, D_ONE);
    lin(t, "sisa.attn.W_Q.weight", 384, 384);
    lin(t, "sisa.attn.W_K.weight", 384, 384);
    lin(t, "sisa.attn.W_V.weight", 384, 384);
    lin(t, "sisa.attn.W_O.weight", 384, 384);
    lin(t, "sisa.attn.W_B.weight", 192, 384);
    lin(t, "sisa.attn.W_C.weight", 192, 384);
    lin(t, "sisa.attn.theta_proj.weight", 96, 384);
    lin(t, "sisa.attn.alpha_proj.weight", 6, 384);
    t1(t, "sisa.attn.alpha_proj.bias", 6, D_ZERO);
    lin(t, "sisa.attn.forget_proj.weight", 6, 384);
    t1(t, "sisa.attn.forget_proj.bias", 6, D_ZERO);
    t1(t, "sisa.attn.lambda_raw", 6, D_ZERO);
    lin(t, "sisa.ffn.w_gate.weight", 960, 384);
    lin(t, "sisa.ffn.w_up.weight", 960, 384);
    lin(t, "sisa.ffn.w_down.weight", 384, 960);
    t1(t, "head_norm.weight", 384, D_ONE);
    lin(t, "head.0.weight", 128, 384);
    t1(t, "head.0.bias", 128, D_ZERO);
    lin(t, "head.3.weight", 1, 128);
    t1(t, "head.3.bias", 1, D_ZERO);
}

/* Writes the table as `magic` container (tensor count, then name, rank, dims, element count, fp32 values per
 * tensor) drawing values in table order from one seeded stream.  0 on success, -1 on I/O failure. */
static int write_table(const char* path, const char* magic, const Table* t, uint64_t seed, char hex[65],
                       long long* params_out, size_t* bytes_out) {
    FILE* f = fopen(path, "wb");
    if (!f) return -1;
    shv_sha256 h;
    shv_sha256_init(&h);
    Rng r;
    rng_seed(&r, seed);
    long long params = 0;
    size_t bytes = 0;
    int ok = 1;
#define PUT(p, n)                                              \
    do {                                                       \
        if (fwrite((p), 1, (n), f) != (size_t)(n)) ok = 0;     \
        shv_sha256_update(&h, (p), (n));                       \
        bytes += (n);                                          \
    } while (0)
    PUT(magic, 8);
    const uint32_t count = (uint32_t)t->n;
    PUT(&count, 4);
    for (int i = 0; i < t->n && ok; ++i) {
        const Spec* s = &t->v[i];
        const uint32_t nl = (uint32_t)strlen(s->name), rank = (uint32_t)s->rank;
        PUT(&nl, 4);
        PUT(s->name, nl);
        PUT(&rank, 4);
        for (int d = 0; d < s->rank; ++d) { const uint32_t dim = (uint32_t)s->dims[d]; PUT(&dim, 4); }
        const uint64_t e = numel(s);
        PUT(&e, 8);
        float* buf = (float*)malloc(sizeof(float) * e);
        fill(s, buf, &r);
        PUT(buf, sizeof(float) * e);
        free(buf);
        if (s->param) params += (long long)e;
    }
#undef PUT
    if (fclose(f) != 0) ok = 0;
    uint8_t dg[32];
    shv_sha256_final(&h, dg);
    shv_sha256_hex(dg, hex);
    if (params_out) *params_out = params;
    if (bytes_out) *bytes_out = bytes;
    return ok ? 0 : -1;
}

/* ---------------------------------------------------------------------------------------------- C API */
/* Writes `path` (SHLDV001) and `path`.json.  Returns 0 on success, -1 on I/O failure.  sha_hex (65 bytes) may be
 * NULL; parameter/tensor totals may be NULL. */
SHV_SYNTH_API int shv_synth_weights(const char* path, uint64_t seed, double threshold, char* sha_hex,
                                     long long* parameters, int* tensors) {
    Table t = {0};
    build_table(&t);
    char hex[65];
    long long params = 0;
    size_t bytes = 0;
    int ok = write_table(path, "SHLDV001", &t, seed, hex, &params, &bytes) == 0;
    if (ok) {
        char jp[4096];
        snprintf(jp, sizeof jp, "%s.json", path);
        FILE* j = fopen(jp, "w");
        if (!j) ok = 0;
        else {
            fprintf(j,
                    "{\n \"format\": \"SHLDV001\",\n \"generator\": \"shv_synth_weights\",\n \"seed\": %llu,\n"
                    " \"threshold\": %.17g,\n \"parameters\": %lld,\n \"tensor_count\": %d,\n"
                    " \"output_bytes\": %zu,\n \"output_sha256\": \"%s\"\n}\n",
                    (unsigned long long)seed, threshold, params, t.n, bytes, hex);
            if (fclose(j) != 0) ok = 0;
        }
    }
    if (sha_hex) memcpy(sha_hex, hex, 65);
    if (parameters) *parameters = params;
    if (tensors) *tensors = t.n;
    free(t.v);
    return ok ? 0 : -1;
}

/* The SHIELD-A frontend's tensors, names and shapes as engine/audio/frontend.cpp:148-160 validates them (the
 * export's frontend.window and frontend.fb included, engine/audio/export.py:35) */
static void bn_drawn(Table* t, const char* prefix, int c) {
    char n[96];
    int d[1] = {c};
    snprintf(n, sizeof n, "%s.weight", prefix); add(t, n, 1, d, D_BN_W, 0, 0, 1);
    snprintf(n, sizeof n, "%s.bias", prefix); add(t, n, 1, d, D_BN_B, 0, 0, 1);
    snprintf(n, sizeof n, "%s.running_mean", prefix); add(t, n, 1, d, D_BN_B, 0, 0, 0);
    snprintf(n, sizeof n, "%s.running_var", prefix); add(t, n, 1, d, D_BN_VAR, 0, 0, 0);
}
static void build_audio_frontend_table(Table* t) {
    char n[96];
    t1(t, "frontend.mean", 80, D_MEL_MEAN);
    t1(t, "frontend.std", 80, D_MEL_STD);
    { int d[1] = {400}; add(t, "frontend.window", 1, d, D_WINDOW, 0, 0, 0); }
    { int d[2] = {80, 257}; add(t, "frontend.fb", 2, d, D_MELFB, 0, 0, 0); }
    conv(t, "cnn.stem.0.weight", 32, 1, 3);
    bn_drawn(t, "cnn.stem.1", 32);
    static const int channels[4] = {48, 96, 160, 192};
    int ci = 32;
    for (int s = 0; s < 4; ++s)
        for (int b = 0; b < 2; ++b) {
            const int co = channels[s], hid = 2 * ci;
            snprintf(n, sizeof n, "cnn.stages.%d.%d.pw1.0.weight", s, b); conv(t, n, hid, ci, 1);
            snprintf(n, sizeof n, "cnn.stages.%d.%d.pw1.1", s, b); bn_drawn(t, n, hid);
            snprintf(n, sizeof n, "cnn.stages.%d.%d.dw.0.weight", s, b); conv(t, n, hid, 1, 3);
            snprintf(n, sizeof n, "cnn.stages.%d.%d.dw.1", s, b); bn_drawn(t, n, hid);
            snprintf(n, sizeof n, "cnn.stages.%d.%d.pw2.0.weight", s, b); conv(t, n, co, hid, 1);
            snprintf(n, sizeof n, "cnn.stages.%d.%d.pw2.1", s, b); bn_drawn(t, n, co);
            ci = co;
        }
    conv(t, "cnn.freq_attn.weight", 1, 192, 1);
    t1(t, "cnn.freq_attn.bias", 1, D_ZERO);
    lin(t, "cnn.proj.weight", 384, 192);
}

/* The whole SHIELD-A model (SHLDA001): the sequence-stage tensors drawn exactly as shv_synth_audio_weights draws
 * them from the same seed, then the frontend's.  0 on success, -1 on I/O failure; sha_hex may be NULL. */
SHV_SYNTH_API int shv_synth_audio_model_weights(const char* path, uint64_t seed, char* sha_hex, int* tensors) {
    Table t = {0};
    build_audio_table(&t);
    build_audio_frontend_table(&t);
    char hex[65];
    const int rc = write_table(path, "SHLDA001", &t, seed, hex, NULL, NULL);
    if (sha_hex) memcpy(sha_hex, hex, 65);
    if (tensors) *tensors = t.n;
    free(t.v);
    return rc;
}

/* SHIELD-A sequence-stage weights (SHLDA001) at `path`.  0 on success, -1 on I/O failure; sha_hex may be NULL. */
SHV_SYNTH_API int shv_synth_audio_weights(const char* path, uint64_t seed, char* sha_hex, int* tensors) {
    Table t = {0};
    build_audio_table(&t);
    char hex[65];
    const int rc = write_table(path, "SHLDA001", &t, seed, hex, NULL, NULL);
    if (sha_hex) memcpy(sha_hex, hex, 65);
    if (tensors) *tensors = t.n;
    free(t.v);
    return rc;
}

/* n uniform bytes on {0..255} from `seed` (crops: 172800 bytes per frame, 20 frames per clip). */
SHV_SYNTH_API void shv_synth_bytes(uint8_t* out, size_t n, uint64_t seed) {
    Rng r;
    rng_seed(&r, seed);
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        const uint64_t x = rng_next(&r);
        memcpy(out + i, &x, 8);
    }
    if (i < n) {
        const uint64_t x = rng_next(&r);
        memcpy(out + i, &x, n - i);
    }
}

/* SHA-256 of a buffer (hex), for fixture checks of generated inputs. */
SHV_SYNTH_API void shv_synth_sha256(const void* data, size_t n, char* hex) {
    shv_sha256 h;
    uint8_t dg[32];
    shv_sha256_init(&h);
    shv_sha256_update(&h, data, n);
    shv_sha256_final(&h, dg);
    shv_sha256_hex(dg, hex);
}
