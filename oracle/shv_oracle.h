/* TEST INFRASTRUCTURE ONLY -- never linked into the engine, never called by its product path.
 *
 * Scalar C restatement of the SHIELD-V forward of the reference CPU engine in its exact (FP32) tier
 * (engine/model/isa_impl.hpp + engine/model/runtime.cpp).  Every output element is produced by the same
 * sequence of IEEE float operations as the reference (K blocks of 64 in GEMMs, the 16-lane partial sums and
 * fixed reduction tree of its vector code, Cephes exp for SiLU, libm expf/log1pf/sincosf for the gates), so on
 * the same libm it is bit-identical to the reference; tests/ pin it against the compiled reference engine.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. */
#ifndef SHV_ORACLE_H
#define SHV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_model orc_model;
typedef void (*orc_dump_fn)(void* ctx, const char* name, const float* data, size_t n);

/* GEMM epilogues (engine/model/net.hpp:162-172) */
enum { ORC_STORE = 0, ORC_RELU = 1, ORC_HS = 2, ORC_RES = 3, ORC_ACC = 4, ORC_ACC_DIV2 = 5, ORC_SWIGLU = 6,
       ORC_HSIG = 7, ORC_SILU = 8 };

orc_model* orc_load(const char* weights_path);   /* NULL on error (orc_last_error) */
void orc_free(orc_model* m);
const char* orc_last_error(void);

/* rgb [180][320][3] -> tokens [16][384] */
int orc_encode_frame(const orc_model* m, const uint8_t* rgb, float* tokens, orc_dump_fn dump, void* ctx);
/* tok[20] -> 16x384 blocks; logit out */
int orc_classify(const orc_model* m, const float* const* tok, float* logit, orc_dump_fn dump, void* ctx);

/* building blocks (same arithmetic as inside the forward) */
/* C[m][n] = epi(sum_k A[m][k] W[n][k]); W row-major [N][K]; SWIGLU: W rows interleaved in 16-row panels
 * (gate panel, up panel, ...) as the reference packs them; C column j for panel pair j/16. */
void orc_gemm(const float* A, int lda, int M, const float* W, const float* bias, int N, int K, float* C, int ldc,
              int epi, const float* R, int ldr);
float orc_exp(float x);     /* Cephes-style exp of the reference's vector code */
float orc_silu(float x);
float orc_hswish(float x);
/* gated delta rule of one head over T tokens (q, k already normalised, q scaled): q,k [T][64], v [T][128] */
void orc_delta_rule(const float* q, const float* k, const float* v, const float* decay, const float* beta, int T,
                    int ldq, int ldv, float* o, int ldo);

#ifdef __cplusplus
}
#endif
#endif
