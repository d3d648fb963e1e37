/* Exhaustive check of the division-by-6 formula the HIP kernels use for hardswish / hardsigmoid
 * (shield-sisa_amd/csrc/dev_common.hpp: div6): q = v * fp32(1/6); q = fma(fma(-q, 6, v), fp32(1/6), q).
 * For every finite fp32 v the result is compared with the IEEE quotient v / 6.0f.  Prints the number of
 * mismatches and the largest |v| that mismatches; the kernels fall back to the division below that bound. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

int main(void) {
    const float r = 0.16666667163372039794921875f;
    unsigned long long bad = 0;
    float worst = 0.0f;
#pragma omp parallel for reduction(+ : bad) reduction(max : worst) schedule(static)
    for (long long u = 0; u <= 0xFFFFFFFFLL; ++u) {
        const uint32_t b = (uint32_t)u;
        float v;
        memcpy(&v, &b, 4);
        if (!isfinite(v)) continue;
        const float ref = v / 6.0f;
        float q = v * r;
        q = fmaf(fmaf(-q, 6.0f, v), r, q);
        if (memcmp(&ref, &q, 4) != 0) {
            bad++;
            if (fabsf(v) > worst) worst = fabsf(v);
        }
    }
    printf("%llu %.9g\n", bad, (double)worst);
    return 0;
}
