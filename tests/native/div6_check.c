/* Exhaustive check of the division by 6 the HIP kernels use for hardswish / hardsigmoid
 * (shield-sisa_amd/csrc/dev_common.hpp: div6_step, div6): the step q = v * fp32(1/6);
 * q = fma(fma(-q, 6, v), fp32(1/6), q), zero returned as itself, and the IEEE division where 0 < |v| < 2.4e-38.
 * For every finite fp32 v both the plain step and the whole function are compared with the IEEE quotient
 * v / 6.0f.  Prints the plain step's mismatch count, the largest |v| among them, and the whole function's mismatch
 * count (which must be 0). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

int main(void) {
    const float r = 0.16666667163372039794921875f;
    unsigned long long bad = 0, bad_fn = 0;
    float worst = 0.0f;
#pragma omp parallel for reduction(+ : bad, bad_fn) reduction(max : worst) schedule(static)
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
        float f = v == 0.0f ? v : q;
        if (fabsf(v) < 2.4e-38f && v != 0.0f) f = v / 6.0f;
        if (memcmp(&ref, &f, 4) != 0) bad_fn++;
    }
    printf("%llu %.9g %llu\n", bad, (double)worst, bad_fn);
    return 0;
}
