/* Exhaustive check of the fp32 division by 6 the HIP kernels use for HardSwish (div6 in
 * vknn_amd/csrc/kernels/common.h): q = t * (1/6); r = fma(-q, 6, t); q' = fma(r, 1/6, q), keeping q
 * when q' is NaN. For every fp32 bit pattern t it compares q' with the correctly rounded t / 6.0f
 * (q kept when r is 0 or q' is NaN) and counts the inputs where they differ in a way an fp16 store could see: different bits,
 * unless both are NaN, or both lie below 2^-25 in magnitude with the same sign (then both round
 * to the same signed fp16 zero). The kernels' fma and multiply are IEEE round-to-nearest-even,
 * as is this host code built with -ffp-contract=off. Prints the count (0 expected). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float div6(float t) {
    const float inv6 = 1.0f / 6.0f;
    const float q    = t * inv6;
    const float r    = fmaf(-q, 6.0f, t);
    const float q2   = fmaf(r, inv6, q);
    return (r == 0.f || q2 != q2) ? q : q2;
}

int main(void) {
    unsigned long long bad = 0, subnormal_diff = 0;
#pragma omp parallel for reduction(+ : bad, subnormal_diff) schedule(static)
    for (long long i = 0; i < (1LL << 32); ++i) {
        const uint32_t u = (uint32_t) i;
        float t, a, b;
        memcpy(&t, &u, 4);
        a = t / 6.0f;
        b = div6(t);
        uint32_t ua, ub;
        memcpy(&ua, &a, 4);
        memcpy(&ub, &b, 4);
        if (ua == ub || (a != a && b != b)) continue;
        if (fabsf(a) < 0x1p-25f && fabsf(b) < 0x1p-25f && signbit(a) == signbit(b)) {
            ++subnormal_diff;
            continue;
        }
        ++bad;
    }
    printf("%llu %llu\n", bad, subnormal_diff);
    return 0;
}
