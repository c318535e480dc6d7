/* libm_check.c - CPU checks of the device restatements of expf/exp (qmsg_libm.h) against the
 * C library the reference links (glibc: src/model.c:424 expf, src/model.c:1049 exp).
 * Test infrastructure: part of liboracle.so, called only by tests/. */
#include "qmsg_libm.h"

#include <math.h>
#include <stdint.h>
#include <string.h>

static inline int same_f(float a, float b)
{
    uint32_t ua, ub;
    memcpy(&ua, &a, 4);
    memcpy(&ub, &b, 4);
    return ua == ub || (isnan(a) && isnan(b));
}

static inline int same_d(double a, double b)
{
    uint64_t ua, ub;
    memcpy(&ua, &a, 8);
    memcpy(&ub, &b, 8);
    return ua == ub || (isnan(a) && isnan(b));
}

/* Inputs with bit patterns in [lo, hi) (hi up to 2^32) where qmsg_expf differs from expf. */
uint64_t orc_expf_mismatches(uint64_t lo, uint64_t hi)
{
    uint64_t bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static, 1 << 20)
    for (int64_t i = (int64_t)lo; i < (int64_t)hi; i++) {
        const uint32_t u = (uint32_t)i;
        float x;
        memcpy(&x, &u, 4);
        bad += !same_f(qmsg_expf(x), expf(x));
    }
    return bad;
}

/* n seeded inputs where qmsg_exp differs from exp: uniform on [-60, 0] and [-800, 0] (the
 * softmax's x - max range, through the scaled paths near underflow), differences of two
 * floats (what the softmax actually forms), and arbitrary bit patterns. */
uint64_t orc_exp_mismatches(uint64_t seed, int64_t n)
{
    uint64_t bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static, 1 << 16)
    for (int64_t i = 0; i < n; i++) {
        uint64_t z = (seed + (uint64_t)i) * 0x9e3779b97f4a7c15ull;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        z ^= z >> 31;
        double x;
        switch (i & 3) {
        case 0: x = -(double)(z >> 11) * 0x1p-53 * 60.0; break;
        case 1: x = -(double)(z >> 11) * 0x1p-53 * 800.0; break;
        case 2: {
            const float a = (float)((double)(z >> 40) * 0x1p-24 * 20.0);
            const float b = (float)((double)((z >> 16) & 0xffffff) * 0x1p-24 * 20.0);
            x = (double)a - (double)b;
            if (x > 0) x = -x;
            break;
        }
        default: memcpy(&x, &z, 8); break;
        }
        bad += !same_d(qmsg_exp(x), exp(x));
    }
    return bad;
}
