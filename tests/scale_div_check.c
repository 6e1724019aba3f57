/* CPU check of the quantisers' shared-scale division (quant.hip, ScaleDiv):
 * for a block scale s = amax/448 with finite s >= 2^-64, r = 1/s and
 *   q0 = x*r,  q1 = q0 + (x - q0*s)*r,  q2 = q1 + (x - q1*s)*r  (FMAs),
 * with x's sign, must equal the IEEE quotient x/s wherever |x/s| >= 2^-12
 * (the range in which the fp32 quotient can change an E4M3 code) and be
 * below 2^-11 with the same sign elsewhere. Scales are drawn over the whole
 * fp32 range, near 1 and near the 2^-64 bound; x runs through every bf16
 * value of magnitude <= amax and random fp32 values below amax, both signs.
 * Usage: scale_div_check <number of scales> ; exit status 0 when no case
 * fails. Built with -ffp-contract=off so x*r and x/s round on their own. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static uint64_t state = 88172645463325252ull;
static uint64_t rnd(void) { state ^= state << 13; state ^= state >> 7; state ^= state << 17; return state; }
static long long bad = 0, total = 0;

static void check(float x, float s, float r)
{
    volatile float want = x / s;
    const float q0 = x * r;
    const float q1 = fmaf(fmaf(-q0, s, x), r, q0);
    const float q2 = copysignf(fmaf(fmaf(-q1, s, x), r, q1), x);
    int ok;
    if (fabsf(want) >= 0x1p-12f)
        ok = f2u(q2) == f2u(want);
    else
        ok = fabsf(q2) < 0x1p-11f && signbit(q2) == signbit(want);
    total++;
    if (!ok) {
        if (bad < 10)
            printf("x=%a s=%a want=%a got=%a\n", x, s, want, q2);
        bad++;
    }
}

int main(int argc, char** argv)
{
    const int nscales = argc > 1 ? atoi(argv[1]) : 1000;
    for (int t = 0; t < nscales; t++) {
        uint32_t au = (uint32_t)(rnd() % 0x7F7FFFFFu) + 1u;
        if (t % 4 == 0)
            au = 0x1FE00000u + (uint32_t)(rnd() % 0x01000000u); /* s near 2^-64 */
        if (t % 4 == 1)
            au = 0x3F000000u + (uint32_t)(rnd() % 0x02000000u); /* amax near 1 */
        const float amax = u2f(au);
        const float s = amax / 448.0f;
        if (!(s >= 0x1p-64f))
            continue; /* the kernels divide for these scales */
        const float r = 1.0f / s;
        for (uint32_t h = 0; h < 0x7F80u; h++) {
            const float x = u2f(h << 16);
            if (x > amax)
                break;
            check(x, s, r);
            check(-x, s, r);
        }
        for (int k = 0; k < 20000; k++) {
            const float x = u2f((uint32_t)(rnd() % ((uint64_t)au + 1)));
            check(x, s, r);
            check(-x, s, r);
        }
        check(amax, s, r);
        check(-amax, s, r);
    }
    printf("checked %lld quotients, %lld mismatches\n", total, bad);
    return bad != 0;
}
