/* The soft cap's tanhf (gemma4.c:518-519 calls the host libm's tanhf), as the
 * device computes it, checked against the host libm.
 *
 * The method is glibc's single-precision tanh (sysdeps/ieee754/flt-32/
 * s_tanhf.c, from Sun's fdlibm) with its expm1f (s_expm1f.c):
 *   tanh(x) = sign(x) (1 - 2 / (expm1(2|x|) + 2))   for 1 <= |x| < 22,
 *           = sign(x) (-t / (t + 2)), t = expm1(-2|x|) for |x| < 1,
 *   = x (1 + x) below 2^-55, +-1 from 22 on, tanh(+-0) = +-0;
 *   expm1(x): x = k ln2 + r (ln2 split in a 24-bit-exact high part and a low
 *   part, k = +-1 directly near +-ln2), the rational form
 *   r1 = 1 + h (Q1 + h (Q2 + h (Q3 + h (Q4 + h Q5)))), h = r^2 / 2, and the
 *   reconstruction 2^k (1 + r - ...) - 1 arranged by the size of k.
 * Every operation is one rounded fp32 operation (no contraction), as in the
 * device code (built with -ffp-contract=off).
 *
 *   tanhf_method_check            every float with |x| < 22 (both signs):
 *                                 prints "<differing> <tested>"
 *   tanhf_method_check constants  prints Q1..Q5, ln2_hi, ln2_lo, invln2 as hex
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float from_bits(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static uint32_t to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

#ifdef PLANT_ERROR /* the test's planted mistake: Q1 one ulp off (246 inputs
                      change; one ulp in Q2..Q5 changes none: below rounding) */
static const uint32_t kQ[5] = {0xbd08888au, 0x3ad00d01u, 0xb8a670cdu, 0x36867e54u, 0xb457edbbu};
#else
static const uint32_t kQ[5] = {0xbd088889u, 0x3ad00d01u, 0xb8a670cdu, 0x36867e54u, 0xb457edbbu};
#endif
static const uint32_t kLn2Hi = 0x3f317180u, kLn2Lo = 0x3717f7d1u, kInvLn2 = 0x3fb8aa3bu;

/* expm1 for the arguments tanh passes: finite, |x| < 44 */
static float expm1_method(float x) {
    const float Q1 = from_bits(kQ[0]), Q2 = from_bits(kQ[1]), Q3 = from_bits(kQ[2]),
                Q4 = from_bits(kQ[3]), Q5 = from_bits(kQ[4]);
    const float ln2_hi = from_bits(kLn2Hi), ln2_lo = from_bits(kLn2Lo), invln2 = from_bits(kInvLn2);
    const uint32_t ux = to_bits(x), ax = ux & 0x7fffffffu;
    const int negative = (int)(ux >> 31);
    if (negative && ax >= 0x4195b844u) return -1.0f; /* x <= -27 ln2 */
    int k;
    float c = 0.0f;
    if (ax > 0x3eb17218u) {      /* |x| > ln2 / 2 */
        float hi, lo;
        if (ax < 0x3f851592u) { /* |x| < 3 ln2 / 2 */
            hi = negative ? x + ln2_hi : x - ln2_hi;
            lo = negative ? -ln2_lo : ln2_lo;
            k = negative ? -1 : 1;
        } else {
            k = (int)(invln2 * x + (negative ? -0.5f : 0.5f));
            const float t = (float)k;
            hi = x - t * ln2_hi; /* exact */
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (ax < 0x33000000u) { /* |x| < 2^-25 */
        return x;
    } else {
        k = 0;
    }
    const float hfx = 0.5f * x, hxs = x * hfx;
    const float r1 = 1.0f + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    float t = 3.0f - r1 * hfx;
    float e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = x * (e - c) - c;
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) return x < -0.25f ? -2.0f * (e - (x + 0.5f)) : 1.0f + 2.0f * (x - e);
    float y;
    if (k <= -2 || k > 56) {
        y = 1.0f - (e - x);
        y = from_bits(to_bits(y) + ((uint32_t)k << 23));
        return y - 1.0f;
    }
    if (k < 23) {
        t = from_bits(0x3f800000u - (0x1000000u >> k)); /* 1 - 2^-k */
        y = t - (e - x);
    } else {
        t = from_bits((uint32_t)(0x7f - k) << 23); /* 2^-k */
        y = x - (e + t);
        y += 1.0f;
    }
    return from_bits(to_bits(y) + ((uint32_t)k << 23));
}

static float tanh_method(float x) {
    const uint32_t ux = to_bits(x), ax = ux & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (ux >> 31) ? 1.0f / x - 1.0f : 1.0f / x + 1.0f;
    float z;
    if (ax < 0x41b00000u) { /* |x| < 22 */
        if (ax == 0) return x;
        if (ax < 0x24000000u) return x * (1.0f + x); /* |x| < 2^-55 */
        const float a = from_bits(ax);
        if (ax >= 0x3f800000u) { /* |x| >= 1 */
            const float t = expm1_method(2.0f * a);
            z = 1.0f - 2.0f / (t + 2.0f);
        } else {
            const float t = expm1_method(-2.0f * a);
            z = -t / (t + 2.0f);
        }
    } else {
        z = 1.0f;
    }
    return (ux >> 31) ? -z : z;
}

int main(int argc, char **argv) {
    if (argc > 1 && !strcmp(argv[1], "constants")) {
        for (int i = 0; i < 5; i++) printf("0x%08x\n", kQ[i]);
        printf("0x%08x\n0x%08x\n0x%08x\n", kLn2Hi, kLn2Lo, kInvLn2);
        return 0;
    }
    const uint32_t end = 0x41b00000u; /* 22.0f */
    long long bad = 0, tested = 0;
#pragma omp parallel for schedule(dynamic, 1 << 16) reduction(+ : bad, tested)
    for (long long u = 0; u < (long long)end; u++) {
        for (uint32_t sign = 0; sign < 2; sign++) {
            const float x = from_bits((uint32_t)u | (sign << 31));
            const float a = tanh_method(x), b = tanhf(x);
            tested++;
            if (to_bits(a) != to_bits(b)) {
                if (bad < 5) fprintf(stderr, "x %a: method %a libm %a\n", x, a, b);
                bad++;
            }
        }
    }
    printf("%lld %lld\n", bad, tested);
    return 0;
}
