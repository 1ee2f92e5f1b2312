/*
 * Exhaustive check that the expf method used by the device kernels (the
 * table-driven exp2 method of ARM's optimized-routines, double evaluation with
 * the range reduction fused into fma) returns exactly the host libm's expf for
 * every float in the method's main path, (-103.97, 88.72).  Prints the number
 * of mismatches; exit status 0 when there are none.
 *
 * The table is recomputed here from its definition (2^(i/32) rounded to
 * double) by long division-free bisection in 128-bit integers, so a wrong
 * table entry in the device source also shows up as a mismatch: the device
 * table is compared against this one by tests/test_expf_method.py.
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static uint64_t table[32];

/* floor(2^(i/32) * 2^52) by bisection on y^32 <= 2^(i + 52*32), exact in
 * multiprecision arithmetic of 64-bit limbs (y < 2^53, y^32 < 2^1696). */
typedef struct { uint64_t w[28]; } big;
static void big_mul(big *r, const big *a, uint64_t b) {
    unsigned __int128 carry = 0;
    for (int i = 0; i < 28; i++) {
        unsigned __int128 p = (unsigned __int128)a->w[i] * b + carry;
        r->w[i] = (uint64_t)p;
        carry = p >> 64;
    }
}
static int big_cmp(const big *a, const big *b) {
    for (int i = 27; i >= 0; i--)
        if (a->w[i] != b->w[i]) return a->w[i] < b->w[i] ? -1 : 1;
    return 0;
}
static void pow2_big(big *r, int e) {
    memset(r, 0, sizeof(*r));
    r->w[e / 64] = 1ull << (e % 64);
}
static int y32_le(uint64_t y, const big *limit) {
    big acc;
    memset(&acc, 0, sizeof(acc));
    acc.w[0] = 1;
    for (int k = 0; k < 32; k++) big_mul(&acc, &acc, y);
    return big_cmp(&acc, limit) <= 0;
}
static void make_table(void) {
    for (int i = 0; i < 32; i++) {
        /* y = 2^(i/32) * 2^52 in [2^52, 2^53): y^32 = 2^(i + 1664) */
        big limit;
        pow2_big(&limit, i + 52 * 32);
        uint64_t lo = 1ull << 52, hi = 1ull << 53;
        while (hi - lo > 1) {
            uint64_t mid = lo + (hi - lo) / 2;
            if (y32_le(mid, &limit)) lo = mid; else hi = mid;
        }
        /* round to nearest: compare (lo + 1/2)^32 = ((2 lo + 1)/2)^32 with 2^(i+1664),
         * i.e. (2 lo + 1)^32 with 2^(i + 1664 + 32) */
        big lim2;
        pow2_big(&lim2, i + 52 * 32 + 32);
        uint64_t m = y32_le(2 * lo + 1, &lim2) ? lo + 1 : lo;
        if (i == 0) m = 1ull << 52;
        uint64_t bits = (1023ull << 52) | (m - (1ull << 52));
        table[i] = bits - ((uint64_t)i << 47);
    }
}

static float expf_method(float x) {
    uint32_t ux;
    memcpy(&ux, &x, 4);
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    double xd = x, kd = fma(inv_ln2_n, xd, shift), r, s, z, y;
    uint64_t ki, t;
    memcpy(&ki, &kd, 8);
    kd -= shift;
    r = fma(inv_ln2_n, xd, -kd);
    t = table[ki & 31] + (ki << 47);
    memcpy(&s, &t, 8);
    z = fma(c0, r, c1);
    y = fma(c2, r, 1.0);
    y = fma(z, r * r, y);
    return (float)(y * s);
}

int main(int argc, char **argv) {
    make_table();
    if (argc > 1) { /* print the table for comparison with the device source */
        for (int i = 0; i < 32; i++) printf("0x%016llx\n", (unsigned long long)table[i]);
        return 0;
    }
    long bad = 0, tested = 0;
#pragma omp parallel for reduction(+ : bad, tested) schedule(static)
    for (int64_t u = 0; u < (1ll << 32); u++) {
        uint32_t bits = (uint32_t)u;
        float x;
        memcpy(&x, &bits, 4);
        if (!(x > -0x1.9fe368p6f && x < 0x1.62e42ep6f)) continue;
        tested++;
        float a = expf(x), b = expf_method(x);
        if (memcmp(&a, &b, 4)) bad++;
    }
    printf("%ld %ld\n", bad, tested);
    return bad != 0;
}
