/* Exhaustive check of the identity the int4 quantizer kernels use in place
 * of a per-element fp16 division.  For every positive finite fp16 s and
 * every finite fp16 x, with r = fl32(1 / s) (correctly rounded):
 *
 *   (a) fp16_rn(x * r) == fp16_rn(x / s) whenever |x / s| >= 2^-14, both
 *       when the product x * r is exact before the one rounding to fp16
 *       (v_fma_mix*_f16) and when it is first rounded to fp32 (fp32
 *       multiply, then v_cvt_f16_f32);
 *   (b) the int4 code clamp(round_half_even(fp16(.)), -8, 7) of x * r
 *       equals that of x / s for every pair (also when the quotient is an
 *       fp16 subnormal: those codes are all 0).
 *
 * fp16(x / s) is the correctly rounded quotient that the reference's __hdiv
 * returns (signrot/kernels/fused.cu:100-104).  Why (a) holds: a quotient of
 * two 11-bit significands is never a normal-range fp16 rounding midpoint
 * (the midpoint's odd 12-bit significand cannot divide an 11-bit one) and
 * lies at relative distance > 2^-23 from each, while x * r is within
 * 2^-23 (relative) of x / s.  Subnormal-range midpoints have fewer bits, so
 * (a) can fail there (e.g. 3*2^-24 / 6 = 2^-25), which (b) makes harmless.
 *
 * Prints "<mismatches> <pairs checked>" and exits non-zero on a mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

/* fp16 bits -> double (exact). */
static double h2d(uint16_t h) {
    const int e = (h >> 10) & 0x1F, m = h & 0x3FF;
    const double v = e == 0 ? ldexp((double)m, -24) : ldexp((double)(m | 0x400), e - 25);
    return (h & 0x8000) ? -v : v;
}

/* double -> fp16 bits, round to nearest, ties to even, by integer
 * arithmetic on the double's fields (finite input; overflow -> inf). */
static uint16_t d2h(double d) {
    uint64_t b;
    memcpy(&b, &d, 8);
    const uint16_t sign = (uint16_t)((b >> 48) & 0x8000);
    const int ex = (int)((b >> 52) & 0x7FF);
    uint64_t man = b & ((1ull << 52) - 1);
    if (ex == 0 && man == 0) return sign;
    int e;
    if (ex == 0) { /* double subnormal: far below fp16's range */
        return sign;
    }
    man |= 1ull << 52;
    e = ex - 1023;
    if (e > 15) return sign | 0x7C00;
    int shift = 42; /* 52 - 10 fraction bits */
    if (e < -14) shift += -14 - e;
    if (shift > 60) return sign; /* below half the smallest subnormal */
    uint64_t q = man >> shift;
    const uint64_t rem = man & ((1ull << shift) - 1), half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) q += 1;
    if (e < -14) return sign | (uint16_t)q; /* q == 1024 is the smallest normal */
    if (q == 2048) { q = 1024; e += 1; }
    if (e > 15) return sign | 0x7C00;
    return sign | (uint16_t)(((e + 15) << 10) | (int)(q - 1024));
}

/* clamp(round_half_even(v), -8, 7) of an fp16 value; rint rounds ties to even. */
static int code(uint16_t h) {
    double r = rint(h2d(h));
    if (r < -8) r = -8;
    if (r > 7) r = 7;
    return (int)r;
}

/* The converter itself: exact on every fp16 value, ties to even at every
 * midpoint between neighbours, and to the nearer neighbour just off it. */
static int check_d2h(void) {
    for (uint32_t h = 0; h < 0x7C00; ++h) {
        if (d2h(h2d((uint16_t)h)) != h || d2h(-h2d((uint16_t)h)) != (h | 0x8000)) return 1;
        if (h + 1 < 0x7C00) {
            const double lo = h2d((uint16_t)h), hi = h2d((uint16_t)(h + 1)), mid = (lo + hi) / 2;
            const uint16_t even = (h & 1) ? (uint16_t)(h + 1) : (uint16_t)h;
            if (d2h(mid) != even) return 1;
            if (d2h(nextafter(mid, 0.0)) != h || d2h(nextafter(mid, 1e9)) != h + 1) return 1;
        }
    }
    if (d2h(65519.0) != 0x7BFF || d2h(65520.0) != 0x7C00) return 1;
    return 0;
}

int main(void) {
    if (check_d2h()) {
        printf("fp16 converter self-check failed\n");
        return 2;
    }
    uint64_t checked = 0, bad = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : checked, bad)
    for (uint32_t sb = 1; sb < 0x7C00; ++sb) {
        const double s = h2d((uint16_t)sb);
        const float r = 1.0f / (float)s;
        for (uint32_t xb = 0; xb < 0x7C00; ++xb) {
            const double x = h2d((uint16_t)xb);
            const double quot = x / s; /* 53-bit quotient: never a double-rounding hazard */
            const uint16_t want = d2h(quot);
            const uint16_t fused = d2h(x * (double)r);             /* exact product */
            const uint16_t twostep = d2h((double)((float)x * r));  /* fp32 product */
            checked += 1;
            int ok = code(fused) == code(want) && code(twostep) == code(want);
            if (quot >= 0x1p-14) ok = ok && fused == want && twostep == want;
            if (!ok) {
#pragma omp critical
                if (bad < 10)
                    printf("mismatch s=%04x x=%04x want=%04x fused=%04x twostep=%04x\n", sb, xb,
                           want, fused, twostep);
                ++bad;
            }
        }
    }
    printf("%llu %llu\n", (unsigned long long)bad, (unsigned long long)checked);
    return bad != 0;
}
