/* Exhaustive checks of the correctly rounded exp and log: TEST INFRASTRUCTURE ONLY (see gemvq_oracle.h).
 *
 * Every binary32 bit pattern is evaluated. The correctly rounded result is taken from an 80-bit libm evaluation
 * (expl / logl, error about one unit in 2^-63) rounded once to binary32; where that value lies within 16 units of
 * its last place of a binary32 rounding boundary, the quad-precision evaluation (expq / logq, 113 bits) decides. */
#include "gemvq_oracle.h"

#include <math.h>
#include <quadmath.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t fbits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline float bitsf(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* the binary32 value nearest to v (long double), and whether v is within 16 of its units of a rounding boundary */
static float round_ld(long double v, int * near_boundary) {
    const float f = (float)v;
    *near_boundary = 0;
    const long double fd = (long double)f;
    if (fd == v || isinf(f) || f == 0.0f) {
        /* on a binary32 value (a boundary is half a binary32 unit away), or at the ends of the range */
        if (isinf(f) || f == 0.0f) *near_boundary = fd != v;  /* decide the ends in quad precision */
        return f;
    }
    const uint32_t b = fbits(f);
    const float g = bitsf(fabsl(v) > fabsl(fd) ? b + 1 : b - 1);
    const long double mid = 0.5L * (fd + (long double)g);
    int e;
    frexpl(v, &e);
    const long double unit = ldexpl(1.0L, e - 64);
    *near_boundary = fabsl(v - mid) <= 16.0L * unit;
    return f;
}

static float cr_reference(int fn, float x, int * hard) {
    int near;
    const float f = round_ld(fn == 0 ? expl((long double)x) : logl((long double)x), &near);
    *hard = near;
    if (!near) return f;
    const __float128 q = fn == 0 ? expq((__float128)x) : logq((__float128)x);
    return (float)q;
}

static int same(float a, float b) { return (a != a && b != b) || fbits(a) == fbits(b); }

static float orc_cr(int fn, float x) { return fn == 0 ? orc_cr_expf(x) : orc_cr_logf(x); }

/* Inputs whose evaluation is not a special case: exp on [-110, 89], log on positive finite values. */
static int interesting(int fn, float x) {
    if (x != x) return 0;
    return fn == 0 ? (x >= -110.0f && x <= 89.0f) : (x > 0.0f && x < INFINITY);
}

void orc_crmath_check(int fn, int n_threads, uint64_t out[4]) {
    uint64_t bad = 0, libm = 0, hard = 0, n = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : bad, libm, hard, n) num_threads(n_threads > 0 ? n_threads : 1)
    for (int64_t hi = 0; hi < (1 << 16); ++hi) {
        for (uint32_t lo = 0; lo < (1u << 16); ++lo) {
            const float x = bitsf((uint32_t)(hi << 16) | lo);
            const float y = orc_cr(fn, x);
            const float l = fn == 0 ? expf(x) : logf(x);
            libm += !same(y, l);
            if (!interesting(fn, x)) {
                /* the special cases: NaN, zero, infinity, overflow and underflow ends */
                const float r = fn == 0 ? (x != x ? x : x > 89.0f ? INFINITY : 0.0f)
                                        : (x != x || x < 0.0f ? NAN : x == 0.0f ? -INFINITY : x);
                bad += !same(y, r);
                continue;
            }
            int h;
            const float r = cr_reference(fn, x, &h);
            hard += (uint64_t)h;
            bad += !same(y, r);
            ++n;
        }
    }
    out[0] = bad;
    out[1] = libm;
    out[2] = hard;
    out[3] = n;
}

uint64_t orc_crmath_compare(int fn, float (*other)(float), int n_threads) {
    uint64_t diff = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : diff) num_threads(n_threads > 0 ? n_threads : 1)
    for (int64_t hi = 0; hi < (1 << 16); ++hi)
        for (uint32_t lo = 0; lo < (1u << 16); ++lo) {
            const float x = bitsf((uint32_t)(hi << 16) | lo);
            diff += !same(orc_cr(fn, x), other(x));
        }
    return diff;
}

/* Block hashes over all inputs: block b covers the bit patterns b 2^20 .. b 2^20 + 2^20 - 1; its hash is the sum
 * modulo 2^64 of bits(f(x)) * (2 i + 1) over the block's patterns i (NaN results count as 0x7fc00000). */
void orc_crmath_hash(int fn, uint64_t * hashes, int n_threads) {
#pragma omp parallel for schedule(dynamic, 8) num_threads(n_threads > 0 ? n_threads : 1)
    for (int blk = 0; blk < 4096; ++blk) {
        uint64_t h = 0;
        for (uint32_t i = 0; i < (1u << 20); ++i) {
            const float y = orc_cr(fn, bitsf(((uint32_t)blk << 20) | i));
            const uint32_t yb = y != y ? 0x7fc00000u : fbits(y);
            h += (uint64_t)yb * (2ull * i + 1ull);
        }
        hashes[blk] = h;
    }
}
