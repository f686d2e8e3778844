/* Correctly rounded binary32 exp and log for the reference-arithmetic decoder: TEST INFRASTRUCTURE ONLY (see
 * gemvq_oracle.h).
 *
 * The reference's CPU path evaluates exp and log with the host's libm (std::exp / std::log on float,
 * fpga/src/gemvq_ref.h:298-342 and 367). glibc's expf / logf are not correctly rounded and their constants are not
 * in this tree, so no independent implementation can reproduce them bit for bit. The reference-arithmetic decoder
 * therefore uses the correctly rounded functions, which a device can evaluate with the same bits: the result is the
 * binary32 value nearest to the exact e^x or log x (ties to even), which is what any libm approximates.
 *
 * Method (double-double evaluation, then one rounding to binary32):
 *   exp: x = k ln2/32 + r, |r| <= ln2/64 (+ rounding), with ln2/32 split in a 39-bit part (k times it is exact) and
 *        a double; r carried as a double-double. e^r - 1 = r + r^2/2 + ... + r^7/5040 (the quadratic and higher terms
 *        in double); e^x = 2^(k >> 5) * T[k & 31] * (1 + (e^r - 1)), T[j] = 2^(j/32) as double-doubles. Relative
 *        error below 2^-64.
 *   log: x = 2^e m, m in [sqrt(1/2), sqrt(2)); c = 1 + i/64 nearest to m (i = -19 .. 27); s = (m - c) / (m + c) as a
 *        double-double (m - c and m + c are exact); log m = log c + 2 atanh(s) = log c + 2 s + 2 s^3/3 + .. + 2 s^9/9
 *        (|s| <= 1/181); log x = e ln2 + log m, the large terms added exactly (two-sums). Relative error below 2^-64.
 *   rounding: the double-double hi + lo goes to binary32 as hi does, except where hi is exactly halfway between two
 *        binary32 values, where the sign of lo decides (and lo = 0 keeps the even one).
 * Exhaustive checks (tests/test_oracle_crmath.py): every binary32 input against an 80-bit libm evaluation (quad
 * precision where that one is within a few units of a rounding boundary); the library's device code against these
 * functions on every input, on the host and on the GPU. */
#include "gemvq_oracle.h"

#include <math.h>
#include <stdint.h>
#include <string.h>

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
static inline double pow2d(int m) { /* 2^m, -1022 <= m <= 1023 */
    const uint64_t u = (uint64_t)(m + 1023) << 52;
    double d;
    memcpy(&d, &u, 8);
    return d;
}

/* s + e = a + b exactly (Knuth's two-sum; no ordering needed) */
static inline void two_sum(double a, double b, double * s, double * e) {
    const double x = a + b, bv = x - a, av = x - bv;
    *s = x;
    *e = (a - av) + (b - bv);
}
/* p + e = a * b exactly (the fused multiply-add's single rounding gives the low part) */
static inline void two_prod(double a, double b, double * p, double * e) {
    const double x = a * b;
    *p = x;
    *e = fma(a, b, -x);
}

/* hi + lo rounded to binary32 (see the file comment) */
static float dd_to_float(double hi, double lo) {
    const float f = (float)hi;
    const double fd = (double)f;
    if (fd == hi) return f;
    /* the binary32 neighbour of f on hi's side: larger magnitude when |hi| > |f| */
    const uint32_t b = fbits(f);
    const float g = bitsf(fabs(hi) > fabs(fd) ? b + 1 : b - 1);
    const double mid = 0.5 * (fd + (double)g);
    if (hi != mid || lo == 0.0) return f;
    return ((lo > 0.0) == (fd > hi)) ? f : g;
}

static const double LN2_32_HI = 0x1.62e42fefa4000p-6;   /* ln2 / 32, 39 significant bits */
static const double LN2_32_LO = -0x1.8432a1b0e2634p-48; /* ln2 / 32 - LN2_32_HI */
static const double INV_LN2_32 = 0x1.71547652b82fep+5;  /* 32 / ln2 */
static const double EXP_T[32][2] = {  /* 2^(j/32) = hi + lo */
    {0x1.0000000000000p+0, 0x0.0p+0},
    {0x1.059b0d3158574p+0, 0x1.d73e2a475b465p-55},
    {0x1.0b5586cf9890fp+0, 0x1.8a62e4adc610bp-54},
    {0x1.11301d0125b51p+0, -0x1.6c51039449b3ap-54},
    {0x1.172b83c7d517bp+0, -0x1.19041b9d78a76p-55},
    {0x1.1d4873168b9aap+0, 0x1.e016e00a2643cp-54},
    {0x1.2387a6e756238p+0, 0x1.9b07eb6c70573p-54},
    {0x1.29e9df51fdee1p+0, 0x1.612e8afad1255p-55},
    {0x1.306fe0a31b715p+0, 0x1.6f46ad23182e4p-55},
    {0x1.371a7373aa9cbp+0, -0x1.63aeabf42eae2p-54},
    {0x1.3dea64c123422p+0, 0x1.ada0911f09ebcp-55},
    {0x1.44e086061892dp+0, 0x1.89b7a04ef80d0p-59},
    {0x1.4bfdad5362a27p+0, 0x1.d4397afec42e2p-56},
    {0x1.5342b569d4f82p+0, -0x1.07abe1db13cadp-55},
    {0x1.5ab07dd485429p+0, 0x1.6324c054647adp-54},
    {0x1.6247eb03a5585p+0, -0x1.383c17e40b497p-54},
    {0x1.6a09e667f3bcdp+0, -0x1.bdd3413b26456p-54},
    {0x1.71f75e8ec5f74p+0, -0x1.16e4786887a99p-55},
    {0x1.7a11473eb0187p+0, -0x1.41577ee04992fp-55},
    {0x1.82589994cce13p+0, -0x1.d4c1dd41532d8p-54},
    {0x1.8ace5422aa0dbp+0, 0x1.6e9f156864b27p-54},
    {0x1.93737b0cdc5e5p+0, -0x1.75fc781b57ebcp-57},
    {0x1.9c49182a3f090p+0, 0x1.c7c46b071f2bep-56},
    {0x1.a5503b23e255dp+0, -0x1.d2f6edb8d41e1p-54},
    {0x1.ae89f995ad3adp+0, 0x1.7a1cd345dcc81p-54},
    {0x1.b7f76f2fb5e47p+0, -0x1.5584f7e54ac3bp-56},
    {0x1.c199bdd85529cp+0, 0x1.11065895048ddp-55},
    {0x1.cb720dcef9069p+0, 0x1.503cbd1e949dbp-56},
    {0x1.d5818dcfba487p+0, 0x1.2ed02d75b3707p-55},
    {0x1.dfc97337b9b5fp+0, -0x1.1a5cd4f184b5cp-54},
    {0x1.ea4afa2a490dap+0, -0x1.e9c23179c2893p-54},
    {0x1.f50765b6e4540p+0, 0x1.9d3e12dd8a18bp-54},
};

float orc_cr_expf(float x) {
    if (x != x) return x + x;
    if (x > 89.0f) return INFINITY;  /* e^89 > 2^128 */
    if (x < -110.0f) return 0.0f;    /* e^-110 < 2^-158 */
    const double xd = (double)x;
    const double kd = rint(xd * INV_LN2_32);
    double r0, re;
    two_sum(xd, -(kd * LN2_32_HI), &r0, &re);  /* kd * LN2_32_HI is exact (13 + 39 bits) */
    double rh, rl;
    two_sum(r0, -(kd * LN2_32_LO), &rh, &rl);
    rl += re;
    /* e^r - 1 = rh + (rl + rh rl + rh^2 (1/2 + rh / 6 + .. + rh^5 / 5040)) */
    const double q = (rh * rh) * (0.5 + rh * (1.0 / 6 + rh * (1.0 / 24 + rh * (1.0 / 120 + rh * (1.0 / 720 + rh * (1.0 / 5040))))));
    double ph, pl;
    two_sum(rh, rl + (rh * rl + q), &ph, &pl);
    const int k = (int)kd, j = k & 31, m = (k - j) / 32;
    const double th = EXP_T[j][0], tl = EXP_T[j][1];
    /* T (1 + p) = th + th ph + (th pl + tl + tl ph) */
    double ah, al, sh, sl, yh, yl;
    two_prod(th, ph, &ah, &al);
    two_sum(th, ah, &sh, &sl);
    two_sum(sh, sl + (al + (th * pl + (tl + tl * ph))), &yh, &yl);
    const double s = pow2d(m);  /* -159 <= m <= 128: exact scaling */
    return dd_to_float(yh * s, yl * s);
}

static const double LN2_HI = 0x1.62e42fefa3a00p-1;    /* ln2, 44 significant bits */
static const double LN2_LO = -0x1.0ca86c3898d00p-49;  /* ln2 - LN2_HI */
static const double SQRT2 = 0x1.6a09e667f3bcdp+0;
static const double LOG_C[47][2] = {  /* log(1 + i/64) = hi + lo, i = -19 .. 27 */
    {-0x1.68ac83e9c6a14p-2, -0x1.a64eadd740178p-58},
    {-0x1.522ae0738a3d8p-2, 0x1.8f7e9b38a6979p-57},
    {-0x1.3c25277333184p-2, 0x1.2ad27e50a8ec6p-56},
    {-0x1.269621134db92p-2, -0x1.e0efadd9db02bp-56},
    {-0x1.1178e8227e47cp-2, 0x1.0e63a5f01c691p-57},
    {-0x1.f991c6cb3b379p-3, -0x1.f665066f980a2p-57},
    {-0x1.d1037f2655e7bp-3, -0x1.60629242471a2p-57},
    {-0x1.a93ed3c8ad9e3p-3, -0x1.bcafa9de97203p-57},
    {-0x1.823c16551a3c2p-3, 0x1.1232ce70be781p-57},
    {-0x1.5bf406b543db2p-3, 0x1.1f5b44c0df7e7p-61},
    {-0x1.365fcb0159016p-3, -0x1.7d411a5b944adp-58},
    {-0x1.1178e8227e47cp-3, 0x1.0e63a5f01c691p-58},
    {-0x1.da727638446a2p-4, -0x1.401fa71733019p-58},
    {-0x1.9335e5d594989p-4, 0x1.478a85704ccb7p-58},
    {-0x1.4d3115d207eacp-4, -0x1.769f42c7842ccp-58},
    {-0x1.08598b59e3a07p-4, 0x1.dd7009902bf32p-58},
    {-0x1.894aa149fb343p-5, -0x1.a8be97660a23dp-60},
    {-0x1.0415d89e74444p-5, -0x1.c05cf1d753622p-59},
    {-0x1.0205658935847p-6, -0x1.27c8e8416e71fp-60},
    {0x0.0p+0, 0x0.0p+0},
    {0x1.fc0a8b0fc03e4p-7, -0x1.83092c59642a1p-62},
    {0x1.f829b0e783300p-6, 0x1.33e3f04f1ef23p-60},
    {0x1.77458f632dcfcp-5, 0x1.18d3ca87b9296p-59},
    {0x1.f0a30c01162a6p-5, 0x1.85f325c5bbacdp-59},
    {0x1.341d7961bd1d1p-4, -0x1.b599f227becbbp-58},
    {0x1.6f0d28ae56b4cp-4, -0x1.906d99184b992p-58},
    {0x1.a926d3a4ad563p-4, 0x1.942f48aa70ea9p-58},
    {0x1.e27076e2af2e6p-4, -0x1.61578001e0162p-60},
    {0x1.0d77e7cd08e59p-3, 0x1.9a5dc5e9030acp-57},
    {0x1.29552f81ff523p-3, 0x1.301771c407dbfp-57},
    {0x1.44d2b6ccb7d1ep-3, 0x1.9f4f6543e1f88p-57},
    {0x1.5ff3070a793d4p-3, -0x1.bc60efafc6f6ep-58},
    {0x1.7ab890210d909p-3, 0x1.be36b2d6a0608p-59},
    {0x1.9525a9cf456b4p-3, 0x1.d904c1d4e2e26p-57},
    {0x1.af3c94e80bff3p-3, -0x1.398cff3641985p-58},
    {0x1.c8ff7c79a9a22p-3, -0x1.4f689f8434012p-57},
    {0x1.e27076e2af2e6p-3, -0x1.61578001e0162p-59},
    {0x1.fb9186d5e3e2bp-3, -0x1.caaae64f21acbp-57},
    {0x1.0a324e27390e3p-2, 0x1.7dcfde8061c03p-56},
    {0x1.1675cababa60ep-2, 0x1.ce63eab883717p-61},
    {0x1.22941fbcf7966p-2, -0x1.76f5eb09628afp-56},
    {0x1.2e8e2bae11d31p-2, -0x1.8f4cdb95ebdf9p-56},
    {0x1.3a64c556945eap-2, -0x1.c68651945f97cp-57},
    {0x1.4618bc21c5ec2p-2, 0x1.f42decdeccf1dp-56},
    {0x1.51aad872df82dp-2, 0x1.3927ac19f55e3p-59},
    {0x1.5d1bdbf5809cap-2, 0x1.4236383dc7fe1p-56},
    {0x1.686c81e9b14afp-2, -0x1.ddea0f7f58e3dp-57},
};

float orc_cr_logf(float x) {
    if (x != x) return x + x;
    if (x < 0.0f) return NAN;
    if (x == 0.0f) return -INFINITY;
    uint32_t b = fbits(x);
    if (b == 0x7f800000u) return x;
    int e;
    if (b < 0x00800000u) {  /* subnormal: scale into the normal range (exact) */
        b = fbits(x * 8388608.0f);
        e = (int)(b >> 23) - 150;
    } else {
        e = (int)(b >> 23) - 127;
    }
    double md = (double)bitsf((b & 0x7fffffu) | 0x3f800000u);  /* [1, 2) */
    if (md > SQRT2) {
        md *= 0.5;
        e += 1;
    }
    const int i = (int)rint((md - 1.0) * 64.0);  /* -19 .. 27 */
    const double c = 1.0 + (double)i * 0.015625;
    const double f = md - c, g = md + c;          /* both exact */
    const double sh = f / g, sl = fma(-sh, g, f) / g;
    const double s2 = sh * sh;
    const double tail = (sh * s2) * (2.0 / 3 + s2 * (2.0 / 5 + s2 * (2.0 / 7 + s2 * (2.0 / 9))));
    const double ed = (double)e;
    double b1, e1, c1, e2, hi, lo;
    two_sum(ed * LN2_HI, LOG_C[i + 19][0], &b1, &e1);  /* ed * LN2_HI is exact (8 + 44 bits) */
    two_sum(b1, 2.0 * sh, &c1, &e2);
    two_sum(c1, e1 + e2 + (ed * LN2_LO + (LOG_C[i + 19][1] + (2.0 * sl + tail))), &hi, &lo);
    return dd_to_float(hi, lo);
}
