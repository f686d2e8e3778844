/* CPU oracle for the batch-1 decode path: TEST INFRASTRUCTURE ONLY (see gemvq_oracle.h).
 * Each function cites the reference file:line whose arithmetic it restates. Paths are relative to the reference
 * repository (ohrz/fpga-llama-gguf). Built with -ffp-contract=off so no multiply-add is fused. */
#include "gemvq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------------------------ */
/* fp16 <-> fp32: gemvq_ref.h:16-52 (IEEE half, round to nearest even; overflow and NaN give infinity there).   */
float orc_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; ++sh; }
            /* value = m0 * 2^-24 with the leading bit moved to position 10 after sh shifts */
            bits = sign | ((uint32_t)(127 - 15 - sh + 1) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_float_to_half(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    const int e = (int)((bits >> 23) & 0xff) - 127 + 15;
    uint32_t m = bits & 0x7fffffu;
    if (e >= 31) return sign | 0x7c00u;
    if (e <= 0) {
        if (e < -10) return sign;
        m |= 0x800000u;
        const int sh = 14 - e;
        uint32_t r = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return sign | (uint16_t)r;
    }
    uint32_t out = ((uint32_t)e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (out & 1u))) ++out; /* a carry moves into the exponent */
    return sign | (uint16_t)out;
}

/* ggml nearest_int (gemvq_ref.h:54-60): round half to even through the FP32 addition of 1.5 * 2^23. */
int orc_nearest_int(float v) {
    const float biased = v + 12582912.f;
    int32_t b;
    memcpy(&b, &biased, 4);
    return (b & 0x007fffff) - 0x00400000;
}

/* ------------------------------------------------------------------------------------------------------------ */
/* exp / log of the canonical arithmetic. ggml uses expf/logf (gemvq_ref.h:305, 337-339); CPU and GPU libraries
 * differ in the last ulp, so both sides evaluate these formulas instead (within 2 ulp of the correctly rounded
 * value, checked against libm in the tests).
 * exp: Cody-Waite reduction x = n ln2 + r, |r| <= ln2/2, e^r by its Taylor series to r^7/7! (Horner, fused
 * multiply-adds), then the exact scaling by 2^n. Results below the normal range are flushed to +0. */
static const float ORC_LOG2E = 1.44269504088896341f;
static const float ORC_LN2_HI = 0.693145751953125f;          /* 15 significant bits: n * LN2_HI is exact */
static const float ORC_LN2_LO = 1.42860682030941723212e-6f;  /* ln 2 - LN2_HI */

static float orc_pow2i(int n) { /* 2^n for -126 <= n <= 127 */
    uint32_t b = (uint32_t)(n + 127) << 23;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

float orc_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -87.0f) return 0.0f;
    const float n = rintf(x * ORC_LOG2E);
    float r = fmaf(-n, ORC_LN2_HI, x);
    r = fmaf(-n, ORC_LN2_LO, r);
    float p = 1.0f / 5040.0f;
    p = fmaf(p, r, 1.0f / 720.0f);
    p = fmaf(p, r, 1.0f / 120.0f);
    p = fmaf(p, r, 1.0f / 24.0f);
    p = fmaf(p, r, 1.0f / 6.0f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const int ni = (int)n;
    if (ni > 127) return (p * 2.0f) * orc_pow2i(ni - 1);
    return p * orc_pow2i(ni);
}

/* log for x > 0: x = m 2^e with m in [sqrt(1/2), sqrt(2)), log m = 2 atanh(s), s = (m - 1) / (m + 1), series to
 * s^9/9, result e ln2 + log m with ln2 split in two parts. */
float orc_logf(float x) {
    if (x != x || x < 0.0f) return NAN;
    if (x == 0.0f) return -INFINITY;
    if (x == INFINITY) return x;
    uint32_t b;
    memcpy(&b, &x, 4);
    int e;
    if ((b >> 23) == 0) { /* subnormal: scale up by 2^23 exactly */
        const float xs = x * 8388608.0f;
        memcpy(&b, &xs, 4);
        e = (int)(b >> 23) - 127 - 23;
    } else {
        e = (int)(b >> 23) - 127;
    }
    uint32_t mb = (b & 0x7fffffu) | 0x3f800000u; /* m in [1, 2) */
    float m;
    memcpy(&m, &mb, 4);
    if (m > 1.41421353816986083984f) { m = m * 0.5f; e += 1; }
    const float f = m - 1.0f;
    const float s = f / (2.0f + f);
    const float s2 = s * s;
    float p = 1.0f / 9.0f;
    p = fmaf(p, s2, 1.0f / 7.0f);
    p = fmaf(p, s2, 1.0f / 5.0f);
    p = fmaf(p, s2, 1.0f / 3.0f);
    p = p * s2;
    /* log m = 2s + 2s * p */
    const float two_s = 2.0f * s;
    const float logm = fmaf(two_s, p, two_s);
    const float ef = (float)e;
    return fmaf(ef, ORC_LN2_HI, fmaf(ef, ORC_LN2_LO, logm));
}

/* SiLU, sigmoid, softplus in ggml's forms (gemvq_ref.h:332-342, gemvqc_ops.h:64-79). */
float orc_silu(float x) { return x / (1.0f + orc_expf(-x)); }
float orc_sigmoid(float x) { return 1.0f / (1.0f + orc_expf(-x)); }
float orc_softplus(float x) { return x > 20.0f ? x : orc_logf(1.0f + orc_expf(x)); }

/* Canonical FP32 reduction: pairwise tree over element indices on a power-of-two padded copy (the order of the
 * reference kernel's tree16/tree8 word sums, gemvqc_ops.h:51-60, gemvqc_gdn.h:48-56, extended to any length). */
float orc_pair_sum(const float * a, int n) {
    if (n <= 0) return 0.0f;
    int p = 1;
    while (p < n) p <<= 1;
    float stack[1024];
    float * t = p <= 1024 ? stack : (float *)malloc(sizeof(float) * (size_t)p);
    memcpy(t, a, (size_t)n * sizeof(float));
    for (int i = n; i < p; ++i) t[i] = 0.0f;
    for (int s = 1; s < p; s *= 2)
        for (int i = 0; i < p; i += 2 * s) t[i] = t[i] + t[i + s];
    const float r = t[0];
    if (t != stack) free(t);
    return r;
}

size_t orc_row_bytes(int fmt, int cols) {
    switch (fmt) {
    case ORC_Q4_0: return (size_t)(cols / 32) * 18;
    case ORC_Q4_1: return (size_t)(cols / 32) * 20;
    case ORC_Q8_0: return (size_t)(cols / 32) * 34;
    case ORC_Q5_K: return (size_t)(cols / 256) * 176;
    case ORC_Q6_K: return (size_t)(cols / 256) * 210;
    default: return 0;
    }
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Activation quantizers. Q8_0: gemvq_ref.h:236-245 (d = amax / 127, id = 1 / d, roundf half away from zero, the
 * scale stored as fp16; gemvqw_engine.h:95-158 does the same). */
void orc_quantize_q8_0(const float * x, int n, int8_t * q, uint16_t * d_bits) {
    for (int b = 0; b < n / 32; ++b) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[b * 32 + j]));
        const float s = amax / 127.0f, id = s != 0.0f ? 1.0f / s : 0.0f;
        d_bits[b] = orc_float_to_half(s);
        for (int j = 0; j < 32; ++j) q[b * 32 + j] = (int8_t)roundf(x[b * 32 + j] * id);
    }
}

/* Q8_1 (gemvq_ref.h:201-212, ggml quantize_row_q8_1_ref): d = amax / 127, q = roundf(x / d), d_bits = fp16(d),
 * s_bits = fp16(sum(q) * d) with the FP32 d. */
void orc_quantize_q8_1(const float * x, int n, int8_t * q, uint16_t * d_bits, uint16_t * s_bits) {
    for (int b = 0; b < n / 32; ++b) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[b * 32 + j]));
        const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
        int sum = 0;
        for (int j = 0; j < 32; ++j) {
            q[b * 32 + j] = (int8_t)roundf(x[b * 32 + j] * id);
            sum += q[b * 32 + j];
        }
        d_bits[b] = orc_float_to_half(d);
        s_bits[b] = orc_float_to_half((float)sum * d);
    }
}

/* Q8_K: gemvq_ref.h:62-81 (ggml quantize_row_q8_K_ref), plus ggml's bsums (sum of each 16 quants). */
void orc_quantize_q8_K(const float * x, int n, int8_t * q, float * d, int16_t * bsums) {
    for (int b = 0; b < n / 256; ++b) {
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < 256; ++j) {
            const float ax = fabsf(x[b * 256 + j]);
            if (ax > amax) { amax = ax; max = x[b * 256 + j]; }
        }
        if (amax == 0.0f) {
            d[b] = 0.0f;
            for (int j = 0; j < 256; ++j) q[b * 256 + j] = 0;
        } else {
            const float iscale = -127.0f / max;
            for (int j = 0; j < 256; ++j) {
                const int v = orc_nearest_int(iscale * x[b * 256 + j]);
                q[b * 256 + j] = (int8_t)(v < 127 ? v : 127);
            }
            d[b] = 1.0f / iscale;
        }
        if (bsums) {
            for (int g = 0; g < 16; ++g) {
                int s = 0;
                for (int i = 0; i < 16; ++i) s += q[b * 256 + g * 16 + i];
                bsums[b * 16 + g] = (int16_t)s;
            }
        }
    }
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Reference GEMV, restating gemvq_ref.h line by line in C. */

/* gemvq_ref.h:84-92: 6-bit scale and min of sub-block j of a Q4_K/Q5_K super-block. */
static void scale_min_k4(int j, const uint8_t * q, int * sc, int * m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

static uint16_t rd16(const uint8_t * p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Dequantized integer weights of one super-block (gemvq_ref.h:103-108 Q5_K, 157-165 Q6_K). */
static void q5k_weights(const uint8_t * blk, int * a) {
    const uint8_t * qh = blk + 16, * qs = blk + 48;
    for (int s = 0; s < 8; ++s)
        for (int e = 0; e < 32; ++e) {
            const uint8_t byte = qs[32 * (s / 2) + e];
            a[32 * s + e] = ((s & 1) ? (byte >> 4) : (byte & 15)) + (((qh[e] >> s) & 1) ? 16 : 0);
        }
}

static void q6k_weights(const uint8_t * blk, int * a) {
    const uint8_t * ql = blk, * qh = blk + 128;
    for (int n = 0; n < 2; ++n)
        for (int l = 0; l < 32; ++l) {
            const uint8_t h = qh[32 * n + l];
            a[128 * n + l] = (int8_t)((ql[64 * n + l] & 0xF) | (((h >> 0) & 3) << 4)) - 32;
            a[128 * n + l + 32] = (int8_t)((ql[64 * n + l + 32] & 0xF) | (((h >> 2) & 3) << 4)) - 32;
            a[128 * n + l + 64] = (int8_t)((ql[64 * n + l] >> 4) | (((h >> 4) & 3) << 4)) - 32;
            a[128 * n + l + 96] = (int8_t)((ql[64 * n + l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32;
        }
}

/* gemvq_ref.h:95-134 (ggml_vec_dot_q5_K_q8_K_generic). */
static float ref_dot_q5_k(const uint8_t * row, const int8_t * q8, const float * d8, int nsb, double * magnitude) {
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float sumf = 0.0f;
    for (int sb = 0; sb < nsb; ++sb) {
        const uint8_t * block = row + (size_t)sb * 176;
        const uint8_t * scales = block + 4;
        const int8_t * y = q8 + (size_t)sb * 256;
        int a[256];
        q5k_weights(block, a);
        int sumi = 0;
        for (int j = 0; j < 16; ++j) {
            int bsum = 0, sc, m;
            for (int i = 0; i < 16; ++i) bsum += y[16 * j + i];
            scale_min_k4(j / 2, scales, &sc, &m);
            sumi += bsum * m;
        }
        int aux32[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int j = 0; j < 8; ++j) {
            int sc, m;
            scale_min_k4(j, scales, &sc, &m);
            for (int i = 0; i < 32; ++i) aux32[i % 8] += sc * (y[32 * j + i] * a[32 * j + i]);
        }
        const float d = orc_half_to_float(rd16(block)) * d8[sb];
        double part = 0.0;
        for (int l = 0; l < 8; ++l) {
            sums[l] += d * (float)aux32[l];
            part += (double)aux32[l];
        }
        const float dmin = orc_half_to_float(rd16(block + 2)) * d8[sb];
        sumf -= dmin * (float)sumi;
        *magnitude += fabs((double)d * part) + fabs((double)dmin * sumi);
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

/* gemvq_ref.h:149-181 (ggml_vec_dot_q6_K_q8_K_generic). */
static float ref_dot_q6_k(const uint8_t * row, const int8_t * q8, const float * d8, int nsb, double * magnitude) {
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int sb = 0; sb < nsb; ++sb) {
        const uint8_t * block = row + (size_t)sb * 210;
        const int8_t * scales = (const int8_t *)(block + 192);
        const int8_t * y = q8 + (size_t)sb * 256;
        int a[256];
        q6k_weights(block, a);
        int aux32[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int j = 0; j < 16; ++j)
            for (int i = 0; i < 16; ++i) aux32[i % 8] += scales[j] * (y[16 * j + i] * a[16 * j + i]);
        const float d = orc_half_to_float(rd16(block + 208)) * d8[sb];
        double part = 0.0;
        for (int l = 0; l < 8; ++l) {
            sums[l] += d * (float)aux32[l];
            part += (double)aux32[l];
        }
        *magnitude += fabs((double)d * part);
    }
    float sumf = 0.0f;
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

/* gemvq_ref.h:196-229 (Q4_1 against Q8_1). */
static void ref_q4_1(const uint8_t * w, const float * x, int rows, int cols, float * y, double * mag) {
    const int nb = cols / 32;
    int8_t * q = (int8_t *)malloc((size_t)cols);
    float * d8 = (float *)malloc(sizeof(float) * (size_t)nb), * s8 = (float *)malloc(sizeof(float) * (size_t)nb);
    for (int b = 0; b < nb; ++b) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[b * 32 + j]));
        const float d = amax / 127, id = d != 0.0f ? 1.0f / d : 0.0f;
        int sum = 0;
        for (int j = 0; j < 32; ++j) {
            q[b * 32 + j] = (int8_t)roundf(x[b * 32 + j] * id);
            sum += q[b * 32 + j];
        }
        d8[b] = orc_half_to_float(orc_float_to_half(d));
        s8[b] = orc_half_to_float(orc_float_to_half((float)sum * d));
    }
    for (int r = 0; r < rows; ++r) {
        float sum = 0.0f;
        double m = 0.0;
        for (int b = 0; b < nb; ++b) {
            const uint8_t * blk = &w[((size_t)r * nb + b) * 20];
            int sumi = 0;
            for (int j = 0; j < 16; ++j) sumi += (blk[4 + j] & 0x0F) * q[b * 32 + j] + (blk[4 + j] >> 4) * q[b * 32 + j + 16];
            const float dw = orc_half_to_float(rd16(blk)), mw = orc_half_to_float(rd16(blk + 2));
            const float term = (dw * d8[b]) * (float)sumi + mw * s8[b];
            sum += term;
            m += fabsf((dw * d8[b]) * (float)sumi) + fabsf(mw * s8[b]); /* a float sum, as std::fabs(float) gives */
        }
        y[r] = sum;
        if (mag) mag[r] = m;
    }
    free(q); free(d8); free(s8);
}

/* gemvq_ref.h:231-265 (dispatch; Q4_0 and Q8_0 sequential FP32 rows, term = sumi * (dw * dx)). */
void orc_ref_gemv(int fmt, const uint8_t * w, const float * x, int rows, int cols, float * y, double * mag) {
    if (fmt == ORC_Q5_K || fmt == ORC_Q6_K) {
        int8_t * q = (int8_t *)malloc((size_t)cols);
        float * d = (float *)malloc(sizeof(float) * (size_t)(cols / 256));
        orc_quantize_q8_K(x, cols, q, d, NULL);
        const int nsb = cols / 256;
        for (int r = 0; r < rows; ++r) {
            double m = 0.0;
            y[r] = fmt == ORC_Q5_K ? ref_dot_q5_k(w + (size_t)r * nsb * 176, q, d, nsb, &m)
                                   : ref_dot_q6_k(w + (size_t)r * nsb * 210, q, d, nsb, &m);
            if (mag) mag[r] = m;
        }
        free(q); free(d);
        return;
    }
    if (fmt == ORC_Q4_1) { ref_q4_1(w, x, rows, cols, y, mag); return; }
    const int nb = cols / 32, bb = fmt == ORC_Q4_0 ? 18 : 34;
    int8_t * q = (int8_t *)malloc((size_t)cols);
    uint16_t * dh = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)nb);
    orc_quantize_q8_0(x, cols, q, dh);
    for (int r = 0; r < rows; ++r) {
        float sum = 0.0f;
        double m = 0.0;
        for (int b = 0; b < nb; ++b) {
            const uint8_t * blk = &w[((size_t)r * nb + b) * bb];
            int sumi = 0;
            for (int j = 0; j < 32; ++j) {
                const int wv = fmt == ORC_Q4_0 ? (int)(j < 16 ? (blk[2 + j] & 15) : (blk[2 + j - 16] >> 4)) - 8
                                               : (int)(int8_t)blk[2 + j];
                sumi += wv * q[b * 32 + j];
            }
            const float term = (float)sumi * (orc_half_to_float(rd16(blk)) * orc_half_to_float(dh[b]));
            sum += term;
            m += fabs(term);
        }
        y[r] = sum;
        if (mag) mag[r] = m;
    }
    free(q); free(dh);
}

/* gemvq_ref.h:269-272 */
int orc_ref_within_tolerance(float got, float ref, double mag) {
    const double err = fabs((double)got - (double)ref);
    return err <= 1e-6 + 1e-5 * fabs((double)ref) + 1e-6 * mag;
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Canonical fixed-point GEMV (the reference kernel's arithmetic, gemvqw_engine.h:352-445): a scale is split into
 * an integer significand and a power of two, the block sum times the significand product is exact, and the
 * product is truncated (floor) to the accumulator LSB 2^-40 (stream_common.h:59-62). The row sum is the exact
 * integer sum of these terms, rounded to FP32 once (stream_common.h:92-126: round to nearest even). */
typedef struct { int neg; int64_t m; int e; } orc_parts;

static orc_parts half_parts(uint16_t h) { /* gemvqw_engine.h:373-383 */
    orc_parts p;
    const int ex = (h >> 10) & 31, f = h & 1023;
    p.neg = (h >> 15) & 1;
    p.m = ex == 0 ? f : (f | 1024);
    p.e = ex == 0 ? -24 : ex - 25;
    return p;
}

static orc_parts float_parts(float v) { /* gemvqw_engine.h:385-394 (FP32 subnormals count as zero) */
    uint32_t b;
    memcpy(&b, &v, 4);
    orc_parts p;
    const int ex = (b >> 23) & 255;
    p.neg = (b >> 31) & 1;
    p.m = ex == 0 ? 0 : ((b & 0x7fffffu) | 0x800000u);
    p.e = ex - 150;
    return p;
}

/* floor(p * 2^(e + 40)), computed exactly in 128 bits; aborts if the result leaves the int64 range. */
static int64_t fixed_of(__int128 p, int e) {
    const int sh = e + 40;
    __int128 v;
    if (sh >= 0) {
        if (sh > 100) abort();
        v = p * ((__int128)1 << sh);
    } else {
        v = sh < -120 ? (p < 0 ? -1 : 0) : (p >> (-sh)); /* arithmetic shift: floor */
    }
    if (v > (__int128)INT64_MAX || v < (__int128)INT64_MIN) abort();
    return (int64_t)v;
}

float orc_fixed_to_float(int64_t acc) { return (float)acc * 9.094947017729282379e-13f; /* 2^-40, exact */ }

void orc_fx_gemv_q(int fmt, const uint8_t * w, const int8_t * xq, const uint16_t * xd16, const float * xd32,
                   const int16_t * xbsums, int rows, int cols, float * y, int32_t * blocksums, int64_t * acc_out) {
    const size_t rb = orc_row_bytes(fmt, cols);
    for (int r = 0; r < rows; ++r) {
        const uint8_t * row = w + (size_t)r * rb;
        __int128 acc = 0;
        if (fmt == ORC_Q4_1) {
            /* Q4_1 x Q8_1 (gemvq_ref.h:194-229): term = floor(sumi * d_w * d_x * 2^40) + floor(m_w * s_x * 2^40), both
             * products of fp16 values exact; xbsums carries the fp16 bits of each block's s_x. */
            const int nb = cols / 32;
            const uint16_t * xs16 = (const uint16_t *)xbsums;
            for (int b = 0; b < nb; ++b) {
                const uint8_t * blk = row + (size_t)b * 20;
                int sumi = 0;
                for (int j = 0; j < 16; ++j)
                    sumi += (blk[4 + j] & 15) * xq[b * 32 + j] + (blk[4 + j] >> 4) * xq[b * 32 + j + 16];
                if (blocksums) blocksums[(size_t)r * nb + b] = sumi;
                const orc_parts pw = half_parts(rd16(blk)), pm = half_parts(rd16(blk + 2));
                const orc_parts px = half_parts(xd16[b]), ps = half_parts(xs16[b]);
                __int128 p1 = (__int128)sumi * (pw.m * px.m);
                if (pw.neg != px.neg) p1 = -p1;
                acc += fixed_of(p1, pw.e + px.e);
                __int128 p2 = (__int128)(pm.m * ps.m);
                if (pm.neg != ps.neg) p2 = -p2;
                acc += fixed_of(p2, pm.e + ps.e);
            }
        } else if (fmt == ORC_Q4_0 || fmt == ORC_Q8_0) {
            const int nb = cols / 32, bb = fmt == ORC_Q4_0 ? 18 : 34;
            for (int b = 0; b < nb; ++b) {
                const uint8_t * blk = row + (size_t)b * bb;
                int sumi = 0;
                for (int j = 0; j < 32; ++j) {
                    const int wv = fmt == ORC_Q4_0 ? (int)(j < 16 ? (blk[2 + j] & 15) : (blk[2 + j - 16] >> 4)) - 8
                                                   : (int)(int8_t)blk[2 + j];
                    sumi += wv * xq[b * 32 + j];
                }
                if (blocksums) blocksums[(size_t)r * nb + b] = sumi;
                const orc_parts pw = half_parts(rd16(blk)), px = half_parts(xd16[b]);
                __int128 p = (__int128)sumi * (pw.m * px.m);
                if (pw.neg != px.neg) p = -p;
                acc += fixed_of(p, pw.e + px.e);
            }
        } else if (fmt == ORC_Q5_K || fmt == ORC_Q6_K) {
            const int nsb = cols / 256;
            for (int sb = 0; sb < nsb; ++sb) {
                const int8_t * x8 = xq + (size_t)sb * 256;
                int a[256];
                int64_t S = 0, M = 0;
                uint16_t dbits, mbits = 0;
                if (fmt == ORC_Q5_K) {
                    const uint8_t * blk = row + (size_t)sb * 176;
                    q5k_weights(blk, a);
                    for (int s = 0; s < 8; ++s) {
                        int sc, m;
                        scale_min_k4(s, blk + 4, &sc, &m);
                        int dot = 0;
                        for (int i = 0; i < 32; ++i) dot += a[32 * s + i] * x8[32 * s + i];
                        S += (int64_t)sc * dot;
                        M += (int64_t)m * (xbsums[sb * 16 + 2 * s] + xbsums[sb * 16 + 2 * s + 1]);
                    }
                    dbits = rd16(blk);
                    mbits = rd16(blk + 2);
                } else {
                    const uint8_t * blk = row + (size_t)sb * 210;
                    const int8_t * sc = (const int8_t *)(blk + 192);
                    q6k_weights(blk, a);
                    for (int g = 0; g < 16; ++g) {
                        int dot = 0;
                        for (int i = 0; i < 16; ++i) dot += a[16 * g + i] * x8[16 * g + i];
                        S += (int64_t)sc[g] * dot;
                    }
                    dbits = rd16(blk + 208);
                }
                if (blocksums) {
                    blocksums[((size_t)r * nsb + sb) * 2] = (int32_t)S;
                    blocksums[((size_t)r * nsb + sb) * 2 + 1] = (int32_t)M;
                }
                /* gemvqw_engine.h:430-444: floor(S d dx 2^40) - floor(M dmin dx 2^40) */
                const orc_parts pd = half_parts(dbits), px = float_parts(xd32[sb]);
                __int128 ps = (__int128)S * (pd.m * px.m);
                if (pd.neg != px.neg) ps = -ps;
                acc += fixed_of(ps, pd.e + px.e);
                if (fmt == ORC_Q5_K) {
                    const orc_parts pm = half_parts(mbits);
                    __int128 pmv = (__int128)M * (pm.m * px.m);
                    if (pm.neg != px.neg) pmv = -pmv;
                    acc -= fixed_of(pmv, pm.e + px.e);
                }
            }
        } else {
            abort();
        }
        if (acc > (__int128)INT64_MAX || acc < (__int128)INT64_MIN) abort();
        if (acc_out) acc_out[r] = (int64_t)acc;
        y[r] = orc_fixed_to_float((int64_t)acc);
    }
}

void orc_fx_gemv(int fmt, const uint8_t * w, const float * x, int rows, int cols, float * y, int32_t * blocksums,
                 int64_t * acc) {
    int8_t * q = (int8_t *)malloc((size_t)cols);
    if (fmt == ORC_Q5_K || fmt == ORC_Q6_K) {
        float * d = (float *)malloc(sizeof(float) * (size_t)(cols / 256));
        int16_t * bs = (int16_t *)malloc(sizeof(int16_t) * (size_t)(cols / 16));
        orc_quantize_q8_K(x, cols, q, d, bs);
        orc_fx_gemv_q(fmt, w, q, NULL, d, bs, rows, cols, y, blocksums, acc);
        free(d); free(bs);
    } else if (fmt == ORC_Q4_1) {
        uint16_t * dh = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(cols / 32));
        uint16_t * sh = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(cols / 32));
        orc_quantize_q8_1(x, cols, q, dh, sh);
        orc_fx_gemv_q(fmt, w, q, dh, NULL, (const int16_t *)sh, rows, cols, y, blocksums, acc);
        free(dh); free(sh);
    } else {
        uint16_t * dh = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(cols / 32));
        orc_quantize_q8_0(x, cols, q, dh);
        orc_fx_gemv_q(fmt, w, q, dh, NULL, NULL, rows, cols, y, blocksums, acc);
        free(dh);
    }
    free(q);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Norms. Reference: gemvq_ref.h:288-295 and 310-324 (sums of squares in double, sequential). */
void orc_ref_rmsnorm(const float * x, const float * w, int n, float eps, float * y) {
    double sum = 0.0;
    for (int i = 0; i < n; ++i) sum += (double)x[i] * (double)x[i];
    const float scale = 1.0f / sqrtf((float)(sum / n) + eps);
    for (int i = 0; i < n; ++i) y[i] = (x[i] * scale) * w[i];
}

void orc_ref_rownorm(const float * x, const float * w, int n, int rows, float eps, int flags, float * y) {
    for (int r = 0; r < rows; ++r) {
        const float * xr = x + (size_t)r * n;
        double sum = 0.0;
        for (int i = 0; i < n; ++i) sum += (double)(xr[i] * xr[i]);
        const float scale = (flags & 1) ? 1.0f / fmaxf(sqrtf((float)sum), eps) : 1.0f / sqrtf((float)(sum / n) + eps);
        for (int i = 0; i < n; ++i) y[(size_t)r * n + i] = (flags & 2) ? xr[i] * scale : (xr[i] * scale) * w[i];
    }
}

/* Canonical scale: the squares summed by the pairwise tree; RMS 1 / sqrt(sum / n + eps), L2 1 / max(sqrt(sum), eps)
 * (gemvqc_ops.h:120-126 evaluates the same FP32 expressions). */
float orc_norm_scale(const float * x, int n, float eps, int l2) {
    float * sq = (float *)malloc(sizeof(float) * (size_t)n);
    for (int i = 0; i < n; ++i) sq[i] = x[i] * x[i];
    const float sum = orc_pair_sum(sq, n);
    free(sq);
    return l2 ? 1.0f / fmaxf(sqrtf(sum), eps) : 1.0f / sqrtf(sum / (float)n + eps);
}

/* RMSNORM opcode (gemvqc16.h:46-51, gemvqc_ops.h:169-234): y = (x * scale) * w per row, packed rows out. */
void orc_rownorm(const float * x, const float * w, int n, int rows, int stride, float eps, int flags, float * y) {
    if (stride == 0) stride = n;
    for (int r = 0; r < rows; ++r) {
        const float * xr = x + (size_t)r * stride;
        const float s = orc_norm_scale(xr, n, eps, flags & 1);
        for (int i = 0; i < n; ++i) y[(size_t)r * n + i] = (flags & 2) ? xr[i] * s : (xr[i] * s) * w[i];
    }
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Element-wise ops. SILU_MUL gemvqc_ops.h:88-99 ((g / (1 + e^-g)) * u, sigmoid: (1 / (1 + e^-g)) * u). */
void orc_silu_mul(const float * g, const float * u, int n, int sigmoid, float * y) {
    for (int i = 0; i < n; ++i) y[i] = ((sigmoid ? 1.0f : g[i]) / (1.0f + orc_expf(-g[i]))) * u[i];
}

/* UNARY gemvqc_ops.h:70-79: 1 SiLU, 2 sigmoid, 3 softplus, 4 copy. */
void orc_unary(const float * x, int n, int kind, float * y) {
    for (int i = 0; i < n; ++i) {
        const float v = x[i];
        y[i] = kind == 1 ? orc_silu(v) : kind == 2 ? orc_sigmoid(v) : kind == 3 ? orc_softplus(v) : v;
    }
}

/* The exp and log of the reference arithmetic: the host's libm (the compiled reference path, for the golden
 * vectors) or the correctly rounded functions (the reference-arithmetic decoder, which the GPU reproduces). */
typedef struct {
    float (*exp)(float);
    float (*log)(float);
} orc_math;
static const orc_math MATH_LIBM = {expf, logf};
static const orc_math MATH_CR = {orc_cr_expf, orc_cr_logf};

/* gemvq_ref.h:333-342. */
static void ref_unary(const float * x, int n, int kind, float * y, const orc_math * mt) {
    for (int i = 0; i < n; ++i) {
        const float v = x[i];
        y[i] = kind == 1 ? v / (1.0f + mt->exp(-v)) : kind == 2 ? 1.0f / (1.0f + mt->exp(-v))
             : kind == 3 ? (v > 20.0f ? v : mt->log(1.0f + mt->exp(v))) : v;
    }
}
void orc_ref_unary(const float * x, int n, int kind, float * y) { ref_unary(x, n, kind, y, &MATH_LIBM); }
void orc_ref_unary_cr(const float * x, int n, int kind, float * y) { ref_unary(x, n, kind, y, &MATH_CR); }

/* gemvq_ref.h:303-307: y = g / (1 + e^-g) * u */
void orc_ref_silu_mul_cr(const float * g, const float * u, int n, float * y) {
    for (int i = 0; i < n; ++i) y[i] = g[i] / (1.0f + orc_cr_expf(-g[i])) * u[i];
}

/* CONV (gemvq_ref.h:346-358, gemvqc_ops.h:135-144, 387-431): window [state_c (3), x_c], summed from t = 0. */
static void conv_impl(const float * state, const float * x, const float * w, int ch, int silu, float * y,
                      float * new_state, const orc_math * mt) {
    for (int c = 0; c < ch; ++c) {
        const float in[4] = {state[c * 3], state[c * 3 + 1], state[c * 3 + 2], x[c]};
        float sum = 0.0f;
        for (int t = 0; t < 4; ++t) sum += in[t] * w[c * 4 + t];
        y[c] = silu ? (mt ? sum / (1.0f + mt->exp(-sum)) : orc_silu(sum)) : sum;
        for (int t = 0; t < 3; ++t) new_state[c * 3 + t] = in[t + 1];
    }
}
void orc_conv(const float * state, const float * x, const float * w, int ch, int silu, float * y, float * ns) {
    conv_impl(state, x, w, ch, silu, y, ns, NULL);
}
void orc_ref_conv(const float * state, const float * x, const float * w, int ch, int silu, float * y, float * ns) {
    conv_impl(state, x, w, ch, silu, y, ns, &MATH_LIBM);
}
void orc_ref_conv_cr(const float * state, const float * x, const float * w, int ch, int silu, float * y, float * ns) {
    conv_impl(state, x, w, ch, silu, y, ns, &MATH_CR);
}

/* ROPE (gemvqc_ops.h:275-312): NEOX pairs (i, i + n_dims / 2); cs holds cos, sin of pair i at 2i, 2i + 1. */
void orc_rope(const float * x, const float * cs, int n_dims, int ne0, int rows, float * y) {
    const int half = n_dims / 2;
    for (int r = 0; r < rows; ++r) {
        const float * xr = x + (size_t)r * ne0;
        float * yr = y + (size_t)r * ne0;
        for (int i = 0; i < ne0; ++i) yr[i] = xr[i];
        for (int i = 0; i < half; ++i) {
            const float x0 = xr[i], x1 = xr[i + half], c = cs[2 * i], s = cs[2 * i + 1];
            yr[i] = x0 * c - x1 * s;
            yr[i + half] = x0 * s + x1 * c;
        }
    }
}

/* ------------------------------------------------------------------------------------------------------------ */
/* GDN reference: gemvq_ref.h:363-397 (libm exp, sequential dots). */
void orc_ref_gdn(float * state, const float * q, const float * k, const float * v, const float * g, const float * beta,
                 int hv, int hk, float scale, float * y, double * y_mag, double * s_mag) {
    orc_ref_gdn_mt(state, q, k, v, g, beta, hv, hk, scale, y, y_mag, s_mag, 1);
}

/* The value heads are independent, so they split over threads without changing any result. */
static void ref_gdn(float * state, const float * q, const float * k, const float * v, const float * g,
                    const float * beta, int hv, int hk, float scale, float * y, double * y_mag, double * s_mag,
                    int n_threads, const orc_math * mt) {
    const int S = 128;
#pragma omp parallel for schedule(static) num_threads(n_threads > 0 ? n_threads : 1)
    for (int h = 0; h < hv; ++h) {
        const float * qh = q + (h % hk) * S, * kh = k + (h % hk) * S;
        const float decay = mt->exp(g[h]);
        for (int j = 0; j < S; ++j) {
            float * row = &state[((size_t)h * S + j) * S];
            double dmag = 0.0;
            float dot = 0.0f;
            for (int i = 0; i < S; ++i) {
                row[i] *= decay;
                dot += row[i] * kh[i];
                dmag += fabs((double)row[i] * kh[i]);
            }
            const float delta = (v[h * S + j] - dot) * beta[h];
            const double delta_mag = (fabs((double)v[h * S + j]) + dmag) * fabs((double)beta[h]);
            float out = 0.0f;
            double omag = 0.0;
            for (int i = 0; i < S; ++i) {
                if (s_mag) s_mag[((size_t)h * S + j) * S + i] = fabs((double)row[i]) + fabs((double)kh[i]) * delta_mag;
                row[i] += kh[i] * delta;
                out += row[i] * qh[i];
                omag += (fabs((double)row[i]) + fabs((double)kh[i]) * delta_mag) * fabs((double)qh[i]);
            }
            y[h * S + j] = out * scale;
            if (y_mag) y_mag[h * S + j] = omag * scale;
        }
    }
}
void orc_ref_gdn_mt(float * state, const float * q, const float * k, const float * v, const float * g,
                    const float * beta, int hv, int hk, float scale, float * y, double * y_mag, double * s_mag,
                    int n_threads) {
    ref_gdn(state, q, k, v, g, beta, hv, hk, scale, y, y_mag, s_mag, n_threads, &MATH_LIBM);
}
void orc_ref_gdn_cr_mt(float * state, const float * q, const float * k, const float * v, const float * g,
                       const float * beta, int hv, int hk, float scale, float * y, int n_threads) {
    ref_gdn(state, q, k, v, g, beta, hv, hk, scale, y, NULL, NULL, n_threads, &MATH_CR);
}

/* Canonical fused step: the GDN opcode (gemvqc16.h:60-81) with the input load of gemvqc_gdn.h:223-281, the step of
 * gemvqc_gdn.h:73-187 (x = S_j * decay; delta = (v_j - x . k) * beta; S_j' = x + k * delta; y_j = (S_j' . q) *
 * scale) and the gated output of gemvqc_gdn.h:284-346; dots and sums of squares by the pairwise tree. */
void orc_gdn(float * state, const float * q, const float * k, const float * v, const float * graw, const float * braw,
             const float * dt, const float * a, const float * z, const float * w, int hv, int hk, float scale,
             float l2_eps, float rms_eps, int flags, float * y) {
    orc_gdn_mt(state, q, k, v, graw, braw, dt, a, z, w, hv, hk, scale, l2_eps, rms_eps, flags, y, 1);
}

/* The value heads are independent, so they split over threads without changing any result. */
void orc_gdn_mt(float * state, const float * q, const float * k, const float * v, const float * graw, const float * braw,
                const float * dt, const float * a, const float * z, const float * w, int hv, int hk, float scale,
                float l2_eps, float rms_eps, int flags, float * y, int n_threads) {
    const int S = 128;
    float * qn = (float *)malloc(sizeof(float) * (size_t)hk * S);
    float * kn = (float *)malloc(sizeof(float) * (size_t)hk * S);
    for (int h = 0; h < hk; ++h) {
        const float sq = (flags & 2) ? orc_norm_scale(q + h * S, S, l2_eps, 1) : 1.0f;
        const float sk = (flags & 2) ? orc_norm_scale(k + h * S, S, l2_eps, 1) : 1.0f;
        for (int i = 0; i < S; ++i) {
            qn[h * S + i] = (flags & 2) ? q[h * S + i] * sq : q[h * S + i];
            kn[h * S + i] = (flags & 2) ? k[h * S + i] * sk : k[h * S + i];
        }
    }
#pragma omp parallel for schedule(static) num_threads(n_threads > 0 ? n_threads : 1)
    for (int h = 0; h < hv; ++h) {
        float prod[128], xrow[128];
        const float * qh = qn + (h % hk) * S, * kh = kn + (h % hk) * S;
        float gv = graw[h], bt = braw[h];
        if (flags & 8) {
            gv = orc_softplus(graw[h] + dt[h]) * a[h];
            bt = orc_sigmoid(braw[h]);
        }
        const float decay = orc_expf(gv);
        for (int j = 0; j < S; ++j) {
            float * row = &state[((size_t)h * S + j) * S];
            for (int i = 0; i < S; ++i) {
                xrow[i] = row[i] * decay;
                prod[i] = xrow[i] * kh[i];
            }
            const float dot = orc_pair_sum(prod, S);
            const float delta = (v[h * S + j] - dot) * bt;
            for (int i = 0; i < S; ++i) {
                row[i] = xrow[i] + kh[i] * delta;
                prod[i] = row[i] * qh[i];
            }
            y[h * S + j] = orc_pair_sum(prod, S) * scale;
        }
        if (flags & 4) {
            float * yh = y + h * S;
            const float s = orc_norm_scale(yh, S, rms_eps, 0);
            for (int i = 0; i < S; ++i)
                yh[i] = ((flags & 32) ? z[h * S + i] : orc_silu(z[h * S + i])) * ((yh[i] * s) * w[i]);
        }
    }
    free(qn); free(kn);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Attention core for one token (not on the reference card; ggml semantics with an F16 KV cache). */
void orc_attn(const float * q, const uint16_t * kc, const uint16_t * vc, int nh, int nkvh, int hd, int n_kv,
              float scale, float * out) {
    orc_attn_mt(q, kc, vc, nh, nkvh, hd, n_kv, scale, out, 1);
}

/* The q heads are independent, so they split over threads without changing any result. */
void orc_attn_mt(const float * q, const uint16_t * kc, const uint16_t * vc, int nh, int nkvh, int hd, int n_kv,
                 float scale, float * out, int n_threads) {
    const int group = nh / nkvh, CH = 64, nch = (n_kv + CH - 1) / CH;
#pragma omp parallel for schedule(static) num_threads(n_threads > 0 ? n_threads : 1)
    for (int h = 0; h < nh; ++h) {
        float * q16 = (float *)malloc(sizeof(float) * (size_t)hd);
        float * prod = (float *)malloc(sizeof(float) * (size_t)hd);
        float * s = (float *)malloc(sizeof(float) * (size_t)n_kv);
        float * mc = (float *)malloc(sizeof(float) * (size_t)nch), * lc = (float *)malloc(sizeof(float) * (size_t)nch);
        float * oc = (float *)malloc(sizeof(float) * (size_t)nch * hd);
        const int kh = h / group;
        for (int d = 0; d < hd; ++d) q16[d] = orc_half_to_float(orc_float_to_half(q[h * hd + d]));
        for (int t = 0; t < n_kv; ++t) {
            const uint16_t * kt = kc + ((size_t)t * nkvh + kh) * hd;
            for (int d = 0; d < hd; ++d) prod[d] = q16[d] * orc_half_to_float(kt[d]);
            s[t] = orc_pair_sum(prod, hd) * scale;
        }
        for (int c = 0; c < nch; ++c) {
            const int t0 = c * CH, t1 = t0 + CH < n_kv ? t0 + CH : n_kv;
            float m = s[t0];
            for (int t = t0 + 1; t < t1; ++t) m = fmaxf(m, s[t]);
            mc[c] = m;
            float l = 0.0f;
            float * o = oc + (size_t)c * hd;
            for (int d = 0; d < hd; ++d) o[d] = 0.0f;
            for (int t = t0; t < t1; ++t) {
                const float p = orc_expf(s[t] - m);
                l += p;
                const uint16_t * vt = vc + ((size_t)t * nkvh + kh) * hd;
                for (int d = 0; d < hd; ++d) o[d] += p * orc_half_to_float(vt[d]);
            }
            lc[c] = l;
        }
        float M = mc[0];
        for (int c = 1; c < nch; ++c) M = fmaxf(M, mc[c]);
        float L = 0.0f;
        float * oh = out + (size_t)h * hd;
        for (int d = 0; d < hd; ++d) oh[d] = 0.0f;
        for (int c = 0; c < nch; ++c) {
            const float f = orc_expf(mc[c] - M);
            L += lc[c] * f;
            for (int d = 0; d < hd; ++d) oh[d] += oc[(size_t)c * hd + d] * f;
        }
        for (int d = 0; d < hd; ++d) oh[d] = oh[d] / L;
        free(q16); free(prod); free(s); free(mc); free(lc); free(oc);
    }
}

/* Attention in the shape of ggml's CPU path without flash attention (the reference leaves attention to ggml's CPU
 * backend, README.md:77): q converted to fp16 (the F16 cache's vec_dot type), each score an F16 dot with the float
 * products summed in double (ggml_vec_dot_f16's generic form), times scale; softmax with the max subtracted, libm
 * expf and the sum in double (ggml_vec_soft_max_f32), scaled by 1 / sum; the probabilities converted to fp16 for the
 * product with V (again an F16 dot summed in double). Upstream ggml is not available here, so this form is
 * restated from ggml's published generic code and is not pinned against it. */
void orc_ref_attn(const float * q, const uint16_t * kc, const uint16_t * vc, int nh, int nkvh, int hd, int n_kv,
                  float scale, float * out) {
    orc_ref_attn_mt(q, kc, vc, nh, nkvh, hd, n_kv, scale, out, 1);
}

static void ref_attn(const float * q, const uint16_t * kc, const uint16_t * vc, int nh, int nkvh, int hd, int n_kv,
                     float scale, float * out, int n_threads, const orc_math * mt) {
    const int group = nh / nkvh;
#pragma omp parallel for schedule(static) num_threads(n_threads > 0 ? n_threads : 1)
    for (int h = 0; h < nh; ++h) {
        const int kh = h / group;
        float * q16 = (float *)malloc(sizeof(float) * (size_t)hd);
        float * s = (float *)malloc(sizeof(float) * (size_t)n_kv);
        float * p16 = (float *)malloc(sizeof(float) * (size_t)n_kv);
        for (int d = 0; d < hd; ++d) q16[d] = orc_half_to_float(orc_float_to_half(q[h * hd + d]));
        float mx = -INFINITY;
        for (int t = 0; t < n_kv; ++t) {
            const uint16_t * kt = kc + ((size_t)t * nkvh + kh) * hd;
            double acc = 0.0;
            for (int d = 0; d < hd; ++d) acc += (double)(q16[d] * orc_half_to_float(kt[d]));
            s[t] = (float)acc * scale;
            mx = fmaxf(mx, s[t]);
        }
        double sum = 0.0;
        for (int t = 0; t < n_kv; ++t) {
            const float e = mt->exp(s[t] - mx);
            sum += (double)e;
            s[t] = e;
        }
        const float inv = (float)(1.0 / sum);
        for (int t = 0; t < n_kv; ++t) p16[t] = orc_half_to_float(orc_float_to_half(s[t] * inv));
        for (int d = 0; d < hd; ++d) {
            double acc = 0.0;
            for (int t = 0; t < n_kv; ++t) acc += (double)(orc_half_to_float(vc[((size_t)t * nkvh + kh) * hd + d]) * p16[t]);
            out[h * hd + d] = (float)acc;
        }
        free(q16); free(s); free(p16);
    }
}
void orc_ref_attn_mt(const float * q, const uint16_t * kc, const uint16_t * vc, int nh, int nkvh, int hd, int n_kv,
                     float scale, float * out, int n_threads) {
    ref_attn(q, kc, vc, nh, nkvh, hd, n_kv, scale, out, n_threads, &MATH_LIBM);
}
void orc_ref_attn_cr_mt(const float * q, const uint16_t * kc, const uint16_t * vc, int nh, int nkvh, int hd, int n_kv,
                        float scale, float * out, int n_threads) {
    ref_attn(q, kc, vc, nh, nkvh, hd, n_kv, scale, out, n_threads, &MATH_CR);
}

/* ggml dequantize_row_q6_K: y = d * sc * q evaluated as (d * sc) * q. */
void orc_dequant_row_q6_K(const uint8_t * row, int cols, float * y) {
    for (int sb = 0; sb < cols / 256; ++sb) {
        const uint8_t * blk = row + (size_t)sb * 210;
        const int8_t * sc = (const int8_t *)(blk + 192);
        const float d = orc_half_to_float(rd16(blk + 208));
        int a[256];
        q6k_weights(blk, a);
        for (int i = 0; i < 256; ++i) y[sb * 256 + i] = (d * (float)sc[i / 16]) * (float)a[i];
    }
}

/* ggml_argmax: the first index of the maximum. */
int orc_argmax(const float * x, int n) {
    int best = 0;
    for (int i = 1; i < n; ++i)
        if (x[i] > x[best]) best = i;
    return best;
}
