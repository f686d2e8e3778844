/* Fast rows of the CPU oracle: TEST INFRASTRUCTURE ONLY (see gemvq_oracle.h).
 *
 * The same two arithmetics as gemvq_oracle.c, row by row, with the integer block sums formed by AVX2 int8 dot
 * products instead of scalar loops:
 *   canonical (mode 0): every block term exact and floored to 2^-40, summed exactly, rounded to FP32 once (the
 *     reference kernel's fixed point, gemvqw_engine.h:352-445, as orc_fx_gemv_q states it);
 *   reference (mode 1): the reference's sequential FP32 row sums (gemvq_ref.h:94-265, as orc_ref_gemv states it).
 * An integer block sum does not depend on the order of its products, so only the block sums are vectorized; the
 * per-row combination of the terms is the scalar one, term by term in block order. On hosts with AVX-512 VNNI the
 * Q4_0 / Q4_1 / Q8_0 block sums come from vpdpbusd, 16 blocks at a time (orc_fast_simd). The tests check every
 * format, both arithmetics and both SIMD levels bit for bit against the scalar oracle. */
#include "orc_fast.h"
#include "gemvq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef __AVX2__
#include <immintrin.h>
#endif

static uint16_t rd16(const uint8_t * p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* fp16 bits as significand, exponent and sign: value = (-1)^neg m 2^e (gemvqw_engine.h:373-383) */
static inline void half_me(uint16_t h, int * m, int * e, int * neg) {
    const int ex = (h >> 10) & 31, f = h & 1023;
    *neg = (h >> 15) & 1;
    *m = ex == 0 ? f : (f | 1024);
    *e = ex == 0 ? -24 : ex - 25;
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Activation quantization (the oracle's quantizers) plus per-block data the fast rows use. */
void orc_act_init(orc_act * a, int fmt, const float * x, int cols) {
    memset(a, 0, sizeof(*a));
    a->fmt = fmt;
    a->cols = cols;
    a->q = (int8_t *)malloc((size_t)cols + 64);
    if (fmt == ORC_Q5_K || fmt == ORC_Q6_K) {
        const int nsb = cols / 256;
        a->d32 = (float *)malloc(sizeof(float) * (size_t)nsb);
        a->bs = (int16_t *)malloc(sizeof(int16_t) * (size_t)nsb * 16);
        orc_quantize_q8_K(x, cols, a->q, a->d32, a->bs);
        return;
    }
    const int nb = cols / 32;
    a->d16 = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)nb);
    a->xsum = (int32_t *)malloc(sizeof(int32_t) * (size_t)nb);
    if (fmt == ORC_Q4_1) {
        a->s16 = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)nb);
        orc_quantize_q8_1(x, cols, a->q, a->d16, a->s16);
    } else {
        orc_quantize_q8_0(x, cols, a->q, a->d16);
    }
    a->mx = (int32_t *)malloc(sizeof(int32_t) * (size_t)nb * 2);
    a->ms = a->mx + nb;
    a->ex = (int8_t *)malloc((size_t)nb * 4);
    a->es = a->ex + nb;
    a->nx = a->ex + 2 * nb;
    a->ns = a->ex + 3 * nb;
    a->dxf = (float *)malloc(sizeof(float) * (size_t)nb * 2);
    a->sxf = a->dxf + nb;
    for (int b = 0; b < nb; ++b) {
        int s = 0;
        for (int j = 0; j < 32; ++j) s += a->q[b * 32 + j];
        a->xsum[b] = s;
        int m, e, n;
        half_me(a->d16[b], &m, &e, &n);
        a->mx[b] = m;
        a->ex[b] = (int8_t)e;
        a->nx[b] = (int8_t)n;
        a->dxf[b] = orc_half_to_float(a->d16[b]);
        const uint16_t sb = a->s16 ? a->s16[b] : 0;
        half_me(sb, &m, &e, &n);
        a->ms[b] = m;
        a->es[b] = (int8_t)e;
        a->ns[b] = (int8_t)n;
        a->sxf[b] = orc_half_to_float(sb);
    }
}

void orc_act_free(orc_act * a) {
    free(a->q); free(a->d16); free(a->s16); free(a->d32); free(a->bs); free(a->xsum); free(a->mx); free(a->ex);
    free(a->dxf);
    memset(a, 0, sizeof(*a));
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Integer block sums. */
#ifdef __AVX2__
static inline int hsum8(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
    return _mm_cvtsi128_si32(s);
}
#endif

/* Q6_K super-block: the 256 weights as unsigned 6-bit values u (q = u - 32) in element order. */
static inline void q6k_unsigned(const uint8_t * blk, uint8_t * u) {
    const uint8_t * ql = blk, * qh = blk + 128;
#ifdef __AVX2__
    const __m256i m4 = _mm256_set1_epi8(0x0F), m3 = _mm256_set1_epi8(0x03);
    for (int n = 0; n < 2; ++n) {
        const __m256i l0 = _mm256_loadu_si256((const __m256i *)(ql + 64 * n));
        const __m256i l1 = _mm256_loadu_si256((const __m256i *)(ql + 64 * n + 32));
        const __m256i h = _mm256_loadu_si256((const __m256i *)(qh + 32 * n));
        const __m256i h0 = _mm256_slli_epi16(_mm256_and_si256(h, m3), 4);
        const __m256i h1 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 2), m3), 4);
        const __m256i h2 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 4), m3), 4);
        const __m256i h3 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 6), m3), 4);
        _mm256_storeu_si256((__m256i *)(u + 128 * n), _mm256_or_si256(_mm256_and_si256(l0, m4), h0));
        _mm256_storeu_si256((__m256i *)(u + 128 * n + 32), _mm256_or_si256(_mm256_and_si256(l1, m4), h1));
        _mm256_storeu_si256((__m256i *)(u + 128 * n + 64),
                            _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l0, 4), m4), h2));
        _mm256_storeu_si256((__m256i *)(u + 128 * n + 96),
                            _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l1, 4), m4), h3));
    }
#else
    for (int n = 0; n < 2; ++n)
        for (int l = 0; l < 32; ++l) {
            const uint8_t h = qh[32 * n + l];
            u[128 * n + l] = (uint8_t)((ql[64 * n + l] & 0xF) | (((h >> 0) & 3) << 4));
            u[128 * n + l + 32] = (uint8_t)((ql[64 * n + l + 32] & 0xF) | (((h >> 2) & 3) << 4));
            u[128 * n + l + 64] = (uint8_t)((ql[64 * n + l] >> 4) | (((h >> 4) & 3) << 4));
            u[128 * n + l + 96] = (uint8_t)((ql[64 * n + l + 32] >> 4) | (((h >> 6) & 3) << 4));
        }
#endif
}

/* ------------------------------------------------------------------------------------------------------------ */
/* Canonical fixed-point terms (the oracle's orc_fx_gemv_q: floor(p * 2^(e + 40)), exact). */
static int64_t fixed_slow(__int128 p, int e) {
    const int sh = e + 40;
    __int128 v;
    if (sh >= 0) {
        if (sh > 100) abort();
        v = p * ((__int128)1 << sh);
    } else {
        v = sh < -120 ? (p < 0 ? -1 : 0) : (p >> (-sh));
    }
    if (v > (__int128)INT64_MAX || v < (__int128)INT64_MIN) abort();
    return (int64_t)v;
}

/* p of magnitude below 2^43 */
static inline int64_t fixed_fast(int64_t p, int e) {
    const int sh = e + 40;
    if (sh >= 0) return sh <= 19 ? p * ((int64_t)1 << sh) : fixed_slow(p, e);
    return sh < -62 ? (p < 0 ? -1 : 0) : (p >> (-sh));
}


/* One weight row against T activation rows. Each weight block is loaded, expanded and its scale decoded once, then
 * used for every token; each token's terms are combined in block order, exactly as a single-token row does. */
#ifdef __AVX2__
typedef __m256i wblk;
static inline wblk expand_nibbles(const uint8_t * qs) {
    const __m128i v = _mm_loadu_si128((const __m128i *)qs), m4 = _mm_set1_epi8(0x0F);
    return _mm256_set_m128i(_mm_and_si128(_mm_srli_epi16(v, 4), m4), _mm_and_si128(v, m4));
}
static inline int dot_u8(wblk w, const int8_t * x) {  /* unsigned weights (< 128) times signed quants */
    const __m256i p = _mm256_maddubs_epi16(w, _mm256_loadu_si256((const __m256i *)x));
    return hsum8(_mm256_madd_epi16(p, _mm256_set1_epi16(1)));
}
static inline wblk load_i8(const uint8_t * wq) { return _mm256_loadu_si256((const __m256i *)wq); }
static inline int dot_s8(wblk w, const int8_t * x) {
    const __m256i xv = _mm256_loadu_si256((const __m256i *)x);
    const __m256i p = _mm256_maddubs_epi16(_mm256_sign_epi8(w, w), _mm256_sign_epi8(xv, w));
    return hsum8(_mm256_madd_epi16(p, _mm256_set1_epi16(1)));
}
#else
typedef struct { uint8_t b[32]; } wblk;
static inline wblk expand_nibbles(const uint8_t * qs) {
    wblk w;
    for (int j = 0; j < 16; ++j) { w.b[j] = qs[j] & 15; w.b[j + 16] = qs[j] >> 4; }
    return w;
}
static inline int dot_u8(wblk w, const int8_t * x) {
    int s = 0;
    for (int j = 0; j < 32; ++j) s += w.b[j] * x[j];
    return s;
}
static inline wblk load_i8(const uint8_t * wq) { wblk w; memcpy(w.b, wq, 32); return w; }
static inline int dot_s8(wblk w, const int8_t * x) {
    int s = 0;
    for (int j = 0; j < 32; ++j) s += (int)(int8_t)w.b[j] * x[j];
    return s;
}
#endif

/* fixed-point term of a block sum with pre-decoded scale parts */
static inline int64_t term_parts(int sumi, int mw, int ew, int nw, int mx, int ex, int nx) {
    int64_t p = (int64_t)sumi * (int64_t)(mw * mx);
    if (nw != nx) p = -p;
    return fixed_fast(p, ew + ex);
}

enum { MAXT = 32 };

static void rows_q4q8(int mode, int fmt, const uint8_t * w, const orc_act * const * a, int T, int r0, int r1,
                      float * Y, size_t ys) {
    const int nb = a[0]->cols / 32;
    const int bb = fmt == ORC_Q4_0 ? 18 : fmt == ORC_Q4_1 ? 20 : 34;
    const size_t rb = (size_t)nb * bb;
    for (int r = r0; r < r1; ++r) {
        const uint8_t * row = w + (size_t)r * rb;
        __int128 acc[MAXT];
        float sum[MAXT];
        for (int t = 0; t < T; ++t) { acc[t] = 0; sum[t] = 0.0f; }
        for (int b = 0; b < nb; ++b) {
            const uint8_t * blk = row + (size_t)b * bb;
            const uint16_t hw = rd16(blk);
            const wblk wv = fmt == ORC_Q8_0 ? load_i8(blk + 2) : expand_nibbles(blk + (fmt == ORC_Q4_1 ? 4 : 2));
            int mw, ew, nw, mm = 0, em = 0, nm = 0;
            half_me(hw, &mw, &ew, &nw);
            const uint16_t hm = fmt == ORC_Q4_1 ? rd16(blk + 2) : 0;
            if (fmt == ORC_Q4_1) half_me(hm, &mm, &em, &nm);
            const float dw = orc_half_to_float(hw), mwf = fmt == ORC_Q4_1 ? orc_half_to_float(hm) : 0.0f;
            for (int t = 0; t < T; ++t) {
                const orc_act * x = a[t];
                const int8_t * xq = x->q + 32 * b;
                int sumi = fmt == ORC_Q8_0 ? dot_s8(wv, xq) : dot_u8(wv, xq);
                if (fmt == ORC_Q4_0) sumi -= 8 * x->xsum[b];
                if (mode == 0) {
                    acc[t] += term_parts(sumi, mw, ew, nw, x->mx[b], x->ex[b], x->nx[b]);
                    if (fmt == ORC_Q4_1) acc[t] += term_parts(1, mm, em, nm, x->ms[b], x->es[b], x->ns[b]);
                } else if (fmt == ORC_Q4_1) {
                    /* gemvq_ref.h:218-220 */
                    const float term = (dw * x->dxf[b]) * (float)sumi + mwf * x->sxf[b];
                    sum[t] += term;
                } else {
                    /* gemvq_ref.h:250-258 */
                    const float term = (float)sumi * (dw * x->dxf[b]);
                    sum[t] += term;
                }
            }
        }
        for (int t = 0; t < T; ++t) {
            float v = sum[t];
            if (mode == 0) {
                if (acc[t] > (__int128)INT64_MAX || acc[t] < (__int128)INT64_MIN) abort();
                v = orc_fixed_to_float((int64_t)acc[t]);
            }
            Y[(size_t)t * ys + (r - r0)] = v;
        }
    }
}

/* ---- AVX-512 VNNI rows (x86 hosts that have it; chosen at run time) ------------------------------------------
 * The same per-row arithmetic as rows_q4q8: only the integer block sums, exact whatever their order, come from
 * vpdpbusd (unsigned byte times signed byte, four products per 32-bit lane), 16 blocks at a time; in the reference
 * mode the 16 blocks' FP32 terms are formed with the scalar path's operations (FP32 products, no fusion) and then
 * added to the row sum one by one in block order. Q8_0 weights (signed) go through |w| and x with w's sign. */
#if defined(__x86_64__)
#define ORC_VNNI __attribute__((target("avx512f,avx512bw,avx512vl,avx512vnni")))
#include <immintrin.h>

/* sums of the 8 consecutive 32-bit lanes of each half of r[0..7]: block 2k in lanes 0-7 of r[k], block 2k + 1 in
 * lanes 8-15; out[b] for b < 16 */
ORC_VNNI static inline void block_sums16(const __m512i * r, int32_t * out) {
    __m512i t[4], u[2];
    for (int k = 0; k < 4; ++k)
        t[k] = _mm512_add_epi32(_mm512_unpacklo_epi32(r[2 * k], r[2 * k + 1]), _mm512_unpackhi_epi32(r[2 * k], r[2 * k + 1]));
    for (int j = 0; j < 2; ++j)
        u[j] = _mm512_add_epi32(_mm512_unpacklo_epi64(t[2 * j], t[2 * j + 1]), _mm512_unpackhi_epi64(t[2 * j], t[2 * j + 1]));
    /* 128-bit lane L of u[j]: lane k of it is a partial sum of r[4j + k]; L 0, 1 the even block, L 2, 3 the odd */
    const __m512i a = _mm512_shuffle_i32x4(u[0], u[1], _MM_SHUFFLE(2, 0, 2, 0));
    const __m512i b = _mm512_shuffle_i32x4(u[0], u[1], _MM_SHUFFLE(3, 1, 3, 1));
    int32_t v[16];
    _mm512_storeu_si512((void *)v, _mm512_add_epi32(a, b));
    /* v: [even of r0..r3 | odd of r0..r3 | even of r4..r7 | odd of r4..r7] */
    for (int k = 0; k < 4; ++k) {
        out[2 * k] = v[k];
        out[2 * k + 1] = v[4 + k];
        out[8 + 2 * k] = v[8 + k];
        out[8 + 2 * k + 1] = v[12 + k];
    }
}

/* the 32 weights of block b as bytes in element order, two blocks per 512-bit vector */
ORC_VNNI static inline __m256i weights32(int fmt, const uint8_t * blk) {
    if (fmt == ORC_Q8_0) return _mm256_loadu_si256((const __m256i *)(blk + 2));
    const __m128i v = _mm_loadu_si128((const __m128i *)(blk + (fmt == ORC_Q4_1 ? 4 : 2))), m4 = _mm_set1_epi8(0x0F);
    return _mm256_set_m128i(_mm_and_si128(_mm_srli_epi16(v, 4), m4), _mm_and_si128(v, m4));
}

ORC_VNNI static void rows_q4q8_vnni(int mode, int fmt, const uint8_t * w, const orc_act * const * a, int T, int r0,
                                    int r1, float * Y, size_t ys) {
    const int nb = a[0]->cols / 32;
    const int bb = fmt == ORC_Q4_0 ? 18 : fmt == ORC_Q4_1 ? 20 : 34;
    const size_t rb = (size_t)nb * bb;
    for (int r = r0; r < r1; ++r) {
        const uint8_t * row = w + (size_t)r * rb;
        __int128 acc[MAXT];
        float sum[MAXT];
        for (int t = 0; t < T; ++t) { acc[t] = 0; sum[t] = 0.0f; }
        for (int b0 = 0; b0 < nb; b0 += 16) {
            __m512i wv[8], neg[8];
            uint16_t hw[16], hm[16];
            for (int k = 0; k < 8; ++k) {
                const uint8_t * p0 = row + (size_t)(b0 + 2 * k) * bb, * p1 = p0 + bb;
                const __m512i v = _mm512_inserti64x4(_mm512_castsi256_si512(weights32(fmt, p0)), weights32(fmt, p1), 1);
                if (fmt == ORC_Q8_0) {
                    neg[k] = _mm512_movm_epi8(_mm512_movepi8_mask(v));
                    wv[k] = _mm512_abs_epi8(v);
                } else {
                    wv[k] = v;
                }
                hw[2 * k] = rd16(p0);
                hw[2 * k + 1] = rd16(p1);
                hm[2 * k] = fmt == ORC_Q4_1 ? rd16(p0 + 2) : 0;
                hm[2 * k + 1] = fmt == ORC_Q4_1 ? rd16(p1 + 2) : 0;
            }
            const __m512 dw = _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i *)hw));
            const __m512 mw = _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i *)hm));
            for (int t = 0; t < T; ++t) {
                const orc_act * x = a[t];
                __m512i rr[8];
                for (int k = 0; k < 8; ++k) {
                    __m512i xv = _mm512_loadu_si512((const void *)(x->q + 32 * (b0 + 2 * k)));
                    if (fmt == ORC_Q8_0) xv = _mm512_sub_epi8(_mm512_xor_si512(xv, neg[k]), neg[k]);  /* x with w's sign */
                    rr[k] = _mm512_dpbusd_epi32(_mm512_setzero_si512(), wv[k], xv);
                }
                int32_t si[16];
                block_sums16(rr, si);
                if (fmt == ORC_Q4_0)
                    for (int j = 0; j < 16; ++j) si[j] -= 8 * x->xsum[b0 + j];
                if (mode == 0) {
                    for (int j = 0; j < 16; ++j) {
                        const int b = b0 + j;
                        int mwp, ewp, nwp;
                        half_me(hw[j], &mwp, &ewp, &nwp);
                        acc[t] += term_parts(si[j], mwp, ewp, nwp, x->mx[b], x->ex[b], x->nx[b]);
                        if (fmt == ORC_Q4_1) {
                            int mm, em, nm;
                            half_me(hm[j], &mm, &em, &nm);
                            acc[t] += term_parts(1, mm, em, nm, x->ms[b], x->es[b], x->ns[b]);
                        }
                    }
                } else {
                    const __m512 dx = _mm512_loadu_ps(x->dxf + b0);
                    const __m512 fs = _mm512_cvtepi32_ps(_mm512_loadu_si512((const void *)si));
                    float term[16];
                    if (fmt == ORC_Q4_1) {  /* (dw * dx) * float(sumi) + m_w * s_x, gemvq_ref.h:218-220 */
                        const __m512 sx = _mm512_loadu_ps(x->sxf + b0);
                        _mm512_storeu_ps(term, _mm512_add_ps(_mm512_mul_ps(_mm512_mul_ps(dw, dx), fs), _mm512_mul_ps(mw, sx)));
                    } else {  /* float(sumi) * (dw * dx), gemvq_ref.h:250-258 */
                        _mm512_storeu_ps(term, _mm512_mul_ps(fs, _mm512_mul_ps(dw, dx)));
                    }
                    float s_ = sum[t];
                    for (int j = 0; j < 16; ++j) s_ += term[j];
                    sum[t] = s_;
                }
            }
        }
        for (int t = 0; t < T; ++t) {
            float v = sum[t];
            if (mode == 0) {
                if (acc[t] > (__int128)INT64_MAX || acc[t] < (__int128)INT64_MIN) abort();
                v = orc_fixed_to_float((int64_t)acc[t]);
            }
            Y[(size_t)t * ys + (r - r0)] = v;
        }
    }
}
#endif

/* The SIMD level of the fast rows: ORC_SIMD_AVX512_VNNI where the host has it (and the rows are whole groups of 16
 * blocks), else ORC_SIMD_AVX2; orc_fast_set_simd lowers it (tests compare both against the scalar oracle). */
static int g_simd = -1;

static int simd_available(void) {
#if defined(__x86_64__)
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") && __builtin_cpu_supports("avx512vl") &&
        __builtin_cpu_supports("avx512vnni"))
        return ORC_SIMD_AVX512_VNNI;
#endif
    return ORC_SIMD_AVX2;
}

int orc_fast_simd(void) {
    if (g_simd < 0) g_simd = simd_available();
    return g_simd;
}

int orc_fast_set_simd(int level) {
    const int avail = simd_available();
    g_simd = level < avail ? level : avail;
    return g_simd;
}

static void rows_q6k(int mode, const uint8_t * w, const orc_act * const * a, int T, int r0, int r1, float * Y, size_t ys) {
    const int nsb = a[0]->cols / 256;
    const size_t rb = (size_t)nsb * 210;
    for (int r = r0; r < r1; ++r) {
        const uint8_t * row = w + (size_t)r * rb;
        __int128 acc[MAXT];
        float sums[MAXT][8];
        for (int t = 0; t < T; ++t) {
            acc[t] = 0;
            for (int l = 0; l < 8; ++l) sums[t][l] = 0.0f;
        }
        for (int sb = 0; sb < nsb; ++sb) {
            const uint8_t * blk = row + (size_t)sb * 210;
            const int8_t * sc = (const int8_t *)(blk + 192);
            uint8_t u[256];
            q6k_unsigned(blk, u);
            const uint16_t hd = rd16(blk + 208);
            int md, ed, nd;
            half_me(hd, &md, &ed, &nd);
            for (int t = 0; t < T; ++t) {
                const orc_act * x = a[t];
                const int8_t * xq = x->q + 256 * sb;
                if (mode == 0) {
                    int64_t off = 0;
                    for (int g = 0; g < 16; ++g) off += (int64_t)sc[g] * x->bs[16 * sb + g];
#ifdef __AVX2__
                    __m256i s32 = _mm256_setzero_si256();
                    for (int v = 0; v < 8; ++v) {
                        const __m256i p = _mm256_maddubs_epi16(_mm256_loadu_si256((const __m256i *)(u + 32 * v)),
                                                               _mm256_loadu_si256((const __m256i *)(xq + 32 * v)));
                        const __m256i scv = _mm256_set_m128i(_mm_set1_epi16(sc[2 * v + 1]), _mm_set1_epi16(sc[2 * v]));
                        s32 = _mm256_add_epi32(s32, _mm256_madd_epi16(p, scv));
                    }
                    const int64_t S = (int64_t)hsum8(s32) - 32 * off;
#else
                    int64_t S = 0;
                    for (int g = 0; g < 16; ++g) {
                        int d = 0;
                        for (int i = 0; i < 16; ++i) d += u[16 * g + i] * xq[16 * g + i];
                        S += (int64_t)sc[g] * d;
                    }
                    S -= 32 * off;
#endif
                    uint32_t xb;
                    memcpy(&xb, &x->d32[sb], 4);
                    const int xe = (xb >> 23) & 255;
                    const int64_t xm = xe == 0 ? 0 : ((xb & 0x7fffffu) | 0x800000u);
                    __int128 p = (__int128)S * (md * xm);
                    if (nd != (int)(xb >> 31)) p = -p;
                    acc[t] += fixed_slow(p, ed + xe - 150);
                } else {
                    /* gemvq_ref.h:148-181: aux32[l] holds elements l and l + 8 of every group of 16 (integers:
                     * exact in any order) */
                    int aux32[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#ifdef __AVX2__
                    const __m256i c32 = _mm256_set1_epi16(32);
                    __m256i acc8 = _mm256_setzero_si256();
                    for (int j = 0; j < 16; ++j) {
                        const __m256i xv = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(xq + 16 * j)));
                        const __m256i uv = _mm256_sub_epi16(
                            _mm256_cvtepu8_epi16(_mm_loadu_si128((const __m128i *)(u + 16 * j))), c32);
                        const __m256i p = _mm256_mullo_epi16(xv, uv);  /* |x (u - 32)| <= 127 * 32 */
                        const __m128i pr = _mm_add_epi16(_mm256_castsi256_si128(p), _mm256_extracti128_si256(p, 1));
                        acc8 = _mm256_add_epi32(acc8, _mm256_mullo_epi32(_mm256_cvtepi16_epi32(pr), _mm256_set1_epi32(sc[j])));
                    }
                    _mm256_storeu_si256((__m256i *)aux32, acc8);
#else
                    for (int j = 0; j < 16; ++j) {
                        int pr[8];
                        for (int i = 0; i < 8; ++i)
                            pr[i] = xq[16 * j + i] * ((int)u[16 * j + i] - 32) + xq[16 * j + i + 8] * ((int)u[16 * j + i + 8] - 32);
                        for (int i = 0; i < 8; ++i) aux32[i] += sc[j] * pr[i];
                    }
#endif
                    const float d = orc_half_to_float(hd) * x->d32[sb];
                    for (int l = 0; l < 8; ++l) sums[t][l] += d * (float)aux32[l];
                }
            }
        }
        for (int t = 0; t < T; ++t) {
            float v;
            if (mode == 0) {
                if (acc[t] > (__int128)INT64_MAX || acc[t] < (__int128)INT64_MIN) abort();
                v = orc_fixed_to_float((int64_t)acc[t]);
            } else {
                v = 0.0f;
                for (int l = 0; l < 8; ++l) v += sums[t][l];
            }
            Y[(size_t)t * ys + (r - r0)] = v;
        }
    }
}

int orc_fast_supported(int fmt) { return fmt == ORC_Q4_0 || fmt == ORC_Q4_1 || fmt == ORC_Q8_0 || fmt == ORC_Q6_K; }

void orc_fast_rows_multi(int mode, int fmt, const uint8_t * w, const orc_act * const * a, int T, int r0, int r1,
                         float * y, size_t ys) {
    if (T < 1 || T > MAXT) abort();
    if (fmt == ORC_Q6_K) {
        rows_q6k(mode, w, a, T, r0, r1, y, ys);
    } else if (fmt == ORC_Q4_0 || fmt == ORC_Q4_1 || fmt == ORC_Q8_0) {
#if defined(__x86_64__)
        if (orc_fast_simd() == ORC_SIMD_AVX512_VNNI && (a[0]->cols / 32) % 16 == 0) {
            rows_q4q8_vnni(mode, fmt, w, a, T, r0, r1, y, ys);
            return;
        }
#endif
        rows_q4q8(mode, fmt, w, a, T, r0, r1, y, ys);
    } else { /* Q5_K: the scalar oracle row by row */
        if (mode != 0) abort(); /* the scalar reference path quantizes itself: use orc_ref_gemv */
        const size_t rb = orc_row_bytes(fmt, a[0]->cols);
        for (int t = 0; t < T; ++t)
            for (int r = r0; r < r1; ++r)
                orc_fx_gemv_q(fmt, w + (size_t)r * rb, a[t]->q, a[t]->d16, a[t]->d32, a[t]->bs, 1, a[t]->cols,
                              y + (size_t)t * ys + (r - r0), NULL, NULL);
    }
}

void orc_fast_rows(int mode, int fmt, const uint8_t * w, const orc_act * a, int r0, int r1, float * y) {
    orc_fast_rows_multi(mode, fmt, w, &a, 1, r0, r1, y, 0);
}

void orc_fast_gemv(int mode, int fmt, const uint8_t * w, const float * x, int rows, int cols, float * y) {
    if (mode == 1 && !orc_fast_supported(fmt)) {
        orc_ref_gemv(fmt, w, x, rows, cols, y, NULL);
        return;
    }
    orc_act a;
    orc_act_init(&a, fmt, x, cols);
    orc_fast_rows(mode, fmt, w, &a, 0, rows, y);
    orc_act_free(&a);
}

void orc_fast_gemv_mt(int mode, int fmt, const uint8_t * w, const float * x, int rows, int cols, float * y,
                      int n_threads) {
    if (n_threads < 1) n_threads = 1;
    const size_t rb = orc_row_bytes(fmt, cols);
    const int parts = 4 * n_threads;  /* row ranges, dealt to the threads statically */
    if (mode == 1 && !orc_fast_supported(fmt)) {
#pragma omp parallel for num_threads(n_threads) schedule(static)
        for (int c = 0; c < parts; ++c) {
            const int r0 = (int)((long long)rows * c / parts), r1 = (int)((long long)rows * (c + 1) / parts);
            if (r1 > r0) orc_ref_gemv(fmt, w + (size_t)r0 * rb, x, r1 - r0, cols, y + r0, NULL);
        }
        return;
    }
    orc_act a;
    orc_act_init(&a, fmt, x, cols);
#pragma omp parallel for num_threads(n_threads) schedule(static)
    for (int c = 0; c < parts; ++c) {
        const int r0 = (int)((long long)rows * c / parts), r1 = (int)((long long)rows * (c + 1) / parts);
        if (r1 > r0) orc_fast_rows(mode, fmt, w, &a, r0, r1, y + r0);
    }
    orc_act_free(&a);
}
