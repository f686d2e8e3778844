/* CPU oracle for the batch-1 decode path: TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and only as the
 * checker (or as the timed CPU baseline). The product library never links it.
 *
 * Two arithmetics are restated here:
 *   ref_*  the reference's plain-C++ CPU path (fpga/src/gemvq_ref.h): ggml's generic quantize_row_q8_0/q8_K and
 *          vec_dot_*_generic with sequential FP32 row sums, double-precision norm sums, sequential GDN dots.
 *   fx_* / canonical ops  the arithmetic the GPU reproduces bit for bit: exact integer block dots, each block (or
 *          super-block) term exact and truncated to a fixed-point LSB of 2^-40 as the reference kernel does
 *          (fpga/src/gemvqw_engine.h:352-445, fpga/src/stream_common.h:59-126), summed exactly in integers and
 *          rounded to FP32 once; FP32 reductions (norms, GDN dots) as a pairwise tree over element indices; own
 *          exp/log (Cody-Waite reduction + Taylor/atanh series) so CPU and GPU evaluate the same formulas.
 * The ref_* path pins the canonical one within the reference's own tolerances (gemvq_ref.h:267-284, 399-402).
 */
#ifndef GEMVQ_ORACLE_H
#define GEMVQ_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (gemvqw.h:6-10) */
enum { ORC_Q4_0 = 2, ORC_Q4_1 = 3, ORC_Q8_0 = 8, ORC_Q5_K = 13, ORC_Q6_K = 14 };

/* ---- scalar helpers ---- */
float orc_half_to_float(uint16_t h);
uint16_t orc_float_to_half(float f);
int orc_nearest_int(float v);
float orc_expf(float x);
float orc_logf(float x);
float orc_silu(float x);
float orc_sigmoid(float x);
float orc_softplus(float x);
/* Canonical FP32 sum (pairwise): pad to the next power of two P with +0, then for s = 1, 2, .. P/2:
 * a[i] += a[i + s] for i = 0, 2s, 4s, ..; the result is a[0]. Every aligned power-of-two chunk is a subtree. */
float orc_pair_sum(const float * a, int n);
size_t orc_row_bytes(int fmt, int cols);

/* ---- correctly rounded exp and log (orc_crmath.c): the binary32 value nearest to e^x / log x ---- */
float orc_cr_expf(float x);
float orc_cr_logf(float x);
/* Exhaustive checks over every binary32 input (orc_crcheck.c); fn 0 exp, 1 log. out: [0] inputs where orc_cr_* is
 * not the correctly rounded result, [1] inputs where the host libm (expf / logf) differs from orc_cr_*, [2] inputs
 * the 80-bit reference left to quad precision, [3] inputs off the special cases. */
void orc_crmath_check(int fn, int n_threads, uint64_t out[4]);
/* Inputs where other() differs from orc_cr_* (NaN equals NaN). */
uint64_t orc_crmath_compare(int fn, float (*other)(float), int n_threads);
/* hashes[b], b < 4096: sum mod 2^64 over i < 2^20 of bits(f(bits b 2^20 + i)) (2 i + 1), NaN as 0x7fc00000. */
void orc_crmath_hash(int fn, uint64_t * hashes, int n_threads);

/* ---- activation quantizers (gemvq_ref.h:62-81, 236-245) ---- */
/* Q8_0: per 32 values d_bits = fp16(amax / 127), q = roundf(x * (1 / (amax / 127))). */
void orc_quantize_q8_0(const float * x, int n, int8_t * q, uint16_t * d_bits);
/* Q8_1 (for Q4_1 weights): Q8_0's quants, d_bits = fp16(amax / 127), s_bits = fp16(sum(q) * (amax / 127)). */
void orc_quantize_q8_1(const float * x, int n, int8_t * q, uint16_t * d_bits, uint16_t * s_bits);
/* Q8_K: per 256 values iscale = -127 / max (signed value of largest magnitude, first on ties), q = min(127,
 * nearest_int(iscale * x)), d = 1 / iscale; bsums per 16 values. */
void orc_quantize_q8_K(const float * x, int n, int8_t * q, float * d, int16_t * bsums);

/* ---- GEMV, reference path (gemvq_ref.h:94-265): sequential FP32; mag = sum of |block terms| per row ---- */
void orc_ref_gemv(int fmt, const uint8_t * w, const float * x, int rows, int cols, float * y, double * mag);
int orc_ref_within_tolerance(float got, float ref, double mag);

/* ---- GEMV, canonical fixed-point path ----
 * y[r] = fp32(sum_b floor(term_b * 2^40)) * 2^-40. blocksums (optional): per row the integer block sums, Q4_0/Q4_1/
 * Q8_0 one int32 per 32-block (sum_j w_j * q8_j with the Q4_0 weights minus 8; Q4_1 (this build's extension of the
 * kernel arithmetic, which has no Q4_1): term = floor(sumi d_w d_x 2^40) + floor(m_w s_x 2^40)), Q5_K/Q6_K two int32 per super-block
 * (S = sum sc * (q . q8), M = sum m * bsum, M = 0 for Q6_K). acc (optional): the int64 fixed-point row sums. */
void orc_fx_gemv(int fmt, const uint8_t * w, const float * x, int rows, int cols, float * y, int32_t * blocksums,
                 int64_t * acc);
/* Same on an already quantized x (Q8_0: q + fp16 scale bits; Q8_1: q + fp16 d bits + the fp16 s bits passed as
 * xbsums; Q8_K: q + FP32 d + bsums). */
void orc_fx_gemv_q(int fmt, const uint8_t * w, const int8_t * xq, const uint16_t * xd16, const float * xd32,
                   const int16_t * xbsums, int rows, int cols, float * y, int32_t * blocksums, int64_t * acc);
float orc_fixed_to_float(int64_t acc);

/* ---- norms ---- */
void orc_ref_rmsnorm(const float * x, const float * w, int n, float eps, float * y);               /* gemvq_ref.h:288 */
void orc_ref_rownorm(const float * x, const float * w, int n, int rows, float eps, int flags, float * y); /* :310 */
/* Canonical row norm (RMSNORM opcode): flags bit0 L2, bit1 no weight; rows of n floats every stride floats. */
float orc_norm_scale(const float * x, int n, float eps, int l2);
void orc_rownorm(const float * x, const float * w, int n, int rows, int stride, float eps, int flags, float * y);

/* ---- element-wise (gemvq_ref.h:297-358, gemvqc_ops.h:64-99, 387-431) ---- */
void orc_silu_mul(const float * g, const float * u, int n, int sigmoid, float * y);
void orc_unary(const float * x, int n, int kind, float * y);
void orc_conv(const float * state, const float * x, const float * w, int ch, int silu, float * y, float * new_state);
void orc_rope(const float * x, const float * cs, int n_dims, int ne0, int rows, float * y);
void orc_ref_conv(const float * state, const float * x, const float * w, int ch, int silu, float * y, float * new_state);
void orc_ref_unary(const float * x, int n, int kind, float * y);
/* The same with the correctly rounded exp / log in place of libm's (the reference-arithmetic decoder). */
void orc_ref_conv_cr(const float * state, const float * x, const float * w, int ch, int silu, float * y, float * new_state);
void orc_ref_unary_cr(const float * x, int n, int kind, float * y);
void orc_ref_silu_mul_cr(const float * g, const float * u, int n, float * y);

/* ---- Gated DeltaNet step ---- */
/* Reference (gemvq_ref.h:363-397): state [hv][128][128] in place, q/k [hk][128], v [hv][128], g, beta [hv] (g is
 * the log decay, beta already the gate); y [hv][128]; y_mag / s_mag may be NULL. */
void orc_ref_gdn(float * state, const float * q, const float * k, const float * v, const float * g, const float * beta,
                 int hv, int hk, float scale, float * y, double * y_mag, double * s_mag);
void orc_ref_gdn_mt(float * state, const float * q, const float * k, const float * v, const float * g,
                    const float * beta, int hv, int hk, float scale, float * y, double * y_mag, double * s_mag,
                    int n_threads);
void orc_ref_gdn_cr_mt(float * state, const float * q, const float * k, const float * v, const float * g,
                       const float * beta, int hv, int hk, float scale, float * y, int n_threads);
/* Canonical fused step (GDN opcode): flags bit1 L2-normalize q/k (l2_eps), bit2 gated output norm
 * (rms_eps, w[128], z[hv*128]), bit3 gates from raw projections (beta = sigmoid(b), g = softplus(a_raw + dt) * a),
 * bit5 z already holds silu(z).
 * state updated in place, y receives the (gated) output. */
void orc_gdn(float * state, const float * q, const float * k, const float * v, const float * graw, const float * braw,
             const float * dt, const float * a, const float * z, const float * w, int hv, int hk, float scale,
             float l2_eps, float rms_eps, int flags, float * y);
void orc_gdn_mt(float * state, const float * q, const float * k, const float * v, const float * graw, const float * braw,
                const float * dt, const float * a, const float * z, const float * w, int hv, int hk, float scale,
                float l2_eps, float rms_eps, int flags, float * y, int n_threads);

/* ---- attention core (one token, GQA, F16 KV cache) ----
 * q [nh][hd] fp32 (rounded to fp16 like ggml's F16 vec_dot type), kc/vc [n_kv][nkvh][hd] fp16 bits (positions
 * 0..n_kv-1), softmax in chunks of 64 positions (online max per chunk, combined over chunks in order), out [nh][hd]. */
void orc_attn(const float * q, const uint16_t * kc, const uint16_t * vc, int nh, int nkvh, int hd, int n_kv,
              float scale, float * out);
void orc_attn_mt(const float * q, const uint16_t * kc, const uint16_t * vc, int nh, int nkvh, int hd, int n_kv,
                 float scale, float * out, int n_threads);
/* The reference-arithmetic decoder's attention: ggml's CPU path without flash attention (fp16 q, F16 dots summed in
 * double, softmax with libm expf and a double sum, fp16 probabilities times V). */
void orc_ref_attn(const float * q, const uint16_t * kc, const uint16_t * vc, int nh, int nkvh, int hd, int n_kv,
                  float scale, float * out);
void orc_ref_attn_mt(const float * q, const uint16_t * kc, const uint16_t * vc, int nh, int nkvh, int hd, int n_kv,
                     float scale, float * out, int n_threads);
void orc_ref_attn_cr_mt(const float * q, const uint16_t * kc, const uint16_t * vc, int nh, int nkvh, int hd, int n_kv,
                        float scale, float * out, int n_threads);

/* ---- Q6_K row dequantize (ggml dequantize_row_q6_K) and argmax ---- */
void orc_dequant_row_q6_K(const uint8_t * row, int cols, float * y);
int orc_argmax(const float * x, int n);

#ifdef __cplusplus
}
#endif
#endif
