/* Fast rows of the CPU oracle (TEST INFRASTRUCTURE ONLY, see gemvq_oracle.h): the oracle's two GEMV arithmetics
 * with the integer block sums formed by int8 SIMD dot products. Bit-identical to orc_fx_gemv (mode 0) and
 * orc_ref_gemv (mode 1). */
#ifndef ORC_FAST_H
#define ORC_FAST_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* A quantized activation row: Q8_0 (Q4_0 / Q8_0 weights), Q8_1 (Q4_1) or Q8_K (Q5_K / Q6_K). */
typedef struct {
    int fmt, cols;
    int8_t * q;
    uint16_t * d16;   /* Q8_0 / Q8_1 fp16 scale bits */
    uint16_t * s16;   /* Q8_1 fp16 s bits */
    float * d32;      /* Q8_K scales */
    int16_t * bs;     /* Q8_K bsums */
    int32_t * xsum;   /* Q8_0 / Q8_1 sum of each block's quants */
    /* Q8_0 / Q8_1: the fp16 scale d (and Q8_1 s) split into significand, exponent and sign, and as FP32 */
    int32_t * mx, * ms;
    int8_t * ex, * es, * nx, * ns;
    float * dxf, * sxf;
} orc_act;

/* SIMD level of the fast rows: the highest the host supports unless lowered (returns the level in effect). */
enum { ORC_SIMD_AVX2 = 0, ORC_SIMD_AVX512_VNNI = 1 };
int orc_fast_simd(void);
int orc_fast_set_simd(int level);

void orc_act_init(orc_act * a, int weight_fmt, const float * x, int cols);
void orc_act_free(orc_act * a);
int orc_fast_supported(int fmt);
/* y[0 .. r1 - r0) = rows r0 .. r1 - 1 of w (GGUF layout) times the activation; mode 0 canonical, 1 reference. */
void orc_fast_rows(int mode, int fmt, const uint8_t * w, const orc_act * a, int r0, int r1, float * y);
/* The same for T <= 32 activation rows at once (each weight row read once): token t's results at y + t * ys. */
void orc_fast_rows_multi(int mode, int fmt, const uint8_t * w, const orc_act * const * a, int T, int r0, int r1,
                         float * y, size_t ys);
/* Quantizes x and runs every row (the pinning entry point of the tests). */
void orc_fast_gemv(int mode, int fmt, const uint8_t * w, const float * x, int rows, int cols, float * y);
/* The same with the rows split over n_threads OpenMP threads (placement from OMP_PLACES / OMP_PROC_BIND). */
void orc_fast_gemv_mt(int mode, int fmt, const uint8_t * w, const float * x, int rows, int cols, float * y,
                      int n_threads);

#ifdef __cplusplus
}
#endif
#endif
