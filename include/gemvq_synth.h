/* Synthetic data for the decode path: a portable counter-based RNG and ggml's reference weight quantizers, so that
 * every run (this machine, the GPU host) produces the same bytes from a seed. Host-only C ABI, no GPU calls.
 * Not part of the decode hot path; the reference consumes GGUF files instead (llama.cpp model loading). */
#ifndef GEMVQ_SYNTH_H
#define GEMVQ_SYNTH_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Value i of stream `stream` under `seed`: SplitMix64 of (key + (i + 1) * golden gamma), key derived from seed and
 * stream. Normals by Box-Muller in double on pairs (2p, 2p + 1). */
uint64_t gqs_u64(uint64_t seed, uint64_t stream, uint64_t i);
void gqs_normal(uint64_t seed, uint64_t stream, uint64_t first, size_t n, float mean, float stddev, float * out);
void gqs_uniform(uint64_t seed, uint64_t stream, uint64_t first, size_t n, float lo, float hi, float * out);

/* ggml quantize_row_{q4_0,q4_1,q8_0,q5_K,q6_K}_ref on `rows` rows of `cols` floats (GGUF block bytes out). type is
 * the ggml type id (2, 3, 8, 13, 14). Returns the bytes written, 0 for an unsupported type or shape. */
size_t gqs_quantize(int type, const float * x, int64_t rows, int64_t cols, uint8_t * out);
size_t gqs_row_bytes(int type, int64_t cols);

/* A rows x cols matrix drawn from N(mean, stddev^2) (element (r, c) is value r * cols + c of the stream) and
 * quantized to `type`, generated in parallel by n_threads. */
size_t gqs_matrix(int type, int64_t rows, int64_t cols, uint64_t seed, uint64_t stream, float mean, float stddev,
                  uint8_t * out, int n_threads);

#ifdef __cplusplus
}
#endif
#endif
