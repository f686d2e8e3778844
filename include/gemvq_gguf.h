/* GGUF model files on the host (no GPU call): the reader that hands GGUF weight rows to gemvq_upload_weight, and the
 * inverse of ggml's CPU_REPACK Q4_0x8 layout.
 *
 * The reference receives its weights from llama.cpp, which reads the GGUF file and may hold Q4_0 tensors in the
 * CPU_REPACK buffer type; its backend turns those back into GGUF rows before repacking them for the card
 * (ggml-xrt.cpp:675-710, xrt_gguf). These entry points give a caller of this backend the same two steps. The file is
 * memory-mapped read-only; tensor data pointers stay valid until gemvq_gguf_close. Format: GGUF version 2 or 3 (magic
 * "GGUF", key/value metadata, tensor infos with ne0 first, data aligned to general.alignment, default 32). */
#ifndef GEMVQ_GGUF_H
#define GEMVQ_GGUF_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gemvq_gguf gemvq_gguf;

/* Opens and parses a file; NULL on error (gemvq_gguf_last_error() says why). */
gemvq_gguf * gemvq_gguf_open(const char * path);
void gemvq_gguf_close(gemvq_gguf * f);
const char * gemvq_gguf_last_error(void);

int gemvq_gguf_version(const gemvq_gguf * f);
int gemvq_gguf_n_tensors(const gemvq_gguf * f);
/* Tensor i: name (NUL-terminated, truncated to name_cap), ggml type, dimensions (ne[0] innermost, unused = 1),
 * data pointer into the mapping, size in bytes. Returns 0, or -1 for a bad index. */
int gemvq_gguf_tensor(const gemvq_gguf * f, int i, char * name, size_t name_cap, int * type, int64_t ne[4],
                      const void ** data, uint64_t * nbytes);
/* Byte offset of tensor i's data from the start of the file, or -1. */
int64_t gemvq_gguf_file_offset(const gemvq_gguf * f, int i);
/* Index of the tensor named `name`, or -1. */
int gemvq_gguf_find(const gemvq_gguf * f, const char * name);
/* Scalar metadata: 0 and the value if `key` exists with a numeric type (converted), -1 otherwise. */
int gemvq_gguf_get_f64(const gemvq_gguf * f, const char * key, double * out);
/* String metadata: a pointer to the NUL-terminated value (valid until close), or NULL. */
const char * gemvq_gguf_get_str(const gemvq_gguf * f, const char * key);

/* block_q4_0x8 (8 rows interleaved: 8 fp16 scales, then 16 chunks of 8 quant bytes, chunk c = bytes 8 (c / 8)..
 * of row c % 8, each byte XOR 0x88) -> GGUF block_q4_0 rows (fp16 scale, 16 bytes of quants), lossless
 * (ggml-xrt.cpp:675-710). rows % 8 == 0, cols % 32 == 0. Returns 0 or -1. */
int gemvq_unrepack_q4_0x8(int rows, int cols, const void * x8, void * gguf_rows);

#ifdef __cplusplus
}
#endif
#endif
