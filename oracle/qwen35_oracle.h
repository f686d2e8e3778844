/* CPU oracle of the synthetic Qwen3.5-shaped hybrid decoder (TEST INFRASTRUCTURE ONLY, see gemvq_oracle.h).
 * One token per call through the whole model with the canonical arithmetic of gemvq_oracle.c; the greedy token is
 * the argmax of the logits. The layer structure follows llama.cpp's qwen35 graph as the reference offloads it
 * (llama.cpp/patches/0006-qwen35-graph-order.patch: qkv/z/beta/alpha after the norm for DeltaNet layers, q/k/v for
 * attention layers) and the reference's fused op forms (fpga/src/gemvqc16.h:26-91). */
#ifndef QWEN35_ORACLE_H
#define QWEN35_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int32_t n_layer, n_embd, n_ff, n_vocab;
    int32_t n_head, n_head_kv, head_dim, n_rot;
    int32_t ssm_k_heads, ssm_v_heads, ssm_head_dim, ssm_conv;
    int32_t attn_interval, n_ctx;
    float eps, rope_base;
} orc_qw_config;

/* One tensor of a model blob: ggml type id (0 F32, 2 Q4_0, 8 Q8_0, 13 Q5_K, 14 Q6_K), ne0 = columns, ne1 = rows. */
typedef struct {
    char name[64];
    int32_t type, ne0, ne1, pad;
    uint64_t offset, nbytes;
} orc_tensor_desc;

void * orc_model_create(const orc_qw_config * cfg, const orc_tensor_desc * table, int n_tensors, const uint8_t * blob,
                        int n_threads);
/* Runs token at position pos; logits (n_vocab floats) may be NULL. Returns the greedy token, or -1 on error. */
int orc_model_decode(void * model, int token, int pos, float * logits);
/* Hidden state after the last layer (before the output norm) of the latest decode, n_embd floats. */
const float * orc_model_hidden(void * model);
void orc_model_destroy(void * model);

/* ggml's rope cache for one position (NEOX, ext_factor 0, freq_scale 1, attn_factor 1): n_dims floats, cos and sin of
 * pair i at 2i, 2i + 1, theta advanced by theta *= base^(-2 / n_dims) as ggml does. */
void orc_rope_cache(int pos, int n_dims, float base, float * cs);

#ifdef __cplusplus
}
#endif
#endif
