/* CPU oracle of the synthetic Qwen3.5-shaped hybrid decoder (TEST INFRASTRUCTURE ONLY, see gemvq_oracle.h).
 * Tokens run through the whole model in the canonical arithmetic of gemvq_oracle.c (or, in reference mode, the
 * reference's CPU arithmetic); the greedy token is the argmax of the logits. The layer structure follows llama.cpp's qwen35 graph as the reference offloads it
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
/* Arithmetic of the following tokens (the states carry over): the canonical one the GPU reproduces bit for bit
 * (default); the reference's sequential FP32 rows and double sums of squares with correctly rounded exp / log (the
 * GPU's reference-arithmetic mode reproduces it bit for bit); or the same with the host libm's expf / logf. */
enum { ORC_MODE_CANONICAL = 0, ORC_MODE_REFERENCE = 1, ORC_MODE_REFERENCE_LIBM = 2 };
int orc_model_set_mode(void * model, int mode);
/* Planted wiring mistakes, for tests that show the independent checks catch them (0: none). */
enum {
    ORC_FAULT_NONE = 0,
    ORC_FAULT_ATTN_RESIDUAL = 1,  /* the attention output replaces the residual stream instead of adding to it */
    ORC_FAULT_QGATE_SWAP = 2,     /* q read from the gate half of the interleaved q + gate rows, and the gate from q */
    ORC_FAULT_GATES_SWAP = 3,     /* the DeltaNet beta and alpha projections exchanged */
    ORC_FAULT_FFN_SWAP = 4,       /* ffn_gate and ffn_up exchanged (SiLU on the wrong one) */
    ORC_FAULT_ROPE_K = 5,         /* keys cached without their RoPE rotation */
    ORC_FAULT_SSM_RESIDUAL = 6,   /* the ssm_out output replaces the residual stream */
    ORC_FAULT_LAST = 6
};
int orc_model_set_fault(void * model, int fault);
/* out (NULL: off) receives, for the last token of every later call, the residual stream before layer 0 and after
 * each layer: (n_layer + 1) x n_embd floats. */
int orc_model_set_trace(void * model, float * out);
/* Clears the recurrent states and the KV cache. */
int orc_model_reset(void * model);
/* Runs token at position pos; logits (n_vocab floats) may be NULL. Returns the greedy token, or -1 on error. */
int orc_model_decode(void * model, int token, int pos, float * logits);
/* Runs n tokens at positions pos0 .. pos0 + n - 1 in chunks of up to 32 (each weight row read once per chunk), no
 * logits; the states and caches afterwards equal those of n decode steps bit for bit. */
int orc_model_prefill(void * model, const int32_t * tokens, int n, int pos0);
/* Greedy decode from a reset model: the prompt (prefill of all but its last token), then n_gen decode steps. out
 * receives n_prompt + n_gen ids; last_logits (may be NULL) the logits of the last step. */
int orc_model_generate(void * model, const int32_t * prompt, int n_prompt, int n_gen, int32_t * out, float * last_logits);
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
