/* Batch-1 greedy decode of a Qwen3.5-shaped hybrid model (Gated DeltaNet and gated-attention layers in a fixed
 * interval) on the command-list backend of gemvq_hip.h.
 *
 * This is the work the reference's ggml backend does for every token (ggml-xrt.cpp:2190-2745: node fusion into
 * command lists, operand placement in the activation buffer, GDN state traffic), done once: the model's per-token
 * command list is built at create time, validated, and captured as one hipGraph. A token is one replay. The token
 * id, its position and the greedy argmax stay on the device (NEXT_TOKEN), so a whole prompt + generation is a
 * sequence of replays with no host round trip. Tensor names follow GGUF / llama.cpp's qwen35 conventions. */
#ifndef GEMVQ_QWEN35_H
#define GEMVQ_QWEN35_H
#include <stddef.h>
#include <stdint.h>

#include "gemvq_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int32_t n_layer, n_embd, n_ff, n_vocab;
    int32_t n_head, n_head_kv, head_dim, n_rot;
    int32_t ssm_k_heads, ssm_v_heads, ssm_head_dim, ssm_conv;
    int32_t attn_interval, n_ctx;  /* layer il is full attention when (il + 1) % attn_interval == 0 */
    float eps, rope_base;
} gemvq_qw_config;

/* One tensor of a model blob (GGUF-style): ggml type id, ne0 = columns, ne1 = rows, byte offset and size. */
typedef struct {
    char name[64];
    int32_t type, ne0, ne1, pad;
    uint64_t offset, nbytes;
} gemvq_tensor_desc;

typedef struct gemvq_qwen35 gemvq_qwen35;

/* Context sizes a model needs (activation floats, weight bytes, GDN state rows). */
int gemvq_qwen35_sizes(const gemvq_qw_config * cfg, const gemvq_tensor_desc * table, int n_tensors,
                       size_t * act_floats, size_t * weight_bytes, size_t * state_rows);
/* Uploads the weights into ctx, allocates KV buffers, lays out the activation buffer and builds the per-token
 * command list. Returns NULL on failure (gemvq_last_error(ctx) says why). */
gemvq_qwen35 * gemvq_qwen35_create(gemvq_ctx * ctx, const gemvq_qw_config * cfg, const gemvq_tensor_desc * table,
                                   int n_tensors, const uint8_t * blob);
void gemvq_qwen35_destroy(gemvq_qwen35 * m);
/* Clears recurrent states and KV, stores the prompt (n >= 1 ids) and sets position 0 with token prompt[0]. */
int gemvq_qwen35_reset(gemvq_qwen35 * m, const int32_t * prompt, int n);
/* Enqueues n decode steps (replays of the per-token graph, captured by the first step after create or after a
 * reset with a new prompt length); asynchronous. */
int gemvq_qwen35_step(gemvq_qwen35 * m, int n);
/* Runs the next n prompt positions (all before the last prompt token) in chunks of up to GEMVQ_GEMM_MAX_TOK tokens
 * per weight read (GEMM commands; the reference plans this batched path, ROADMAP.md:78-96, and has no counterpart):
 * afterwards the model is where n decode steps would have left it (states, KV cache, position, token ids), bit for
 * bit, without the logits. GEMVQ_EINVAL when a projection has no batched form (Q4_0 / Q4_1 / Q8_0 with columns a
 * multiple of 512; decode steps then do the same work) or the positions pass the last prompt token but one; synchronizes. */
int gemvq_qwen35_prefill(gemvq_qwen35 * m, int n);
/* Token ids at positions 0 .. n - 1 (prompt tokens, then generated ones); synchronizes. */
int gemvq_qwen35_tokens(gemvq_qwen35 * m, int32_t * out, int n);
/* Logits of the last step (n_vocab floats); synchronizes. */
int gemvq_qwen35_logits(gemvq_qwen35 * m, float * out);
/* Hidden state after the last layer of the last step (n_embd floats); synchronizes. */
int gemvq_qwen35_hidden(gemvq_qwen35 * m, float * out);
/* The per-token command list (words) and the number of commands; n_words = 0 queries the size. */
int gemvq_qwen35_commands(gemvq_qwen35 * m, uint32_t * words, size_t n_words);
/* The captured graph id (for gemvq_graph_time); -1 before the first step. */
int gemvq_qwen35_graph(gemvq_qwen35 * m);
/* The arithmetic of the model's steps and prefill from now on (gemvq_set_arith on its context; the graphs are
 * captured again): GEMVQ_ARITH_REFERENCE decodes with the tokens and logits of the reference's CPU path. The
 * states carry over. 0 or GEMVQ_EINVAL. */
int gemvq_qwen35_set_arith(gemvq_qwen35 * m, int arith);
/* Lockstep decode of n_seq (2..GEMVQ_GEMM_MAX_TOK) sequences (the multi-sequence path the reference plans,
 * ROADMAP.md:78-96; no counterpart in its code): every step reads each weight row once for all sequences (GEMM
 * commands over their n_seq token rows), with CONV, the DeltaNet step and attention in their sequences forms, so
 * each sequence keeps its own conv windows, state rows, KV region (n_ctx positions) and position, and its ids and
 * logits are those of a single-sequence model decoding its prompt, bit for bit. Prompts are consumed by the same
 * steps (a sequence takes its next prompt token while it has one, then its argmax). Layer projections must have a
 * batched form (Q4_0 / Q4_1 / Q8_0, columns a multiple of 512); a head of another type runs one GEMV per sequence.
 * gemvq_qwen35_batch_sizes gives the context sizes; gemvq_qwen35_step, _set_arith, _commands, _graph and _destroy
 * apply to the batch model (in the reference arithmetic each sequence's ids and logits are those of a
 * single-sequence model decoding in it), the single-sequence _reset, _prefill, _tokens, _logits and _hidden return
 * GEMVQ_EINVAL for it
 * (gemvq_qwen35_batch_create with n_seq 1 is gemvq_qwen35_create). */
int gemvq_qwen35_batch_sizes(const gemvq_qw_config * cfg, const gemvq_tensor_desc * table, int n_tensors, int n_seq,
                             size_t * act_floats, size_t * weight_bytes, size_t * state_rows);
gemvq_qwen35 * gemvq_qwen35_batch_create(gemvq_ctx * ctx, const gemvq_qw_config * cfg,
                                         const gemvq_tensor_desc * table, int n_tensors, const uint8_t * blob,
                                         int n_seq);
/* Clears states and KV; sequence s gets prompts[offsets[s] .. offsets[s + 1]) (1..n_ctx ids) and position 0. */
int gemvq_qwen35_batch_reset(gemvq_qwen35 * m, const int32_t * prompts, const int32_t * offsets);
/* Sequence seq's token ids at positions 0 .. n - 1; its logits of the last step (n_vocab floats); synchronize. */
int gemvq_qwen35_batch_tokens(gemvq_qwen35 * m, int seq, int32_t * out, int n);
int gemvq_qwen35_batch_logits(gemvq_qwen35 * m, int seq, float * out);
/* The per-token command list gemvq_qwen35_create would build, without a device: weights placed as
 * gemvq_upload_weight places them in table order, KV buffers numbered in layer order. Returns the number of commands
 * (words copied when n_words is large enough), or GEMVQ_EINVAL. */
int gemvq_qwen35_dry_commands(const gemvq_qw_config * cfg, const gemvq_tensor_desc * table, int n_tensors,
                              uint32_t * words, size_t n_words);

#ifdef __cplusplus
}
#endif
#endif
