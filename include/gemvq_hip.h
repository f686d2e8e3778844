/* MI355X (gfx950) batch-1 decode backend: the C ABI between the C++ host side and the HIP kernels.
 *
 * It replaces the boundary between the reference's ggml backend and its FPGA kernel:
 *   - gemvq_run()            replaces the kernel call gemvqc16(w0..w19, act, cmds, n_cmds, st..., act_rd)
 *                            (fpga/src/gemvqc16.h:136-149) and its launch by xrt_qc_launch (ggml-xrt.cpp:1241-1280);
 *   - gemvq_upload_weight()  replaces xrt_qc_weight_offset + gemvqw_layout::repack (ggml-xrt.cpp:735-765,
 *                            fpga/src/gemvqw_layout.h:137-157): one layout-only repack at load;
 *   - gemvq_act_write/read() replace the act BO syncs of xrt_qc_flush (ggml-xrt.cpp:1399-1478);
 *   - gemvq_state_*()        replace the XRT_RS buffer I/O (ggml-xrt.cpp:439-475, 535-552);
 *   - gemvq_graph_*()        a per-token command list captured once as a hipGraph and replayed per token (the
 *                            reference starts the kernel once per list, ggml-xrt.cpp:1241-1280);
 *   - gemvq_features()       the n_cmds == 0 feature probe (gemvqc16.cpp:1076-1082, ggml-xrt.cpp:1284-1300).
 * Plain C types only; a context is not re-entrant (one host thread at a time, as the reference's backend mutex).
 *
 * Command list: GEMVQ_CMD_WORDS uint32 words per command, the opcodes and word layouts of gemvqc16.h:26-98, act
 * offsets and lengths in floats and multiples of 16 as there (gemvqc16.h:24-25), with these differences: a GEMV's
 * w_off lo/hi is the weight offset returned by gemvq_upload_weight (the matrix keeps its rows/cols/format from the
 * upload and the command must repeat them); GDN state rows index the state buffer (128 floats per row); there is no
 * STATE_LOAD prefetch need (the opcode is accepted and does nothing) and TRACE is accepted and does nothing. Opcodes
 * added for the parts the reference leaves on the CPU (attention core, embedding rows, greedy sampling) are listed
 * below.
 *
 *   GEMV      [1, format | flags, rows, cols, w_off lo, w_off hi, x_off, y_off]
 *             format 2 Q4_0, 3 Q4_1 (Q8_1 activations), 8 Q8_0, 13 Q5_K, 14 Q6_K; flags GEMVQ_GEMV_SWIGLU
 *             (0x100), GEMVQ_GEMV_CONV (0x200), GEMVQ_GEMV_ADD (0x400) as gemvqc16.h:31-45, and
 *             GEMVQ_GEMV_ARGMAX (0x800): the next command is an
 *             ARGMAX over this GEMV's y (consumed; y is written), and GEMVQ_GEMV_SILU (0x1000): y = silu(W x) =
 *             v / (1 + e^-v) (the UNARY SiLU folded into the GEMV, no command consumed). Groups of up to 4 GEMVs with
 *             the same x_off, cols and format run as one pass; a group ends after a GEMV whose y overlaps x.
 *   RMSNORM   [2, n, x_off, w_off, y_off, eps bits, rows, flags]  flags bit0 L2, bit1 no weight, bit2 deferred
 *             (the following GEMVs with x_off == y_off and cols == n quantize the normalized row), bits 23:8 row
 *             stride in 16-float words (0: packed).
 *   ADD 3, SILU_MUL 4, MUL 5, UNARY 6, CONV 8, ROPE 10 as gemvqc16.h:52-59, 85-91; ROPE word 7 (pos_off): if
 *             nonzero, cs_off is a table of n_dims floats per position and the row is selected by the int32
 *             position stored at act[pos_off]. CONV word 7 bits 31:16 (0 or 1: one token): n_tok packed token
 *             rows of x and y run in order, each window ending at its token (up to GEMVQ_GEMM_MAX_TOK); with word 7
 *             bit1 (GEMVQ_CONV_SEQS) token t is the one token of sequence t instead, its window (3 * ch floats) at
 *             the state offsets + 3 * ch * t.
 *   GDN       [7, H_v | H_k << 16, q_off, k_off, v_off, g_off, beta_off, y_off]
 *             + [src_row, dst_row, scale bits, flags, l2_eps bits, rms_eps bits, w_off, z_off]
 *             (+ [dt_off, a_off, n_tok, qkv_stride, gb_stride, 0, 0, 0] with GEMVQ_GDN_GATES) as gemvqc16.h:60-81;
 *             n_tok (0 or 1: one token; up to GEMVQ_GEMM_MAX_TOK) tokens run in order on the same state, token t's
 *             q / k / v at t * qkv_stride, its g / beta at t * gb_stride, its y and z rows packed (hv * 128 apart);
 *             the gated norm then covers every token's heads. GEMVQ_GDN_WITH_GEMV is accepted (the results are
 *             those of the commands run one by one). GEMVQ_GDN_WITH_OUT (16, as gemvqc16.h:75-81) on a one-token
 *             GDN with the gated norm asks for the step, the norm, the ssm_out GEMV that follows and its residual
 *             ADD in one launch when the list has the shape [GDN (H_v a multiple of 4, at most 32), GEMV (Q4_0 /
 *             Q8_0, x = the step's y, rows a multiple of 16, at least 16 H_v, at most 16384) + GEMVQ_GEMV_ADD,
 *             its ADD into y2], y2 being the residual itself or apart from it, and neither meeting the step's
 *             operands or y; other shapes run unfused. Either way the results are the bits of the commands run
 *             one by one.
 *             GEMVQ_GDN_Z_SILU (32): z_off already holds silu(z), the gated norm multiplies by it directly. A GDN with
 *             the gated norm followed by a Q4_0 / Q8_0 GEMV reading its y applies the norm in that GEMV's activation
 *             prologue (one launch less; y is still written).
 *             GEMVQ_GDN_SEQS (64) with n_tok > 1: the tokens belong to n_tok sequences decoded in lockstep (no
 *             counterpart in the reference): token t is the one token of sequence t and runs on its own state rows,
 *             src_row / dst_row + t * H_v * 128, all tokens in one launch.
 *   ATTN      [12, n_head | n_head_kv << 16, q_off, kv, y_off, head_dim | n_rot << 16, pos_off, flags]
 *             + [k_off, v_off, scale bits, eps bits, qn_off, kn_off, cs_off, gate_off]
 *             One token of GQA attention (q head h reads KV head h / (n_head / n_head_kv)). q rows (head_dim floats)
 *             start every 2 * head_dim floats when flags bit0 (gate interleaved, Qwen3.5 Q+gate projection), else
 *             every head_dim floats. Per head: RMS norm with weight (qn_off / kn_off, eps), NEOX RoPE on the first
 *             n_rot floats with the cos/sin table at cs_off (n_rot floats per position), K and V stored as fp16 in
 *             KV buffer kv at the position act[pos_off], softmax(q k^T * scale) V over positions 0..pos, then
 *             flags bit0: y = sigmoid(gate) * y with the gate rows at gate_off (stride 2 * head_dim).
 *             flags bits 16..23 = n_tok (0 or 1: one token; at most GEMVQ_GEMM_MAX_TOK): tokens t < n_tok at positions
 *             act[pos_off] + t, as n_tok one-token commands run in order (token t sees the keys of tokens < t), with
 *             packed rows: token t's q and gate rows start t * n_head * (q row stride) floats on, its k and v rows
 *             t * n_head_kv * head_dim, its output t * n_head * head_dim. Results are bit-identical to those commands.
 *             flags bit1 (GEMVQ_ATTN_SEQS) with n_tok > 1: token t is the one token of sequence t of n_tok decoded in
 *             lockstep (no counterpart in the reference): its position is act_i32[pos_off + 16 t], and KV buffer kv
 *             (n_ctx a multiple of n_tok) holds the sequences in n_tok equal regions of n_ctx / n_tok positions, token
 *             t storing and reading region t; each token's results are those of a one-token command on its region.
 *   GET_ROWS  [13, format | n_tok << 16, rows, cols, w_off lo, w_off hi, id_off, y_off]  y = dequantized row
 *             act_i32[id_off]; with n_tok (2..GEMVQ_GEMM_MAX_TOK) token t's id is act_i32[id_off + 16 t] and its row
 *             goes to y_off + t * cols.
 *   ARGMAX    [14, n, x_off, key_off, rows, row_stride, 0, 0]  max(packed key at act[key_off..+1]) with the first
 *             index of the maximum of x; the key must be cleared (NEXT_TOKEN does it). rows (0 or 1: one; at most
 *             GEMVQ_GEMM_MAX_TOK): row r at x_off + r * row_stride, its key at key_off + 16 r.
 *   NEXT_TOKEN [15, key_off, tok_off, pos_off, prompt_off, n_prompt, out_off, 0]  token = argmax of the key, or
 *             the prompt token act_i32[prompt_off + pos + 1] while pos + 1 < n_prompt; act_i32[out_off + pos + 1]
 *             = token; act_i32[tok_off] = token; act_i32[pos_off] = pos + 1; the key is cleared.
 *             Word 7 = n_seq | cap << 8 with n_seq > 1: n_seq sequences in lockstep, sequence s with its key, token
 *             and position at key_off, tok_off, pos_off + 16 s, its prompt length at act_i32[n_prompt + 16 s] (word
 *             5 is then an offset), its prompt at prompt_off + s * cap and its token ids at out_off + s * cap.
 *   FILL      [16, n, y_off, value bits, 0, 0, 0, 0]  y = value.
 *   GEMM      [17, format | flags, rows, cols, w_off lo, w_off hi, x_off, y_off]
 *             + [n_tok, x_stride, y_stride, res_off, res_stride, norm_w_off, eps bits, norm_flags]
 *             The batched GEMV (the reference's planned batched path, ROADMAP.md:78-96; no counterpart in its
 *             kernel): n_tok (1..GEMVQ_GEMM_MAX_TOK) token rows read each weight row once. Token t's input row is at
 *             x_off + t * x_stride and its output row at y_off + t * y_stride; each output row equals, bit for bit,
 *             what a GEMV command on that token row writes. Format 2 Q4_0, 3 Q4_1 or 8 Q8_0, cols a multiple of
 *             512; or 13 Q5_K or 14 Q6_K with cols a multiple of 512 up to 12288, no SwiGLU pair, and y not over x
 *             or the norm weight (these run in launches of up to 4 tokens, each reading the weights once).
 *             flags: GEMVQ_GEMV_SWIGLU (the next command is the u GEMM with the same format, rows, cols, x_off,
 *             n_tok, x_stride and norm words and no flags; y = silu(g) * u goes to the u command's y_off /
 *             y_stride), GEMVQ_GEMV_ADD (y = W x + res, token t's residual at res_off + t * res_stride) or
 *             GEMVQ_GEMV_SILU. norm_flags GEMVQ_NORM_DEFER: every token row is RMS-normalized first (weight at
 *             norm_w_off unless GEMVQ_NORM_NO_WEIGHT, GEMVQ_NORM_L2 for the L2 norm, eps), as a deferred RMSNORM
 *             before a GEMV. The rows are read before any output is written, so y may overlap x (K-quant
 *             formats excepted).
 *             Consecutive GEMMs of one format on the same rows and norm words quantize the rows once and run as one
 *             launch of up to four members, unless one is a SwiGLU pair or a member's output overlaps an earlier
 *             member's output or residual; the results are those of the commands one by one.
 */
#ifndef GEMVQ_HIP_H
#define GEMVQ_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GEMVQ_CMD_WORDS 8u
#define GEMVQ_OP_GEMV 1u
#define GEMVQ_OP_RMSNORM 2u
#define GEMVQ_OP_ADD 3u
#define GEMVQ_OP_SILU_MUL 4u
#define GEMVQ_OP_MUL 5u
#define GEMVQ_OP_UNARY 6u
#define GEMVQ_OP_GDN 7u
#define GEMVQ_OP_CONV 8u
#define GEMVQ_OP_STATE_LOAD 9u
#define GEMVQ_OP_ROPE 10u
#define GEMVQ_OP_TRACE 11u
#define GEMVQ_OP_ATTN 12u
#define GEMVQ_OP_GET_ROWS 13u
#define GEMVQ_OP_ARGMAX 14u
#define GEMVQ_OP_NEXT_TOKEN 15u
#define GEMVQ_OP_FILL 16u
#define GEMVQ_OP_GEMM 17u
#define GEMVQ_GEMM_MAX_TOK 32u
#define GEMVQ_GEMV_SWIGLU 0x100u
#define GEMVQ_GEMV_CONV 0x200u
#define GEMVQ_GEMV_ADD 0x400u
#define GEMVQ_GEMV_ARGMAX 0x800u
#define GEMVQ_GEMV_SILU 0x1000u
#define GEMVQ_GROUP 4u
#define GEMVQ_GDN_WITH_GEMV 1u
#define GEMVQ_GDN_L2_QK 2u
#define GEMVQ_GDN_GATED 4u
#define GEMVQ_GDN_GATES 8u
#define GEMVQ_GDN_WITH_OUT 16u
#define GEMVQ_GDN_Z_SILU 32u
#define GEMVQ_GDN_SEQS 64u
#define GEMVQ_CONV_SEQS 2u
#define GEMVQ_ATTN_SEQS 2u
#define GEMVQ_NORM_L2 1u
#define GEMVQ_NORM_NO_WEIGHT 2u
#define GEMVQ_NORM_DEFER 4u
#define GEMVQ_SILU_MUL_SIGMOID 1u
#define GEMVQ_MAX_COLS 16384u
#define GEMVQ_MAX_CMDS 4096u
/* Feature words (gemvqc16.h:126-134 layout, marker 0x6B51 / 0x6B52). */
#define GEMVQ_FEATURES 0x6B51FFFFu /* every format bit of the first word, Q4_1 (bit 2) included */
#define GEMVQ_FEATURES2 0x6B52000Fu /* bit0 SILU_MUL sigmoid + strided g, bit1 ATTN/GET_ROWS/ARGMAX/NEXT_TOKEN,
                                       bit2 GEMM, bit3 ATTN and GET_ROWS n_tok */

typedef struct gemvq_ctx gemvq_ctx;

/* Status: 0 ok; > 0 the 1-based index of the first invalid command (nothing ran); GEMVQ_MAX_CMDS + 1 for a list
 * that is too long; < 0 a HIP error (negated hipError_t), an argument error (GEMVQ_EINVAL), a wait for the device
 * that passed its limit (GEMVQ_ETIMEDOUT), or a call on a context that a failed or timed-out device operation made
 * unusable (GEMVQ_EUNUSABLE).
 * Failure handling (replaces ggml-xrt.cpp:69-78, the GGML_XRT_WAIT_TIMEOUT_MS bound on every kernel wait, and the
 * runtime_valid latch of ggml-xrt.cpp:1258-1264, 2761-2770): every wait for the device is bounded (default 180000
 * ms, GEMVQ_WAIT_TIMEOUT_MS in the environment at create, or gemvq_set_wait_timeout). A HIP error from a launch, a
 * copy or the stream, or a timed-out wait, latches the context unusable: every later call that would touch the
 * device returns GEMVQ_EUNUSABLE (gemvq_last_error keeps the first failure) until gemvq_ctx_destroy, which waits for
 * the device's outstanding work before it frees memory. Command lists rejected by validation (nothing launched) and
 * argument errors do not latch. */
#define GEMVQ_EINVAL (-10000)
#define GEMVQ_ETIMEDOUT (-10001)
#define GEMVQ_EUNUSABLE (-10002)

/* Creates a context on HIP device `device` with an activation buffer of act_floats floats, a weight arena of
 * weight_bytes, and state_rows GDN state rows of 128 floats. Returns NULL on failure. */
gemvq_ctx * gemvq_ctx_create(int device, size_t act_floats, size_t weight_bytes, size_t state_rows);
void gemvq_ctx_destroy(gemvq_ctx * ctx);
/* Last error message of the context (or of the last failed create when ctx is NULL). */
const char * gemvq_last_error(const gemvq_ctx * ctx);
void gemvq_features(gemvq_ctx * ctx, uint32_t out[2]);

/* Repacks rows x cols GGUF rows of ggml type `type` (2, 8, 13, 14) into the weight arena and returns the weight
 * offset for GEMV / GET_ROWS commands in *w_off. The bits are the original ones; only their order changes. */
int gemvq_upload_weight(gemvq_ctx * ctx, int type, int rows, int cols, const void * gguf_rows, uint64_t * w_off);
/* Bytes of the arena in use (weights uploaded so far, with alignment). */
uint64_t gemvq_weight_bytes_used(const gemvq_ctx * ctx);
/* The load-time layout on the host (no GPU call): gemvq_repack writes the device layout of rows x cols GGUF rows
 * into dst (the same number of bytes); gemvq_unpack is its inverse. Returns 0 or GEMVQ_EINVAL. */
int gemvq_repack(int type, int rows, int cols, const void * gguf_rows, void * dst);
int gemvq_unpack(int type, int rows, int cols, const void * packed, void * gguf_rows);

/* Activation buffer I/O (offsets and counts in floats; int32 data may be written through the same calls). */
int gemvq_act_write(gemvq_ctx * ctx, size_t off, const void * src, size_t n);
int gemvq_act_read(gemvq_ctx * ctx, size_t off, void * dst, size_t n);
/* GDN state rows (128 floats each). */
int gemvq_state_write(gemvq_ctx * ctx, size_t row, const float * src, size_t rows);
int gemvq_state_read(gemvq_ctx * ctx, size_t row, float * dst, size_t rows);
int gemvq_state_clear(gemvq_ctx * ctx);

/* KV buffer for ATTN: n_ctx positions of n_head_kv x head_dim fp16 keys and values. Returns its id (>= 0). */
int gemvq_kv_create(gemvq_ctx * ctx, int n_ctx, int n_head_kv, int head_dim);
int gemvq_kv_read(gemvq_ctx * ctx, int kv, int pos0, int npos, uint16_t * k, uint16_t * v);
int gemvq_kv_clear(gemvq_ctx * ctx);

/* Runs a command list now (validated first; synchronous). */
int gemvq_run(gemvq_ctx * ctx, const uint32_t * cmds, unsigned n_cmds);
/* Validates and captures a command list as a hipGraph; *graph receives its id. */
int gemvq_graph_create(gemvq_ctx * ctx, const uint32_t * cmds, unsigned n_cmds, int * graph);
/* Launches a captured graph `times` times back to back (asynchronous; gemvq_sync waits). */
int gemvq_graph_replay(gemvq_ctx * ctx, int graph, int times);
int gemvq_graph_destroy(gemvq_ctx * ctx, int graph);
int gemvq_sync(gemvq_ctx * ctx);
/* The bound of every wait for the device, in milliseconds (> 0). */
int gemvq_set_wait_timeout(gemvq_ctx * ctx, unsigned ms);
/* 1 while the context accepts device work, 0 after a failed or timed-out device operation (or for NULL). */
int gemvq_usable(const gemvq_ctx * ctx);
/* Free and total HBM of a device (hipMemGetInfo); 0 or a negative HIP error. */
int gemvq_device_memory(int device, size_t * free_bytes, size_t * total_bytes);

/* Number of kernel launches the last validated list compiled to (after fusion). */
int gemvq_last_launch_count(const gemvq_ctx * ctx);

/* Debug: the integer block sums of the next GEMV pass's first matrix are written to dst (int32 per 32-block for
 * Q4_0 / Q8_0, two int32 S, M per super-block for Q5_K / Q6_K); cleared after that pass. */
int gemvq_debug_blocksums(gemvq_ctx * ctx, int32_t * dst, size_t n);

/* Timing: average device time in microseconds of the kernels of `graph` over `times` replays, measured with
 * HIP events on the context stream (the replays run back to back between the events). */
int gemvq_graph_time(gemvq_ctx * ctx, int graph, int times, double * us_per_replay);

/* Profiling (the counterpart of the reference's TRACE opcode and XRT-TIMING totals, gemvqc16.h:92-98,
 * ggml-xrt.cpp:285-314, 1302-1397): runs a command list `reps` times, each kernel launched with device start/stop
 * events (hipExtLaunchKernelGGL), and reports per launch the kernel, the commands it executes, its algorithmic
 * bytes (GGUF-sized weights, fp32 vectors read and written once, state and KV cache traffic) and its median
 * duration over the repetitions. The list's side effects happen `reps` times. Returns the number of launches (>= 0) or a status. */
typedef struct {
    char name[40];
    int32_t first_cmd, n_cmds;
    uint64_t bytes;
    double us;
} gemvq_launch_stat;
int gemvq_profile(gemvq_ctx * ctx, const uint32_t * cmds, unsigned n_cmds, int reps, gemvq_launch_stat * out,
                  int max_out);

/* Arithmetic of the lists compiled after the call (graphs keep the arithmetic they were captured in).
 * GEMVQ_ARITH_CANONICAL (default): the reference kernel's fixed-point GEMV rows (each block term exact and floored to
 * 2^-40, summed exactly, rounded once; fpga/src/gemvqw_engine.h:352-445) and pairwise-tree FP32 reductions.
 * GEMVQ_ARITH_REFERENCE: the reference's CPU path (fpga/src/gemvq_ref.h), as its ggml backend checks the kernel
 * against it (the XRT-VERIFY mode, ggml-xrt.cpp:1153-1202): GEMV rows as FP32 block terms added in block order (the
 * K-quants' eight FP32 partial sums), norm sums of FP32 squares in double in index order, the DeltaNet step's dots in
 * order, attention with double sums (ggml's CPU path), and correctly rounded exp / log (gemvq_cr_expf / _logf) where
 * the reference calls libm. Every command keeps its meaning; the fused forms whose arithmetic differs (the gated norm
 * in the next GEMV's prologue, GEMVQ_GDN_WITH_OUT) run unfused (the gated norm, in the reference's order, in the
 * DeltaNet step's own launch), a GEMM runs token by token as GEMV commands, and CONV, GDN and ATTN with several
 * tokens run token by token. Debug block sums are not written in this mode.
 * Returns 0 or GEMVQ_EINVAL. */
#define GEMVQ_ARITH_CANONICAL 0
#define GEMVQ_ARITH_REFERENCE 1
int gemvq_set_arith(gemvq_ctx * ctx, int arith);
int gemvq_arith(const gemvq_ctx * ctx);
/* The reference arithmetic's exp and log on the host: the binary32 value nearest to e^x / log x (ties to even), the
 * same code the device evaluates. */
float gemvq_cr_expf(float x);
float gemvq_cr_logf(float x);
/* Test hook: the device's correctly rounded exp (fn 0) or log (fn 1) over every binary32 input, as 4096 block
 * hashes (block b: the inputs with bits b 2^20 .. b 2^20 + 2^20 - 1; hash = sum mod 2^64 of bits(f(x)) (2 i + 1) over
 * the block's i, NaN results as 0x7fc00000). Synchronous; 0 or a negative status. */
int gemvq_crmath_hash(gemvq_ctx * ctx, int fn, uint64_t * hashes);

/* No counterpart in the reference: for callers that cannot allocate device memory (code under hipGraph capture,
 * serving loops, harnesses that forbid hipMalloc). The batched GEMV of the GEMM command (plain epilog) on
 * caller-owned device memory, allocating nothing: y[t * y_stride + r] = row r of the matrix times token row t of x
 * (at x + t * x_stride), bit for bit what a GEMM command computes. w: the matrix in the device layout of
 * gemvq_repack (type 2 Q4_0, 3 Q4_1 or 8 Q8_0; rows x cols, cols a multiple of 512 up to GEMVQ_MAX_COLS),
 * 256-byte aligned; x and y 64-byte aligned, strides multiples of 16 floats; 1 <= n_tok <= GEMVQ_GEMM_MAX_TOK.
 * Runs on the current device, asynchronously on `stream` (a hipStream_t; NULL for the null stream). The quantized
 * activation rows are staged in a fixed device array of GEMVQ_STATIC_SCRATCH_BYTES per device, held until the
 * process ends, so calls that overlap on one device race. Returns 0, GEMVQ_EINVAL (nothing launched: a size beyond
 * the limits, a misaligned or NULL pointer) or a negated HIP error. */
#define GEMVQ_STATIC_SCRATCH_BYTES 655360u
int gemvq_gemm_static(int type, int rows, int cols, const void * w, const float * x, int n_tok, int x_stride,
                      float * y, int y_stride, void * stream);

#ifdef __cplusplus
}
#endif
#endif
