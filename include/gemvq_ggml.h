/* ggml-facing backend over the gemvq command lists (gemvq_hip.h): the part of the reference's ggml backend that
 * turns a graph split into fused command lists (ggml-xrt.cpp:1813-2745), with its device and backend interface
 * (:2773-3063), its recurrent-state buffer type (:405-622) and its public pair (ggml-xrt.h:11-16).
 *
 * ggml itself is not part of this library. A split is described in a ggml-shaped graph IR: gqg_tensor carries the
 * ggml_tensor fields the planner reads, under ggml's names and meanings (type ids are ggml's; ops are named as
 * ggml's and numbered here). A ggml build wraps this backend with a translation of ggml_tensor into gqg_tensor
 * (one field copy per node; the integration notes show it), so the planner's results are the same either way.
 *
 * What a split compiles to (the reference's fused forms, gemvqc16.h):
 *   - MUL_MAT of a Q4_0 / Q4_1 / Q8_0 / Q5_K / Q6_K weight on one F32 token row: GEMV; GEMVs on one row group;
 *     GLU(SWIGLU) of two such GEMVs read by nothing else: a SwiGLU pair; ADD of a GEMV read only by that ADD: the
 *     GEMV's ADD epilog; RMS_NORM (+ MUL by an F32 weight) read only by GEMVs: a deferred RMSNORM; SILU of a GEMV
 *     read only by that SILU: the GEMV's SiLU epilog.
 *   - The one-token DeltaNet chain (ggml-xrt.cpp:1819-2060): GET_ROWS of the conv state from a recurrent-state
 *     buffer, CONCAT with the qkv projection, SSM_CONV, SILU, and the CPY of the new window: one CONV epilog on the
 *     qkv GEMV; L2_NORM of q and k, the gates SIGMOID(beta) and MUL(SOFTPLUS(ADD(alpha, dt)), a), GATED_DELTA_NET on
 *     the state rows of a recurrent-state buffer, the gated norm MUL(MUL(RMS_NORM(y), w), SILU(z)) and the CPY of
 *     the new state: one GDN command.
 *   - One-token gated attention (Qwen3.5; the reference leaves it on the host): RMS_NORM + MUL of the q and k heads,
 *     ROPE (NEOX) of both, SET_ROWS of k and v into a KV buffer of this backend, FLASH_ATTN_EXT over the cache and
 *     the SIGMOID gate MUL: one ATTN command (q and gate interleaved as Qwen3.5's q projection writes them).
 *   - GET_ROWS of a quantized weight by I32 ids: GET_ROWS; RMS_NORM, MUL, ADD, UNARY (SILU, SIGMOID, SOFTPLUS), CONT
 *     of strided rows, ROPE: their commands.
 * Every split compiles to one command list, run as a captured hipGraph: the plan (the list, where every input and
 * output sits in the activation buffer, what is copied back) is cached under a structural signature of the split
 * (every node's fields, its operands as node positions or outside tensors; the role of the reference's plan key,
 * ggml-xrt.cpp:2133-2188) and the graph is replayed when the same split comes again. An
 * output is copied back to its host tensor only when it is a graph output or a split output (the reference's
 * readback filter, :1399-1478).
 *
 * Errors: a failed call latches the backend invalid; every later compute returns GQG_STATUS_FAILED
 * (ggml-xrt.cpp:2747-2770). Status values are ggml's (GGML_STATUS_*). */
#ifndef GEMVQ_GGML_H
#define GEMVQ_GGML_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (the GGUF ids) of the types the planner handles. */
enum {
    GQG_TYPE_F32 = 0, GQG_TYPE_F16 = 1, GQG_TYPE_Q4_0 = 2, GQG_TYPE_Q4_1 = 3, GQG_TYPE_Q8_0 = 8,
    GQG_TYPE_Q5_K = 13, GQG_TYPE_Q6_K = 14, GQG_TYPE_I32 = 26, GQG_TYPE_I64 = 27
};

/* ggml ops, named as in ggml.h (numbered here). Views (VIEW, RESHAPE, PERMUTE, TRANSPOSE) compute nothing. */
enum {
    GQG_OP_NONE = 0, GQG_OP_ADD, GQG_OP_MUL, GQG_OP_SCALE, GQG_OP_RMS_NORM, GQG_OP_L2_NORM, GQG_OP_MUL_MAT,
    GQG_OP_CPY, GQG_OP_CONT, GQG_OP_RESHAPE, GQG_OP_VIEW, GQG_OP_PERMUTE, GQG_OP_TRANSPOSE, GQG_OP_GET_ROWS,
    GQG_OP_SET_ROWS, GQG_OP_CONCAT, GQG_OP_ROPE, GQG_OP_FLASH_ATTN_EXT, GQG_OP_SSM_CONV, GQG_OP_GATED_DELTA_NET,
    GQG_OP_UNARY, GQG_OP_GLU, GQG_OP_SOFT_MAX, GQG_OP_COUNT
};
enum { GQG_UNARY_SILU = 1, GQG_UNARY_SIGMOID = 2, GQG_UNARY_SOFTPLUS = 3 }; /* op_params[0] of UNARY */
enum { GQG_GLU_SWIGLU = 1 };                                               /* op_params[0] of GLU; [1] swapped */
enum { GQG_ROPE_TYPE_NEOX = 2 };                                           /* op_params[2] of ROPE (ggml's) */

/* ggml tensor flags, with GGML_TENSOR_FLAG_SPLIT_OUTPUT of the reference's scheduler patch (0002). */
enum { GQG_FLAG_INPUT = 1, GQG_FLAG_OUTPUT = 2, GQG_FLAG_SPLIT_OUTPUT = 1 << 8 };

/* Where a tensor's data lives (ggml's buffer and its usage). */
enum {
    GQG_BUF_HOST = 0,    /* host memory: split inputs are copied in, outputs copied back */
    GQG_BUF_WEIGHTS = 1, /* a weights buffer: quantized matrices and F32 constants are uploaded once, keyed by tensor */
    GQG_BUF_RS = 2,      /* a recurrent-state buffer of this backend (gqg_rs_buffer_alloc) */
    GQG_BUF_KV = 3       /* a KV buffer of this backend (gqg_kv_buffer_alloc) */
};

#define GQG_MAX_DIMS 4
#define GQG_MAX_SRC 10
#define GQG_MAX_OP_PARAMS 16

typedef struct gqg_tensor {
    int32_t type;
    int32_t op;
    int64_t ne[GQG_MAX_DIMS]; /* elements per dimension */
    size_t nb[GQG_MAX_DIMS];  /* bytes per step in each dimension */
    int32_t op_params[GQG_MAX_OP_PARAMS];
    int32_t flags;
    int32_t buffer; /* GQG_BUF_* */
    struct gqg_tensor * src[GQG_MAX_SRC];
    struct gqg_tensor * view_src;
    size_t view_offs;
    void * data;
    char name[64];
} gqg_tensor;

typedef struct {
    int n_nodes;
    gqg_tensor ** nodes;
} gqg_cgraph;

enum { GQG_STATUS_ALLOC_FAILED = -2, GQG_STATUS_FAILED = -1, GQG_STATUS_SUCCESS = 0 };

typedef struct gqg_backend gqg_backend;

typedef struct {
    int device;
    size_t act_floats;    /* activation buffer (split inputs and outputs, resident constants and conv states) */
    size_t weight_bytes;  /* weight arena (quantized matrices, uploaded on first use) */
    size_t state_rows;    /* recurrent state rows of 128 floats */
    int dry;              /* nonzero: plan only, no device (weights and constants get offsets, nothing runs) */
} gqg_params;

/* ggml-xrt.cpp:2970-2976: NULL on failure (one backend per process, as the reference). */
gqg_backend * gqg_backend_init(const gqg_params * params);
void gqg_backend_free(gqg_backend * b);
const char * gqg_backend_error(const gqg_backend * b);

/* ggml-xrt.cpp:2998-3015 (and offload_op): whether this backend runs the node. */
int gqg_supports_op(const gqg_backend * b, const gqg_tensor * op);
/* ggml-xrt.cpp:2747-2771: runs one split (the nodes of one backend in graph order); GQG_STATUS_*. */
int gqg_graph_compute(gqg_backend * b, gqg_cgraph * graph);
/* The command words the split compiles to (without running it; also in a dry backend): returns the number of
 * commands (words = GEMVQ_CMD_WORDS per command, copied when cap is large enough), or a negative GQG_STATUS. */
int gqg_graph_plan(gqg_backend * b, gqg_cgraph * graph, uint32_t * words, size_t cap);
/* Plan cache counters: plans built, plans reused. */
void gqg_plan_stats(const gqg_backend * b, uint64_t out[2]);
/* The host data a split's plan copies in before its run (ins) and copies back after it (outs: the readback filter,
 * ggml-xrt.cpp:1399-1478): counts[0] and counts[1] receive how many, and up to cap of each are stored. Plans (or reuses)
 * the split; returns 0 or a negative GQG_STATUS. */
int gqg_graph_io(gqg_backend * b, gqg_cgraph * graph, const void ** ins, const void ** outs, size_t cap, int counts[2]);

/* Recurrent-state buffer type (ggml-xrt.cpp:562-611; ggml_backend_xrt_rs_buffer_type): a host address range
 * reserved without access rights; gqg_rs_init_tensor places a tensor named cache_s_l* on state rows (128 floats a
 * row) and any other (cache_r_l*, conv windows) in the activation buffer's resident region. Data moves only
 * through set/get/memset/clear or the backend's own commands. */
typedef struct gqg_buffer gqg_buffer;
gqg_buffer * gqg_rs_buffer_alloc(gqg_backend * b, size_t size);
/* KV buffer of this backend (cache_k_l*, cache_v_l*: F16 rows of n_head_kv * head_dim); gqg_kv_init_tensor pairs
 * the k and v tensors of a layer into one device KV cache of n_ctx positions. */
gqg_buffer * gqg_kv_buffer_alloc(gqg_backend * b, size_t size);
void * gqg_buffer_base(const gqg_buffer * buf);
int gqg_buffer_init_tensor(gqg_buffer * buf, gqg_tensor * t);
int gqg_buffer_set(gqg_buffer * buf, const gqg_tensor * t, const void * data, size_t offset, size_t size);
int gqg_buffer_get(gqg_buffer * buf, const gqg_tensor * t, void * data, size_t offset, size_t size);
int gqg_buffer_clear(gqg_buffer * buf, uint8_t value);
void gqg_buffer_free(gqg_buffer * buf);

/* Registration (ggml-xrt.cpp:3030-3063, ggml-xrt.h:11-16): the device and backend interface a ggml wrapper
 * forwards to. get_memory reports the device's free and total HBM. */
typedef struct {
    const char * name;
    const char * (*get_description)(void);
    void (*get_memory)(size_t * free_bytes, size_t * total_bytes);
    int device_type; /* 2: GPU, so that -ngl selects the device (ggml's GGML_BACKEND_DEVICE_TYPE_GPU) */
    gqg_backend * (*init_backend)(const gqg_params * params);
    void (*free_backend)(gqg_backend * b);
    int (*supports_op)(const gqg_backend * b, const gqg_tensor * op);
    int (*offload_op)(const gqg_backend * b, const gqg_tensor * op);
    int (*graph_compute)(gqg_backend * b, gqg_cgraph * graph);
    gqg_buffer * (*rs_buffer_alloc)(gqg_backend * b, size_t size);
    gqg_buffer * (*kv_buffer_alloc)(gqg_backend * b, size_t size);
} gqg_backend_reg;

const gqg_backend_reg * gqg_backend_get_reg(void);

#ifdef __cplusplus
}
#endif
#endif
