// Launch descriptors of the gfx950 kernels (shared by the kernels and the host command processor).
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gq {

enum : int { T_Q4_0 = 2, T_Q4_1 = 3, T_Q8_0 = 8, T_Q5_K = 13, T_Q6_K = 14 };

// Repacked weight layout (layout only, original bits): the GGUF block fields of all rows split into
// field-major regions, each row-major, so that lane l of a wave reads unit l of a row from consecutive bytes.
//   Q4_0: qs[rows][nb][16], d[rows][nb] (u16)
//   Q4_1: qs[rows][nb][16], dm[rows][nb] (u32: d | m << 16)
//   Q8_0: qs_lo[rows][nb][16] (bytes 0..15 of each block's quants), qs_hi[rows][nb][16], d[rows][nb]
//   Q5_K: qs[rows][nsb][128], qh[rows][nsb][32], meta[rows][nsb][16] (d, dmin, 12 scale bytes)
//   Q6_K: ql[rows][nsb][128], qh[rows][nsb][64], sc[rows][nsb][16], d[rows][nsb] (u16)
struct WeightView {
    const uint8_t * a;  // first region
    const uint8_t * b;
    const uint8_t * c;
    const uint8_t * d;
};

enum : int { EPI_PLAIN = 0, EPI_SWIGLU = 1, EPI_ADD = 2, EPI_CONV = 3, EPI_SILU = 4 };
// XSRC_GATED: gate_silu says whether z is silu(z).
enum : int { XSRC_RAW = 0, XSRC_NORM = 1, XSRC_GATED = 2 };
// Prologue kinds of the GEMV kernel instances.
enum : int { XS_PLAIN = 0, XS_GATED = 1 };

struct GemvMember {
    WeightView w;    // matrix (g of a SwiGLU pair)
    WeightView w2;   // u of a SwiGLU pair
    float * y;
    const float * res;        // ADD residual
    const float * conv_src;   // CONV state [rows][3]
    float * conv_dst;
    const float * conv_w;     // CONV kernel [rows][4]
    int rows;
    int task_begin;  // first row of the member in the group's row order
    int wave_begin;  // set at launch: the member's first wave within each XCD slice
    int waves;       // set at launch: the member's waves per slice; wave w takes the slice's rows w, w + waves, ...
    const float * ea;  // set at launch: epilog operand addresses (see epilog_operands)
    const float * eb;
    int e_sa, e_sb, e_split, e_lane;
    int epi;
    int conv_silu;
};

struct GemvArgs {
    const float * x;          // activation (act + x_off); XSRC_GATED: the raw DeltaNet output
    const float * norm_w;     // deferred norm weight (NULL: no weight); XSRC_GATED: the gated norm's weight [128]
    float norm_eps;
    int xsrc;                 // XSRC_RAW, XSRC_NORM or XSRC_GATED
    const float * gate_z;     // XSRC_GATED: z (the output gate) [cols]
    float * x_out;            // XSRC_GATED: the gated activation is also written here (by workgroup 0)
    int gate_silu;            // XSRC_GATED: gate_z holds silu(z) already
    int norm_l2;
    int cols;
    int n_members;
    int total_tasks;
    GemvMember m[4];
    unsigned long long * argmax_key;  // non-NULL: argmax over member 0's y
    int32_t * dbg;                    // non-NULL: integer block sums of member 0
    float wbound[4];  // per member (Q4_0 / Q4_1 / Q8_0): the largest block term magnitude over |d_x| * 2^40
};

struct NormArgs {
    const float * x;
    const float * w;
    float * y;
    int n, rows, stride;  // stride in floats
    float eps;
    int flags;
};

enum : int { EW_ADD = 0, EW_MUL = 1, EW_SILU_MUL = 2, EW_SIGMOID_MUL = 3, EW_SILU = 4, EW_SIGMOID = 5,
             EW_SOFTPLUS = 6, EW_COPY = 7, EW_FILL = 8 };

struct EwArgs {
    const float * a;   // first operand (g for SILU_MUL, x for UNARY)
    const float * b;   // second operand (u for SILU_MUL)
    float * y;
    int n;
    int row, stride;   // a is rows of `row` floats every `stride` floats (row 0: contiguous)
    int op;
    float value;       // FILL
};

struct ConvArgs {
    const float * x;
    const float * w;
    const float * s_src;
    float * s_dst;
    float * y;
    int ch;
    int silu;
    int n_tok;  // token rows of x and y (ch floats apart), run in order: each token's window ends at its row
    int seqs;   // nonzero: token t belongs to sequence t, whose window is at s_src / s_dst + 3 * ch * t
};

struct RopeArgs {
    const float * x;
    const float * cs;     // n_dims floats, or a table with n_dims floats per position
    const int32_t * pos;  // non-NULL: row of the table
    float * y;
    int n_dims, ne0, rows;
};

struct GdnArgs {
    const float * q;
    const float * k;
    const float * v;
    const float * g;      // log decay, or alpha raw with gates
    const float * beta;   // beta, or beta raw with gates
    const float * dt;
    const float * a;
    float * y;
    const float * src;    // state rows (128 floats each), head h row j at (h * 128 + j) * 128
    float * dst;
    int hv, hk;
    float scale, l2_eps;
    int flags;
    int n_tok;             // tokens run in order on the same state
    int s_qkv, s_gb, s_y;  // row strides (floats) between tokens of q / k / v, of g / beta, of y
    int seqs;              // nonzero: the tokens belong to n_tok sequences, token t on its own state rows (src and
                           // dst + t * hv * 128 rows), all in one launch
    // reference arithmetic with the gated output norm (GEMVQ_GDN_GATED): the step's launch also applies the norm to
    // its token's heads (z rows hv * 128 apart per token, the norm weight [128], the RMS eps); NULL gz: not applied
    const float * gz;
    const float * gw;
    float rms_eps;
};

// The DeltaNet step, its gated output norm, the ssm_out product and its residual sum in one launch (the reference's
// GDN_WITH_OUT, gemvqc16.h:75-81, gemvqc16.cpp:872-903): out = ssm_out(gated norm(step)) + res. Workgroup h < hv
// steps value head h (its state rows read and written once, in place when src == dst), normalizes, gates and
// quantizes the head's 128 outputs and publishes the quants in the exchange area; every workgroup holds 16 rows of
// ssm_out in registers, waits for all heads and forms its rows (exact fixed-point sums, rounded once, plus res).
constexpr int GDN_OUT_MAX_HEADS = 32;   // value heads (hv a multiple of 4)
constexpr int GDN_OUT_MAX_ROWS = 16384;
// Exchange area: two slots, each GDN_XCH_COPIES copies (one per XCD) of GDN_XCH_SLOT 64-bit words; head h's words
// are h * 36 + j: its 32 words of quants, then its 4 block words, each as tag | word (tag zero: not yet published).
constexpr int GDN_XCH_SLOT = 36 * GDN_OUT_MAX_HEADS;
constexpr int GDN_XCH_COPIES = 8;
constexpr int GDN_XCH_WORDS = 2 * GDN_XCH_COPIES * GDN_XCH_SLOT;
struct GdnOutArgs {
    GdnArgs g;                  // one token; g.y is not used
    const float * z;            // the output gate (silu(z) when z_silu)
    const float * nw;           // the gated norm's weight [128]
    float rms_eps;
    int z_silu;
    float * y;                  // the gated output [hv * 128] (the GDN command's y)
    WeightView w;               // ssm_out, rows x (hv * 128), Q4_0 or Q8_0
    int rows;                   // a multiple of 16, at least 16 * hv
    const float * res;          // residual [rows]
    float * out;                // ssm_out + res [rows] (res itself, or apart from it)
    unsigned long long * xch;   // exchange area (GDN_XCH_WORDS), both slots' tags zero before the list's first launch
    int slot;                   // the exchange slot of this launch (0 or 1, in turn over a list's fused launches)
    uint32_t * fault;           // host word set to 1 when a workgroup's wait for the heads ran out of polls
    unsigned polls;             // the bound of that wait
};
bool gdn_out_fits(int hv, int rows);  // the fused launch serves hv value heads and `rows` ssm_out rows

struct GatedNormArgs {    // per head of 128: y = silu(z) * ((y * s) * w), s = 1 / sqrt(mean(y^2) + eps)
    float * y;
    const float * z;          // z, or silu(z) when z_silu
    const float * w;
    int heads;
    float eps;
    int z_silu;
};

struct AttnArgs {
    const float * q;      // q rows
    const float * k;      // new key rows (n_head_kv x head_dim)
    const float * v;
    const float * qn;     // q norm weight (head_dim)
    const float * kn;
    const float * cs;     // cos/sin table, n_rot floats per position
    const int32_t * pos;
    const float * gate;   // NULL or gate rows (stride 2 * head_dim)
    float * y;
    uint16_t * kc;        // [n_ctx][n_head_kv][head_dim]
    uint16_t * vc;
    float * part;         // partials: [n_head][max_chunks][2 + head_dim]
    unsigned int * counter;  // [n_head_kv * ATTN_MAXG]: finished chunks per q head
    int n_head, n_head_kv, head_dim, n_rot, q_stride, n_ctx;
    float scale, eps;
    // n_tok > 1: tokens at positions *pos + t, t < n_tok, in one launch pair. Token t's q (and gate) rows start
    // t * n_head * q_stride floats on, its new key and value t * n_head_kv * head_dim, its output t * n_head *
    // head_dim; its partials and counters follow those of token t - 1 (part and counter hold n_tok sets).
    int n_tok;
    float * qr;           // n_tok > 1: normalized, rotated, fp16-rounded q rows [n_tok][n_head][head_dim]
    // seq_ctx > 0: token t belongs to sequence t: its position is pos[16 t], and its keys and values are positions
    // [t * seq_ctx, (t + 1) * seq_ctx) of the cache (n_ctx is then the capacity of one sequence, seq_ctx)
    int seq_ctx;
};

struct GetRowsArgs {
    WeightView w;
    const int32_t * id;   // token t's id at id[16 t]
    float * y;            // token t's row at y + t * cols
    int rows, cols, type;
    int n_tok;
};

struct NextTokenArgs {
    unsigned long long * key;
    int32_t * tok;
    int32_t * pos;
    const int32_t * prompt;
    int n_prompt;
    int32_t * out;
    int max_pos;
    // n_seq > 1: sequence t's key, token and position at key + 8 t (16 floats), tok + 16 t, pos + 16 t; its prompt
    // (n_prompt_of[16 t] ids) at prompt + t * seq_cap and its token ids at out + t * seq_cap (max_pos = seq_cap)
    int n_seq;
    const int32_t * n_prompt_of;
    int seq_cap;
};

// Batched GEMV (n_tok tokens per weight read): the activation rows are quantized once into Q8_0 blocks whose 32
// quants are stored in the MFMA operand order (8-byte group g holds quants 4g..4g+3 and 16+4g..16+4g+3), with
// d * 2^40 per block as FP32; token rows n_tok..n_pad-1 are zero.
struct GemmQuantArgs {
    const float * x;       // token t's row at x + t * x_stride
    const float * norm_w;  // per-token RMS norm folded into the quantization: its weight (NULL: none)
    int8_t * q;            // [n_pad][cols]
    float * d40;           // [n_pad][cols / 32]
    float * s40;           // [n_pad][cols / 32]: the Q8_1 s = fp16(sum of the block's quants * d), times 2^40
    int n_tok, n_pad, cols, x_stride;
    int norm, norm_l2;
    float eps;
};

constexpr int GEMM_MAX_MORE = 3;  // a GEMM group has at most four members

struct GemmMore {  // a further member of a GEMM group: its own matrix, output rows and epilog, the same activation
    WeightView w;
    float * y;
    const float * res;
    int rows, y_stride, res_stride, epi;
    int tile0;  // its first 16-row tile in the group's grid
};

struct GemmArgs {
    WeightView w;       // matrix (g of a SwiGLU pair)
    WeightView w2;      // u of a SwiGLU pair
    const int8_t * q;   // the quantized activation (GemmQuantArgs)
    const float * d40;
    const float * s40;  // Q4_1 weights: the activation blocks' Q8_1 s * 2^40
    float * y;          // token t, row r at y[t * y_stride + r]
    const float * res;  // ADD: res[t * res_stride + r]
    int rows, cols, n_tok, y_stride, res_stride;
    int epi;            // EPI_PLAIN, EPI_SWIGLU, EPI_ADD or EPI_SILU
    int n_more;         // members after the first (not with a SwiGLU pair); tiles of member i + 1 follow member i's
    GemmMore more[GEMM_MAX_MORE];
    float wbound[GEMM_MAX_MORE + 1];  // per member: the largest block term magnitude over |d_x| * 2^40 (INFINITY:
                                      // unknown, every round's terms are summed in int64)
};

// The GEMM command for 2-4 tokens on the single-token GEMV's structure: each lane keeps its activation blocks of
// every token in registers, so each weight row is streamed and unpacked once for all of them, and the tokens are
// quantized in the launch's own prologue (no separate quantization launch).
constexpr int TOK_MAX = 4;
struct TokMember {
    WeightView w;       // matrix (g of a SwiGLU pair)
    WeightView w2;      // u of a SwiGLU pair (the matrix again otherwise)
    float * y;          // token t, row r at y[t * y_stride + r]
    const float * res;  // ADD: res[t * res_stride + r]; otherwise y (read, not used)
    int rows, y_stride, res_stride, epi;
    int wave_begin, waves;  // set at launch, as GemvMember's
};
struct TokArgs {
    const float * x;       // token t's row at x + t * x_stride
    const float * norm_w;  // per-token RMS norm folded into the quantization: its weight (NULL: none)
    float eps;
    int norm, norm_l2;
    int cols, n_tok, x_stride;
    int n_members;
    TokMember m[4];
    float wbound[4];  // per member: the largest block term magnitude over |d_x| * 2^40
};

constexpr int GEMV_MAXK = 16384;  // GEMV columns at most
constexpr int GEMM_MAX_TOK = 32;  // tokens of one batched GEMV (two tiles of 16)
constexpr int ATTN_CHUNK = 64;
constexpr int ATTN_MAXG = 8;  // q heads per KV head
constexpr int GDN_MAX_HEADS = 64;  // value heads of one GDN command

// Profiling: when set (by gemvq_profile on the calling thread), launchers start kernels through
// hipExtLaunchKernelGGL with these events, which record the kernel's own start and end on the device.
extern thread_local hipEvent_t g_prof_start, g_prof_stop;

#define GQ_LAUNCH(kernel, grid, block, shmem, stream, ...)                                                         \
    do {                                                                                                            \
        if (::gq::g_prof_start)                                                                                     \
            hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, ::gq::g_prof_start, ::gq::g_prof_stop, 0,     \
                                  __VA_ARGS__);                                                                     \
        else                                                                                                        \
            hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                                    \
    } while (0)

hipError_t launch_gemv(const GemvArgs & a, int type, hipStream_t s);
hipError_t launch_norm(const NormArgs & a, hipStream_t s);
hipError_t launch_ew(const EwArgs & a, hipStream_t s);
hipError_t launch_conv(const ConvArgs & a, hipStream_t s);
hipError_t launch_rope(const RopeArgs & a, hipStream_t s);
hipError_t launch_gdn(const GdnArgs & a, hipStream_t s);
hipError_t launch_gated_norm(const GatedNormArgs & a, hipStream_t s);
hipError_t launch_gdn_out(const GdnOutArgs & a, int type, hipStream_t s);
hipError_t launch_attn(const AttnArgs & a, hipStream_t s);
hipError_t launch_get_rows(const GetRowsArgs & a, hipStream_t s);
hipError_t launch_argmax(const float * x, int n, unsigned long long * key, int rows, int stride, hipStream_t s);
hipError_t launch_next_token(const NextTokenArgs & a, hipStream_t s);
hipError_t launch_gemm_quant(const GemmQuantArgs & a, hipStream_t s);
hipError_t launch_gemm(const GemmArgs & a, int type, hipStream_t s);
// Whether launch_gemv_tok has an instance for this weight type, width, token count and member kind (a SwiGLU pair).
bool gemv_tok_ok(int type, int cols, int n_tok, bool pair);
hipError_t launch_gemv_tok(const TokArgs & a, int type, hipStream_t s);

// Layout helpers (host and device).
__host__ __device__ inline size_t gguf_row_bytes(int type, int cols) {
    switch (type) {
    case T_Q4_0: return size_t(cols / 32) * 18;
    case T_Q4_1: return size_t(cols / 32) * 20;
    case T_Q8_0: return size_t(cols / 32) * 34;
    case T_Q5_K: return size_t(cols / 256) * 176;
    case T_Q6_K: return size_t(cols / 256) * 210;
    default: return 0;
    }
}

__host__ __device__ inline WeightView weight_view(const uint8_t * base, int type, int rows, int cols) {
    WeightView v;
    const size_t R = size_t(rows);
    if (type == T_Q4_0 || type == T_Q4_1) {
        const size_t nb = size_t(cols / 32);
        v.a = base;
        v.b = base + R * nb * 16;
        v.c = v.d = nullptr;
    } else if (type == T_Q8_0) {
        const size_t nb = size_t(cols / 32);
        v.a = base;
        v.b = base + R * nb * 16;
        v.c = base + R * nb * 32;
        v.d = nullptr;
    } else if (type == T_Q5_K) {
        const size_t ns = size_t(cols / 256);
        v.a = base;
        v.b = base + R * ns * 128;
        v.c = base + R * ns * 160;
        v.d = nullptr;
    } else {
        const size_t ns = size_t(cols / 256);
        v.a = base;
        v.b = base + R * ns * 128;
        v.c = base + R * ns * 192;
        v.d = base + R * ns * 208;
    }
    return v;
}

}  // namespace gq
