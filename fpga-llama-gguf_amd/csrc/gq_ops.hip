// Non-GEMV kernels of the decode command stream for gfx950: row norms, element-wise ops, conv, RoPE, the Gated
// DeltaNet step, its gated output norm, the attention core, embedding rows, argmax and the greedy token step.
// Reductions follow the pairwise tree over element indices; see gq_device.h for the scalar arithmetic.
#include "gq_device.h"
#include "gq_gdn.h"
#include "gq_kernels.h"

namespace gq {
namespace {

// ---- RMSNORM opcode (gemvqc_ops.h:169-234): one workgroup of 256 per row ----
__global__ __launch_bounds__(256) void norm_kernel(NormArgs a) {
    __shared__ float red[4];
    const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float * x = a.x + size_t(r) * a.stride;
    const int nw = a.n / 16, rounds = (nw + 255) / 256;  // n <= 16384: at most 4 rounds
    float rs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        if (g >= rounds) break;
        const int w = g * 256 + tid;
        float ws = 0.0f;
        if (w < nw) {
            float sq[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float v = x[16 * w + i];
                sq[i] = v * v;
            }
            ws = tree<16>(sq);
        }
        ws = pair_sum_lanes<64>(ws);
        if (lane == 0) red[wave] = ws;
        __syncthreads();
        rs[g] = (red[0] + red[1]) + (red[2] + red[3]);
        __syncthreads();
    }
    const float sum = (rs[0] + rs[1]) + (rs[2] + rs[3]);
    const float s = (a.flags & 1) ? 1.0f / fmaxf(sqrtf(sum), a.eps) : 1.0f / sqrtf(sum / float(a.n) + a.eps);
    float * y = a.y + size_t(r) * a.n;
    for (int i = tid; i < a.n; i += 256) y[i] = (a.flags & 2) ? x[i] * s : (x[i] * s) * a.w[i];
}

// ---- element-wise (gemvqc_ops.h:314-385) ----
__global__ void ew_kernel(EwArgs a) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += gridDim.x * blockDim.x) {
        const float av = a.op == EW_FILL ? 0.0f
                       : a.row ? a.a[size_t(i / a.row) * a.stride + i % a.row] : a.a[i];
        float r;
        switch (a.op) {
        case EW_ADD: r = av + a.b[i]; break;
        case EW_MUL: r = av * a.b[i]; break;
        case EW_SILU_MUL: r = (av / (1.0f + expf_(-av))) * a.b[i]; break;
        case EW_SIGMOID_MUL: r = (1.0f / (1.0f + expf_(-av))) * a.b[i]; break;
        case EW_SILU: r = silu_(av); break;
        case EW_SIGMOID: r = sigmoid_(av); break;
        case EW_SOFTPLUS: r = softplus_(av); break;
        case EW_COPY: r = av; break;
        default: r = a.value; break;
        }
        a.y[i] = r;
    }
}

// ---- CONV opcode (gemvqc_ops.h:387-431): window [state (3), x], summed from t = 0; n_tok tokens in order, the
// state moving one place per token ----
// With seqs, token t is the one token of sequence t (grid y): its own window in, its own window out.
__global__ void conv_kernel(ConvArgs a) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= a.ch) return;
    if (a.seqs) {
        const size_t t = blockIdx.y, so = 3 * size_t(a.ch) * t;
        a.s_src += so;
        a.s_dst += so;
        a.x += t * size_t(a.ch);
        a.y += t * size_t(a.ch);
        a.n_tok = 1;
    }
    float s0 = a.s_src[3 * c], s1 = a.s_src[3 * c + 1], s2 = a.s_src[3 * c + 2];
    const float w0 = a.w[4 * c], w1 = a.w[4 * c + 1], w2 = a.w[4 * c + 2], w3 = a.w[4 * c + 3];
    // every token's input is requested before the first output is stored (y may be x: a token's output replaces
    // only its own input)
    float xs[GEMM_MAX_TOK];
#pragma unroll
    for (int t = 0; t < GEMM_MAX_TOK; ++t) xs[t] = t < a.n_tok ? a.x[size_t(t) * a.ch + c] : 0.0f;
#pragma unroll
    for (int t = 0; t < GEMM_MAX_TOK; ++t) {
        if (t < a.n_tok) {
            const float x = xs[t];
            float sum = 0.0f;
            sum += s0 * w0;
            sum += s1 * w1;
            sum += s2 * w2;
            sum += x * w3;
            a.y[size_t(t) * a.ch + c] = a.silu ? silu_(sum) : sum;
            s0 = s1;
            s1 = s2;
            s2 = x;
        }
    }
    a.s_dst[3 * c] = s0;
    a.s_dst[3 * c + 1] = s1;
    a.s_dst[3 * c + 2] = s2;
}

// ---- ROPE opcode (gemvqc_ops.h:275-312): NEOX pairs (i, i + n_dims / 2) ----
__global__ void rope_kernel(RopeArgs a) {
    const int r = blockIdx.x;
    const float * cs = a.pos ? a.cs + size_t(*a.pos) * a.n_dims : a.cs;
    const float * x = a.x + size_t(r) * a.ne0;
    float * y = a.y + size_t(r) * a.ne0;
    const int half = a.n_dims / 2, i = threadIdx.x;  // blockDim.x >= ne0
    float out = 0.0f;
    if (i < a.ne0) {
        if (i < half) {
            out = x[i] * cs[2 * i] - x[i + half] * cs[2 * i + 1];
        } else if (i < a.n_dims) {
            const int j = i - half;
            out = x[j] * cs[2 * j + 1] + x[i] * cs[2 * j];
        } else {
            out = x[i];
        }
    }
    __syncthreads();  // y may be x
    if (i < a.ne0) y[i] = out;
}

// ---- GDN step (gemvqc_gdn.h:73-187 with the input load of :223-281) ----
// Workgroup (value head h, chunk of 8 state rows), 128 threads: 16 lanes per row, 8 consecutive floats per lane, one
// row per thread (512 workgroups for 32 heads: the per-token chain of dependent reductions is latency-bound, so more
// waves per SIMD hide it).
// The rows of a head are independent given q, k, v, beta and the decay, so a chunk needs nothing from the others.
// n_tok tokens run in order with the chunk's state in registers (loaded once, stored once); each token's inputs
// are requested two tokens ahead, so their latency overlaps the updates of the tokens before.
constexpr int GDN_ROWS = 8;
constexpr int GDN_IT = GDN_ROWS / 8;

struct GdnIn {  // one token's inputs of this thread
    float q[8], k[8], v[GDN_IT];
    float g, b;
};

__device__ __forceinline__ void gdn_load(const GdnArgs & a, int tk, int h, int kh, int chunk, int l16, int grp, GdnIn & o) {
    const float * qt = a.q + size_t(tk) * a.s_qkv, * kt = a.k + size_t(tk) * a.s_qkv, * vt = a.v + size_t(tk) * a.s_qkv;
    const float4 * qp = reinterpret_cast<const float4 *>(qt + kh * 128 + 8 * l16);
    const float4 * kp = reinterpret_cast<const float4 *>(kt + kh * 128 + 8 * l16);
    const float4 q0 = qp[0], q1 = qp[1], k0 = kp[0], k1 = kp[1];
    o.q[0] = q0.x; o.q[1] = q0.y; o.q[2] = q0.z; o.q[3] = q0.w; o.q[4] = q1.x; o.q[5] = q1.y; o.q[6] = q1.z; o.q[7] = q1.w;
    o.k[0] = k0.x; o.k[1] = k0.y; o.k[2] = k0.z; o.k[3] = k0.w; o.k[4] = k1.x; o.k[5] = k1.y; o.k[6] = k1.z; o.k[7] = k1.w;
#pragma unroll
    for (int it = 0; it < GDN_IT; ++it) o.v[it] = vt[h * 128 + chunk * GDN_ROWS + it * 8 + grp];
    o.g = a.g[size_t(tk) * a.s_gb + h];
    o.b = a.beta[size_t(tk) * a.s_gb + h];
}

// One token on the state rows x (gemvq_ref.h:360-397): decay, delta rule, output row dot.
__device__ __forceinline__ void gdn_token(const GdnArgs & a, const GdnIn & in, int tk, int h, int chunk, int l16, int grp,
                                          float dtv, float av, float (&x)[GDN_IT][8]) {
    float q[8], k[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        q[i] = in.q[i];
        k[i] = in.k[i];
    }
    if (a.flags & 2) gdn_l2_qk(q, k, a.l2_eps);  // L2 norm of q and k per key head (ggml_l2_norm)
    float bt;
    const float decay = gdn_gates(a.flags & 8, in.g, in.b, dtv, av, bt);
    float out[GDN_IT];
    gdn_step_rows<GDN_IT>(q, k, in.v, decay, bt, x, out);
    if (l16 == 0) {
#pragma unroll
        for (int it = 0; it < GDN_IT; ++it) a.y[size_t(tk) * a.s_y + h * 128 + chunk * GDN_ROWS + it * 8 + grp] = out[it] * a.scale;
    }
}

// With SEQS (args.seqs), grid y is the token: token t is the one token of sequence t on its own state rows.
// The state rows, the first token's inputs and the key head count are leading scalar arguments (preloaded into SGPRs
// where the firmware supports it), so without SEQS the state and input loads wait for no load of the argument
// segment.
template <bool SEQS>
__global__ __launch_bounds__(128) void gdn_kernel(const float * src, const float * q, const float * k, const float * v,
                                                  const float * g, const float * beta, int hk, GdnArgs args) {
    constexpr int IT = GDN_IT;
    GdnArgs a = args;
    a.src = src;
    a.q = q;
    a.k = k;
    a.v = v;
    a.g = g;
    a.beta = beta;
    a.hk = hk;
    if constexpr (SEQS) {
        const size_t t = blockIdx.y, so = size_t(a.hv) * 128 * 128 * t;
        a.src += so;
        a.dst += so;
        a.q += t * size_t(a.s_qkv);
        a.k += t * size_t(a.s_qkv);
        a.v += t * size_t(a.s_qkv);
        a.g += t * size_t(a.s_gb);
        a.beta += t * size_t(a.s_gb);
        a.y += t * size_t(a.s_y);
        a.n_tok = 1;
    }
    const int chunks = 128 / GDN_ROWS;
    const int h = blockIdx.x / chunks, chunk = blockIdx.x % chunks, kh = h % a.hk;
    const int l16 = threadIdx.x & 15, grp = threadIdx.x >> 4;  // 8 row groups
    // all state rows of this thread are requested before any is written (src and dst may be the same rows)
    float x[IT][8];
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int j = chunk * GDN_ROWS + it * 8 + grp;
        const size_t row = (size_t(h) * 128 + j) * 128 + 8 * l16;
        const float4 s0 = *reinterpret_cast<const float4 *>(a.src + row);
        const float4 s1 = *reinterpret_cast<const float4 *>(a.src + row + 4);
        x[it][0] = s0.x; x[it][1] = s0.y; x[it][2] = s0.z; x[it][3] = s0.w;
        x[it][4] = s1.x; x[it][5] = s1.y; x[it][6] = s1.z; x[it][7] = s1.w;
    }
    // a ring of three token inputs: token tk + 2 is requested before token tk runs (uniform branches: only tokens
    // that exist are loaded); the first token's are requested before the gate parameters
    GdnIn r0, r1, r2;
    gdn_load(a, 0, h, kh, chunk, l16, grp, r0);
    const int n = a.n_tok;
    if (n > 1) gdn_load(a, 1, h, kh, chunk, l16, grp, r1);
    float dtv = 0.0f, av = 0.0f;
    if (a.flags & 8) {
        dtv = a.dt[h];
        av = a.a[h];
    }
    for (int tk = 0; tk < n; tk += 3) {
        if (tk + 2 < n) gdn_load(a, tk + 2, h, kh, chunk, l16, grp, r2);
        gdn_token(a, r0, tk, h, chunk, l16, grp, dtv, av, x);
        if (tk + 1 >= n) break;
        if (tk + 3 < n) gdn_load(a, tk + 3, h, kh, chunk, l16, grp, r0);
        gdn_token(a, r1, tk + 1, h, chunk, l16, grp, dtv, av, x);
        if (tk + 2 >= n) break;
        if (tk + 4 < n) gdn_load(a, tk + 4, h, kh, chunk, l16, grp, r1);
        gdn_token(a, r2, tk + 2, h, chunk, l16, grp, dtv, av, x);
    }
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int j = chunk * GDN_ROWS + it * 8 + grp;
        const size_t row = (size_t(h) * 128 + j) * 128 + 8 * l16;
        *reinterpret_cast<float4 *>(a.dst + row) = make_float4(x[it][0], x[it][1], x[it][2], x[it][3]);
        *reinterpret_cast<float4 *>(a.dst + row + 4) = make_float4(x[it][4], x[it][5], x[it][6], x[it][7]);
    }
}

// ---- gated output norm (gemvqc_gdn.h:284-346): one wave per head, lane l holds elements 2l, 2l + 1 ----
__global__ __launch_bounds__(64) void gated_norm_kernel(GatedNormArgs a) {
    const int h = blockIdx.x, l = threadIdx.x;
    float * y = a.y + h * 128;
    const float y0 = y[2 * l], y1 = y[2 * l + 1];
    const float sum = pair_sum_lanes<64>(y0 * y0 + y1 * y1);
    const float s = 1.0f / sqrtf(sum / 128.0f + a.eps);
    const float z0 = a.z[h * 128 + 2 * l], z1 = a.z[h * 128 + 2 * l + 1];
    const float g0 = a.z_silu ? z0 : silu_(z0), g1 = a.z_silu ? z1 : silu_(z1);
    const float o0 = g0 * ((y0 * s) * a.w[2 * l]);
    const float o1 = g1 * ((y1 * s) * a.w[2 * l + 1]);
    y[2 * l] = o0;
    y[2 * l + 1] = o1;
}

// ---- attention core (one token, GQA, fp16 KV) ----
// Workgroup (q head, chunk of 64 positions), 256 threads; HD = head_dim, a power of two in [16, 256]. The G q heads
// of a KV head and chunk run on workgroups that are dealt to the same XCD, whose L2 then serves the chunk's keys and
// values to all of them. Every global read of a phase is issued in one round (a dependent chain of global loads
// costs about a microsecond per link, far more than the arithmetic here):
//   1. the chunk's cached keys and values (thread t holds 16-byte piece t % (HD / 8) of rows t / (HD / 8) + k *
//      (2048 / HD)), the head's q row, the new key and value, the norm weights and the RoPE row;
//   2. RMS norm with weight and NEOX RoPE of q and the new key (element e in thread e), fp16 rounding; the first
//      q head of the KV head stores the new key and value in the cache;
//   3. scores from registers: 8 products and their adjacent tree in the thread, the tree over the HD / 8 pieces
//      of a row across lanes (together the pairwise sum over head_dim), times scale;
//   4. the chunk max, e^(s - max), then thread d sums p and p * v[d] over the positions in order and writes the
//      partials (max, sum, o[hd]);
//   5. the last workgroup of the q head loads all chunks' partials (32 chunks per round), forms M = max m_c,
//      f_c = e^(m_c - M), L = sum l_c f_c and O = sum o_c f_c in chunk order, and writes O / L times the sigmoid
//      of the gate.
constexpr int ATT_T = 256;
// 16 bytes of keys or values: a native vector, which the compiler keeps in registers (HIP's uint4 struct kept the
// chunk's arrays out of SROA, in scratch)
typedef unsigned kv16 __attribute__((ext_vector_type(4)));
constexpr int MAXCH = 64;  // chunks a combine round handles (wave 0's lanes)
constexpr int CMB = 32;    // chunks per load round of the combine (each round is a dependent load)

// ---- new keys, values and queries of n_tok tokens (step 2 below, one vector per workgroup) ----
// Workgroup (slot s, token t): s < n_head normalizes and rotates q head s and writes it, fp16-rounded, to qr; the
// others do the same for the new key of KV head s - n_head and store it and the value in the cache at *pos + t.
// Same operations in the same order as the single-token kernel, so the cache and the rounded queries are the bits
// that n_tok single-token launches would produce.
template <int HD>
__global__ __launch_bounds__(ATT_T) void attn_append_kernel(AttnArgs a) {
    __shared__ float xs[HD];
    __shared__ float red[4];
    const int s = blockIdx.x, t = blockIdx.y, pos = a.seq_ctx ? a.pos[16 * t] : *a.pos + t;
    if (pos < 0 || pos >= a.n_ctx) return;  // positions past the KV capacity are not stored
    const bool isq = s < a.n_head;
    const int h = isq ? s : s - a.n_head;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = a.n_rot / 2;
    const bool el = tid < HD;
    const int e = el ? tid : 0;
    const size_t kvo = (size_t(t) * a.n_head_kv + h) * HD + e;
    const float x = !el ? 0.0f : isq ? a.q[size_t(t) * a.n_head * a.q_stride + size_t(h) * a.q_stride + e] : a.k[kvo];
    const float w = isq ? a.qn[e] : a.kn[e];
    const float vv = isq ? 0.0f : a.v[kvo];
    const int pi = e < half ? e : e - half;
    const bool rot = e < a.n_rot;
    const float cs0 = rot ? a.cs[size_t(pos) * a.n_rot + 2 * pi] : 0.0f;
    const float cs1 = rot ? a.cs[size_t(pos) * a.n_rot + 2 * pi + 1] : 0.0f;
    float sq[1] = {x * x};
    pair_sum_lanes_n<64, 1>(sq);
    if (lane == 0) red[wave] = sq[0];
    __syncthreads();
    const float sum = (red[0] + red[1]) + (red[2] + red[3]);
    const float sc = 1.0f / sqrtf(sum / float(HD) + a.eps);
    if (el) xs[e] = (x * sc) * w;
    __syncthreads();
    const float x0 = xs[pi], x1 = xs[pi + half];
    const float rv = e < half ? x0 * cs0 - x1 * cs1 : (rot ? x0 * cs1 + x1 * cs0 : xs[e]);
    if (!el) return;
    if (isq) {
        a.qr[(size_t(t) * a.n_head + h) * HD + e] = h2f(f2h(rv));
    } else {
        const size_t cpos = a.seq_ctx ? size_t(t) * a.seq_ctx + pos : size_t(pos);  // the token's sequence region
        const size_t off = (cpos * a.n_head_kv + h) * HD + e;
        a.kc[off] = uint16_t(f2h(rv));
        a.vc[off] = uint16_t(f2h(vv));
    }
}

// Chunk partials: agent-scope atomic accesses (coherent across the XCDs' L2 caches). The combine orders them with a
// wait for the stores' completion (s_waitcnt 0) before the counter update: on gfx9 vector stores are counted in
// vmcnt, so that wait covers them. Later architectures count stores separately (vscnt), which s_waitcnt 0 does not
// wait for, so the code is restricted to the gfx9 CDNA parts it was written for.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__) && !defined(__gfx942__)
#error "the attention combine relies on gfx9 store counting (vmcnt); build for gfx950 (or gfx942)"
#endif
__device__ __forceinline__ void part_store(float * p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float part_load(const float * p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Steps 3-4 of one token on a loaded chunk (rows t0 .. t0 + nt - 1): kr holds the chunk's key pieces, vs its values,
// qs[0] the rounded q and, with NEW, qs[1] the new key of row pos. Leaves the chunk max in mx and gives thread e
// (< HD) the chunk's sums l and o over its positions in order.
template <int HD, bool NEW>
__device__ __forceinline__ void attn_chunk(const AttnArgs & a, const kv16 (&kr)[(ATTN_CHUNK + ATT_T / (HD / 8) - 1) / (ATT_T / (HD / 8))],
                                           const uint16_t * vs, const float (*qs)[HD], float * pr, float & mx, int pos,
                                           int t0, int nt, float & o, float & l) {
    constexpr int PER = HD / 8, RPP = ATT_T / PER, NP = (ATTN_CHUNK + RPP - 1) / RPP;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, pc = tid % PER;
    const bool el = tid < HD;
    const int e = el ? tid : 0;
    // ---- 3. scores ----
    float qv[8], kn[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        qv[i] = qs[0][pc * 8 + i];
        kn[i] = qs[1][pc * 8 + i];
    }
    float dots[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        const bool is_new = NEW && t0 + tid / PER + j * RPP == pos;
        const uint32_t kw[4] = {kr[j].x, kr[j].y, kr[j].z, kr[j].w};
        float t[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] = qv[i] * (is_new ? kn[i] : h2f((kw[i / 2] >> (16 * (i % 2))) & 0xffffu));
        dots[j] = tree<8>(t);
    }
    pair_sum_lanes_n<PER, NP>(dots);
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        const int ti = tid / PER + j * RPP;
        if (pc == 0 && ti < nt) pr[ti] = dots[j] * a.scale;
    }
    __syncthreads();
    // ---- 4. chunk softmax numerators, partial sums in position order ----
    if (wave == 0) {
        const float sv = lane < nt ? pr[lane] : -__builtin_inff();
        float m = sv;
#pragma unroll
        for (int st = 32; st >= 1; st >>= 1) m = fmaxf(m, __shfl_xor(m, st, WAVE));
        if (lane < nt) pr[lane] = expf_(sv - m);
        if (lane == 0) mx = m;
    }
    __syncthreads();
    o = 0.0f;
    l = 0.0f;
    if (el) {
#pragma unroll 8
        for (int i = 0; i < nt; ++i) {
            const float p = pr[i];
            l += p;
            o += p * h2f(vs[i * HD + e]);
        }
    }
}

// Steps 3-5 of one token on a loaded chunk (as attn_chunk); the partials go to set th, and the workgroup that
// completes the set's nc chunks combines them into the output row (and clears the set's counter).
template <int HD, bool NEW>
__device__ __forceinline__ void attn_token(const AttnArgs & a, const kv16 (&kr)[(ATTN_CHUNK + ATT_T / (HD / 8) - 1) / (ATT_T / (HD / 8))],
                                           const uint16_t * vs, const float (*qs)[HD], float * pr, float & mx, float * fcs,
                                           float * lcs, int & last, int pos, int t0, int chunk, int th, int nt, int nc, float gt) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool el = tid < HD;
    const int e = el ? tid : 0;
    float o, l;
    attn_chunk<HD, NEW>(a, kr, vs, qs, pr, mx, pos, t0, nt, o, l);
    const int pstride = 2 + HD, nchmax = (a.n_ctx + ATTN_CHUNK - 1) / ATTN_CHUNK;
    if (el) {
        float * pp = a.part + (size_t(th) * nchmax + chunk) * pstride;
        part_store(pp + 2 + e, o);
        if (e == 0) {
            part_store(pp, mx);
            part_store(pp + 1, l);
        }
    }
    // The partials are agent-scope atomic stores, coherent across the XCDs without an L2 writeback; every thread
    // waits until its stores have completed before the barrier, so the counter update that follows it is ordered
    // after all of them (a release without the writeback of the whole L2 that a release fence performs). The last
    // workgroup's partial loads are agent-scope atomic loads issued after its counter update returned, so they need
    // no acquire fence (no L2 invalidation) either.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
        last = __hip_atomic_fetch_add(a.counter + th, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == unsigned(nc - 1);
    __syncthreads();
    if (!last) return;
    // ---- 5. combine (last workgroup of the q head): M over every chunk, then L and O in chunk order, MAXCH
    //      chunks a round (wave 0 forms a round's f_c and l_c in LDS) ----
    const float * pk = a.part + size_t(th) * nchmax * pstride;
    const int nr0 = min(nc, MAXCH);  // chunks of the first round
    float ov[CMB];
    float mc = -__builtin_inff(), lc = 0.0f;
    if (wave == 0 && lane < nr0) {
        mc = part_load(pk + size_t(lane) * pstride);
        lc = part_load(pk + size_t(lane) * pstride + 1);
    }
#pragma unroll
    for (int c = 0; c < CMB; ++c) ov[c] = c < nc ? part_load(pk + size_t(c) * pstride + 2 + e) : 0.0f;
    if (wave == 0) {
        float M = mc;
        for (int r0 = MAXCH; r0 < nc; r0 += MAXCH)  // contexts past MAXCH chunks: the later rounds' maxima
            M = fmaxf(M, r0 + lane < nc ? part_load(pk + size_t(r0 + lane) * pstride) : -__builtin_inff());
#pragma unroll
        for (int st = 32; st >= 1; st >>= 1) M = fmaxf(M, __shfl_xor(M, st, WAVE));
        if (lane < nr0) {
            fcs[lane] = expf_(mc - M);
            lcs[lane] = lc;
        }
        if (lane == 0) mx = M;
    }
    __syncthreads();
    float O = 0.0f, L = 0.0f;
    for (int r0 = 0;;) {
        const int rn = min(MAXCH, nc - r0);
        for (int c0 = 0;;) {  // the round's chunks, CMB value rows a dependent load
#pragma unroll
            for (int c = 0; c < CMB; ++c) {
                if (c0 + c >= rn) break;
                const float f = fcs[c0 + c];
                L += lcs[c0 + c] * f;
                O += ov[c] * f;
            }
            c0 += CMB;
            if (c0 >= rn) break;
#pragma unroll
            for (int c = 0; c < CMB; ++c)
                ov[c] = c0 + c < rn ? part_load(pk + size_t(r0 + c0 + c) * pstride + 2 + e) : 0.0f;
        }
        r0 += MAXCH;
        if (r0 >= nc) break;
        const int rn2 = min(MAXCH, nc - r0);
        __syncthreads();  // every thread has read this round's f_c and l_c
        if (wave == 0 && lane < rn2) {
            const float m2 = part_load(pk + size_t(r0 + lane) * pstride);
            fcs[lane] = expf_(m2 - mx);
            lcs[lane] = part_load(pk + size_t(r0 + lane) * pstride + 1);
        }
#pragma unroll
        for (int c = 0; c < CMB; ++c)
            ov[c] = c < rn2 ? part_load(pk + size_t(r0 + c) * pstride + 2 + e) : 0.0f;
        __syncthreads();
    }
    if (el) {
        float out = O / L;
        if (a.gate) out = (1.0f / (1.0f + expf_(-gt))) * out;
        a.y[size_t(th) * HD + e] = out;
    }
    if (tid == 0) a.counter[th] = 0u;
}

// The position, the q rows, the cache and the head counts are leading scalar arguments (preloaded into SGPRs where
// the firmware supports it): the position and q loads wait for no load of the argument segment.
template <int HD>
__global__ __launch_bounds__(ATT_T) void attn_kernel(const int32_t * pos_p, const float * q, uint16_t * kc, uint16_t * vc,
                                                     int n_head, int n_head_kv, int q_stride, int n_ctx, AttnArgs args) {
    AttnArgs a = args;
    a.pos = pos_p;
    a.q = q;
    a.kc = kc;
    a.vc = vc;
    a.n_head = n_head;
    a.n_head_kv = n_head_kv;
    a.q_stride = q_stride;
    a.n_ctx = n_ctx;
    constexpr int PER = HD / 8;                    // 16-byte pieces per row
    constexpr int RPP = ATT_T / PER;               // rows per pass
    constexpr int NP = (ATTN_CHUNK + RPP - 1) / RPP;  // passes
    __shared__ __align__(16) uint16_t vs[ATTN_CHUNK * HD];
    __shared__ __align__(16) float qs[2][HD];  // q and the new key: normalized, then rotated + rounded
    __shared__ float pr[ATTN_CHUNK];           // scores, then e^(s - max)
    __shared__ float red[2][4];
    __shared__ float mx, fcs[MAXCH], lcs[MAXCH];
    __shared__ int last;
    // workgroup b: unit u = (KV head, chunk) with u % 8 == b % 8 (one XCD), q head g of the unit's KV head
    const int G = a.n_head / a.n_head_kv, b = blockIdx.x;
    const int u = (b / (8 * G)) * 8 + (b & 7), g = (b >> 3) % G;
    const int kvh = u % a.n_head_kv, chunk = u / a.n_head_kv, hq = kvh * G + g;
    const int th = hq;  // the q head's partials set
    const int pos = *a.pos, nc = (pos + ATTN_CHUNK) / ATTN_CHUNK;
    if (pos < 0 || pos >= a.n_ctx || chunk >= nc) return;  // positions past the KV capacity are not stored
    const int tid = threadIdx.x, half = a.n_rot / 2;
    const int lane = tid & 63, wave = tid >> 6, pc = tid % PER;
    const int t0 = chunk * ATTN_CHUNK, nt = min(ATTN_CHUNK, pos + 1 - t0);
    const bool has_new = chunk == nc - 1;  // this chunk holds pos
    const float * qrow = a.q + size_t(hq) * a.q_stride;
    // ---- 1. loads ----
    kv16 kr[NP], vr[NP];  // rows past the chunk re-read its last row (stored memory); they are not used
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        const int ti = min(tid / PER + j * RPP, nt - 1);
        const size_t off = (size_t(t0 + ti) * a.n_head_kv + kvh) * HD + pc * 8;
        kr[j] = *reinterpret_cast<const kv16 *>(a.kc + off);
        vr[j] = *reinterpret_cast<const kv16 *>(a.vc + off);
    }
    const bool el = tid < HD;
    const int e = el ? tid : 0;  // element of the head this thread holds
    float xv[2];
    xv[0] = el ? qrow[e] : 0.0f;
    xv[1] = (has_new && el) ? a.k[size_t(kvh) * HD + e] : 0.0f;
    const float wq = a.qn[e], wk = a.kn[e];
    const float vv = has_new ? a.v[size_t(kvh) * HD + e] : 0.0f;
    const float gt = a.gate ? a.gate[size_t(hq) * 2 * HD + e] : 0.0f;
    const int pi = e < half ? e : e - half;  // the RoPE pair of this element
    const bool rot = e < a.n_rot;
    const float cs0 = rot ? a.cs[size_t(pos) * a.n_rot + 2 * pi] : 0.0f;
    const float cs1 = rot ? a.cs[size_t(pos) * a.n_rot + 2 * pi + 1] : 0.0f;
#pragma unroll
    for (int j = 0; j < NP; ++j) {  // values to LDS (the row of pos is overwritten with the new value below)
        const int ti = tid / PER + j * RPP;
        if (ti < nt) *reinterpret_cast<kv16 *>(vs + ti * HD + pc * 8) = vr[j];
    }
    // ---- 2. norms (pairwise over head_dim), RoPE, fp16 rounding ----
    {
        float sq[2] = {xv[0] * xv[0], xv[1] * xv[1]};
        pair_sum_lanes_n<64, 2>(sq);
        if (lane == 0) {
            red[0][wave] = sq[0];
            red[1][wave] = sq[1];
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float sum = (red[h][0] + red[h][1]) + (red[h][2] + red[h][3]);
            const float sc = 1.0f / sqrtf(sum / float(HD) + a.eps);
            if (el) qs[h][e] = (xv[h] * sc) * (h == 0 ? wq : wk);
        }
        __syncthreads();
        float rv[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float x0 = qs[h][pi], x1 = qs[h][pi + half];
            rv[h] = e < half ? x0 * cs0 - x1 * cs1 : (rot ? x0 * cs1 + x1 * cs0 : qs[h][e]);
        }
        __syncthreads();
        if (el) {
            qs[0][e] = h2f(f2h(rv[0]));
            qs[1][e] = h2f(f2h(rv[1]));
            if (has_new) {
                const uint32_t kb = f2h(rv[1]), vb = f2h(vv);
                vs[(pos - t0) * HD + e] = uint16_t(vb);
                if (g == 0) {  // one q head per KV head stores the new key and value
                    const size_t off = (size_t(pos) * a.n_head_kv + kvh) * HD + e;
                    a.kc[off] = uint16_t(kb);
                    a.vc[off] = uint16_t(vb);
                }
            }
        }
    }
    __syncthreads();
    attn_token<HD, true>(a, kr, vs, qs, pr, mx, fcs, lcs, last, pos, t0, chunk, th, nt, nc, gt);
}

// ---- embedding rows (ggml dequantize_row_*) ----
// The ids are a leading scalar argument (preloaded into SGPRs where the firmware supports it): the id load waits for
// no load of the argument segment.
__global__ void get_rows_kernel(const int32_t * ids, GetRowsArgs a) {
    const int id = ids[16 * blockIdx.y];
    if (id < 0 || id >= a.rows) return;
    float * const yt = a.y + size_t(blockIdx.y) * a.cols;  // this token's row
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < a.cols; i += gridDim.x * blockDim.x) {
        float y;
        if (a.type == T_Q6_K) {
            const int nsb = a.cols / 256, sb = i / 256, e = i % 256;
            const size_t sbi = size_t(id) * nsb + sb;
            const int n = e / 128, r = e % 128, quarter = r / 32, l = r % 32;
            // unit j = 2n + (quarter & 1) holds quarter & 1 (group A) and quarter | 2 (group B); its high bits and
            // scale bytes are contiguous in the repacked layout
            const int j = 2 * n + (quarter & 1), grp = quarter >> 1;
            const uint8_t ql = a.w.a[sbi * 128 + 64 * n + l + 32 * (quarter & 1)];
            const uint8_t qh = a.w.b[sbi * 64 + 16 * j + 4 * ((l >> 2) & 3) + (l & 3)];
            const int lo = quarter < 2 ? (ql & 0xF) : (ql >> 4);
            const int q = (lo | (((qh >> (2 * (l >> 4) + 4 * grp)) & 3) << 4)) - 32;
            const int8_t scv = int8_t(a.w.c[sbi * 16 + 4 * j + 2 * grp + l / 16]);
            const float d = h2f(*reinterpret_cast<const uint16_t *>(a.w.d + sbi * 2));
            y = (d * float(scv)) * float(q);
        } else if (a.type == T_Q4_0) {
            const int nb = a.cols / 32, b = i / 32, j = i % 32;
            const size_t bi = size_t(id) * nb + b;
            const uint8_t byte = a.w.a[bi * 16 + (j & 15)];
            const int q = (j < 16 ? (byte & 15) : (byte >> 4)) - 8;
            y = float(q) * h2f(*reinterpret_cast<const uint16_t *>(a.w.b + bi * 2));
        } else {  // Q8_0
            const int nb = a.cols / 32, b = i / 32, j = i % 32;
            const size_t bi = size_t(id) * nb + b;
            const int8_t q = int8_t(j < 16 ? a.w.a[bi * 16 + j] : a.w.b[bi * 16 + j - 16]);
            y = float(q) * h2f(*reinterpret_cast<const uint16_t *>(a.w.c + bi * 2));
        }
        yt[i] = y;
    }
}

// Grid y: row r of x (stride floats apart), its key at key + 8 r (16 floats).
__global__ __launch_bounds__(256) void argmax_kernel(const float * x, int n, unsigned long long * key, int stride) {
    __shared__ unsigned long long red[4];
    x += size_t(blockIdx.y) * stride;
    key += size_t(blockIdx.y) * 8;
    unsigned long long best = 0;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
        const unsigned long long k = argmax_key(x[i], uint32_t(i));
        best = k > best ? k : best;
    }
    for (int s = 32; s >= 1; s >>= 1) {
        const unsigned long long o = __shfl_xor(best, s, WAVE);
        best = o > best ? o : best;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long b = red[0];
        for (int i = 1; i < 4; ++i) b = red[i] > b ? red[i] : b;
        atomicMax(key, b);
    }
}

// With n_seq > 1, thread t serves sequence t.
__global__ void next_token_kernel(NextTokenArgs a) {
    if (a.n_seq > 1) {
        const int t = threadIdx.x;
        if (t >= a.n_seq) return;
        a.key += 8 * t;
        a.tok += 16 * t;
        a.pos += 16 * t;
        a.prompt += size_t(t) * a.seq_cap;
        a.out += size_t(t) * a.seq_cap;
        a.n_prompt = a.n_prompt_of[16 * t];
        a.max_pos = a.seq_cap;
    }
    const int pos = *a.pos;
    const unsigned long long k = *a.key;
    int tok = int(0xffffffffu - uint32_t(k & 0xffffffffu));
    // a sequence's prompt occupies at most its seq_cap slots, whatever its length word says
    const int plim = a.n_seq > 1 ? min(a.n_prompt, a.seq_cap) : a.n_prompt;
    if (pos + 1 < plim) tok = a.prompt[pos + 1];
    if (pos + 1 < a.max_pos) a.out[pos + 1] = tok;
    *a.tok = tok;
    *a.pos = pos + 1;
    *a.key = 0ull;
}

}  // namespace

hipError_t launch_norm(const NormArgs & a, hipStream_t s) {
    GQ_LAUNCH(norm_kernel, dim3(a.rows), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_ew(const EwArgs & a, hipStream_t s) {
    int grid = (a.n + 255) / 256;
    grid = grid < 1024 ? grid : 1024;
    GQ_LAUNCH(ew_kernel, dim3(grid), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_conv(const ConvArgs & a, hipStream_t s) {
    GQ_LAUNCH(conv_kernel, dim3((a.ch + 255) / 256, a.seqs ? a.n_tok : 1), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_rope(const RopeArgs & a, hipStream_t s) {
    if (a.ne0 > 1024) return hipErrorInvalidValue;
    const int t = ((a.ne0 + 63) / 64) * 64;
    GQ_LAUNCH(rope_kernel, dim3(a.rows), dim3(t), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_gdn(const GdnArgs & a, hipStream_t s) {
    if (a.seqs)
        GQ_LAUNCH(gdn_kernel<true>, dim3(a.hv * (128 / GDN_ROWS), a.n_tok), dim3(128), 0, s, a.src, a.q, a.k, a.v, a.g,
                  a.beta, a.hk, a);
    else
        GQ_LAUNCH(gdn_kernel<false>, dim3(a.hv * (128 / GDN_ROWS), 1), dim3(128), 0, s, a.src, a.q, a.k, a.v, a.g,
                  a.beta, a.hk, a);
    return hipGetLastError();
}

hipError_t launch_gated_norm(const GatedNormArgs & a, hipStream_t s) {
    GQ_LAUNCH(gated_norm_kernel, dim3(a.heads), dim3(64), 0, s, a);
    return hipGetLastError();
}

// ---- attention of a block of tokens (after attn_append_kernel) ----
// Workgroup (unit, q head, group of ATTN_TG tokens): the chunk's keys (registers) and values (LDS) are loaded once,
// for the group's last stored position, and serve the group's tokens in turn; each token runs attn_token on the rows
// up to its own position, with its rounded query from qr, so its partials, combine and output are those of a one-token
// launch. Tokens whose position is outside the KV capacity are skipped.
constexpr int ATTN_TG = 2;

template <int HD>
__global__ __launch_bounds__(ATT_T) void attn_group_kernel(AttnArgs a) {
    constexpr int PER = HD / 8, RPP = ATT_T / PER, NP = (ATTN_CHUNK + RPP - 1) / RPP;
    __shared__ __align__(16) uint16_t vs[ATTN_CHUNK * HD];
    __shared__ __align__(16) float qs[2][HD];  // the token's rounded q (qs[1] unused)
    __shared__ float pr[ATTN_CHUNK];
    __shared__ float mx, fcs[MAXCH], lcs[MAXCH];
    __shared__ int last;
    const int G = a.n_head / a.n_head_kv, b = blockIdx.x;
    const int u = (b / (8 * G)) * 8 + (b & 7), g = (b >> 3) % G;
    const int kvh = u % a.n_head_kv, chunk = u / a.n_head_kv, hq = kvh * G + g;
    // with sequences a group is one token, whose position is its own and whose keys and values are its sequence's
    const int tg = a.seq_ctx ? 1 : ATTN_TG, tk0 = int(blockIdx.y) * tg, tk1 = min(tk0 + tg, a.n_tok);
    const int pos0 = a.seq_ctx ? a.pos[16 * tk0] - tk0 : *a.pos;  // token t at pos0 + t
    if (a.seq_ctx) {
        const size_t ro = size_t(tk0) * a.seq_ctx * a.n_head_kv * HD;
        a.kc += ro;
        a.vc += ro;
    }
    const int first = max(pos0 + tk0, 0), plast = min(pos0 + tk1 - 1, a.n_ctx - 1);  // the group's stored positions
    if (first > plast || chunk >= (plast + ATTN_CHUNK) / ATTN_CHUNK) return;
    const int tid = threadIdx.x, pc = tid % PER;
    const int t0 = chunk * ATTN_CHUNK, ntmax = min(ATTN_CHUNK, plast + 1 - t0);
    kv16 kr[NP], vr[NP];  // rows past ntmax re-read row ntmax - 1; they are not used
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        const int ti = min(tid / PER + j * RPP, ntmax - 1);
        const size_t off = (size_t(t0 + ti) * a.n_head_kv + kvh) * HD + pc * 8;
        kr[j] = *reinterpret_cast<const kv16 *>(a.kc + off);
        vr[j] = *reinterpret_cast<const kv16 *>(a.vc + off);
    }
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        const int ti = tid / PER + j * RPP;
        if (ti < ntmax) *reinterpret_cast<kv16 *>(vs + ti * HD + pc * 8) = vr[j];
    }
    const bool el = tid < HD;
    const int e = el ? tid : 0;
    for (int t = tk0; t < tk1; ++t) {  // uniform over the workgroup
        const int pos = pos0 + t, nc = (pos + ATTN_CHUNK) / ATTN_CHUNK;
        if (pos < 0 || pos >= a.n_ctx || chunk >= nc) continue;
        const int th = t * a.n_head + hq, nt = min(ATTN_CHUNK, pos + 1 - t0);
        if (el) qs[0][e] = a.qr[size_t(th) * HD + e];
        const float gt = a.gate ? a.gate[size_t(t) * a.n_head * a.q_stride + size_t(hq) * 2 * HD + e] : 0.0f;
        __syncthreads();  // qs (and, the first time, vs) written
        attn_token<HD, false>(a, kr, vs, qs, pr, mx, fcs, lcs, last, pos, t0, chunk, th, nt, nc, gt);
        __syncthreads();  // the next token overwrites qs, pr and the combine's shared values
    }
}

// One token: the attention kernel alone. Several: their new keys, values and queries first (one launch), then the
// attention of every (token, q head, chunk).
template <int HD>
hipError_t launch_attn_hd(const AttnArgs & a, dim3 grid, hipStream_t s) {
    if (grid.y == 1) {
        GQ_LAUNCH(attn_kernel<HD>, grid, dim3(ATT_T), 0, s, a.pos, a.q, a.kc, a.vc, a.n_head, a.n_head_kv, a.q_stride,
                  a.n_ctx, a);
        return hipGetLastError();
    }
    GQ_LAUNCH(attn_append_kernel<HD>, dim3(a.n_head + a.n_head_kv, grid.y), dim3(ATT_T), 0, s, a);
    const int tg = a.seq_ctx ? 1 : ATTN_TG;
    GQ_LAUNCH(attn_group_kernel<HD>, dim3(grid.x, (grid.y + tg - 1) / tg), dim3(ATT_T), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_attn(const AttnArgs & a, hipStream_t s) {
    if (a.n_head % a.n_head_kv || a.n_head / a.n_head_kv > ATTN_MAXG)
        return hipErrorInvalidValue;
    // units (KV head, chunk) in groups of 8, each group followed by its q heads: workgroup b serves unit
    // (b / (8 G)) 8 + b % 8 (units past the last are idle) and q head (b / 8) % G of its KV head
    const int units = a.n_head_kv * ((a.n_ctx + ATTN_CHUNK - 1) / ATTN_CHUNK);
    const int n_tok = a.n_tok > 1 ? a.n_tok : 1;
    if (n_tok > GEMM_MAX_TOK || (n_tok > 1 && !a.qr)) return hipErrorInvalidValue;
    const dim3 grid(((units + 7) / 8) * 8 * (a.n_head / a.n_head_kv), n_tok);
    switch (a.head_dim) {
    case 16: return launch_attn_hd<16>(a, grid, s);
    case 32: return launch_attn_hd<32>(a, grid, s);
    case 64: return launch_attn_hd<64>(a, grid, s);
    case 128: return launch_attn_hd<128>(a, grid, s);
    case 256: return launch_attn_hd<256>(a, grid, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_get_rows(const GetRowsArgs & a, hipStream_t s) {
    GQ_LAUNCH(get_rows_kernel, dim3((a.cols + 255) / 256, a.n_tok > 1 ? a.n_tok : 1), dim3(256), 0, s, a.id, a);
    return hipGetLastError();
}

hipError_t launch_argmax(const float * x, int n, unsigned long long * key, int rows, int stride, hipStream_t s) {
    int grid = (n + 255) / 256;
    grid = grid < 256 ? grid : 256;
    GQ_LAUNCH(argmax_kernel, dim3(grid, rows), dim3(256), 0, s, x, n, key, stride);
    return hipGetLastError();
}

hipError_t launch_next_token(const NextTokenArgs & a, hipStream_t s) {
    GQ_LAUNCH(next_token_kernel, dim3(1), dim3(a.n_seq > 1 ? ((a.n_seq + 63) / 64) * 64 : 1), 0, s, a);
    return hipGetLastError();
}

}  // namespace gq
