// Reference-arithmetic kernels other than the GEMV (see gq_ref.h): row norms, the element-wise ops that evaluate exp
// or log, the conv, the DeltaNet step and its gated output norm, attention, and the exhaustive hash of the
// correctly rounded exp / log. They favour the reference's operation order over speed; the mode exists to give the
// reference CPU path's results on the GPU.
#include "gemvq_hip.h"
#include "gq_ref.h"
#include "gq_refmath.h"

namespace gq {
namespace {

// ---- RMSNORM rows (gemvq_ref.h:309-324): one workgroup of 256 per row ----
__global__ __launch_bounds__(256) void norm_ref_kernel(NormArgs a) {
    __shared__ double red[4];
    const int r = blockIdx.x, tid = threadIdx.x;
    const float * x = a.x + size_t(r) * a.stride;
    const int l2 = a.flags & 1;
    const float v = ref_norm_value(x, a.n, l2, red);
    const float s = l2 ? 1.0f / fmaxf(sqrtf(v), a.eps) : 1.0f / sqrtf(v + a.eps);
    float * y = a.y + size_t(r) * a.n;
    for (int i = tid; i < a.n; i += 256) y[i] = (a.flags & 2) ? x[i] * s : (x[i] * s) * a.w[i];
}

// ---- element-wise ops (gemvq_ref.h:297-342), exp / log correctly rounded ----
__global__ void ew_ref_kernel(EwArgs a) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += gridDim.x * blockDim.x) {
        const float av = a.op == EW_FILL ? 0.0f : a.row ? a.a[size_t(i / a.row) * a.stride + i % a.row] : a.a[i];
        float r;
        switch (a.op) {
        case EW_ADD: r = av + a.b[i]; break;
        case EW_MUL: r = av * a.b[i]; break;
        case EW_SILU_MUL: r = av / (1.0f + cr::expf(-av)) * a.b[i]; break;
        case EW_SIGMOID_MUL: r = 1.0f / (1.0f + cr::expf(-av)) * a.b[i]; break;
        case EW_SILU: r = cr::silu(av); break;
        case EW_SIGMOID: r = cr::sigmoid(av); break;
        case EW_SOFTPLUS: r = cr::softplus(av); break;
        case EW_COPY: r = av; break;
        default: r = a.value; break;
        }
        a.y[i] = r;
    }
}

// ---- CONV, one token (gemvq_ref.h:344-358): window [state (3), x] summed from t = 0 ----
__global__ void conv_ref_kernel(ConvArgs a, int tok) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= a.ch) return;
    const size_t so = 3 * size_t(a.ch) * size_t(tok);
    // tokens of one sequence run in order on the same window; sequences each have their own
    const float * src = a.seqs ? a.s_src + so : tok == 0 ? a.s_src : a.s_dst;
    float * dst = a.seqs ? a.s_dst + so : a.s_dst;
    const float x = a.x[size_t(tok) * a.ch + c];
    const float s0 = src[3 * c], s1 = src[3 * c + 1], s2 = src[3 * c + 2];
    float sum = 0.0f;
    sum += s0 * a.w[4 * c];
    sum += s1 * a.w[4 * c + 1];
    sum += s2 * a.w[4 * c + 2];
    sum += x * a.w[4 * c + 3];
    a.y[size_t(tok) * a.ch + c] = a.silu ? cr::silu(sum) : sum;
    dst[3 * c] = s1;
    dst[3 * c + 1] = s2;
    dst[3 * c + 2] = x;
}

// ---- DeltaNet step, one token (gemvq_ref.h:360-397 with ggml's L2_NORM and gate ops around it,
// ggml-xrt.cpp:1977-2000): workgroup = value head h, thread j = state row j ----
__global__ __launch_bounds__(128) void gdn_ref_kernel(GdnArgs a, int tok) {
    __shared__ float ys[128];
    __shared__ double red[2];
    const int h = blockIdx.x, j = threadIdx.x, kh = h % a.hk;
    const float * q = a.q + size_t(tok) * a.s_qkv + kh * 128;
    const float * k = a.k + size_t(tok) * a.s_qkv + kh * 128;
    const float * v = a.v + size_t(tok) * a.s_qkv + h * 128;
    const size_t so = a.seqs ? size_t(tok) * a.hv * 128 * 128 : 0;
    const float * src = a.seqs ? a.src + so : tok == 0 ? a.src : a.dst;
    float * dst = a.dst + so;
    // the thread's state row is requested first: its loads overlap the norms and the gate arithmetic below
    const size_t row = (size_t(h) * 128 + j) * 128;
    float s[128];
#pragma unroll
    for (int i = 0; i < 128; i += 4) {
        const float4 t = *reinterpret_cast<const float4 *>(src + row + i);
        s[i] = t.x;
        s[i + 1] = t.y;
        s[i + 2] = t.z;
        s[i + 3] = t.w;
    }
    // q and k in registers of both waves (element i in lane i % 64 of word i / 64), read back by readlane in the
    // in-order dots below (instead of an LDS read per step); the gate parameters and z requested now
    const auto lane_of = [](float x, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l)); };
    const int l = j & 63;
    float qr[2] = {q[l], q[l + 64]}, kr[2] = {k[l], k[l + 64]};
    const float vj = v[j];
    const float g_in = a.g[size_t(tok) * a.s_gb + h], b_in = a.beta[size_t(tok) * a.s_gb + h];
    const bool gated = a.gz && (a.flags & GEMVQ_GDN_GATED);
    const float zj = gated ? a.gz[(size_t(tok) * a.hv + h) * 128 + j] : 0.0f;
    // the gates (every thread alike): beta = sigmoid(b), g = softplus(alpha + dt) * a
    float beta = b_in, decay = g_in;
    if (a.flags & GEMVQ_GDN_GATES) {
        decay = cr::softplus(decay + a.dt[h]) * a.a[h];
        beta = cr::sigmoid(beta);
    }
    decay = cr::expf(decay);
    if (a.flags & GEMVQ_GDN_L2_QK) {
        // ggml_l2_norm of q and k, 1 / max(sqrt(sum of squares), eps): each double sum of squares formed across the
        // workgroup (thread j: element j) and checked against its rounding bound (the in-order sum where the bound
        // does not fix its FP32 rounding)
        const float xq = j < 64 ? qr[0] : qr[1], xk = j < 64 ? kr[0] : kr[1];
        const float sq = xq * xq, sk = xk * xk;
        const float s0 = 1.0f / fmaxf(sqrtf(ref_norm_reduce(double(sq), q, 128, 1, red)), a.l2_eps);
        const float s1 = 1.0f / fmaxf(sqrtf(ref_norm_reduce(double(sk), k, 128, 1, red)), a.l2_eps);
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            qr[w] = qr[w] * s0;
            kr[w] = kr[w] * s1;
        }
    }
    float dot = 0.0f;
#pragma unroll
    for (int i = 0; i < 128; ++i) {
        s[i] = s[i] * decay;
        dot += s[i] * lane_of(kr[i >> 6], i & 63);
    }
    const float delta = (vj - dot) * beta;
    float out = 0.0f;
#pragma unroll
    for (int i = 0; i < 128; ++i) {
        s[i] += lane_of(kr[i >> 6], i & 63) * delta;
        out += s[i] * lane_of(qr[i >> 6], i & 63);
    }
#pragma unroll
    for (int i = 0; i < 128; i += 4) *reinterpret_cast<float4 *>(dst + row + i) = make_float4(s[i], s[i + 1], s[i + 2], s[i + 3]);
    float yv = out * a.scale;
    if (gated) {
        // the gated output norm of this head (RMS_NORM -> MUL weight -> MUL SILU(z), ggml-xrt.cpp:1952-1975): the
        // double sum of the squares (formed across the workgroup, checked against its rounding bound), then
        // ((y * sc) * w) * silu(z)
        ys[j] = yv;
        const float y2 = yv * yv;
        const float sn = 1.0f / sqrtf(ref_norm_reduce(double(y2), ys, 128, 0, red) + a.rms_eps);
        yv = ((yv * sn) * a.gw[j]) * ((a.flags & GEMVQ_GDN_Z_SILU) ? zj : cr::silu(zj));
    }
    a.y[size_t(tok) * a.s_y + h * 128 + j] = yv;
}

// ---- attention, one token ----
// The token's position, and the cache it stores into and reads (its sequence's region with sequences).
struct AttnTok {
    int pos;
    uint16_t * kc;
    uint16_t * vc;
};
__device__ inline AttnTok attn_tok(const AttnArgs & a, int tok) {
    AttnTok t;
    t.pos = a.seq_ctx ? a.pos[16 * tok] : *a.pos + tok;
    const size_t ro = a.seq_ctx ? size_t(tok) * a.seq_ctx * a.n_head_kv * a.head_dim : 0;
    t.kc = a.kc + ro;
    t.vc = a.vc + ro;
    return t;
}

// Workgroup s < n_head: q head s, normalized (RMS, weight), rotated (NEOX) and rounded to fp16 into qr; the others:
// the new key of KV head s - n_head, normalized and rotated, and the value, stored as fp16 at the position.
__global__ __launch_bounds__(256) void attn_ref_append_kernel(AttnArgs a, int tok) {
    __shared__ float xs[256];
    __shared__ double red[4];
    const AttnTok t = attn_tok(a, tok);
    if (t.pos < 0 || t.pos >= a.n_ctx) return;  // positions past the KV capacity are not stored
    const int s = blockIdx.x, hd = a.head_dim, e = threadIdx.x, half = a.n_rot / 2;
    const bool isq = s < a.n_head;
    const int h = isq ? s : s - a.n_head;
    const float * x = isq ? a.q + size_t(tok) * a.n_head * a.q_stride + size_t(h) * a.q_stride
                          : a.k + (size_t(tok) * a.n_head_kv + h) * hd;
    // the row's double sum of squares formed across the workgroup and checked against its rounding bound (the
    // in-order sum where the bound does not fix the mean's rounding)
    const float xe = e < hd ? x[e] : 0.0f;
    const float sq = xe * xe;
    const float scs = 1.0f / sqrtf(ref_norm_reduce(double(sq), x, hd, 0, red) + a.eps);
    if (e < hd) xs[e] = (xe * scs) * (isq ? a.qn[e] : a.kn[e]);
    __syncthreads();
    if (e >= hd) return;
    const float * cs = a.cs + size_t(t.pos) * a.n_rot;
    const int pi = e < half ? e : e - half;
    float rv = xs[e];
    if (e < half) rv = xs[pi] * cs[2 * pi] - xs[pi + half] * cs[2 * pi + 1];
    else if (e < a.n_rot) rv = xs[pi] * cs[2 * pi + 1] + xs[pi + half] * cs[2 * pi];
    if (isq) {
        a.qr[size_t(h) * hd + e] = h2f(f2h(rv));
    } else {
        const size_t off = (size_t(t.pos) * a.n_head_kv + h) * hd + e;
        t.kc[off] = uint16_t(f2h(rv));
        t.vc[off] = uint16_t(f2h(a.v[(size_t(tok) * a.n_head_kv + h) * hd + e]));
    }
}

// Workgroup = q head, for the positions 0 .. pos:
// - scores: a thread per position, the F16 dot summed in double in index order (the products q * k are exact in
//   FP32); a thread keeps up to three positions' sums (256 apart) interleaved, its key rows read 32 halves at a time
//   with the next 32 requested before the current ones are summed;
// - the max, e^(s - max), their double sum and the fp16 probabilities;
// - values: thread d sums p * v[d] over the positions in order, the values staged in LDS in chunks of RA_CP
//   positions by LDS DMA (each wave requests its share of a chunk's rows at once, the workgroup waits for the chunk
//   once).
// The scores and probabilities sit in LDS up to RA_LDS positions, else in sp (n_ctx floats per q head of scratch).
constexpr int RA_LDS = 6144;
constexpr int RA_CP = 256;  // positions per staged chunk of values: RA_CP * 2 * head_dim bytes of dynamic LDS
// x times the fp16 value in the low (HI = 0) or high half of h, in one instruction (v_fma_mix_f32 with a zero
// addend). The product of an fp16 value and an fp16-valued float is exact in FP32 (22 significant bits, at least
// 2^-48), so for finite values this is the FP32 product h2f(half) * x, but for the sign of a zero product (+0 where
// the product is -0), which no double sum starting at +0 can tell apart.
template <int HI>
__device__ __forceinline__ float mul_f16(float x, uint32_t h) {
    float r;
    if constexpr (HI) asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(x), "v"(h));
    else asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[0,1,0]" : "=v"(r) : "v"(x), "v"(h));
    return r;
}

// The scores of positions p0 + 256 g (g < G; positions at or past n read row n - 1 and store nothing).
template <int HD, int G>
__device__ __forceinline__ void attn_ref_scores(const AttnArgs & a, const AttnTok & t, int kvh, int p0, int n,
                                                const float * qreg, float * sp, float & mx) {
    constexpr int NS = (HD + 31) / 32, NL = HD < 32 ? HD / 8 : 4;  // steps of 32 halves, 16-byte loads per step
    const uint4 * kr[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int p = min(p0 + 256 * g, n - 1);
        kr[g] = reinterpret_cast<const uint4 *>(t.kc + (size_t(p) * a.n_head_kv + kvh) * HD);
    }
    double acc[G];
    uint4 w[2][G][NL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        acc[g] = 0.0;
#pragma unroll
        for (int i = 0; i < NL; ++i) w[0][g][i] = kr[g][i];
    }
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        if (s + 1 < NS) {
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int i = 0; i < NL; ++i) w[(s + 1) & 1][g][i] = kr[g][4 * (s + 1) + i];
        }
#pragma unroll
        for (int i = 0; i < NL; ++i) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int d = 32 * s + 8 * i + j;
                const float qd = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qreg[d >> 6]), d & 63));
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const uint4 & x = w[s & 1][g][i];
                    const uint32_t u = (j >> 1) == 0 ? x.x : (j >> 1) == 1 ? x.y : (j >> 1) == 2 ? x.z : x.w;
                    const float pr = (j & 1) ? mul_f16<1>(qd, u) : mul_f16<0>(qd, u);  // q * k, exact
                    acc[g] += double(pr);
                }
            }
        }
        // this step's sums complete before the loads of the step after next are issued
#pragma unroll
        for (int g = 0; g < G; ++g) asm volatile("" : "+v"(acc[g])::"memory");
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int p = p0 + 256 * g;
        if (p < n) {
            const float sc = float(acc[g]) * a.scale;
            sp[p] = sc;
            mx = fmaxf(mx, sc);
        }
    }
}

// q head blockIdx.x over positions 0 .. n - 1, its scores and probabilities in sp
template <int HD>  // head_dim: a power of two from 16 to 256
__device__ __forceinline__ void attn_ref_head(const AttnArgs & a, int tok, const AttnTok & t, int n, float * sp) {
    __shared__ float qv[256], red[4];
    __shared__ double dred[4];
    constexpr int hd = HD;
    const int h = blockIdx.x, tid = threadIdx.x;
    const int kvh = h / (a.n_head / a.n_head_kv);
    if (tid < hd) qv[tid] = a.qr[size_t(h) * hd + tid];
    __syncthreads();
    // the query in registers, element d in lane d % 64 of word d / 64, read back as a scalar (readlane) at each step
    // of the in-order sums
    // (formed here, where every lane is active: readlane reads lanes that the sums may leave inactive)
    float qreg[(HD + 63) / 64];
#pragma unroll
    for (int k = 0; k < (HD + 63) / 64; ++k) {
        qreg[k] = (tid & 63) + 64 * k < hd ? qv[(tid & 63) + 64 * k] : 0.0f;
        asm volatile("" : "+v"(qreg[k]));
    }
    float mx = -__builtin_inff();
    const int rounds = (n + 255) / 256;
    int r = 0;
    for (; r + 3 <= rounds; r += 3) attn_ref_scores<HD, 3>(a, t, kvh, tid + 256 * r, n, qreg, sp, mx);
    if (rounds - r == 2) attn_ref_scores<HD, 2>(a, t, kvh, tid + 256 * r, n, qreg, sp, mx);
    else if (rounds - r == 1) attn_ref_scores<HD, 1>(a, t, kvh, tid + 256 * r, n, qreg, sp, mx);
#pragma unroll
    for (int st = 32; st >= 1; st >>= 1) mx = fmaxf(mx, __shfl_xor(mx, st, 64));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // e^(s - max) and their double sum, formed across the workgroup; the in-order sum fixes 1 / sum rounded to FP32
    // whenever the tree sum's error bound leaves that rounding open
    double pe = 0.0;
    for (int p = tid; p < n; p += 256) {
        const float e = cr::expf(sp[p] - mx);
        sp[p] = e;
        pe += double(e);
    }
    const double ts = ref_block_sum(pe, dred);  // also the barrier after every e is stored
    const double es = double(n + 64) * 2.220446049250313080847e-16 * ts;
    const float ilo = float(1.0 / (ts + es)), ihi = float(1.0 / (ts - es));
    float inv = ilo;
    if (!(ilo == ihi)) {  // the same on every thread
        __syncthreads();
        if (tid == 0) {
            double sum = 0.0;
            int p = 0;
            for (; p + 8 <= n; p += 8) {
                float e[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) e[i] = sp[p + i];
#pragma unroll
                for (int i = 0; i < 8; ++i) sum += double(e[i]);
            }
            for (; p < n; ++p) sum += double(sp[p]);
            dred[0] = sum;
        }
        __syncthreads();
        inv = float(1.0 / dred[0]);
    }
    for (int p = tid; p < n; p += 256) sp[p] = h2f(f2h(sp[p] * inv));
    // values: chunks of RA_CP positions staged in LDS as rows of head_dim halves (a 1 KiB DMA instruction holds
    // rpi = 512 / head_dim rows; lane l takes 16 bytes of row l / (head_dim / 8)); rows past pos read row pos
    extern __shared__ __attribute__((aligned(16))) uint16_t vst[];
    const unsigned vst_lds = unsigned(reinterpret_cast<uintptr_t>(vst));
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int lpr = hd / 8, rpi = 64 / lpr;  // lanes per row, rows per instruction
    double acc = 0.0;
    for (int c0 = 0; c0 < n; c0 += RA_CP) {
        const int cp = min(RA_CP, n - c0), ninst = (cp + rpi - 1) / rpi;
        __syncthreads();  // the probabilities are written, and the previous chunk's values are read
        for (int i = wave; i < ninst; i += 4) {
            const int r = min(c0 + i * rpi + lane / lpr, n - 1);
            const uint16_t * src = t.vc + (size_t(r) * a.n_head_kv + kvh) * hd + (lane % lpr) * 8;
            asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(vst_lds + unsigned(i) * 1024u),
                         "v"(src)
                         : "memory", "m0");
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid < hd) {
            // in position order, the next 16 positions' values and probabilities read from LDS while the current
            // 16 are added
            const uint16_t * vc = vst + tid;
            const float * pc = sp + c0;
            const int ng = cp / 16;
            uint16_t v0[16], v1[16];
            float p0[16], p1[16];
            const auto load = [&](int q0, uint16_t * v, float * pp) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    v[i] = vc[(q0 + i) * hd];
                    pp[i] = pc[q0 + i];
                }
            };
            const auto add = [&](const uint16_t * v, const float * pp) {
#pragma unroll
                for (int i = 0; i < 16; ++i) acc += double(mul_f16<0>(pp[i], v[i]));  // p * v, exact
                asm volatile("" : "+v"(acc)::"memory");  // these sums complete before the loads after them
            };
            if (ng > 0) load(0, v0, p0);
            for (int g = 0; g < ng; g += 2) {
                if (g + 1 < ng) load(16 * (g + 1), v1, p1);
                add(v0, p0);
                if (g + 1 < ng) {
                    if (g + 2 < ng) load(16 * (g + 2), v0, p0);
                    add(v1, p1);
                }
            }
            for (int q = 16 * ng; q < cp; ++q) acc += double(h2f(vc[q * hd]) * pc[q]);
        }
    }
    if (tid >= hd) return;
    float o = float(acc);
    if (a.gate) o = cr::sigmoid(a.gate[size_t(tok) * a.n_head * a.q_stride + size_t(h) * 2 * hd + tid]) * o;
    a.y[(size_t(tok) * a.n_head + h) * hd + tid] = o;
}

template <int HD>
__global__ __launch_bounds__(256) void attn_ref_kernel(AttnArgs a, int tok) {
    __shared__ float spl[RA_LDS];
    const AttnTok t = attn_tok(a, tok);
    if (t.pos < 0 || t.pos >= a.n_ctx) return;
    const int n = t.pos + 1;
    // the scores in LDS (read and written by LDS instructions) or, past RA_LDS positions, in the head's scratch row
    if (n <= RA_LDS) attn_ref_head<HD>(a, tok, t, n, spl);
    else attn_ref_head<HD>(a, tok, t, n, a.part + size_t(blockIdx.x) * a.n_ctx);
}

// ---- exhaustive hash of the correctly rounded exp / log (block b: inputs b 2^20 .. b 2^20 + 2^20 - 1) ----
__global__ __launch_bounds__(256) void crmath_hash_kernel(int fn, unsigned long long * hashes) {
    __shared__ unsigned long long red[4];
    const uint32_t blk = blockIdx.x;
    unsigned long long h = 0;
    for (uint32_t i = threadIdx.x; i < (1u << 20); i += 256) {
        const float x = cr::bitsf((blk << 20) | i);
        const float y = fn == 0 ? cr::expf(x) : cr::logf(x);
        const uint32_t yb = y != y ? 0x7fc00000u : cr::fbits(y);
        h += (unsigned long long)yb * (2ull * i + 1ull);
    }
#pragma unroll
    for (int st = 32; st >= 1; st >>= 1) h += (unsigned long long)shfl_xor_i64((long long)h, st);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = h;
    __syncthreads();
    if (threadIdx.x == 0) hashes[blk] = red[0] + red[1] + red[2] + red[3];
}

}  // namespace

hipError_t launch_norm_ref(const NormArgs & a, hipStream_t s) {
    GQ_LAUNCH(norm_ref_kernel, dim3(a.rows), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_ew_ref(const EwArgs & a, hipStream_t s) {
    int grid = (a.n + 255) / 256;
    grid = grid < 1024 ? grid : 1024;
    GQ_LAUNCH(ew_ref_kernel, dim3(grid), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_conv_ref(const ConvArgs & a, int tok, hipStream_t s) {
    GQ_LAUNCH(conv_ref_kernel, dim3((a.ch + 255) / 256), dim3(256), 0, s, a, tok);
    return hipGetLastError();
}

hipError_t launch_gdn_ref(const GdnArgs & a, int tok, hipStream_t s) {
    GQ_LAUNCH(gdn_ref_kernel, dim3(a.hv), dim3(128), 0, s, a, tok);
    return hipGetLastError();
}


template <int HD>
hipError_t launch_attn_ref_hd(const AttnArgs & a, int tok, hipStream_t s) {
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&attn_ref_kernel<HD>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, RA_CP * 2 * HD);
    if (attr != hipSuccess) return attr;
    GQ_LAUNCH(attn_ref_kernel<HD>, dim3(a.n_head), dim3(256), size_t(RA_CP) * 2 * HD, s, a, tok);
    return hipGetLastError();
}

hipError_t launch_attn_ref(const AttnArgs & a, int tok, hipStream_t s) {
    if (a.head_dim > 256 || a.n_head % a.n_head_kv) return hipErrorInvalidValue;
    GQ_LAUNCH(attn_ref_append_kernel, dim3(a.n_head + a.n_head_kv), dim3(256), 0, s, a, tok);
    switch (a.head_dim) {
    case 16: return launch_attn_ref_hd<16>(a, tok, s);
    case 32: return launch_attn_ref_hd<32>(a, tok, s);
    case 64: return launch_attn_ref_hd<64>(a, tok, s);
    case 128: return launch_attn_ref_hd<128>(a, tok, s);
    case 256: return launch_attn_ref_hd<256>(a, tok, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_crmath_hash(int fn, unsigned long long * hashes, hipStream_t s) {
    hipLaunchKernelGGL(crmath_hash_kernel, dim3(4096), dim3(256), 0, s, fn, hashes);
    return hipGetLastError();
}

}  // namespace gq
