#pragma once
// Fused GEMV pass for gfx950 (the kernel templates; each gq_gemv_*.hip instantiates the weight types it serves) (the GEMV command and its groups and epilogs, fpga/src/gemvqc16.h:26-45).
//
// One workgroup of 4 waves. The prologue quantizes the activation once into LDS exactly as ggml does for the
// weight type (Q8_0 for Q4_0 / Q8_0, Q8_K for Q5_K / Q6_K), optionally folding a deferred RMS norm into the values
// it quantizes. Each wave then streams whole rows: lane l owns the units u = l + 64k of every row (a unit is one
// 32-weight block for Q4_0 / Q8_0, 64 weights for the K-quants) and keeps their activations in registers. Block
// dots are int8 v_dot4 sums; each block (super-block) term is exact and truncated to the fixed-point LSB 2^-40
// (the reference kernel's arithmetic, gemvqw_engine.h:352-445), so the int64 row sum does not depend on the lane
// or reduction order, and is rounded to FP32 once. Epilogs (SwiGLU pair, residual add, conv, argmax) run on the
// row result before it is stored.
#include "gq_device.h"
#include "gq_kernels.h"

namespace gq {
namespace {

constexpr int NT = 256;        // threads per workgroup
constexpr int NWAVES = NT / WAVE;
constexpr int MAXK = GEMV_MAXK;

struct Lds {
    int8_t xq[MAXK];           // quantized activation
    uint32_t info[MAXK / 32];  // Q8_0: fp16 scale | (sum of the block's quants) << 16; Q8_K: FP32 d bits per super-block
    int16_t bs[MAXK / 16];     // Q8_K bsums
    uint16_t s1[MAXK / 32];    // Q8_1: fp16 of (sum of the block's quants) * d, for Q4_1 weights
    float red[2 * NWAVES + 64];
    unsigned long long key[NWAVES];
};

// The fields the prologue's first loads need, passed as leading scalar kernel arguments (ahead of GemvArgs, which
// is read through the kernel argument segment) so that they can arrive in SGPRs with the wave instead of through a
// dependent scalar load before the activation can be requested.
struct GemvHot {
    const float * x;
    const float * norm_w;
    const float * gate_z;
    int cols;
    int xsrc;
};

// Pairwise tree over the workgroup's per-wave values (NWAVES, a power of two, consecutive).
__device__ __forceinline__ float wave_tree(const float * r) {
    float t[NWAVES];
#pragma unroll
    for (int i = 0; i < NWAVES; ++i) t[i] = r[i];
    return tree<NWAVES>(t);
}

// Canonical norm scale over n floats (pairwise tree of the squares; words of 16 floats per thread, NT words per
// round, rounds combined pairwise with zero padding).
__device__ float block_norm_scale(const float * x, int n, float eps, int l2, Lds & s) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nw = n / 16, rounds = (nw + NT - 1) / NT;  // n <= 16384: at most 4 rounds
    float rs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        if (g < rounds) {  // uniform over the workgroup
        const int w = g * NT + tid;
        float ws = 0.0f;
        if (w < nw) {
            const float4 * p = reinterpret_cast<const float4 *>(x + size_t(w) * 16);
            float sq[16];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 v = p[i];
                sq[4 * i] = v.x * v.x;
                sq[4 * i + 1] = v.y * v.y;
                sq[4 * i + 2] = v.z * v.z;
                sq[4 * i + 3] = v.w * v.w;
            }
            ws = tree<16>(sq);
        }
        ws = pair_sum_lanes<64>(ws);
        if (lane == 0) s.red[wave] = ws;
        __syncthreads();
        rs[g] = wave_tree(s.red);
        __syncthreads();
        }
    }
    // pairwise over the rounds; absent rounds are +0 and leave the tree's values unchanged
    const float sum = (rs[0] + rs[1]) + (rs[2] + rs[3]);
    return l2 ? 1.0f / fmaxf(sqrtf(sum), eps) : 1.0f / sqrtf(sum / float(n) + eps);
}

// Q8_0 of the activation (gemvq_ref.h:236-245) on half-blocks: thread t holds items t + 256 g (an item is 16
// consecutive floats; the two halves of a 32-block sit in adjacent lanes). The loads are issued by prologue_fetch
// before the first weight rows are requested, so they are not queued behind them; prologue_finish then folds the
// deferred norm or the gated output norm and quantizes into LDS.
template <int R, int XS>  // rounds of NT items the registers hold (cols <= 16 NT R); the prologue kind
struct XF {
    float v[R][16];
    float w[R <= 2 ? R : 1][16];  // NORM: the norm weight (the activation again without one); GATED: the gated
                                  // norm's weight (one head, item % 8)
    float z[XS == XS_GATED ? R : 1][16];  // GATED: the output gate
};

__device__ __forceinline__ void load16(const float * p, float * v) {
    const float4 * q = reinterpret_cast<const float4 *>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 t = q[i];
        v[4 * i] = t.x;
        v[4 * i + 1] = t.y;
        v[4 * i + 2] = t.z;
        v[4 * i + 3] = t.w;
    }
}

// Item index clamped into the vector (threads past the end load a valid item and store nothing).
__device__ __forceinline__ int item_of(int g, int n16) {
    const int i = int(threadIdx.x) + NT * g;
    return i < n16 ? i : n16 - 1;
}

// Every load is unconditional (an operand a source does not use is read from the activation itself), so the loads
// cannot be moved into the branches that use them, behind the weight loads.
template <int R, int XS>
__device__ __forceinline__ void prologue_fetch(const GemvHot & h, const GemvArgs & a, XF<R, XS> & f) {
    const int n16 = h.cols / 16;
    const bool normw = h.xsrc == XSRC_NORM && h.norm_w != nullptr;
#pragma unroll
    for (int g = 0; g < R; ++g) {
        const int i = item_of(g, n16);
        const float * xi = h.x + size_t(i) * 16;
        load16(xi, f.v[g]);
        if constexpr (XS == XS_GATED) {
            load16(h.gate_z + size_t(i) * 16, f.z[g]);
            load16(h.norm_w + size_t(i & 7) * 16, f.w[g]);
        } else if constexpr (R <= 2) {
            load16(normw ? h.norm_w + size_t(i) * 16 : xi, f.w[g]);
        }
    }
}

// Q8_0 of one 32-block held as two halves by lanes l and l ^ 1: d = amax / 127 over the block, q = round(v / d)
// (half away from zero), the block's quant sum, and for Q4_1 weights the Q8_1 s = fp16(sum * d).
// The arithmetic of one half-block (both lanes of the pair must run it): its 16 quants packed little-endian, the
// block's quant sum, and the block's FP32 d.
__device__ __forceinline__ float quantize_half_core(const float * v, uint32_t * packed, int & sum) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) amax = fmaxf(amax, fabsf(v[j]));
    amax = fmaxf(amax, dpp_f32<DPP_XOR1>(amax));
    const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t w = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // roundf (half away from zero) as y + copysign(0.5 - 2^-25, y) truncated: equal for every |y| <= 128,
            // and |y| <= 127 (1 + 2^-22) here
            const float y = v[4 * i + j] * id;
            const int q = int(y + copysignf(0.49999997f, y));
            sum += q;
            w |= (uint32_t(q) & 0xffu) << (8 * j);
        }
        packed[i] = w;
    }
    sum += __shfl_xor(sum, 1, WAVE);
    return d;
}

// Stores into the quants xq, the words info (fp16 d | quant sum << 16) and the Q8_1 s values s1 of one vector.
__device__ __forceinline__ void quantize_half(const float * v, int item, bool valid, int8_t * xq, uint32_t * info,
                                              uint16_t * s1) {
    uint32_t packed[4];
    int sum;
    const float d = quantize_half_core(v, packed, sum);
    if (valid) {
        *reinterpret_cast<uint4 *>(xq + size_t(item) * 16) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
        if ((item & 1) == 0) {
            info[item >> 1] = f2h(d) | (uint32_t(sum & 0xffff) << 16);
            s1[item >> 1] = uint16_t(f2h(float(sum) * d));  // ggml quantize_row_q8_1: s = fp16(sum * d), FP32 d
        }
    }
}
__device__ __forceinline__ void quantize_half(const float * v, int item, bool valid, Lds & s) {
    quantize_half(v, item, valid, s.xq, s.info, s.s1);
}

// Norm scale over the whole vector: tree over each item's 16 squares, pairwise over the 64 items of a wave, the 4
// waves of a round and the rounds (padded to a power of two with zeros): the canonical pairwise tree over n.
template <int R, int XS>
__device__ __forceinline__ float norm_scale_items(const GemvArgs & a, const XF<R, XS> & f, Lds & s) {
    const int n16 = a.cols / 16, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float r[R];
#pragma unroll
    for (int g = 0; g < R; ++g) {
        float sq[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) sq[j] = f.v[g][j] * f.v[g][j];
        r[g] = int(threadIdx.x) + NT * g < n16 ? tree<16>(sq) : 0.0f;
    }
    pair_sum_lanes_n<64, R>(r);
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < R; ++g) s.red[NWAVES * g + wave] = r[g];
    }
    __syncthreads();
    float rs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < R; ++g)
        rs[g] = wave_tree(s.red + NWAVES * g);
    const float sum = R == 1 ? rs[0] : R == 2 ? rs[0] + rs[1] : (rs[0] + rs[1]) + (rs[2] + rs[3]);
    return a.norm_l2 ? 1.0f / fmaxf(sqrtf(sum), a.norm_eps) : 1.0f / sqrtf(sum / float(a.cols) + a.norm_eps);
}

// Without the gated norm the three sources share one path: v = (x * scale) * w with scale and w exactly 1 where a
// source has no norm or no weight (x * 1 is x), so no branch separates the loads.
template <int R, int XS>
__device__ __forceinline__ void prologue_finish(const GemvArgs & a, XF<R, XS> & f, Lds & s) {
    const int n16 = a.cols / 16;
    if constexpr (XS == XS_GATED) {
        // the DeltaNet gated output norm (gemvqc_gdn.h:284-346): per head of 128 (8 items, 8 lanes), x =
        // silu(z) * ((y * sc) * w) with sc = 1 / sqrt(sum(y^2) / 128 + eps); workgroup 0 also stores x, which the
        // separate norm would have written
        float hs[R];
#pragma unroll
        for (int g = 0; g < R; ++g) {
            float sq[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) sq[j] = f.v[g][j] * f.v[g][j];
            hs[g] = tree<16>(sq);
        }
        pair_sum_lanes_n<8, R>(hs);
#pragma unroll
        for (int g = 0; g < R; ++g) {
            const float sc = 1.0f / sqrtf(hs[g] / 128.0f + a.norm_eps);
            float * v = f.v[g];
            if (a.gate_silu) {
#pragma unroll
                for (int j = 0; j < 16; ++j) v[j] = f.z[g][j] * ((v[j] * sc) * f.w[g][j]);
            } else {
#pragma unroll
                for (int j = 0; j < 16; ++j) v[j] = silu_(f.z[g][j]) * ((v[j] * sc) * f.w[g][j]);
            }
            const int i = int(threadIdx.x) + NT * g;
            if (blockIdx.x == 0 && i < n16) {
                float4 * o = reinterpret_cast<float4 *>(a.x_out + size_t(i) * 16);
#pragma unroll
                for (int k = 0; k < 4; ++k) o[k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
            }
            quantize_half(v, i, i < n16, s);
        }
    } else {
        const bool norm = a.xsrc == XSRC_NORM, normw = norm && a.norm_w != nullptr;
        const float sc = norm ? norm_scale_items<R, XS>(a, f, s) : 1.0f;  // the same on every thread
#pragma unroll
        for (int g = 0; g < R; ++g) {
            const int i = int(threadIdx.x) + NT * g;
            float * v = f.v[g];
            if constexpr (R <= 2) {
#pragma unroll
                for (int j = 0; j < 16; ++j) v[j] = (v[j] * sc) * (normw ? f.w[g][j] : 1.0f);
            } else if (normw) {  // wide vectors: the weight is read now (registers hold only the activation)
                float w[16];
                load16(a.norm_w + size_t(item_of(g, n16)) * 16, w);
#pragma unroll
                for (int j = 0; j < 16; ++j) v[j] = (v[j] * sc) * w[j];
            } else {
#pragma unroll
                for (int j = 0; j < 16; ++j) v[j] = v[j] * sc;
            }
            quantize_half(v, i, i < n16, s);
        }
    }
}

// Q8_K of the activation (gemvq_ref.h:62-81): one wave per 256-block, 4 values per lane; the signed value of the
// largest magnitude at the first index; bsums per 16.
// x: cols floats; with norm, v = (x * scale) * w (w = norm_w, or 1 without one) before quantizing. Writes the quants
// xq, the bsums bs and the FP32 d bits info of each super-block.
__device__ void quantize_q8_K(const float * x, int cols, bool norm, const float * norm_w, float scale, int8_t * xq,
                              int16_t * bs, uint32_t * info) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nsb = cols / 256;
    for (int sb = wave; sb < nsb; sb += NWAVES) {
        const int base = sb * 256 + lane * 4;
        const float4 t = *reinterpret_cast<const float4 *>(x + base);
        float v[4] = {t.x, t.y, t.z, t.w};
        if (norm) {
            if (norm_w) {
                const float4 w = *reinterpret_cast<const float4 *>(norm_w + base);
                v[0] = (v[0] * scale) * w.x;
                v[1] = (v[1] * scale) * w.y;
                v[2] = (v[2] * scale) * w.z;
                v[3] = (v[3] * scale) * w.w;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = v[j] * scale;
            }
        }
        float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
        for (int st = 32; st >= 1; st >>= 1) amax = fmaxf(amax, __shfl_xor(amax, st, WAVE));
        int cand = 1 << 20;
#pragma unroll
        for (int j = 3; j >= 0; --j)
            if (fabsf(v[j]) == amax) cand = lane * 4 + j;
#pragma unroll
        for (int st = 32; st >= 1; st >>= 1) cand = min(cand, __shfl_xor(cand, st, WAVE));
        float vmax = 0.0f;
        {
            const int src = (cand >> 2) & 63, j = cand & 3;
            const float c0 = __shfl(v[0], src, WAVE), c1 = __shfl(v[1], src, WAVE), c2 = __shfl(v[2], src, WAVE),
                        c3 = __shfl(v[3], src, WAVE);
            vmax = j == 0 ? c0 : j == 1 ? c1 : j == 2 ? c2 : c3;
        }
        uint32_t packed = 0;
        int part = 0;
        float d = 0.0f;
        if (amax != 0.0f) {
            const float iscale = -127.0f / vmax;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float biased = iscale * v[j] + 12582912.0f;
                int q = int(__float_as_uint(biased) & 0x007fffffu) - 0x00400000;
                q = q < 127 ? q : 127;
                part += q;
                packed |= (uint32_t(q) & 0xffu) << (8 * j);
            }
            d = 1.0f / iscale;
        }
        *reinterpret_cast<uint32_t *>(xq + base) = packed;
        part += __shfl_xor(part, 1, WAVE);
        part += __shfl_xor(part, 2, WAVE);
        if ((lane & 3) == 0) bs[sb * 16 + (lane >> 2)] = int16_t(part);
        if (lane == 0) info[sb] = __float_as_uint(d);
    }
}

// ---- per-lane activation slices ----
struct XB {  // one 32-block (Q4_0 / Q4_1 / Q8_0)
    uint32_t q[8];
    float dx40;  // the block's fp16 scale times 2^40 (exact)
    int sum;     // sum of its quants (for the Q4_0 offset of 8)
    float sx40;  // Q4_1: the block's fp16 s (Q8_1) times 2^40 (exact)
};
struct XK {  // one 64-weight unit (Q5_K / Q6_K)
    uint32_t q[16];
    int bs[4];
    int m, e, neg;
};

// Lanes past the last block hold a zero block (zero quants and scales), whose terms are exactly zero.
template <int TYPE>
__device__ __forceinline__ void load_xb(const int8_t * xq, const uint32_t * info, const uint16_t * s1, int b, int nb,
                                        XB & x) {
    const bool in = b < nb;
    b = in ? b : nb - 1;
    const uint4 * p = reinterpret_cast<const uint4 *>(xq + size_t(b) * 32);
    const uint4 lo = p[0], hi = p[1];
    x.q[0] = lo.x; x.q[1] = lo.y; x.q[2] = lo.z; x.q[3] = lo.w;
    x.q[4] = hi.x; x.q[5] = hi.y; x.q[6] = hi.z; x.q[7] = hi.w;
#pragma unroll
    for (int i = 0; i < 8; ++i) x.q[i] = in ? x.q[i] : 0u;
    const uint32_t inf = in ? info[b] : 0u;
    x.dx40 = h2f(inf & 0xffffu) * 1099511627776.0f;  // * 2^40
    x.sum = int(int16_t(inf >> 16));
    x.sx40 = TYPE == T_Q4_1 && in ? h2f(s1[b]) * 1099511627776.0f : 0.0f;
}
template <int TYPE>
__device__ __forceinline__ void load_xb(const Lds & s, int b, int nb, XB & x) {
    load_xb<TYPE>(s.xq, s.info, s.s1, b, nb, x);
}

template <int TYPE>
__device__ __forceinline__ void load_xk(const int8_t * xq, const int16_t * bsv, const uint32_t * info, int u, int nu,
                                        XK & x) {
    u = u < nu ? u : nu - 1;
    const int sb = u >> 2, part = u & 3;
    int off0, off1, g0, g1;
    if (TYPE == T_Q6_K) {
        const int n = part >> 1, p = part & 1;
        off0 = sb * 256 + 128 * n + 32 * p;
        off1 = off0 + 64;
        g0 = (128 * n + 32 * p) / 16;
        g1 = g0 + 4;
    } else {
        off0 = sb * 256 + 64 * part;
        off1 = off0 + 32;
        g0 = (64 * part) / 16;
        g1 = g0 + 2;
    }
    const uint4 * p0 = reinterpret_cast<const uint4 *>(xq + off0);
    const uint4 * p1 = reinterpret_cast<const uint4 *>(xq + off1);
    const uint4 a0 = p0[0], a1 = p0[1], b0 = p1[0], b1 = p1[1];
    x.q[0] = a0.x; x.q[1] = a0.y; x.q[2] = a0.z; x.q[3] = a0.w;
    x.q[4] = a1.x; x.q[5] = a1.y; x.q[6] = a1.z; x.q[7] = a1.w;
    x.q[8] = b0.x; x.q[9] = b0.y; x.q[10] = b0.z; x.q[11] = b0.w;
    x.q[12] = b1.x; x.q[13] = b1.y; x.q[14] = b1.z; x.q[15] = b1.w;
    x.bs[0] = bsv[sb * 16 + g0];
    x.bs[1] = bsv[sb * 16 + g0 + 1];
    x.bs[2] = bsv[sb * 16 + g1];
    x.bs[3] = bsv[sb * 16 + g1 + 1];
    const float d = __uint_as_float(info[sb]);
    float_parts(d, x.m, x.e);
    x.neg = d < 0.0f;
}
template <int TYPE>
__device__ __forceinline__ void load_xk(const Lds & s, int u, int nu, XK & x) {
    load_xk<TYPE>(s.xq, s.bs, s.info, u, nu, x);
}

// ---- weight loads and unit dots ----
struct WB {  // one 32-block: Q4_0 / Q4_1 use lo (16 quant bytes), Q8_0 lo and hi (32 quant bytes)
    uint4 lo, hi;
    uint32_t d;  // fp16 d (Q4_1: d | m << 16)
};
struct WK {  // one 64-weight K-quant unit
    uint4 a0, a1;         // Q6_K ql bytes / Q5_K qs bytes of the unit
    uint4 h0, h1;         // high-bit bytes
    uint32_t s0, s1, s2;  // Q6_K: scale byte pairs of groups A and B; Q5_K: the 12 packed scale bytes
    uint32_t d;           // Q6_K: d; Q5_K: d | dmin << 16
};

// Weight loads are non-temporal: each byte is read once per token, so the stream should not displace what L2 holds
// for reuse (activations, states, the KV cache).
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld16(const uint8_t * p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t ld2(const uint8_t * p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint16_t *>(p));
}
__device__ __forceinline__ uint32_t ld4(const uint8_t * p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p));
}

template <int TYPE>
__device__ __forceinline__ void load_wb(const WeightView & w, size_t idx, WB & o) {
    o.lo = ld16(w.a + idx * 16);
    if (TYPE == T_Q4_0) {
        o.d = ld2(w.b + idx * 2);
    } else if (TYPE == T_Q4_1) {
        o.d = ld4(w.b + idx * 4);
    } else {
        o.hi = ld16(w.b + idx * 16);
        o.d = ld2(w.c + idx * 2);
    }
}

// Integer block sum (gemvq_ref.h:250-257, 218-220): Q4_0 (nibble - 8), Q4_1 (nibble) or Q8_0 weights times the
// Q8_0 / Q8_1 activation block.
template <int TYPE>
__device__ __forceinline__ int dot_block(const WB & w, const XB & x) {
    int s = 0;
    if (TYPE == T_Q4_1) {
        const uint32_t q[4] = {w.lo.x, w.lo.y, w.lo.z, w.lo.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) s = sdot4(q[i] & 0x0F0F0F0Fu, x.q[i], s);
#pragma unroll
        for (int i = 0; i < 4; ++i) s = sdot4((q[i] >> 4) & 0x0F0F0F0Fu, x.q[4 + i], s);
    } else if (TYPE == T_Q4_0) {
        const uint32_t q[4] = {w.lo.x, w.lo.y, w.lo.z, w.lo.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) s = sdot4(q[i] & 0x0F0F0F0Fu, x.q[i], s);
#pragma unroll
        for (int i = 0; i < 4; ++i) s = sdot4((q[i] >> 4) & 0x0F0F0F0Fu, x.q[4 + i], s);
        s -= 8 * x.sum;
    } else {
        const uint32_t q[8] = {w.lo.x, w.lo.y, w.lo.z, w.lo.w, w.hi.x, w.hi.y, w.hi.z, w.hi.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) s = sdot4(q[i], x.q[i], s);
    }
    return s;
}

// floor(sumi * dw * dx * 2^40) (gemvqw_engine.h:417-427) as an integer-valued double: dw * dx * 2^40 is exact in
// FP32 (two 11-bit significands), its product with the 20-bit sumi exact in FP64, floor exact.
template <int TYPE>
__device__ __forceinline__ double block_term(int sumi, uint32_t dw, const XB & x) {
    const float s = float(__builtin_bit_cast(_Float16, uint16_t(dw))) * x.dx40;  // exact conversion
    const double t = floor(double(sumi) * double(s));
    if (TYPE != T_Q4_1) return t;
    // Q4_1: + floor(m * s_x * 2^40), the product of two fp16 values exact in FP32
    const float ms = float(__builtin_bit_cast(_Float16, uint16_t(dw >> 16))) * x.sx40;
    return t + floor(double(ms));
}

template <int TYPE>
__device__ __forceinline__ void load_wk(const WeightView & w, size_t sbi, int part, WK & o) {
    if (TYPE == T_Q6_K) {  // the unit's ql bytes, its own 16 high-bit bytes and 4 scale bytes (the repacked layout)
        const int n = part >> 1, p = part & 1;
        const uint8_t * ql = w.a + sbi * 128 + 64 * n + 32 * p;
        o.a0 = ld16(ql);
        o.a1 = ld16(ql + 16);
        o.h0 = ld16(w.b + sbi * 64 + 16 * part);
        o.h1 = o.h0;
        o.s0 = ld4(w.c + sbi * 16 + 4 * part);
        o.s1 = o.s2 = 0;
        o.d = ld2(w.d + sbi * 2);
    } else {
        const uint8_t * qs = w.a + sbi * 128 + 32 * part;
        const uint8_t * qh = w.b + sbi * 32;
        o.a0 = ld16(qs);
        o.a1 = ld16(qs + 16);
        o.h0 = ld16(qh);
        o.h1 = ld16(qh + 16);
        const uint4 meta = ld16(w.c + sbi * 16);
        o.d = meta.x;
        o.s0 = meta.y;
        o.s1 = meta.z;
        o.s2 = meta.w;
    }
}

__device__ __forceinline__ uint32_t pick(const uint4 & v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Scale bytes of a Q5_K super-block (6-bit scale and min of sub-block j, gemvq_ref.h:84-92).
__device__ __forceinline__ int sbyte(const WK & w, int i) {
    const uint32_t v = i < 4 ? w.s0 : i < 8 ? w.s1 : w.s2;
    return int((v >> (8 * (i & 3))) & 0xffu);
}
__device__ __forceinline__ void scale_min_k4(const WK & w, int j, int & sc, int & m) {
    if (j < 4) {
        sc = sbyte(w, j) & 63;
        m = sbyte(w, j + 4) & 63;
    } else {
        sc = (sbyte(w, j + 4) & 0xF) | ((sbyte(w, j - 4) >> 6) << 4);
        m = (sbyte(w, j + 4) >> 4) | ((sbyte(w, j) >> 6) << 4);
    }
}

// Integer sums of one unit: S = sum sc * (q . q8), M = sum m * bsum (gemvq_ref.h:95-192).
template <int TYPE>
__device__ __forceinline__ void dot_unit(const WK & w, const XK & x, int part, int & S, int & M) {
    if (TYPE == T_Q6_K) {
        int dA0 = 0, dA1 = 0, dB0 = 0, dB1 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            // quants 4i .. 4i + 3 of the unit's groups: low nibbles from ql word i, high bits from word i & 3 of its
            // high-bit bytes (group A at bit 2 (i >> 2) of each byte, group B 4 bits above)
            const uint32_t ql = pick(i < 4 ? w.a0 : w.a1, i & 3), qh = pick(w.h0, i & 3);
            const int sh = 2 * (i >> 2);
            const uint32_t qa = (ql & 0x0F0F0F0Fu) | (((qh >> sh) & 0x03030303u) << 4);
            const uint32_t qb = ((ql >> 4) & 0x0F0F0F0Fu) | (((qh >> (sh + 4)) & 0x03030303u) << 4);
            if (i < 4) {
                dA0 = sdot4(qa, x.q[i], dA0);
                dB0 = sdot4(qb, x.q[8 + i], dB0);
            } else {
                dA1 = sdot4(qa, x.q[i], dA1);
                dB1 = sdot4(qb, x.q[8 + i], dB1);
            }
        }
        const int scA0 = int(int8_t(w.s0 & 0xff)), scA1 = int(int8_t((w.s0 >> 8) & 0xff));
        const int scB0 = int(int8_t((w.s0 >> 16) & 0xff)), scB1 = int(int8_t(w.s0 >> 24));
        S = scA0 * (dA0 - 32 * x.bs[0]) + scA1 * (dA1 - 32 * x.bs[1]) + scB0 * (dB0 - 32 * x.bs[2]) +
            scB1 * (dB1 - 32 * x.bs[3]);
        M = 0;
    } else {
        const int j = part;
        int d0 = 0, d1 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t qs = pick(i < 4 ? w.a0 : w.a1, i & 3), qh = pick(i < 4 ? w.h0 : w.h1, i & 3);
            const uint32_t q0 = (qs & 0x0F0F0F0Fu) | (((qh >> (2 * j)) & 0x01010101u) << 4);
            const uint32_t q1 = ((qs >> 4) & 0x0F0F0F0Fu) | (((qh >> (2 * j + 1)) & 0x01010101u) << 4);
            d0 = sdot4(q0, x.q[i], d0);
            d1 = sdot4(q1, x.q[8 + i], d1);
        }
        int sc0, m0, sc1, m1;
        scale_min_k4(w, 2 * j, sc0, m0);
        scale_min_k4(w, 2 * j + 1, sc1, m1);
        S = sc0 * d0 + sc1 * d1;
        M = m0 * (x.bs[0] + x.bs[1]) + m1 * (x.bs[2] + x.bs[3]);
    }
}

// floor(S * d * dx * 2^40) - floor(M * dmin * dx * 2^40) (gemvqw_engine.h:429-444), exact in int64 (the FP32 dx
// has a 24-bit significand, so these products do not fit a double).
template <int TYPE>
__device__ __forceinline__ long long superblock_term(int S, int M, const WK & w, const XK & x) {
    int md, ed;
    half_parts(w.d & 0xffffu, md, ed);
    const int negs = int((w.d >> 15) & 1) ^ x.neg;
    const long long ps = (long long)(negs ? -S : S) * ((long long)md * (long long)x.m);
    long long t = fixed_term(ps, ed + x.e);
    if (TYPE == T_Q5_K) {
        int mm, em;
        half_parts(w.d >> 16, mm, em);
        const int negm = int((w.d >> 31) & 1) ^ x.neg;
        const long long pm = (long long)(negm ? -M : M) * ((long long)mm * (long long)x.m);
        t -= fixed_term(pm, em + x.e);
    }
    return t;
}

// ---- rows: a wave owns a range of rows of one member and keeps D of them in flight ----
// Per-row register cost decides D (1 to 4): the weight slots of D rows stay near 64 VGPRs.
template <int TYPE, int NU, bool PAIR>
constexpr int slots() {
    const int per = (TYPE == T_Q5_K || TYPE == T_Q6_K ? 20 : TYPE == T_Q8_0 ? 9 : 5) * NU * (PAIR ? 2 : 1);
    const int d = 64 / per;
    return d < 1 ? 1 : d > 4 ? 4 : d;
}

template <int TYPE, int NU, bool PAIR>
struct Slot {  // one row in flight
    static constexpr bool KQ = TYPE == T_Q5_K || TYPE == T_Q6_K;
    WB wb[KQ ? 1 : NU], wb2[(KQ || !PAIR) ? 1 : NU];  // g (or the matrix) and u of a SwiGLU pair
    WK wk[KQ ? NU : 1], wk2[(KQ && PAIR) ? NU : 1];
    float e;  // epilog operands: ADD residual (every lane); CONV: lanes 0-2 the state, lanes 3-6 the kernel
};

// Loads of row r: the same code for every epilog kind, so that no branch surrounds a load (a load behind a branch
// makes the waits after the branch count it conservatively). The second matrix of a pair kernel is the member's own
// matrix for members that are not SwiGLU, and the epilog operand address (ea/eb, set at launch) falls back to the
// row's output for kinds without one.
template <int TYPE, int NU, bool PAIR>
__device__ __forceinline__ void load_slot(const GemvMember & m, int r, int lane, int nb, int nu, Slot<TYPE, NU, PAIR> & o) {
    if constexpr (Slot<TYPE, NU, PAIR>::KQ) {
        const int nsb = nu >> 2;
#pragma unroll
        for (int k = 0; k < NU; ++k) {
            const int u0 = lane + 64 * k, u = u0 < nu ? u0 : nu - 1;
            load_wk<TYPE>(m.w, size_t(r) * nsb + (u >> 2), u & 3, o.wk[k]);
            if constexpr (PAIR) load_wk<TYPE>(m.w2, size_t(r) * nsb + (u >> 2), u & 3, o.wk2[k]);
        }
    } else {
#pragma unroll
        for (int k = 0; k < NU; ++k) {
            const int b = lane + 64 * k, bb = b < nb ? b : nb - 1;
            load_wb<TYPE>(m.w, size_t(r) * nb + bb, o.wb[k]);
            if constexpr (PAIR) load_wb<TYPE>(m.w2, size_t(r) * nb + bb, o.wb2[k]);
        }
    }
    const int l = (lane < 7 ? lane : 6) * m.e_lane;
    const float * pa = m.ea + (size_t(r) * m.e_sa + l);
    const float * pb = m.eb + (size_t(r) * m.e_sb + (l - m.e_split));
    o.e = *(lane < m.e_split ? pa : pb);
}

// Per-lane partial of one row (its lane's units). The block terms are exact integers in FP64, summed in FP64 (exact
// while every partial stays below 2^53 LSB, |partial| < 8192 in output units), or with EXACT (a wave whose partials
// could pass that) each term t is split as t = 2^32 h + l (h = floor(t / 2^32), 0 <= l < 2^32, both exact) and the
// h and the l are summed in two FP64 accumulators, exact for NU <= 8 terms below 2^63 LSB. dbg (block sums for the
// tests) is written only for a row that exists.
template <int TYPE, int NU, bool EXACT>
__device__ __forceinline__ long long lane_blocks(const WB * wb, int r, bool valid, int nb, const XB * xb, int lane,
                                                 int32_t * dbg) {
    double acc = 0.0, hi = 0.0;
#pragma unroll
    for (int k = 0; k < NU; ++k) {
        const int b = lane + 64 * k;
        const int si = dot_block<TYPE>(wb[k], xb[k]);
        const double t = block_term<TYPE>(si, wb[k].d, xb[k]);  // units past the row's end hold a zero activation
        if constexpr (EXACT) {
            const double h = floor(t * 2.3283064365386963e-10);  // t / 2^32
            hi += h;
            acc += t - h * 4294967296.0;
        } else {
            acc += t;
        }
        if (dbg && valid && b < nb) dbg[size_t(r) * nb + b] = si;
    }
    if constexpr (EXACT) return (dint_to_i64(hi) << 32) + dint_to_i64(acc);
    return dint_to_i64(acc);
}

template <int TYPE, int NU>
__device__ __forceinline__ long long lane_units(const WK * wk, int r, bool valid, int nu, const XK * xk, int lane,
                                                int32_t * dbg) {
    const int nsb = nu >> 2;
    long long acc = 0;
#pragma unroll
    for (int k = 0; k < NU; ++k) {
        const int u = lane + 64 * k;
        int S = 0, M = 0;
        dot_unit<TYPE>(wk[k], xk[k], u & 3, S, M);
        if (u >= nu) S = M = 0;
        S = sum_lanes4_i32(S);
        M = sum_lanes4_i32(M);
        const long long t = superblock_term<TYPE>(S, M, wk[k], xk[k]);
        acc += (u < nu && (u & 3) == 0) ? t : 0;
        if (dbg && valid && u < nu && (u & 3) == 0) {
            const size_t i = (size_t(r) * nsb + (u >> 2)) * 2;
            dbg[i] = S;
            dbg[i + 1] = M;
        }
    }
    return acc;
}

struct Ctx {  // per-wave state shared by the row loops
    int lane, nb, nu;
    unsigned long long best;
    bool exact;  // wave-uniform: block terms are summed in int64 (a lane's FP64 partial could pass 2^53 LSB)
};

__device__ __forceinline__ float lane_value(float v, int j) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
}

template <int TYPE, int NU, bool PAIR, int EPI, bool EXACT = false>
__device__ __forceinline__ void lane_partials(const Slot<TYPE, NU, PAIR> & R, int r, bool valid, const XB * xb,
                                              const XK * xk, Ctx & c, int32_t * dbg, long long & p, long long & p2) {
    if constexpr (Slot<TYPE, NU, PAIR>::KQ) {
        p = lane_units<TYPE, NU>(R.wk, r, valid, c.nu, xk, c.lane, dbg);
        if constexpr (PAIR && EPI == EPI_SWIGLU) p2 = lane_units<TYPE, NU>(R.wk2, r, valid, c.nu, xk, c.lane, nullptr);
    } else {
        p = lane_blocks<TYPE, NU, EXACT>(R.wb, r, valid, c.nb, xb, c.lane, dbg);
        if constexpr (PAIR && EPI == EPI_SWIGLU) p2 = lane_blocks<TYPE, NU, EXACT>(R.wb2, r, valid, c.nb, xb, c.lane, nullptr);
    }
}

// The n (<= DS <= 4) rows base, base + stride, ... of a batch: the row totals are reduced together (lane group g holds
// row g), the epilog runs once for all of them on the groups' first lanes, which store; CONV, whose operands sit in
// lanes 0-6 of ev[j], is finished row by row on lane 0. ev holds the rows' epilog operands, taken from the slots
// before they were refilled.
template <int TYPE, int NU, bool PAIR, int EPI, int DS>
__device__ __forceinline__ void finish_chunk(const GemvMember & m, bool argmax, int base, int stride, int n,
                                             const long long * p, const long long * p2, const float * ev, Ctx & c) {

    constexpr int G = DS == 1 ? 1 : DS == 2 ? 2 : 4;
    constexpr int GW = 64 / G;
    long long pp[G], qq[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        pp[j] = j < DS ? p[j < DS ? j : 0] : 0;
        qq[j] = j < DS ? p2[j < DS ? j : 0] : 0;
    }
    const long long tot = reduce_rows<G>(pp);
    if constexpr (EPI == EPI_CONV) {
#pragma unroll
        for (int j = 0; j < DS; ++j) {
            if (j < n) {
                float e[7];
#pragma unroll
                for (int k = 0; k < 7; ++k) e[k] = lane_value(ev[j], k);
                const float v = fixed_to_float(readlane_i64(tot, j * GW));
                if (c.lane == 0) {  // gemvqc_ops.h:387-431 on the row result
                    const int r = base + j * stride;
                    float sum = 0.0f;
                    sum += e[0] * e[3];
                    sum += e[1] * e[4];
                    sum += e[2] * e[5];
                    sum += v * e[6];
                    m.y[r] = m.conv_silu ? silu_(sum) : sum;
                    m.conv_dst[3 * r] = e[1];
                    m.conv_dst[3 * r + 1] = e[2];
                    m.conv_dst[3 * r + 2] = v;
                }
            }
        }
    } else {
        const int g = c.lane / GW;
        const float v = fixed_to_float(tot);
        float out = v;
        if constexpr (PAIR && EPI == EPI_SWIGLU) {
            const long long tot2 = reduce_rows<G>(qq);
            out = (v / (1.0f + expf_(-v))) * fixed_to_float(tot2);  // gemvqc_ops.h:88-92
        } else if constexpr (EPI == EPI_ADD) {
            uint32_t eb = 0;  // the residual of row g (every lane of a slot holds its row's), gathered bitwise
#pragma unroll
            for (int j = 0; j < DS; ++j) eb |= (g == j ? 0xffffffffu : 0u) & __float_as_uint(ev[j]);
            out = v + __uint_as_float(eb);  // gemvqc16.cpp:282-301
        } else if constexpr (EPI == EPI_SILU) {
            out = silu_(v);  // gemvqc_ops.h:70-79 (UNARY SiLU) on the row result
        }
        if ((c.lane & (GW - 1)) == 0 && g < n) {
            const int r = base + g * stride;
            m.y[r] = out;
            if (argmax) {
                const unsigned long long key = argmax_key(out, uint32_t(r));
                c.best = key > c.best ? key : c.best;
            }
        }
    }
}

// Rows reduced and finished together: the partials of a batch of RB rows (RB/DS chunks of the DS rows in flight)
// are kept and go through one cross-lane reduction and one epilog, whose cost is then shared by RB rows even when
// fewer are in flight (finish_chunk takes at most 4 rows, and RB is a multiple of DS). Not for activations of more
// than 8192 columns (NU >= 5): their larger per-lane activation and the batch's partials together pass 256 VGPRs
// and halve the waves per SIMD.
template <int DS, int NU>
constexpr int batch_rows() { return DS >= 3 || NU >= 5 ? DS : 4; }

// The n rows w, w + S, w + 2 S, ... of one member (k-th row w + k S): slot j holds row k = kb + i for the chunk of
// rows i = ch DS + j of the batch starting at kb; a slot is refilled with the row DS further on as soon as its
// partial is formed (unconditionally while a full batch follows, so the compiler's waits stay exact), and each
// batch is reduced and finished once.
template <int TYPE, int NU, bool PAIR, int EPI, int DS>
__device__ __forceinline__ void run_rows(const GemvArgs & a, const GemvMember & m, int mi, int w, int S, int n,
                                         Slot<TYPE, NU, PAIR> * sl, const XB * xb, const XK * xk, Ctx & c) {
    constexpr int RB = batch_rows<DS, NU>(), CH = RB / DS;
    const bool argmax = EPI == EPI_PLAIN && a.argmax_key != nullptr && mi == 0;
    int32_t * dbg = mi == 0 ? a.dbg : nullptr;
    long long p[RB], p2[RB];
    float ev[RB];
    int kb = 0;
    for (; kb + RB < n; kb += RB) {  // full batches with rows after them
#pragma unroll
        for (int ch = 0; ch < CH; ++ch)
#pragma unroll
            for (int j = 0; j < DS; ++j) {
                const int i = ch * DS + j, k = kb + i;
                p2[i] = 0;
                lane_partials<TYPE, NU, PAIR, EPI>(sl[j], w + k * S, true, xb, xk, c, dbg, p[i], p2[i]);
                ev[i] = sl[j].e;
                load_slot<TYPE, NU, PAIR>(m, w + min(k + DS, n - 1) * S, c.lane, c.nb, c.nu, sl[j]);
            }
        finish_chunk<TYPE, NU, PAIR, EPI, RB>(m, argmax, w + kb * S, S, RB, p, p2, ev, c);
    }
    // the last batch (1 to RB rows): chunks past the last row are skipped, and a slot is refilled only for a chunk
    // that has rows
#pragma unroll
    for (int i = 0; i < RB; ++i) {
        p[i] = p2[i] = 0;
        ev[i] = 0.0f;
    }
#pragma unroll
    for (int ch = 0; ch < CH; ++ch) {
        if (ch > 0 && kb + ch * DS >= n) break;
#pragma unroll
        for (int j = 0; j < DS; ++j) {
            const int i = ch * DS + j, k = kb + i;
            lane_partials<TYPE, NU, PAIR, EPI>(sl[j], w + k * S, k < n, xb, xk, c, dbg, p[i], p2[i]);
            ev[i] = sl[j].e;
            if (ch + 1 < CH && kb + (ch + 1) * DS < n)
                load_slot<TYPE, NU, PAIR>(m, w + min(k + DS, n - 1) * S, c.lane, c.nb, c.nu, sl[j]);
        }
    }
    finish_chunk<TYPE, NU, PAIR, EPI, RB>(m, argmax, w + kb * S, S, min(RB, n - kb), p, p2, ev, c);
}

// The rows of a wave whose block terms could pass 2^53 LSB (see the kernel): one row at a time, each loaded, summed
// exactly and finished. Kept apart from the pipelined loop above, which it would otherwise slow.
template <int TYPE, int NU, bool PAIR, int EPI>
__device__ __forceinline__ void exact_rows(const GemvArgs & a, const GemvMember & m, int mi, int w, int S, int n,
                                        const XB * xb, Ctx & c) {
    const bool argmax = EPI == EPI_PLAIN && a.argmax_key != nullptr && mi == 0;
    int32_t * dbg = mi == 0 ? a.dbg : nullptr;
    for (int k = 0; k < n; ++k) {
        Slot<TYPE, NU, PAIR> sl;
        load_slot<TYPE, NU, PAIR>(m, w + k * S, c.lane, c.nb, c.nu, sl);
        long long p = 0, p2 = 0;
        lane_partials<TYPE, NU, PAIR, EPI, true>(sl, w + k * S, true, xb, nullptr, c, dbg, p, p2);
        const float ev = sl.e;
        finish_chunk<TYPE, NU, PAIR, EPI, 1>(m, argmax, w + k * S, S, 1, &p, &p2, &ev, c);
    }
}

// Waves are assigned to members in order: member i owns the global waves wave_begin .. wave_begin + waves - 1;
// waves past the last member only take part in the prologue.
template <int TYPE, int NU, bool PAIR, int XS, int DS>
__global__ __launch_bounds__(NT) void gemv_kernel(const float * x, const float * norm_w, const float * gate_z, int cols,
                                                  int xsrc, int n_members, int wb1, int wb2, int wb3, GemvArgs a) {
    __shared__ Lds s;
    constexpr bool KQ = TYPE == T_Q5_K || TYPE == T_Q6_K;
    // Leading scalar arguments: preloaded into SGPRs where the firmware supports it, so the activation loads and the
    // member choice wait for no load of the kernel argument segment.
    const GemvHot h{x, norm_w, gate_z, cols, xsrc};
    constexpr int RX = KQ ? 1 : (128 * NU + NT - 1) / NT;  // rounds of 16 NT activation floats (cols <= 2048 NU)
    XF<RX, XS> xf;
    if constexpr (!KQ) prologue_fetch<RX, XS>(h, a, xf);  // the activation is requested first
    __builtin_amdgcn_sched_barrier(0);                    // and stays ahead of the member lookup and weight loads
    Ctx c;
    c.lane = threadIdx.x & 63;
    c.nb = h.cols / 32;
    c.nu = h.cols / 64;
    c.best = 0;
    c.exact = false;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: member fields load as scalars
    // Workgroup b serves slice b % 8 of every member's rows (workgroups are dealt to the XCDs in turn, so a slice's
    // rows stream through one XCD's L2; placement only affects speed, never which rows run).
    const int xs = blockIdx.x & 7, lw = (blockIdx.x >> 3) * NWAVES + wave;  // slice, wave index within it
    // member i owns the waves from its wave_begin (wb1..wb3 = a.m[1..3].wave_begin)
    const int mi = n_members > 3 && lw >= wb3 ? 3 : n_members > 2 && lw >= wb2 ? 2 : n_members > 1 && lw >= wb1 ? 1 : 0;
    const GemvMember & m = a.m[mi];
    // The member fields that the first weight and epilog operand loads need, requested in one round of scalar loads
    // (left to itself the compiler waits for the row count before it requests the rest); later reads of the same
    // fields reuse these registers.
    asm volatile("" ::"s"(m.rows), "s"(m.wave_begin), "s"(m.waves), "s"(m.w.a), "s"(m.w.b), "s"(m.w.c), "s"(m.w2.a),
                 "s"(m.w2.b), "s"(m.w2.c), "s"(m.ea), "s"(m.eb), "s"(m.e_sa), "s"(m.e_sb), "s"(m.e_split),
                 "s"(m.e_lane));
    const int s_lo = int((long long)xs * m.rows / 8), len = int((long long)(xs + 1) * m.rows / 8) - s_lo;
    const int wv = lw - m.wave_begin, S = m.waves;  // rows s_lo + wv, s_lo + wv + S, ... of the slice
    // waves past the last member have none; computed without a branch, so that the member's remaining fields are
    // loaded in the same round as these
    const int q = int(unsigned(max(len - 1 - wv, 0)) / unsigned(max(S, 1)));
    const int n = wv < S && wv < len ? q + 1 : 0;
    const int w = s_lo + wv;
    Slot<TYPE, NU, PAIR> sl[DS];  // the first D rows (a wave without rows reloads the member's last row)
#pragma unroll
    for (int j = 0; j < DS; ++j)
        load_slot<TYPE, NU, PAIR>(m, n > 0 ? w + min(j, n - 1) * S : m.rows - 1, c.lane, c.nb, c.nu, sl[j]);
    if constexpr (KQ) {
        const float scale = h.xsrc == XSRC_NORM ? block_norm_scale(h.x, h.cols, a.norm_eps, a.norm_l2, s) : 1.0f;
        quantize_q8_K(h.x, h.cols, h.xsrc == XSRC_NORM, h.norm_w, scale, s.xq, s.bs, s.info);
    } else {
        prologue_finish<RX, XS>(a, xf, s);
    }
    __syncthreads();
    XB xb[KQ ? 1 : NU];
    XK xk[KQ ? NU : 1];
    if constexpr (KQ) {
#pragma unroll
        for (int k = 0; k < NU; ++k) load_xk<TYPE>(s, c.lane + 64 * k, c.nu, xk[k]);
    } else {
#pragma unroll
        for (int k = 0; k < NU; ++k) load_xb<TYPE>(s, c.lane + 64 * k, c.nb, xb[k]);
        // A lane adds its NU block terms in FP64, exact while every partial stays below 2^53 LSB. |term| <= wbound *
        // |d_x| * 2^40 (wbound: the matrix's largest |d_w| times the largest |sum of products| of its type, from the
        // upload), so while wbound * sum |d_x| * 2^40 < 2^52 over a lane's blocks (a factor 2 of margin for the FP32
        // bound) its FP64 sum is exact; a wave with a lane past that sums its terms in int64.
        float dsum = 0.0f;
#pragma unroll
        for (int k = 0; k < NU; ++k) dsum += fabsf(xb[k].dx40);
        c.exact = __builtin_amdgcn_ballot_w64(!(a.wbound[mi] * dsum < 4503599627370496.0f)) != 0;
    }
    if (n > 0 && (KQ || !c.exact)) {
        switch (m.epi) {
        case EPI_SWIGLU:
            if constexpr (PAIR) run_rows<TYPE, NU, PAIR, EPI_SWIGLU, DS>(a, m, mi, w, S, n, sl, xb, xk, c);
            break;
        case EPI_ADD: run_rows<TYPE, NU, PAIR, EPI_ADD, DS>(a, m, mi, w, S, n, sl, xb, xk, c); break;
        case EPI_CONV: run_rows<TYPE, NU, PAIR, EPI_CONV, DS>(a, m, mi, w, S, n, sl, xb, xk, c); break;
        case EPI_SILU: run_rows<TYPE, NU, PAIR, EPI_SILU, DS>(a, m, mi, w, S, n, sl, xb, xk, c); break;
        default: run_rows<TYPE, NU, PAIR, EPI_PLAIN, DS>(a, m, mi, w, S, n, sl, xb, xk, c); break;
        }
    } else if (n > 0) {
        if constexpr (!KQ) {
            switch (m.epi) {
            case EPI_SWIGLU:
                if constexpr (PAIR) exact_rows<TYPE, NU, PAIR, EPI_SWIGLU>(a, m, mi, w, S, n, xb, c);
                break;
            case EPI_ADD: exact_rows<TYPE, NU, PAIR, EPI_ADD>(a, m, mi, w, S, n, xb, c); break;
            case EPI_CONV: exact_rows<TYPE, NU, PAIR, EPI_CONV>(a, m, mi, w, S, n, xb, c); break;
            case EPI_SILU: exact_rows<TYPE, NU, PAIR, EPI_SILU>(a, m, mi, w, S, n, xb, c); break;
            default: exact_rows<TYPE, NU, PAIR, EPI_PLAIN>(a, m, mi, w, S, n, xb, c); break;
            }
        }
    }
    if (a.argmax_key) {
        unsigned long long best = c.best;  // held by the lane-group leaders
#pragma unroll
        for (int st = 1; st < 64; st <<= 1) {
            const unsigned long long o = (unsigned long long)shfl_xor_i64((long long)best, st);
            best = o > best ? o : best;
        }
        if (c.lane == 0) s.key[wave] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long b = s.key[0];
            for (int i = 1; i < NWAVES; ++i) b = s.key[i] > b ? s.key[i] : b;
            if (b) atomicMax(a.argmax_key, b);
        }
    }
}

// Workgroups of `kernel` that fit on the device at once (a grid beyond it runs a second, mostly idle round), at
// most `per_cu` per CU.
template <typename K>
int resident_blocks(K kernel, int per_cu = 1 << 20) {
    int dev = 0, cus = 0, occ = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, NT, 0) != hipSuccess || occ < 1 || cus < 1)
        return 1024;
    return (occ < per_cu ? occ : per_cu) * cus;
}

// Waves per CU a launch may use: every workgroup reads and quantizes the whole activation, so beyond twelve waves
// per CU the extra activation reads cost more than the extra rows in flight gain (measured on the decode layers'
// gate/up pairs and projection groups, about 1 us per launch).
constexpr int GEMV_WAVES_PER_CU = 12;
constexpr int GEMV_WG_PER_CU = GEMV_WAVES_PER_CU / NWAVES > 0 ? GEMV_WAVES_PER_CU / NWAVES : 1;
// Activations of more than 8192 columns (NU >= 5: the 12288-column FFN down projection): two workgroups per CU
// (measured: three cost 1.2 us more per launch, each workgroup reading and quantizing 48 KB).
constexpr int gemv_wg_per_cu(int nu) { return nu >= 5 && GEMV_WG_PER_CU > 2 ? 2 : GEMV_WG_PER_CU; }

// Every member's rows are split into 8 contiguous slices, one per XCD; the same member layout repeats on each XCD
// (workgroups b with b % 8 == x serve slice x). A member's waves per slice: enough for ds rows each when all fit
// on the device at once (every row is requested before the activation prologue ends); otherwise the resident waves,
// shared in proportion to the rows, stream them. A slice's rows are dealt to its waves in turn, so the rows in flight
// form one region of the slice.
template <typename Args>  // GemvArgs or TokArgs: n_members, m[i].rows, m[i].wave_begin, m[i].waves
int plan_waves(Args & a, int cap_blocks, int ds) {
    const int cap_x = cap_blocks / 8 < 1 ? 1 : cap_blocks / 8;  // workgroups per XCD
    int need = 0;
    for (int i = 0; i < a.n_members; ++i) need += ((a.m[i].rows + 7) / 8 + ds - 1) / ds;
    const bool fits = (need + NWAVES - 1) / NWAVES <= cap_x;
    const long long waves = (long long)cap_x * NWAVES;
    long long total = 0;
    for (int i = 0; i < a.n_members; ++i) total += a.m[i].rows;
    int w = 0;
    for (int i = 0; i < a.n_members; ++i) {
        const int per = (a.m[i].rows + 7) / 8;
        long long wi = fits ? (per + ds - 1) / ds : waves * a.m[i].rows / total;
        wi = wi < 1 ? 1 : wi > per ? per : wi;
        a.m[i].wave_begin = w;
        a.m[i].waves = int(wi);
        w += int(wi);
    }
    return 8 * ((w + NWAVES - 1) / NWAVES);
}

// Epilog operand addresses of a member: with l = min(lane, 6) * e_lane, lanes below e_split read ea[r * e_sa + l],
// the others eb[r * e_sb + l - e_split] (CONV: lanes 0-2 the state, lanes 3-6 the kernel; ADD: the residual).
void epilog_operands(GemvMember & m) {
    m.e_lane = 0;
    m.e_split = 64;
    m.e_sa = m.e_sb = 1;
    m.ea = m.eb = m.y;
    if (m.epi == EPI_ADD) {
        m.ea = m.eb = m.res;
    } else if (m.epi == EPI_CONV) {
        m.e_lane = 1;
        m.e_split = 3;
        m.ea = m.conv_src;
        m.e_sa = 3;
        m.eb = m.conv_w;
        m.e_sb = 4;
    }
    if (m.epi != EPI_SWIGLU) m.w2 = m.w;
}

template <int TYPE, int NU, bool PAIR, int XS, int DS>
hipError_t launch_typed(const GemvArgs & a0, hipStream_t st) {
    static const int cap = resident_blocks(gemv_kernel<TYPE, NU, PAIR, XS, DS>, gemv_wg_per_cu(NU));
    GemvArgs a = a0;
    for (int i = 0; i < a.n_members; ++i) epilog_operands(a.m[i]);
    const int grid = plan_waves(a, cap, DS);
    GQ_LAUNCH((gemv_kernel<TYPE, NU, PAIR, XS, DS>), dim3(grid), dim3(NT), 0, st, a.x, a.norm_w, a.gate_z, a.cols,
              a.xsrc, a.n_members, a.n_members > 1 ? a.m[1].wave_begin : 0, a.n_members > 2 ? a.m[2].wave_begin : 0,
              a.n_members > 3 ? a.m[3].wave_begin : 0, a);
    return hipGetLastError();
}

// Rows in flight per wave. A group that all fits in flight at once takes the most slots (its time is latency); a
// larger one takes as few as keep about 16 MB in flight over the resident waves (more in flight than that only
// queues, and streams slower).
template <int TYPE, int NU, bool PAIR, int XS>
hipError_t launch_slots(const GemvArgs & a, hipStream_t st) {
    constexpr int DMAX = slots<TYPE, NU, PAIR>();
    uint64_t rows = 0, bytes = 0;
    for (int i = 0; i < a.n_members; ++i) {
        rows += uint64_t(a.m[i].rows);
        bytes += uint64_t(a.m[i].rows) * gguf_row_bytes(TYPE, a.cols) * (a.m[i].epi == EPI_SWIGLU ? 2 : 1);
    }
    static const int cap_waves = resident_blocks(gemv_kernel<TYPE, NU, PAIR, XS, DMAX>) * NWAVES;
    const uint64_t per_slot = uint64_t(cap_waves) * (bytes / (rows ? rows : 1));  // bytes in flight per slot
    constexpr uint64_t target = uint64_t(16) << 20;
    int d = DMAX;
    if (bytes > target && per_slot * DMAX > target) d = per_slot * 2 <= target ? 2 : 1;
    if constexpr (DMAX > 2) {
        if (d == DMAX) return launch_typed<TYPE, NU, PAIR, XS, DMAX>(a, st);
    }
    if constexpr (DMAX >= 2) {
        if (d >= 2) return launch_typed<TYPE, NU, PAIR, XS, 2>(a, st);
    }
    return launch_typed<TYPE, NU, PAIR, XS, 1>(a, st);
}

// The gated activation prologue exists for Q4_0 / Q8_0 rows of at most 8192 columns without a SwiGLU pair.
template <int TYPE, int NU>
hipError_t launch_pair(const GemvArgs & a, hipStream_t st) {
    bool pair = false;
    for (int i = 0; i < a.n_members; ++i) pair = pair || a.m[i].epi == EPI_SWIGLU;
    if (a.xsrc == XSRC_GATED) {
        if constexpr ((TYPE == T_Q4_0 || TYPE == T_Q8_0) && NU <= 4) {
            if (!pair) return launch_slots<TYPE, NU, false, XS_GATED>(a, st);
        }
        return hipErrorInvalidValue;
    }
    return pair ? launch_slots<TYPE, NU, true, XS_PLAIN>(a, st) : launch_slots<TYPE, NU, false, XS_PLAIN>(a, st);
}

template <int TYPE>
hipError_t launch_nu(const GemvArgs & a, hipStream_t st) {
    constexpr bool KQ = TYPE == T_Q5_K || TYPE == T_Q6_K;
    const int nu = (a.cols / (KQ ? 64 : 32) + 63) / 64;  // cols <= 16384: K-quants nu <= 4, Q4_0 / Q8_0 nu <= 8
    switch (nu) {
    case 1: return launch_pair<TYPE, 1>(a, st);
    case 2: return launch_pair<TYPE, 2>(a, st);
    case 3: return launch_pair<TYPE, 3>(a, st);
    case 4: return launch_pair<TYPE, 4>(a, st);
    default: break;
    }
    if constexpr (!KQ) {
        switch (nu) {
        case 5: return launch_pair<TYPE, 5>(a, st);
        case 6: return launch_pair<TYPE, 6>(a, st);
        case 7: return launch_pair<TYPE, 7>(a, st);
        case 8: return launch_pair<TYPE, 8>(a, st);
        default: break;
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace
}  // namespace gq
