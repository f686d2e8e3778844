// Fused GEMV pass for gfx950 (the GEMV command and its groups and epilogs, fpga/src/gemvqc16.h:26-45).
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
constexpr int MAXK = 16384;

struct Lds {
    int8_t xq[MAXK];           // quantized activation
    uint32_t info[MAXK / 32];  // Q8_0: fp16 scale | (sum of the block's quants) << 16; Q8_K: FP32 d bits per super-block
    int16_t bs[MAXK / 16];     // Q8_K bsums
    uint16_t s1[MAXK / 32];    // Q8_1: fp16 of (sum of the block's quants) * d, for Q4_1 weights
    float red[2 * NWAVES + 64];
    unsigned long long key[NWAVES];
};

// Canonical norm scale over n floats (pairwise tree of the squares; words of 16 floats per thread, 256 words per
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
        rs[g] = (s.red[0] + s.red[1]) + (s.red[2] + s.red[3]);
        __syncthreads();
        }
    }
    // pairwise over the rounds; absent rounds are +0 and leave the tree's values unchanged
    const float sum = (rs[0] + rs[1]) + (rs[2] + rs[3]);
    return l2 ? 1.0f / fmaxf(sqrtf(sum), eps) : 1.0f / sqrtf(sum / float(n) + eps);
}

// Q8_0 of the activation (gemvq_ref.h:236-245), one thread per 32-block, rounds of 256 blocks. With a deferred
// norm the blocks stay in registers while the sum of squares is reduced: tree over the block's 32 squares, pairwise
// over the 64 blocks of a wave, the 4 waves of a round, and the rounds (at most 2 here: n <= 16384), which is the
// canonical pairwise tree over all n elements; then v = (x * scale) * w is quantized.
__device__ __forceinline__ void load_block(const float * p, float * v) {
    const float4 * q = reinterpret_cast<const float4 *>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 t = q[i];
        v[4 * i] = t.x;
        v[4 * i + 1] = t.y;
        v[4 * i + 2] = t.z;
        v[4 * i + 3] = t.w;
    }
}

__device__ __forceinline__ void quantize_block(const float * v, int b, Lds & s) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    uint32_t packed[8];
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t w = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int q = int(roundf(v[4 * i + j] * id));
            sum += q;
            w |= (uint32_t(q) & 0xffu) << (8 * j);
        }
        packed[i] = w;
    }
    uint4 * dst = reinterpret_cast<uint4 *>(s.xq + size_t(b) * 32);
    dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
    s.info[b] = f2h(d) | (uint32_t(sum & 0xffff) << 16);
    s.s1[b] = uint16_t(f2h(float(sum) * d));  // ggml quantize_row_q8_1: s = fp16(sum * d) with the FP32 d
}

// The DeltaNet gated output norm applied while quantizing (gemvqc_gdn.h:284-346): per head of 128, x =
// silu(z) * ((y * s) * w) with s = 1 / sqrt(sum(y^2) / 128 + eps), the sum the pairwise tree over the head (the
// tree over each 32-block, then over the head's 4 consecutive blocks, held by 4 aligned lanes). cols <= 8192 and a
// multiple of 128. Workgroup 0 also stores the gated values, which the separate norm would have written.
__device__ __forceinline__ void prologue_gated(const GemvArgs & a, Lds & s) {
    const int nb = a.cols / 32, b = threadIdx.x;
    if (b >= nb) return;  // whole groups of 4 lanes (nb is a multiple of 4)
    float v[32], z[32], w[32];
    load_block(a.x + size_t(b) * 32, v);
    load_block(a.gate_z + size_t(b) * 32, z);
    load_block(a.norm_w + size_t(b & 3) * 32, w);
    float sq[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) sq[j] = v[j] * v[j];
    const float sum = pair_sum_lanes<4>(tree<32>(sq));
    const float sc = 1.0f / sqrtf(sum / 128.0f + a.norm_eps);
    if (a.gate_silu) {
#pragma unroll
        for (int j = 0; j < 32; ++j) v[j] = z[j] * ((v[j] * sc) * w[j]);
    } else {
#pragma unroll
        for (int j = 0; j < 32; ++j) v[j] = silu_(z[j]) * ((v[j] * sc) * w[j]);
    }
    if (blockIdx.x == 0) {
        float4 * o = reinterpret_cast<float4 *>(a.x_out + size_t(b) * 32);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    }
    quantize_block(v, b, s);
}

template <int ROUNDS>  // rounds of 256 blocks the registers hold (cols <= 8192: 1)
__device__ void prologue_q8_0(const GemvArgs & a, Lds & s) {
    const int nb = a.cols / 32, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (a.xsrc == XSRC_GATED) {
        prologue_gated(a, s);
        return;
    }
    if (a.xsrc != XSRC_NORM) {
        for (int b = tid; b < nb; b += NT) {
            float v[32];
            load_block(a.x + size_t(b) * 32, v);
            quantize_block(v, b, s);
        }
        return;
    }
    float v0[32], v1[ROUNDS > 1 ? 32 : 1];
    const int b0 = tid, b1 = tid + NT;
    float r0 = 0.0f, r1 = 0.0f;
    {
        float sq[32];
        if (b0 < nb) {
            load_block(a.x + size_t(b0) * 32, v0);
#pragma unroll
            for (int j = 0; j < 32; ++j) sq[j] = v0[j] * v0[j];
        } else {
#pragma unroll
            for (int j = 0; j < 32; ++j) v0[j] = sq[j] = 0.0f;
        }
        r0 = pair_sum_lanes<64>(tree<32>(sq));
    }
    if constexpr (ROUNDS > 1) {
        float sq[32];
        if (b1 < nb) {
            load_block(a.x + size_t(b1) * 32, v1);
#pragma unroll
            for (int j = 0; j < 32; ++j) sq[j] = v1[j] * v1[j];
        } else {
#pragma unroll
            for (int j = 0; j < 32; ++j) v1[j] = sq[j] = 0.0f;
        }
        r1 = pair_sum_lanes<64>(tree<32>(sq));
    }
    if (lane == 0) {
        s.red[wave] = r0;
        s.red[4 + wave] = r1;
    }
    __syncthreads();
    const float sum = ((s.red[0] + s.red[1]) + (s.red[2] + s.red[3])) + ((s.red[4] + s.red[5]) + (s.red[6] + s.red[7]));
    const float scale = a.norm_l2 ? 1.0f / fmaxf(sqrtf(sum), a.norm_eps) : 1.0f / sqrtf(sum / float(a.cols) + a.norm_eps);
    if (b0 < nb) {
        if (a.norm_w) {
            float w[32];
            load_block(a.norm_w + size_t(b0) * 32, w);
#pragma unroll
            for (int j = 0; j < 32; ++j) v0[j] = (v0[j] * scale) * w[j];
        } else {
#pragma unroll
            for (int j = 0; j < 32; ++j) v0[j] = v0[j] * scale;
        }
        quantize_block(v0, b0, s);
    }
    if constexpr (ROUNDS > 1) {
      if (b1 < nb) {
        if (a.norm_w) {
            float w[32];
            load_block(a.norm_w + size_t(b1) * 32, w);
#pragma unroll
            for (int j = 0; j < 32; ++j) v1[j] = (v1[j] * scale) * w[j];
        } else {
#pragma unroll
            for (int j = 0; j < 32; ++j) v1[j] = v1[j] * scale;
        }
        quantize_block(v1, b1, s);
      }
    }
}

// Q8_K of the activation (gemvq_ref.h:62-81): one wave per 256-block, 4 values per lane; the signed value of the
// largest magnitude at the first index; bsums per 16.
__device__ void quantize_q8_K(const GemvArgs & a, float scale, Lds & s) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nsb = a.cols / 256;
    for (int sb = wave; sb < nsb; sb += NWAVES) {
        const int base = sb * 256 + lane * 4;
        const float4 t = *reinterpret_cast<const float4 *>(a.x + base);
        float v[4] = {t.x, t.y, t.z, t.w};
        if (a.xsrc == XSRC_NORM) {
            if (a.norm_w) {
                const float4 w = *reinterpret_cast<const float4 *>(a.norm_w + base);
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
        *reinterpret_cast<uint32_t *>(s.xq + base) = packed;
        part += __shfl_xor(part, 1, WAVE);
        part += __shfl_xor(part, 2, WAVE);
        if ((lane & 3) == 0) s.bs[sb * 16 + (lane >> 2)] = int16_t(part);
        if (lane == 0) s.info[sb] = __float_as_uint(d);
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

// Lanes past the last unit load a valid unit (their terms are never added).
template <int TYPE>
__device__ __forceinline__ void load_xb(const Lds & s, int b, int nb, XB & x) {
    b = b < nb ? b : nb - 1;
    const uint4 * p = reinterpret_cast<const uint4 *>(s.xq + size_t(b) * 32);
    const uint4 lo = p[0], hi = p[1];
    x.q[0] = lo.x; x.q[1] = lo.y; x.q[2] = lo.z; x.q[3] = lo.w;
    x.q[4] = hi.x; x.q[5] = hi.y; x.q[6] = hi.z; x.q[7] = hi.w;
    const uint32_t inf = s.info[b];
    x.dx40 = h2f(inf & 0xffffu) * 1099511627776.0f;  // * 2^40
    x.sum = int(int16_t(inf >> 16));
    x.sx40 = TYPE == T_Q4_1 ? h2f(s.s1[b]) * 1099511627776.0f : 0.0f;
}

template <int TYPE>
__device__ __forceinline__ void load_xk(const Lds & s, int u, int nu, XK & x) {
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
    const uint4 * p0 = reinterpret_cast<const uint4 *>(s.xq + off0);
    const uint4 * p1 = reinterpret_cast<const uint4 *>(s.xq + off1);
    const uint4 a0 = p0[0], a1 = p0[1], b0 = p1[0], b1 = p1[1];
    x.q[0] = a0.x; x.q[1] = a0.y; x.q[2] = a0.z; x.q[3] = a0.w;
    x.q[4] = a1.x; x.q[5] = a1.y; x.q[6] = a1.z; x.q[7] = a1.w;
    x.q[8] = b0.x; x.q[9] = b0.y; x.q[10] = b0.z; x.q[11] = b0.w;
    x.q[12] = b1.x; x.q[13] = b1.y; x.q[14] = b1.z; x.q[15] = b1.w;
    x.bs[0] = s.bs[sb * 16 + g0];
    x.bs[1] = s.bs[sb * 16 + g0 + 1];
    x.bs[2] = s.bs[sb * 16 + g1];
    x.bs[3] = s.bs[sb * 16 + g1 + 1];
    const float d = __uint_as_float(s.info[sb]);
    float_parts(d, x.m, x.e);
    x.neg = d < 0.0f;
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

template <int TYPE>
__device__ __forceinline__ void load_wb(const WeightView & w, size_t idx, WB & o) {
    o.lo = *reinterpret_cast<const uint4 *>(w.a + idx * 16);
    if (TYPE == T_Q4_0) {
        o.d = *reinterpret_cast<const uint16_t *>(w.b + idx * 2);
    } else if (TYPE == T_Q4_1) {
        o.d = *reinterpret_cast<const uint32_t *>(w.b + idx * 4);
    } else {
        o.hi = *reinterpret_cast<const uint4 *>(w.b + idx * 16);
        o.d = *reinterpret_cast<const uint16_t *>(w.c + idx * 2);
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
    if (TYPE == T_Q6_K) {
        const int n = part >> 1, p = part & 1;
        const uint4 * ql = reinterpret_cast<const uint4 *>(w.a + sbi * 128 + 64 * n + 32 * p);
        const uint4 * qh = reinterpret_cast<const uint4 *>(w.b + sbi * 64 + 32 * n);
        o.a0 = ql[0];
        o.a1 = ql[1];
        o.h0 = qh[0];
        o.h1 = qh[1];
        const uint8_t * sc = w.c + sbi * 16;
        o.s0 = *reinterpret_cast<const uint16_t *>(sc + 8 * n + 2 * p);
        o.s1 = *reinterpret_cast<const uint16_t *>(sc + 8 * n + 4 + 2 * p);
        o.s2 = 0;
        o.d = *reinterpret_cast<const uint16_t *>(w.d + sbi * 2);
    } else {
        const uint4 * qs = reinterpret_cast<const uint4 *>(w.a + sbi * 128 + 32 * part);
        const uint4 * qh = reinterpret_cast<const uint4 *>(w.b + sbi * 32);
        o.a0 = qs[0];
        o.a1 = qs[1];
        o.h0 = qh[0];
        o.h1 = qh[1];
        const uint4 meta = *reinterpret_cast<const uint4 *>(w.c + sbi * 16);
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
        const int p = part & 1;
        int dA0 = 0, dA1 = 0, dB0 = 0, dB1 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t ql = pick(i < 4 ? w.a0 : w.a1, i & 3), qh = pick(i < 4 ? w.h0 : w.h1, i & 3);
            const uint32_t qa = (ql & 0x0F0F0F0Fu) | (((qh >> (2 * p)) & 0x03030303u) << 4);
            const uint32_t qb = ((ql >> 4) & 0x0F0F0F0Fu) | (((qh >> (2 * p + 4)) & 0x03030303u) << 4);
            if (i < 4) {
                dA0 = sdot4(qa, x.q[i], dA0);
                dB0 = sdot4(qb, x.q[8 + i], dB0);
            } else {
                dA1 = sdot4(qa, x.q[i], dA1);
                dB1 = sdot4(qb, x.q[8 + i], dB1);
            }
        }
        const int scA0 = int(int8_t(w.s0 & 0xff)), scA1 = int(int8_t((w.s0 >> 8) & 0xff));
        const int scB0 = int(int8_t(w.s1 & 0xff)), scB1 = int(int8_t((w.s1 >> 8) & 0xff));
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

// ---- rows: weight loads are issued one task ahead of the compute ----
template <int TYPE, int NU>
struct Rows {
    static constexpr bool KQ = TYPE == T_Q5_K || TYPE == T_Q6_K;
    WB wb[KQ ? 1 : NU], wb2[KQ ? 1 : NU];  // g (or the matrix) and u of a SwiGLU pair
    WK wk[KQ ? NU : 1], wk2[KQ ? NU : 1];
    float e[8];  // epilog operands: ADD residual (e[0]); CONV state (e[0..2]) and kernel (e[4..7])
};

// Loads of one row (and its epilog operands), specialized by epilog kind so that no branch surrounds a load: a
// load behind a branch, or issued after the next row's weights, makes the compute wait for every load before it.
template <int TYPE, int NU, int EPI>
__device__ __forceinline__ void load_row(const GemvMember & m, int r, int lane, int nb, int nu, Rows<TYPE, NU> & R) {
    if constexpr (Rows<TYPE, NU>::KQ) {
        const int nsb = nu >> 2;
#pragma unroll
        for (int k = 0; k < NU; ++k) {
            const int u0 = lane + 64 * k, u = u0 < nu ? u0 : nu - 1;
            load_wk<TYPE>(m.w, size_t(r) * nsb + (u >> 2), u & 3, R.wk[k]);
            if constexpr (EPI == EPI_SWIGLU) load_wk<TYPE>(m.w2, size_t(r) * nsb + (u >> 2), u & 3, R.wk2[k]);
        }
    } else {
#pragma unroll
        for (int k = 0; k < NU; ++k) {
            const int b = lane + 64 * k, bb = b < nb ? b : nb - 1;
            load_wb<TYPE>(m.w, size_t(r) * nb + bb, R.wb[k]);
            if constexpr (EPI == EPI_SWIGLU) load_wb<TYPE>(m.w2, size_t(r) * nb + bb, R.wb2[k]);
        }
    }
    if constexpr (EPI == EPI_ADD) R.e[0] = m.res[r];
    if constexpr (EPI == EPI_CONV) {
        R.e[0] = m.conv_src[3 * r];
        R.e[1] = m.conv_src[3 * r + 1];
        R.e[2] = m.conv_src[3 * r + 2];
        const float4 k = *reinterpret_cast<const float4 *>(m.conv_w + 4 * size_t(r));
        R.e[4] = k.x;
        R.e[5] = k.y;
        R.e[6] = k.z;
        R.e[7] = k.w;
    }
}

template <int TYPE, int NU>
__device__ __forceinline__ void load_row_any(const GemvMember & m, int r, int lane, int nb, int nu, Rows<TYPE, NU> & R) {
    switch (m.epi) {
    case EPI_SWIGLU: load_row<TYPE, NU, EPI_SWIGLU>(m, r, lane, nb, nu, R); break;
    case EPI_ADD: load_row<TYPE, NU, EPI_ADD>(m, r, lane, nb, nu, R); break;
    case EPI_CONV: load_row<TYPE, NU, EPI_CONV>(m, r, lane, nb, nu, R); break;
    default: load_row<TYPE, NU, EPI_PLAIN>(m, r, lane, nb, nu, R); break;
    }
}

template <int TYPE, int NU, bool DBG>
__device__ __forceinline__ long long row_blocks(const WB * wb, int r, int nb, const XB * xb, int lane, int32_t * dbg) {
    double acc = 0.0;
#pragma unroll
    for (int k = 0; k < NU; ++k) {
        const int b = lane + 64 * k;
        const int si = dot_block<TYPE>(wb[k], xb[k]);
        const double t = block_term<TYPE>(si, wb[k].d, xb[k]);
        acc += b < nb ? t : 0.0;
        if constexpr (DBG) {
            if (dbg && b < nb) dbg[size_t(r) * nb + b] = si;
        }
    }
    return wave_sum_i64(dint_to_i64(acc));
}

template <int TYPE, int NU, bool DBG>
__device__ __forceinline__ long long row_units(const WK * wk, int r, int nu, const XK * xk, int lane, int32_t * dbg) {
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
        if constexpr (DBG) {
            if (dbg && u < nu && (u & 3) == 0) {
                const size_t i = (size_t(r) * nsb + (u >> 2)) * 2;
                dbg[i] = S;
                dbg[i + 1] = M;
            }
        }
    }
    return wave_sum_i64(acc);
}

struct Ctx {  // per-wave state shared by the row loops
    int lane, nb, nu;
    unsigned long long best;
};

// One row: dots, exact row sum, epilog (lane 0 stores).
template <int TYPE, int NU, int EPI, bool DBG>
__device__ __forceinline__ void row_compute(const GemvArgs & a, const GemvMember & m, bool argmax, int32_t * dbg, int r,
                                            const Rows<TYPE, NU> & R, const XB * xb, const XK * xk, Ctx & c) {
    long long acc, acc2 = 0;
    if constexpr (Rows<TYPE, NU>::KQ) {
        acc = row_units<TYPE, NU, DBG>(R.wk, r, c.nu, xk, c.lane, dbg);
        if constexpr (EPI == EPI_SWIGLU) acc2 = row_units<TYPE, NU, false>(R.wk2, r, c.nu, xk, c.lane, nullptr);
    } else {
        acc = row_blocks<TYPE, NU, DBG>(R.wb, r, c.nb, xb, c.lane, dbg);
        if constexpr (EPI == EPI_SWIGLU) acc2 = row_blocks<TYPE, NU, false>(R.wb2, r, c.nb, xb, c.lane, nullptr);
    }
    if (c.lane == 0) {
        const float v = fixed_to_float(acc);
        float out = v;
        if constexpr (EPI == EPI_SWIGLU) {
            out = (v / (1.0f + expf_(-v))) * fixed_to_float(acc2);  // gemvqc_ops.h:88-92
        } else if constexpr (EPI == EPI_ADD) {
            out = v + R.e[0];  // gemvqc16.cpp:282-301
        } else if constexpr (EPI == EPI_SILU) {
            out = silu_(v);  // gemvqc_ops.h:70-79 (UNARY SiLU) on the row result
        } else if constexpr (EPI == EPI_CONV) {  // gemvqc_ops.h:387-431 on the row result
            float sum = 0.0f;
            sum += R.e[0] * R.e[4];
            sum += R.e[1] * R.e[5];
            sum += R.e[2] * R.e[6];
            sum += v * R.e[7];
            out = m.conv_silu ? silu_(sum) : sum;
            m.conv_dst[3 * r] = R.e[1];
            m.conv_dst[3 * r + 1] = R.e[2];
            m.conv_dst[3 * r + 2] = v;
        }
        m.y[r] = out;
        if (argmax) {
            const unsigned long long key = argmax_key(out, uint32_t(r));
            c.best = key > c.best ? key : c.best;
        }
    }
}

// Rows r0..r1-1 of one member, two register buffers in turn: the loads of row r + 1 are in flight while row r is
// reduced, and no buffer is copied (a copy of registers that are still being loaded would wait for them). Rows
// past r1 - 1 reload the last row, which the caches serve; their results are not stored.
template <int TYPE, int NU, int EPI, bool DBG>
__device__ __forceinline__ void run_rows(const GemvArgs & a, const GemvMember & m, int mi, int r0, int r1,
                                         Rows<TYPE, NU> & A, const XB * xb, const XK * xk, Ctx & c) {
    const bool argmax = EPI == EPI_PLAIN && a.argmax_key != nullptr && mi == 0;
    int32_t * dbg = (DBG && mi == 0) ? a.dbg : nullptr;
    Rows<TYPE, NU> B;
    for (int r = r0;; r += 2) {
        load_row<TYPE, NU, EPI>(m, min(r + 1, r1 - 1), c.lane, c.nb, c.nu, B);
        row_compute<TYPE, NU, EPI, DBG>(a, m, argmax, dbg, r, A, xb, xk, c);
        if (r + 1 >= r1) break;
        load_row<TYPE, NU, EPI>(m, min(r + 2, r1 - 1), c.lane, c.nb, c.nu, A);
        row_compute<TYPE, NU, EPI, DBG>(a, m, argmax, dbg, r + 1, B, xb, xk, c);
        if (r + 2 >= r1) break;
    }
}

template <int TYPE, int NU, bool DBG>
__global__ __launch_bounds__(NT) void gemv_kernel(GemvArgs a) {
    __shared__ Lds s;
    constexpr bool KQ = TYPE == T_Q5_K || TYPE == T_Q6_K;
    Ctx c;
    c.lane = threadIdx.x & 63;
    c.nb = a.cols / 32;
    c.nu = a.cols / 64;
    c.best = 0;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: member fields load as scalars
    // each wave owns a contiguous range of tasks (streams through consecutive rows)
    const int nwt = gridDim.x * NWAVES, per = (a.total_tasks + nwt - 1) / nwt;
    const int t0 = (blockIdx.x * NWAVES + wave) * per;
    const int t1 = min(a.total_tasks, t0 + per);
    int mi0 = 0;
#pragma unroll
    for (int i = 1; i < 4; ++i)
        if (i < a.n_members && t0 >= a.m[i].task_begin) mi0 = i;
    // the first row's weights are requested before the activation prologue
    Rows<TYPE, NU> cur;
    if (t0 < t1) load_row_any<TYPE, NU>(a.m[mi0], t0 - a.m[mi0].task_begin, c.lane, c.nb, c.nu, cur);
    if constexpr (KQ) {
        const float scale = a.xsrc == XSRC_NORM ? block_norm_scale(a.x, a.cols, a.norm_eps, a.norm_l2, s) : 1.0f;
        quantize_q8_K(a, scale, s);
    } else {
        prologue_q8_0<(NU > 4 ? 2 : 1)>(a, s);
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
    }
    for (int mi = mi0; mi < a.n_members && t0 < t1; ++mi) {
        const GemvMember & m = a.m[mi];
        const int r0 = max(t0, m.task_begin) - m.task_begin, r1 = min(t1, m.task_begin + m.rows) - m.task_begin;
        if (r0 >= r1) continue;
        if (mi != mi0) load_row_any<TYPE, NU>(m, r0, c.lane, c.nb, c.nu, cur);
        switch (m.epi) {
        case EPI_SWIGLU: run_rows<TYPE, NU, EPI_SWIGLU, DBG>(a, m, mi, r0, r1, cur, xb, xk, c); break;
        case EPI_ADD: run_rows<TYPE, NU, EPI_ADD, DBG>(a, m, mi, r0, r1, cur, xb, xk, c); break;
        case EPI_CONV: run_rows<TYPE, NU, EPI_CONV, DBG>(a, m, mi, r0, r1, cur, xb, xk, c); break;
        case EPI_SILU: run_rows<TYPE, NU, EPI_SILU, DBG>(a, m, mi, r0, r1, cur, xb, xk, c); break;
        default: run_rows<TYPE, NU, EPI_PLAIN, DBG>(a, m, mi, r0, r1, cur, xb, xk, c); break;
        }
    }
    if (a.argmax_key) {
        if (c.lane == 0) s.key[wave] = c.best;
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long b = s.key[0];
            for (int i = 1; i < NWAVES; ++i) b = s.key[i] > b ? s.key[i] : b;
            if (b) atomicMax(a.argmax_key, b);
        }
    }
}

// Workgroups of `kernel` that fit on the device at once (a grid beyond it runs a second, mostly idle round).
template <typename K>
int resident_blocks(K kernel) {
    int dev = 0, cus = 0, occ = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, NT, 0) != hipSuccess || occ < 1 || cus < 1)
        return 1024;
    return occ * cus;
}

template <int TYPE, int NU>
hipError_t launch_typed(const GemvArgs & a, hipStream_t st) {
    // about 16 tasks per workgroup (4 per wave) amortize the activation prologue; no more workgroups than fit
    static const int cap = resident_blocks(gemv_kernel<TYPE, NU, false>);
    int grid = (a.total_tasks + 15) / 16;
    grid = grid < 1 ? 1 : grid > cap ? cap : grid;
    if (a.dbg) GQ_LAUNCH((gemv_kernel<TYPE, NU, true>), dim3(grid), dim3(NT), 0, st, a);
    else GQ_LAUNCH((gemv_kernel<TYPE, NU, false>), dim3(grid), dim3(NT), 0, st, a);
    return hipGetLastError();
}

template <int TYPE>
hipError_t launch_nu(const GemvArgs & a, hipStream_t st) {
    constexpr bool KQ = TYPE == T_Q5_K || TYPE == T_Q6_K;
    const int nu = (a.cols / (KQ ? 64 : 32) + 63) / 64;  // cols <= 16384: K-quants nu <= 4, Q4_0 / Q8_0 nu <= 8
    switch (nu) {
    case 1: return launch_typed<TYPE, 1>(a, st);
    case 2: return launch_typed<TYPE, 2>(a, st);
    case 3: return launch_typed<TYPE, 3>(a, st);
    case 4: return launch_typed<TYPE, 4>(a, st);
    default: break;
    }
    if constexpr (!KQ) {
        switch (nu) {
        case 5: return launch_typed<TYPE, 5>(a, st);
        case 6: return launch_typed<TYPE, 6>(a, st);
        case 7: return launch_typed<TYPE, 7>(a, st);
        case 8: return launch_typed<TYPE, 8>(a, st);
        default: break;
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_gemv(const GemvArgs & a, int type, hipStream_t st) {
    if (a.cols <= 0 || a.cols > MAXK || a.total_tasks <= 0) return hipErrorInvalidValue;
    switch (type) {
    case T_Q4_0: return launch_nu<T_Q4_0>(a, st);
    case T_Q4_1: return launch_nu<T_Q4_1>(a, st);
    case T_Q8_0: return launch_nu<T_Q8_0>(a, st);
    case T_Q5_K: return a.cols % 256 ? hipErrorInvalidValue : launch_nu<T_Q5_K>(a, st);
    case T_Q6_K: return a.cols % 256 ? hipErrorInvalidValue : launch_nu<T_Q6_K>(a, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace gq
