// Batched GEMV for gfx950: n_tok tokens share every weight read (prefill, speculative or multi-sequence decode; the
// batched path the reference plans in ROADMAP.md:78-96). Token t's output row is the single-token GEMV's bit for
// bit: the same Q8_0 activation quantizer (gemvq_ref.h:236-245, with a per-token RMS norm folded in as the deferred
// norm of gemvqc16.h:52-59), the same exact block terms floor(sumi * fp16(d_w) * d_x * 2^40) summed in int64 and
// rounded to FP32 once (gemvqw_engine.h:352-445), the same epilogs. Only the block sums change hands: one int8
// v_mfma_i32_16x16x32_i8 per 32-weight block gives them for 16 rows x 16 tokens. A block's 32 quants may be
// permuted as long as the weight and the activation operands agree, so lane group g (lanes 16g..16g+15) takes quants
// 4g..4g+3 and 16+4g..16+4g+3: Q4_0 packs exactly those as the low and high nibbles of quant bytes 4g..4g+3, Q8_0
// holds them as bytes 4g..4g+3 of its two 16-byte halves, and the activation quantizer stores them in that order.
#include "gq_gemv_impl.h"

namespace gq {
namespace {

constexpr int GT = 16;  // rows and tokens per MFMA tile
constexpr int GU = 4;   // blocks per load round of a wave

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// ---- activation: token rows -> Q8_0 blocks in operand order ----
// Workgroup t quantizes token t exactly as the single-token prologue: thread i holds the 16-float items i, i + NT,
// ... (the two halves of a block in adjacent lanes), the norm scale is the canonical pairwise tree over the row, and
// v = (x * scale) * w.
__global__ __launch_bounds__(NT) void gemm_quant_kernel(GemmQuantArgs a) {
    __shared__ Lds s;
    const int tok = blockIdx.x, nb = a.cols / 32, n16 = a.cols / 16;
    int8_t * q = a.q + size_t(tok) * a.cols;
    float * d40 = a.d40 + size_t(tok) * nb;
    if (tok >= a.n_tok) {  // padding tokens: zero quants and scales, whose terms are exactly zero
        for (int i = threadIdx.x; i < n16; i += NT) reinterpret_cast<uint4 *>(q)[i] = make_uint4(0u, 0u, 0u, 0u);
        for (int i = threadIdx.x; i < nb; i += NT) d40[i] = 0.0f;
        return;
    }
    const float * x = a.x + size_t(tok) * a.x_stride;
    const float sc = a.norm ? block_norm_scale(x, a.cols, a.eps, a.norm_l2, s) : 1.0f;
    for (int i = threadIdx.x; i < n16; i += NT) {  // n16 is even: both lanes of a pair run every round
        float v[16];
        load16(x + size_t(i) * 16, v);
        if (a.norm_w) {
            float w[16];
            load16(a.norm_w + size_t(i) * 16, w);
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = (v[j] * sc) * w[j];
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = v[j] * sc;
        }
        uint32_t packed[4];
        int sum;
        const float d = quantize_half_core(v, packed, sum);
        // half h of block b: its word g (quants 16h + 4g .. 16h + 4g + 3) goes to byte 8g + 4h of the block
        const int b = i >> 1, h = i & 1;
        uint32_t * qb = reinterpret_cast<uint32_t *>(q + size_t(b) * 32);
#pragma unroll
        for (int g = 0; g < 4; ++g) qb[2 * g + h] = packed[g];
        if (h == 0) d40[b] = h2f(f2h(d)) * 1099511627776.0f;  // * 2^40, exact
    }
}

// ---- weights and activation operands of one round (GU blocks) of a wave ----
__device__ __forceinline__ uint2 ld8(const uint8_t * p) {
    const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p));
    return make_uint2(v.x, v.y);
}

template <int TYPE>
__device__ __forceinline__ const uint8_t * scale_region(const WeightView & w) {
    return TYPE == T_Q4_0 ? w.b : w.c;
}

// Lane (r, g) (r = lane % 16, g = lane / 16) holds the A operand of weight row r of the tile and the B operand of
// token r of each token tile; its results are rows 4g..4g+3 of the tile for token r, so it also loads those rows'
// scales (4 blocks in 8 bytes) and its token's d * 2^40 (4 blocks in 16 bytes).
template <int TYPE, bool PAIR, int T>
struct Round {
    static constexpr bool Q8 = TYPE == T_Q8_0;
    uint32_t wa[GU], wb[Q8 ? GU : 1];
    uint32_t ua[PAIR ? GU : 1], ub[(PAIR && Q8) ? GU : 1];
    uint2 dw[4], du[PAIR ? 4 : 1];
    uint2 xq[T][GU];
    float4 dx[T];
};

template <int TYPE, bool PAIR, int T>
__device__ __forceinline__ void load_round(const GemmArgs & a, int nb, int ra, const int * ro, int b, int r, int g,
                                           Round<TYPE, PAIR, T> & o) {
#pragma unroll
    for (int j = 0; j < GU; ++j) {
        const size_t blk = size_t(ra) * nb + b + j;
        o.wa[j] = ld4(a.w.a + blk * 16 + 4 * g);
        if constexpr (TYPE == T_Q8_0) o.wb[j] = ld4(a.w.b + blk * 16 + 4 * g);
        if constexpr (PAIR) {
            o.ua[j] = ld4(a.w2.a + blk * 16 + 4 * g);
            if constexpr (TYPE == T_Q8_0) o.ub[j] = ld4(a.w2.b + blk * 16 + 4 * g);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const size_t off = (size_t(ro[i]) * nb + b) * 2;
        o.dw[i] = ld8(scale_region<TYPE>(a.w) + off);
        if constexpr (PAIR) o.du[i] = ld8(scale_region<TYPE>(a.w2) + off);
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const size_t tok = size_t(t * GT + r);
#pragma unroll
        for (int j = 0; j < GU; ++j) o.xq[t][j] = *reinterpret_cast<const uint2 *>(a.q + (tok * nb + b + j) * 32 + 8 * g);
        o.dx[t] = *reinterpret_cast<const float4 *>(a.d40 + tok * nb + b);
    }
}

// The A operand of one block: Q4_0 nibbles (low: quants 4g..4g+3, high: 16+4g..) minus 8 in every byte; Q8_0 its
// two words as they are.
template <int TYPE>
__device__ __forceinline__ long a_operand(uint32_t lo, uint32_t hi) {
    uint32_t w0 = lo, w1 = hi;
    if constexpr (TYPE == T_Q4_0) {
        const uint32_t n0 = lo & 0x0F0F0F0Fu, n1 = (lo >> 4) & 0x0F0F0F0Fu;
        // per byte: ((v | 0x80) - 8) ^ 0x80 = v - 8 as int8 for 0 <= v <= 15, no borrow between bytes
        w0 = ((n0 | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
        w1 = ((n1 | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
    }
    return long((uint64_t(w1) << 32) | w0);
}

__device__ __forceinline__ uint32_t half_of(const uint2 & v, int j) {
    const uint32_t w = (j >> 1) ? v.y : v.x;
    return (j & 1) ? w >> 16 : w & 0xffffu;
}
__device__ __forceinline__ float lane_of(const float4 & v, int j) { return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w; }

// The round's block terms: per block and token tile one MFMA gives the lane's 4 sums (rows 4g + i, token r); each
// term is floor(sumi * s) with s = fp16(d_w) * d_x * 2^40 exact in FP32 and the product exact in FP64; the GU terms
// are summed in FP64 (integers below 2^53) and moved to the int64 totals.
template <int TYPE, bool PAIR, int T>
__device__ __forceinline__ void round_terms(const Round<TYPE, PAIR, T> & o, long long (*tot)[4], long long (*totu)[4]) {
    double acc[T][4], accu[T][4];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] = accu[t][i] = 0.0;
#pragma unroll
    for (int j = 0; j < GU; ++j) {
        uint32_t hw = 0u, hu = 0u;
        if constexpr (TYPE == T_Q8_0) hw = o.wb[j];
        const long aw = a_operand<TYPE>(o.wa[j], hw);
        long au = 0;
        if constexpr (PAIR) {
            if constexpr (TYPE == T_Q8_0) hu = o.ub[j];
            au = a_operand<TYPE>(o.ua[j], hu);
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const long bx = long((uint64_t(o.xq[t][j].y) << 32) | o.xq[t][j].x);
            const float dx = lane_of(o.dx[t], j);
            const v4i zero = {0, 0, 0, 0};
            const v4i sw = __builtin_amdgcn_mfma_i32_16x16x32_i8(aw, bx, zero, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float s = h2f(half_of(o.dw[i], j)) * dx;
                acc[t][i] += floor(double(sw[i]) * double(s));
            }
            if constexpr (PAIR) {
                const v4i su = __builtin_amdgcn_mfma_i32_16x16x32_i8(au, bx, zero, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float s = h2f(half_of(o.du[i], j)) * dx;
                    accu[t][i] += floor(double(su[i]) * double(s));
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            tot[t][i] += dint_to_i64(acc[t][i]);
            if constexpr (PAIR) totu[t][i] += dint_to_i64(accu[t][i]);
        }
}

// Workgroup b: rows 16b .. 16b + 15 (clamped loads past the last row, nothing stored for them); wave w sums the
// blocks w * nb / 4 .. (w + 1) * nb / 4 - 1, and wave 0 adds the other waves' int64 totals (exact in any order),
// applies the epilog and stores token t's row at y + t * y_stride.
template <int TYPE, bool PAIR, int T>
__global__ __launch_bounds__(NT) void gemm_kernel(GemmArgs a) {
    __shared__ long long red[NWAVES - 1][PAIR ? 2 : 1][T][4][WAVE];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int r0 = int(blockIdx.x) * GT;
    const int ra = min(r0 + r, a.rows - 1);
    int ro[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ro[i] = min(r0 + 4 * g + i, a.rows - 1);
    const int nb = a.cols / 32, nbw = nb / NWAVES, b0 = wave * nbw, b1 = b0 + nbw;  // nbw % GU == 0
    long long tot[T][4], totu[PAIR ? T : 1][4];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            tot[t][i] = 0;
            totu[PAIR ? t : 0][i] = 0;
        }
    Round<TYPE, PAIR, T> cur, nxt;
    load_round<TYPE, PAIR, T>(a, nb, ra, ro, b0, r, g, cur);
    for (int b = b0; b + GU < b1; b += GU) {  // the next round is requested before this one's terms
        load_round<TYPE, PAIR, T>(a, nb, ra, ro, b + GU, r, g, nxt);
        round_terms<TYPE, PAIR, T>(cur, tot, totu);
        cur = nxt;
    }
    round_terms<TYPE, PAIR, T>(cur, tot, totu);
    if (wave > 0) {
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                red[wave - 1][0][t][i][lane] = tot[t][i];
                if constexpr (PAIR) red[wave - 1][PAIR ? 1 : 0][t][i][lane] = totu[t][i];
            }
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int tok = t * GT + r;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            long long s = tot[t][i], su = 0;
#pragma unroll
            for (int k = 0; k < NWAVES - 1; ++k) s += red[k][0][t][i][lane];
            if constexpr (PAIR) {
                su = totu[t][i];
#pragma unroll
                for (int k = 0; k < NWAVES - 1; ++k) su += red[k][PAIR ? 1 : 0][t][i][lane];
            }
            const int row = r0 + 4 * g + i;
            if (row >= a.rows || tok >= a.n_tok) continue;
            const float v = fixed_to_float(s);
            float out = v;
            if (PAIR && a.epi == EPI_SWIGLU) {
                out = (v / (1.0f + expf_(-v))) * fixed_to_float(su);  // gemvqc_ops.h:88-92
            } else if (a.epi == EPI_ADD) {
                out = v + a.res[size_t(tok) * a.res_stride + row];  // gemvqc16.cpp:282-301
            } else if (a.epi == EPI_SILU) {
                out = silu_(v);
            }
            a.y[size_t(tok) * a.y_stride + row] = out;
        }
    }
}

template <int TYPE, bool PAIR>
hipError_t launch_tiles(const GemmArgs & a, hipStream_t st) {
    const dim3 grid((a.rows + GT - 1) / GT);
    if (a.n_tok <= GT) GQ_LAUNCH((gemm_kernel<TYPE, PAIR, 1>), grid, dim3(NT), 0, st, a);
    else GQ_LAUNCH((gemm_kernel<TYPE, PAIR, 2>), grid, dim3(NT), 0, st, a);
    return hipGetLastError();
}

template <int TYPE>
hipError_t launch_type(const GemmArgs & a, hipStream_t st) {
    return a.epi == EPI_SWIGLU ? launch_tiles<TYPE, true>(a, st) : launch_tiles<TYPE, false>(a, st);
}

}  // namespace

hipError_t launch_gemm_quant(const GemmQuantArgs & a, hipStream_t s) {
    if (a.n_tok < 1 || a.n_pad < a.n_tok || a.n_pad % GT || a.n_pad > GEMM_MAX_TOK || a.cols % 512 ||
        a.cols > GEMV_MAXK || a.x_stride < a.cols || a.x_stride % 16)
        return hipErrorInvalidValue;
    GQ_LAUNCH(gemm_quant_kernel, dim3(a.n_pad), dim3(NT), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_gemm(const GemmArgs & a, int type, hipStream_t s) {
    // shapes the kernels assume: whole rounds of GU blocks per wave, at most two token tiles
    if (a.rows < 1 || a.n_tok < 1 || a.n_tok > GEMM_MAX_TOK || a.cols % 512 || a.cols > GEMV_MAXK ||
        a.y_stride < a.rows || (a.epi == EPI_ADD && a.res_stride < a.rows))
        return hipErrorInvalidValue;
    switch (type) {
    case T_Q4_0: return launch_type<T_Q4_0>(a, s);
    case T_Q8_0: return launch_type<T_Q8_0>(a, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace gq
