// Batched GEMV for gfx950: n_tok tokens share every weight read (prefill, speculative or multi-sequence decode; the
// batched path the reference plans in ROADMAP.md:78-96). Token t's output row is the single-token GEMV's bit for
// bit: the same Q8_0 activation quantizer (gemvq_ref.h:236-245, with a per-token RMS norm folded in as the deferred
// norm of gemvqc16.h:52-59), the same exact block terms floor(sumi * fp16(d_w) * d_x * 2^40) summed in int64 and
// rounded to FP32 once (gemvqw_engine.h:352-445), the same epilogs. Only the block sums change hands: one int8
// v_mfma_i32_16x16x32_i8 per 32-weight block gives them for 16 rows x 16 tokens. A block's 32 quants may be
// permuted as long as the weight and the activation operands agree, so lane group g (lanes 16g..16g+15) takes quants
// 4g..4g+3 and 16+4g..16+4g+3: Q4_0 and Q4_1 pack exactly those as the low and high nibbles of quant bytes 4g..4g+3,
// Q8_0 holds them as bytes 4g..4g+3 of its two 16-byte halves, and the activation quantizer stores them in that
// order. Q4_1 adds the term floor(m_w * s_x * 2^40) with the Q8_1 s_x of each activation block (gemvq_ref.h:194-229).
#include "gq_gemv_impl.h"

namespace gq {
namespace {

constexpr int GT = 16;                 // rows and tokens per MFMA tile
constexpr int GU = 16;                 // blocks per round of a workgroup (each wave sums GU / NWAVES of them)
constexpr int GW = GU / NWAVES;        // blocks per wave per round
constexpr int ROW_LDS = GU * 16 + 16;  // LDS bytes per staged row: 16 quant bytes per block, padded so that the 16
                                       // rows of an operand read fall in distinct banks

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));  // native vectors (promoted to registers, unlike uint4)
typedef float v4f __attribute__((ext_vector_type(4)));

// Activation scratch: token t's block b, 8-byte group g (quants 4g..4g+3 and 16+4g..16+4g+3) at byte
// ((t * 4 + g) * nb + b) * 8, so a lane's groups of consecutive blocks are contiguous.
__device__ __forceinline__ size_t act_group(int tok, int g, int nb, int b) {
    return ((size_t(tok) * 4 + g) * nb + b) * 8;
}

// ---- activation: token rows -> Q8_0 blocks in operand order ----
// Workgroup t quantizes token t exactly as the single-token prologue: thread i holds the 16-float items i, i + NT,
// ... (the two halves of a block in adjacent lanes), the norm scale is the canonical pairwise tree over the row, and
// v = (x * scale) * w.
__global__ __launch_bounds__(NT) void gemm_quant_kernel(GemmQuantArgs a) {
    __shared__ Lds s;
    const int tok = blockIdx.x, nb = a.cols / 32, n16 = a.cols / 16;
    int8_t * q = a.q;
    float * d40 = a.d40 + size_t(tok) * nb, * s40 = a.s40 + size_t(tok) * nb;
    if (tok >= a.n_tok) {  // padding tokens: zero quants and scales, whose terms are exactly zero
        uint4 * z = reinterpret_cast<uint4 *>(q + act_group(tok, 0, nb, 0));
        for (int i = threadIdx.x; i < n16; i += NT) z[i] = make_uint4(0u, 0u, 0u, 0u);  // 4 groups x nb x 8 bytes
        for (int i = threadIdx.x; i < nb; i += NT) d40[i] = s40[i] = 0.0f;
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
        // half h of block b: its word g (quants 16h + 4g .. 16h + 4g + 3) is word h of group g
        const int b = i >> 1, h = i & 1;
#pragma unroll
        for (int g = 0; g < 4; ++g) *reinterpret_cast<uint32_t *>(q + act_group(tok, g, nb, b) + 4 * h) = packed[g];
        if (h == 0) {
            d40[b] = h2f(f2h(d)) * 1099511627776.0f;                   // * 2^40, exact
            s40[b] = h2f(f2h(float(sum) * d)) * 1099511627776.0f;      // ggml quantize_row_q8_1: fp16(sum * d)
        }
    }
}

// Per-block scale words: fp16 d (Q4_0 in region b, Q8_0 in region c), or d | m << 16 (Q4_1, region b).
template <int TYPE>
__device__ __forceinline__ uint32_t load_scale(const WeightView & w, size_t blk) {
    if constexpr (TYPE == T_Q4_1) return *reinterpret_cast<const uint32_t *>(w.b + blk * 4);
    return *reinterpret_cast<const uint16_t *>((TYPE == T_Q4_0 ? w.b : w.c) + blk * 2);
}

// One round's weights as loaded by the workgroup: thread t takes block t % 16 of the round in row t / 16 of the tile
// (its 16 quant bytes, or 32 for Q8_0, and its fp16 scale), so 16 consecutive threads read 256 contiguous bytes of
// one row.
// (Named members rather than arrays: the register allocator keeps them in VGPRs.)
template <int TYPE, bool PAIR>
struct WRound {
    v4u g0, g1, u0, u1;  // quant bytes (g1 / u1: the high halves of Q8_0 blocks) of the matrix and of u
    uint32_t gd, ud;       // fp16 scales
};

template <int TYPE, bool PAIR>
__device__ __forceinline__ void load_wround(const GemmArgs & a, int nb, int row, int rd, WRound<TYPE, PAIR> & o) {
    const size_t blk = size_t(row) * nb + rd * GU + (threadIdx.x & 15);
    o.g0 = *reinterpret_cast<const v4u *>(a.w.a + blk * 16);
    if constexpr (TYPE == T_Q8_0) o.g1 = *reinterpret_cast<const v4u *>(a.w.b + blk * 16);
    o.gd = load_scale<TYPE>(a.w, blk);
    if constexpr (PAIR) {
        o.u0 = *reinterpret_cast<const v4u *>(a.w2.a + blk * 16);
        if constexpr (TYPE == T_Q8_0) o.u1 = *reinterpret_cast<const v4u *>(a.w2.b + blk * 16);
        o.ud = load_scale<TYPE>(a.w2, blk);
    }
}

template <int TYPE>
__device__ __forceinline__ uint32_t scale_word(uint32_t sw) {
    return TYPE == T_Q4_1 ? sw : __float_as_uint(h2f(sw & 0xffffu));
}

// Thread t's part of a round into an LDS buffer: its 16 quant bytes of every matrix-half at row t / 16, block t % 16
// (rows padded to ROW_LDS bytes), and its scale word: Q4_0 / Q8_0 the fp16 scale as FP32 bits (converted once here,
// not once per token lane), Q4_1 the fp16 pair (d, m) as loaded.
template <int TYPE, bool PAIR>
__device__ __forceinline__ void stage(const WRound<TYPE, PAIR> & w, uint8_t * lq, uint32_t * ld) {
    constexpr int QH = TYPE == T_Q8_0 ? 2 : 1, QBUF = GT * ROW_LDS;
    const int t = threadIdx.x, o = (t >> 4) * ROW_LDS + (t & 15) * 16, od = (t >> 4) * GU + (t & 15);
    *reinterpret_cast<v4u *>(lq + o) = w.g0;
    if constexpr (QH == 2) *reinterpret_cast<v4u *>(lq + QBUF + o) = w.g1;
    ld[od] = scale_word<TYPE>(w.gd);
    if constexpr (PAIR) {
        *reinterpret_cast<v4u *>(lq + QH * QBUF + o) = w.u0;
        if constexpr (QH == 2) *reinterpret_cast<v4u *>(lq + 3 * QBUF + o) = w.u1;
        ld[GT * GU + od] = scale_word<TYPE>(w.ud);
    }
}

// The A operand of one block: Q4_0 nibbles (low: quants 4g..4g+3, high: 16+4g..) minus 8 in every byte; Q4_1 the
// nibbles as they are; Q8_0 its two words as they are.
template <int TYPE>
__device__ __forceinline__ long a_operand(uint32_t lo, uint32_t hi) {
    uint32_t w0 = lo, w1 = hi;
    if constexpr (TYPE == T_Q4_1) {
        w0 = lo & 0x0F0F0F0Fu;
        w1 = (lo >> 4) & 0x0F0F0F0Fu;
    }
    if constexpr (TYPE == T_Q4_0) {
        const uint32_t n0 = lo & 0x0F0F0F0Fu, n1 = (lo >> 4) & 0x0F0F0F0Fu;
        // per byte: ((v | 0x80) - 8) ^ 0x80 = v - 8 as int8 for 0 <= v <= 15, no borrow between bytes
        w0 = ((n0 | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
        w1 = ((n1 | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
    }
    return long((uint64_t(w1) << 32) | w0);
}

// A lane's activation operands of one round: its token's groups g of the wave's GW blocks (GW * 8 contiguous bytes)
// and their d * 2^40.
template <int T>
struct XRound {
    v4u q[T][GW / 2];
    v4f d[T];
    v4f s[T];  // Q4_1 only
};

template <int TYPE, int T>
__device__ __forceinline__ void load_xround(const GemmArgs & a, int nb, int r, int g, int b, XRound<T> & o) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int tok = t * GT + r;
        const v4u * p = reinterpret_cast<const v4u *>(a.q + act_group(tok, g, nb, b));
#pragma unroll
        for (int k = 0; k < GW / 2; ++k) o.q[t][k] = p[k];
        o.d[t] = *reinterpret_cast<const v4f *>(a.d40 + size_t(tok) * nb + b);
        if constexpr (TYPE == T_Q4_1) o.s[t] = *reinterpret_cast<const v4f *>(a.s40 + size_t(tok) * nb + b);
    }
}

__device__ __forceinline__ float lane_of(const v4f & v, int j) { return v[j]; }


// Whether a round needs the int64 path: some lane's wbound * (largest sum of |d_x * 2^40| over a token's GW blocks)
// reaches 2^52 (one ballot, so the branch on it is uniform over the wave).
template <int T>
__device__ __forceinline__ bool round_needs_exact(const XRound<T> & x, float wbound) {
    float dm = 0.0f;
#pragma unroll
    for (int t = 0; t < T; ++t) {
        float ds = 0.0f;
#pragma unroll
        for (int c = 0; c < GW; ++c) ds += fabsf(lane_of(x.d[t], c));
        dm = fmaxf(dm, ds);
    }
    return __builtin_amdgcn_ballot_w64(!(wbound * dm < 4503599627370496.0f)) != 0;
}

// The wave's GW blocks of a staged round: per block and token tile one MFMA gives the lane's 4 sums (rows 4g + i,
// token r); each term is floor(sumi * s) with s = fp16(d_w) * d_x * 2^40 exact in FP32 and the product exact in FP64;
// the GW terms are summed in FP64 and moved to the int64 totals. The FP64 sum is exact while it stays below 2^53 LSB:
// |term| <= wbound * |d_x * 2^40| (wbound: the member's largest |d_w| times its type's largest |sum of products|),
// so a round where a lane's wbound * sum |d_x * 2^40| over a token's GW blocks reaches 2^52 (a factor 2 of margin)
// adds every term of the wave to the int64 totals directly (EXACT).
template <int TYPE, bool PAIR, int T, bool EXACT>
__device__ __forceinline__ void round_terms_k(const uint8_t * lq, const uint32_t * ld, int wave, int r, int g,
                                              const XRound<T> & x, long long (*tot)[4], long long (*totu)[4]) {
    constexpr int NM = PAIR ? 2 : 1, QH = TYPE == T_Q8_0 ? 2 : 1;
    constexpr int QBUF = GT * ROW_LDS, DBUF = GT * GU;  // bytes of one matrix-half's quants, scales of one matrix
    double acc[NM][T][4];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[m][t][i] = 0.0;
    v4u dw[NM][4];  // scale words of rows 4g + i for the wave's GW = 4 blocks
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) dw[m][i] = *reinterpret_cast<const v4u *>(ld + m * DBUF + (4 * g + i) * GU + wave * GW);
#pragma unroll
    for (int j = 0; j < GW; ++j) {
        const int blk = wave * GW + j;
        long aop[NM];
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const uint8_t * p = lq + (m * QH) * QBUF + r * ROW_LDS + blk * 16 + 4 * g;
            const uint32_t lo = *reinterpret_cast<const uint32_t *>(p);
            const uint32_t hi = QH == 2 ? *reinterpret_cast<const uint32_t *>(p + QBUF) : 0u;
            aop[m] = a_operand<TYPE>(lo, hi);
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const v4u qv = x.q[t][j >> 1];
            const long bx = (j & 1) ? long((uint64_t(qv[3]) << 32) | qv[2]) : long((uint64_t(qv[1]) << 32) | qv[0]);
            const float dx = lane_of(x.d[t], j);
            const v4i zero = {0, 0, 0, 0};
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const v4i sm = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop[m], bx, zero, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t sw = dw[m][i][j];
                    const float sc = (TYPE == T_Q4_1 ? h2f(sw & 0xffffu) : __uint_as_float(sw)) * dx;
                    double term = floor(double(sm[i]) * double(sc));
                    if constexpr (TYPE == T_Q4_1)  // + floor(m * s_x * 2^40), the product of two fp16 values exact
                        term += floor(double(h2f(sw >> 16) * lane_of(x.s[t], j)));
                    if constexpr (EXACT) {
                        if (m == 0) tot[t][i] += dint_to_i64(term);
                        else totu[PAIR ? t : 0][i] += dint_to_i64(term);
                    } else {
                        acc[m][t][i] += term;
                    }
                }
            }
        }
    }
    if constexpr (!EXACT) {
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                tot[t][i] += dint_to_i64(acc[0][t][i]);
                if constexpr (PAIR) totu[t][i] += dint_to_i64(acc[PAIR ? 1 : 0][t][i]);
            }
    }
}

// The GW blocks of a round through one of two loops, chosen once per round (not per term, which kept the compiler
// from scheduling the round as one block): the FP64-sum loop, or, where the bound says an FP64 partial could pass
// 2^53 LSB, the one adding every term to the int64 totals.
template <int TYPE, bool PAIR, int T>
__device__ __forceinline__ void round_terms(const uint8_t * lq, const uint32_t * ld, int wave, int r, int g,
                                            const XRound<T> & x, float wbound, long long (*tot)[4],
                                            long long (*totu)[4]) {
    if (round_needs_exact<T>(x, wbound)) round_terms_k<TYPE, PAIR, T, true>(lq, ld, wave, r, g, x, tot, totu);
    else round_terms_k<TYPE, PAIR, T, false>(lq, ld, wave, r, g, x, tot, totu);
}

// Workgroup b: rows 16b .. 16b + 15 (clamped loads past the last row, nothing stored for them), the whole K range in
// rounds of GU blocks. Round rd + 2's weights are requested while round rd is summed (two rounds in flight) and
// round rd + 1's are staged in LDS for the next; wave w sums blocks w * GW .. of each round, and wave 0 adds the
// other waves' int64 totals (exact in any order), applies the epilog and stores token t's row at y + t * y_stride.
// Loads past the last round repeat the last round (cache hits), so every load is unconditional and the waits stay
// exact.
// A group's workgroups are dealt to its members by tile: the member of tile b is the last whose first tile is <= b,
// and its fields replace the first member's (the activation, columns and tokens are shared).
template <int TYPE, bool PAIR, int T>
__global__ __launch_bounds__(NT) void gemm_kernel(GemmArgs a0) {
    constexpr int NM = PAIR ? 2 : 1, QH = TYPE == T_Q8_0 ? 2 : 1;
    constexpr int QBUF = GT * ROW_LDS, DBUF = GT * GU;
    __shared__ __align__(16) uint8_t lq[2][NM * QH * QBUF];
    __shared__ __align__(16) uint32_t ld[2][NM * DBUF];
    __shared__ long long red[NWAVES - 1][NM][T][4][WAVE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    GemmArgs a = a0;
    int tile0 = 0;
    float wbd = a0.wbound[0];  // the member's term bound
    if (!PAIR) {
        int mi = -1;
        for (int i = 0; i < a0.n_more; ++i)
            if (int(blockIdx.x) >= a0.more[i].tile0) mi = i;
        if (mi >= 0) {
            wbd = a0.wbound[mi + 1];
            const GemmMore & o = a0.more[mi];
            a.w = o.w;
            a.y = o.y;
            a.res = o.res;
            a.rows = o.rows;
            a.y_stride = o.y_stride;
            a.res_stride = o.res_stride;
            a.epi = o.epi;
            tile0 = o.tile0;
        }
    }
    const int r0 = (int(blockIdx.x) - tile0) * GT;
    const int nb = a.cols / 32, nr = nb / GU;
    const int lrow = min(r0 + (tid >> 4), a.rows - 1);
    long long tot[T][4], totu[PAIR ? T : 1][4];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            tot[t][i] = 0;
            totu[PAIR ? t : 0][i] = 0;
        }
    // rounds alternate between two LDS buffers and two register slots, so every load lands in a free slot
    WRound<TYPE, PAIR> w0, wa, wb;
    XRound<T> xa, xb;
    load_wround<TYPE, PAIR>(a, nb, lrow, 0, w0);
    load_wround<TYPE, PAIR>(a, nb, lrow, min(1, nr - 1), wb);
    load_xround<TYPE, T>(a, nb, r, g, wave * GW, xa);
    stage<TYPE, PAIR>(w0, lq[0], ld[0]);
    __syncthreads();
    int rd = 0;
    for (; rd + 1 < nr; rd += 2) {
        // round rd from buffer 0 and xa; round rd + 1's weights (wb) go to buffer 1
        load_xround<TYPE, T>(a, nb, r, g, (rd + 1) * GU + wave * GW, xb);
        load_wround<TYPE, PAIR>(a, nb, lrow, min(rd + 2, nr - 1), wa);
        round_terms<TYPE, PAIR, T>(lq[0], ld[0], wave, r, g, xa, wbd, tot, totu);
        stage<TYPE, PAIR>(wb, lq[1], ld[1]);
        __syncthreads();
        // round rd + 1 from buffer 1 and xb; round rd + 2's weights (wa) go to buffer 0
        load_xround<TYPE, T>(a, nb, r, g, min(rd + 2, nr - 1) * GU + wave * GW, xa);
        load_wround<TYPE, PAIR>(a, nb, lrow, min(rd + 3, nr - 1), wb);
        round_terms<TYPE, PAIR, T>(lq[1], ld[1], wave, r, g, xb, wbd, tot, totu);
        stage<TYPE, PAIR>(wa, lq[0], ld[0]);
        __syncthreads();
    }
    if (rd < nr) round_terms<TYPE, PAIR, T>(lq[0], ld[0], wave, r, g, xa, wbd, tot, totu);  // an odd last round
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
            long long sw = tot[t][i], su = 0;
#pragma unroll
            for (int k = 0; k < NWAVES - 1; ++k) sw += red[k][0][t][i][lane];
            if constexpr (PAIR) {
                su = totu[t][i];
#pragma unroll
                for (int k = 0; k < NWAVES - 1; ++k) su += red[k][PAIR ? 1 : 0][t][i][lane];
            }
            const int row = r0 + 4 * g + i;
            if (row >= a.rows || tok >= a.n_tok) continue;
            const float v = fixed_to_float(sw);
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
    int tiles = (a.rows + GT - 1) / GT;
    for (int i = 0; i < a.n_more; ++i) {  // members follow each other, every one at least a tile
        if (a.more[i].tile0 != tiles || a.more[i].rows < 1) return hipErrorInvalidValue;
        tiles += (a.more[i].rows + GT - 1) / GT;
    }
    const dim3 grid(tiles);
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
        a.y_stride < a.rows || (a.epi == EPI_ADD && a.res_stride < a.rows) || a.n_more < 0 || a.n_more > GEMM_MAX_MORE ||
        (a.n_more && a.epi == EPI_SWIGLU))
        return hipErrorInvalidValue;
    for (int i = 0; i < a.n_more; ++i) {
        const GemmMore & o = a.more[i];
        if (o.epi == EPI_SWIGLU || o.y_stride < o.rows || (o.epi == EPI_ADD && o.res_stride < o.rows)) return hipErrorInvalidValue;
    }
    switch (type) {
    case T_Q4_0: return launch_type<T_Q4_0>(a, s);
    case T_Q4_1: return launch_type<T_Q4_1>(a, s);
    case T_Q8_0: return launch_type<T_Q8_0>(a, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace gq
