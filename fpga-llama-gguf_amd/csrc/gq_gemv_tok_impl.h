#pragma once
// The GEMM command for 1-4 tokens (TokArgs) on the single-token GEMV's structure: the same workgroups, XCD slices,
// rows in flight and exact block (K-quant super-block) terms as gemv_kernel, with every lane holding its activation
// blocks (units) of all T tokens in registers. A weight row is streamed and unpacked once and its block terms are
// formed for each token; each token's row total is rounded once and goes through the member's epilog. The tokens
// are quantized in the prologue of every workgroup, each exactly as the single-token prologue quantizes one vector
// (the same norm scale tree and quantizer), so token t's output row is the single-token GEMV's (and the MFMA
// batched GEMV's) bit for bit. For Q4_0 / Q8_0 it replaces a quantization launch plus a batched GEMV whose time is
// that of 16 tokens (one MFMA tile); for the K-quants, which have no MFMA form, one GEMV per token.
#include "gq_gemv_impl.h"

namespace gq {
namespace {

template <bool KQ, int NU>
constexpr int tok_cols() { return (KQ ? 4096 : 2048) * NU; }  // columns at most: 64 NU blocks or units per row

template <int T, int NU, int R, bool KQ>
struct LdsTok {  // T quantized activations: Q8_0 (d | sum words, Q8_1 s) or Q8_K (d bits per super-block, bsums)
    static constexpr int C = tok_cols<KQ, NU>();
    int8_t xq[T][C];
    uint32_t info[T][KQ ? C / 256 : C / 32];
    uint16_t s1[T][KQ ? 1 : C / 32];
    int16_t bs[T][KQ ? C / 16 : 1];
    float red[T * R * NWAVES];
};

struct TokHot {
    const float * x;
    const float * norm_w;
    int cols, x_stride, norm;
};

template <int T, int R>  // R rounds of NT 16-float items per token
struct XT {
    float v[T][R][16];
    float w[R <= 2 ? R : 1][16];  // the norm weight (the activation again without one)
};

// Token t's items, and the norm weight's (R <= 2; wider rows read it when they use it), all issued together and
// without branches.
// h: the preloaded leading kernel arguments (the rows, the norm weight, the columns, the row stride, the norm flag).
template <int T, int R>
__device__ __forceinline__ void tok_fetch(const TokHot & h, XT<T, R> & f) {
    const int n16 = h.cols / 16;
    const bool normw = h.norm && h.norm_w != nullptr;
#pragma unroll
    for (int g = 0; g < R; ++g) {
        const int i = item_of(g, n16);
#pragma unroll
        for (int t = 0; t < T; ++t) load16(h.x + size_t(t) * h.x_stride + size_t(i) * 16, f.v[t][g]);
        if constexpr (R <= 2) load16(normw ? h.norm_w + size_t(i) * 16 : h.x + size_t(i) * 16, f.w[g]);
    }
}

// Each token as the single-token prologue does one vector (XSRC_NORM or the raw rows): the canonical norm scale (a
// tree over each item's 16 squares, pairwise over a wave's 64 items, the 4 waves of a round and the rounds), then
// Q8_0 (and the Q8_1 s) of v = (x * scale) * w into the token's LDS rows, or for K-quant weights Q8_K of the same v
// (quantize_q8_K, which reads the row again in its own layout).
template <int T, int NU, int R, bool KQ>
__device__ __forceinline__ void tok_finish(const TokArgs & a, XT<T, R> & f, LdsTok<T, NU, R, KQ> & s) {
    const int n16 = a.cols / 16, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float sc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) sc[t] = 1.0f;
    if (a.norm) {
        float r[T * R];
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int g = 0; g < R; ++g) {
                float sq[16];
#pragma unroll
                for (int j = 0; j < 16; ++j) sq[j] = f.v[t][g][j] * f.v[t][g][j];
                r[t * R + g] = int(threadIdx.x) + NT * g < n16 ? tree<16>(sq) : 0.0f;
            }
        pair_sum_lanes_n<64, T * R>(r);
        if (lane == 0) {
#pragma unroll
            for (int k = 0; k < T * R; ++k) s.red[NWAVES * k + wave] = r[k];
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < T; ++t) {
            float rs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int g = 0; g < R; ++g) rs[g] = wave_tree(s.red + NWAVES * (t * R + g));
            const float sum = R == 1 ? rs[0] : R == 2 ? rs[0] + rs[1] : (rs[0] + rs[1]) + (rs[2] + rs[3]);
            sc[t] = a.norm_l2 ? 1.0f / fmaxf(sqrtf(sum), a.eps) : 1.0f / sqrtf(sum / float(a.cols) + a.eps);
        }
    }
    if constexpr (KQ) {
#pragma unroll
        for (int t = 0; t < T; ++t)
            quantize_q8_K(a.x + size_t(t) * a.x_stride, a.cols, a.norm != 0, a.norm_w, sc[t], s.xq[t], s.bs[t], s.info[t]);
        return;
    }
    const bool normw = a.norm && a.norm_w != nullptr;
#pragma unroll
    for (int g = 0; g < R; ++g) {
        const int i = int(threadIdx.x) + NT * g;
        float w[16];
        if constexpr (R <= 2) {
#pragma unroll
            for (int j = 0; j < 16; ++j) w[j] = normw ? f.w[g][j] : 1.0f;
        } else if (normw) {
            load16(a.norm_w + size_t(item_of(g, n16)) * 16, w);
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) w[j] = 1.0f;
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            float * v = f.v[t][g];
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = (v[j] * sc[t]) * w[j];
            quantize_half(v, i, i < n16, s.xq[t], s.info[t], s.s1[t]);
        }
    }
}

template <int T>
constexpr int tok_groups() { return T == 1 ? 1 : T == 2 ? 2 : 4; }  // lane groups of a row's reduction

template <int TYPE, int NU, bool PAIR>
struct TSlot {  // one row in flight: its blocks (of g and u for a SwiGLU pair) or K-quant units, and the lane's
                // epilog operand
    static constexpr bool KQ = TYPE == T_Q5_K || TYPE == T_Q6_K;
    WB wb[KQ ? 1 : NU], wb2[(KQ || !PAIR) ? 1 : NU];
    WK wk[KQ ? NU : 1];
    float e;  // ADD: the residual of row r for the lane group's token
};

// Loads of row r. Lane group g (of G groups of 64 / G lanes) takes token min(g, T - 1)'s epilog operand (a
// member without a residual reads its own output row, unused), so no load sits behind a branch.
template <int TYPE, int NU, bool PAIR, int T>
__device__ __forceinline__ void load_tok_slot(const TokMember & m, int r, int lane, int nb, int nu,
                                              TSlot<TYPE, NU, PAIR> & o) {
    constexpr int G = tok_groups<T>(), GW = 64 / G;
    if constexpr (TSlot<TYPE, NU, PAIR>::KQ) {
        const int nsb = nu >> 2;
#pragma unroll
        for (int k = 0; k < NU; ++k) {
            const int u0 = lane + 64 * k, u = u0 < nu ? u0 : nu - 1;
            load_wk<TYPE>(m.w, size_t(r) * nsb + (u >> 2), u & 3, o.wk[k]);
        }
    } else {
#pragma unroll
        for (int k = 0; k < NU; ++k) {
            const int b = lane + 64 * k, bb = b < nb ? b : nb - 1;
            load_wb<TYPE>(m.w, size_t(r) * nb + bb, o.wb[k]);
            if constexpr (PAIR) load_wb<TYPE>(m.w2, size_t(r) * nb + bb, o.wb2[k]);
        }
    }
    const int g = lane / GW, tk = g < T ? g : T - 1;
    o.e = m.res[size_t(tk) * m.res_stride + r];
}

// Row r's T token totals through one cross-lane reduction (lane group g ends with token g's), then the epilog as
// finish_chunk forms it, stored by the groups' first lanes.
template <int T, bool PAIR>
__device__ __forceinline__ void finish_tok_row(const TokMember & m, int r, const long long * p, const long long * p2,
                                               float ev, int lane) {
    constexpr int G = tok_groups<T>(), GW = 64 / G;
    long long pp[G];
#pragma unroll
    for (int j = 0; j < G; ++j) pp[j] = j < T ? p[j < T ? j : 0] : 0;
    const long long tot = reduce_rows<G>(pp);
    const int g = lane / GW;
    const float v = fixed_to_float(tot);
    float out = v;
    if constexpr (PAIR) {
        long long qq[G];
#pragma unroll
        for (int j = 0; j < G; ++j) qq[j] = j < T ? p2[j < T ? j : 0] : 0;
        const long long tot2 = reduce_rows<G>(qq);
        out = (v / (1.0f + expf_(-v))) * fixed_to_float(tot2);  // gemvqc_ops.h:88-92
    } else if (m.epi == EPI_ADD) {
        out = v + ev;  // gemvqc16.cpp:282-301
    } else if (m.epi == EPI_SILU) {
        out = silu_(v);
    }
    if ((lane & (GW - 1)) == 0 && g < T) m.y[size_t(g) * m.y_stride + r] = out;
}

template <int TYPE, int NU, bool PAIR, int T, bool EXACT>
__device__ __forceinline__ void tok_partials(const TSlot<TYPE, NU, PAIR> & sl, int r, int nb, int nu,
                                             const XB (*xb)[NU], const XK (*xk)[NU], int lane, long long * p,
                                             long long * p2) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
        p2[t] = 0;
        if constexpr (TSlot<TYPE, NU, PAIR>::KQ) {
            p[t] = lane_units<TYPE, NU>(sl.wk, r, true, nu, xk[t], lane, nullptr);
        } else {
            p[t] = lane_blocks<TYPE, NU, EXACT>(sl.wb, r, true, nb, xb[t], lane, nullptr);
            if constexpr (PAIR) p2[t] = lane_blocks<TYPE, NU, EXACT>(sl.wb2, r, true, nb, xb[t], lane, nullptr);
        }
    }
}

// The n rows w, w + S, ... of one member with DS in flight: a slot is refilled with the row DS further on as soon
// as its partials are formed (unconditionally while rows follow, so the compiler's waits stay exact).
template <int TYPE, int NU, bool PAIR, int T, int DS, bool EXACT>
__device__ __forceinline__ void tok_rows(const TokMember & m, int w, int S, int n, TSlot<TYPE, NU, PAIR> * sl,
                                         const XB (*xb)[NU], const XK (*xk)[NU], int lane, int nb, int nu) {
    long long p[T], p2[T];
    int k = 0;
    for (; k + DS < n; k += DS) {
#pragma unroll
        for (int j = 0; j < DS; ++j) {
            const int r = w + (k + j) * S;
            tok_partials<TYPE, NU, PAIR, T, EXACT>(sl[j], r, nb, nu, xb, xk, lane, p, p2);
            const float ev = sl[j].e;
            load_tok_slot<TYPE, NU, PAIR, T>(m, w + min(k + j + DS, n - 1) * S, lane, nb, nu, sl[j]);
            finish_tok_row<T, PAIR>(m, r, p, p2, ev, lane);
        }
    }
#pragma unroll
    for (int j = 0; j < DS; ++j) {
        if (k + j < n) {
            const int r = w + (k + j) * S;
            tok_partials<TYPE, NU, PAIR, T, EXACT>(sl[j], r, nb, nu, xb, xk, lane, p, p2);
            finish_tok_row<T, PAIR>(m, r, p, p2, sl[j].e, lane);
        }
    }
}

// Rows in flight per wave: two for plain members of at most 4096 columns (Q4_0 / Q8_0), one for SwiGLU pairs, wider
// rows and K-quant units (whose T tokens' activations already take most of the registers).
template <int TYPE, int NU, bool PAIR>
constexpr int tok_slots() { return PAIR || NU > 2 || TYPE == T_Q5_K || TYPE == T_Q6_K ? 1 : 2; }

// The activation rows, norm weight, columns, row stride, norm flag, member count and the members' first waves are
// leading scalar arguments (preloaded into SGPRs where the firmware supports it), so the activation loads and the
// member choice wait for no load of the argument segment.
template <int TYPE, int NU, bool PAIR, int T>
__global__ __launch_bounds__(NT) void gemv_tok_kernel(const float * x, const float * norm_w, int cols, int x_stride,
                                                      int norm, int n_members, int wb1, int wb2, int wb3, TokArgs a) {
    constexpr bool KQ = TYPE == T_Q5_K || TYPE == T_Q6_K;
    constexpr int DS = tok_slots<TYPE, NU, PAIR>();
    constexpr int R = (tok_cols<KQ, NU>() / 16 + NT - 1) / NT;  // rounds of NT activation items per token
    __shared__ LdsTok<T, NU, R, KQ> s;
    XT<T, R> f;
    tok_fetch<T, R>(TokHot{x, norm_w, cols, x_stride, norm}, f);  // the activations are requested first
    __builtin_amdgcn_sched_barrier(0);  // and stay ahead of the member lookup and the weight loads
    const int lane = threadIdx.x & 63, nb = cols / 32, nu = cols / 64;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // workgroup b serves slice b % 8 of every member's rows (one XCD's L2), as gemv_kernel
    const int xs = blockIdx.x & 7, lw = (blockIdx.x >> 3) * NWAVES + wave;
    const int mi = n_members > 3 && lw >= wb3 ? 3 : n_members > 2 && lw >= wb2 ? 2 : n_members > 1 && lw >= wb1 ? 1 : 0;
    const TokMember & m = a.m[mi];
    // the member fields that the first weight and epilog operand loads need, requested in one round of scalar loads
    asm volatile("" ::"s"(m.rows), "s"(m.wave_begin), "s"(m.waves), "s"(m.w.a), "s"(m.w.b), "s"(m.w.c), "s"(m.w2.a),
                 "s"(m.w2.b), "s"(m.w2.c), "s"(m.res), "s"(m.res_stride));
    const int s_lo = int((long long)xs * m.rows / 8), len = int((long long)(xs + 1) * m.rows / 8) - s_lo;
    const int wv = lw - m.wave_begin, S = m.waves;
    // computed without a branch, so that the member's remaining fields are loaded in the same round as these
    const int q = int(unsigned(max(len - 1 - wv, 0)) / unsigned(max(S, 1)));
    const int n = wv < S && wv < len ? q + 1 : 0;  // waves past the last member have none
    const int w = s_lo + wv;
    TSlot<TYPE, NU, PAIR> sl[DS];
#pragma unroll
    for (int j = 0; j < DS; ++j)
        load_tok_slot<TYPE, NU, PAIR, T>(m, n > 0 ? w + min(j, n - 1) * S : m.rows - 1, lane, nb, nu, sl[j]);
    tok_finish<T, NU, R, KQ>(a, f, s);
    __syncthreads();
    XB xb[T][NU];  // (only the arrays of the weight kind are used; the other is removed by the compiler)
    XK xk[T][NU];
    bool exact = false;
    if constexpr (KQ) {  // super-block terms are summed in int64
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int k = 0; k < NU; ++k) load_xk<TYPE>(s.xq[t], s.bs[t], s.info[t], lane + 64 * k, nu, xk[t][k]);
    } else {
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int k = 0; k < NU; ++k) load_xb<TYPE>(s.xq[t], s.info[t], s.s1[t], lane + 64 * k, nb, xb[t][k]);
        // the single-token kernel's bound on a lane's FP64 partial (below 2^53 LSB), for every token: a wave where
        // it could be passed sums its terms in two FP64 parts (EXACT)
        bool big = false;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            float dsum = 0.0f;
#pragma unroll
            for (int k = 0; k < NU; ++k) dsum += fabsf(xb[t][k].dx40);
            big = big || !(a.wbound[mi] * dsum < 4503599627370496.0f);
        }
        exact = __builtin_amdgcn_ballot_w64(big) != 0;
    }
    if (n > 0) {
        if (!KQ && exact) tok_rows<TYPE, NU, PAIR, T, DS, true>(m, w, S, n, sl, xb, xk, lane, nb, nu);
        else tok_rows<TYPE, NU, PAIR, T, DS, false>(m, w, S, n, sl, xb, xk, lane, nb, nu);
    }
}

template <int TYPE, int NU, bool PAIR, int T>
hipError_t launch_tok_typed(const TokArgs & a0, hipStream_t st) {
    static const int cap = resident_blocks(gemv_tok_kernel<TYPE, NU, PAIR, T>, gemv_wg_per_cu(NU));
    TokArgs a = a0;
    for (int i = 0; i < a.n_members; ++i) {
        TokMember & m = a.m[i];
        if (m.epi != EPI_ADD) {  // the epilog operand load reads the member's own output rows
            m.res = m.y;
            m.res_stride = m.y_stride;
        }
        if (m.epi != EPI_SWIGLU) m.w2 = m.w;
    }
    const int grid = plan_waves(a, cap, tok_slots<TYPE, NU, PAIR>());
    GQ_LAUNCH((gemv_tok_kernel<TYPE, NU, PAIR, T>), dim3(grid), dim3(NT), 0, st, a.x, a.norm_w, a.cols, a.x_stride,
              a.norm, a.n_members, a.n_members > 1 ? a.m[1].wave_begin : 0, a.n_members > 2 ? a.m[2].wave_begin : 0,
              a.n_members > 3 ? a.m[3].wave_begin : 0, a);
    return hipGetLastError();
}

// Instances (gemv_tok_ok states the same): Q4_0 / Q8_0 (NU blocks of 32 per lane) T = 2-4 tokens for rows of at
// most 4096 columns (NU <= 2) and T = 2 up to 12288 (NU <= 6), with SwiGLU pairs; Q5_K / Q6_K (NU units of 64 per
// lane) T = 1-4 up to 4096 columns and T = 1-2 up to 12288, without pairs.
template <int TYPE>
constexpr bool tok_instance(int nu, int t) {
    if constexpr (TYPE == T_Q5_K || TYPE == T_Q6_K) return t >= 1 && t <= TOK_MAX && (nu == 1 || (nu <= 3 && t <= 2));
    return t >= 2 && t <= TOK_MAX && (nu <= 2 || (nu <= 6 && t == 2));
}

template <int TYPE, int NU, int T>
hipError_t launch_tok_nu_t(const TokArgs & a, hipStream_t st) {
    constexpr bool KQ = TYPE == T_Q5_K || TYPE == T_Q6_K;
    if constexpr (tok_instance<TYPE>(NU, T)) {
        if (a.m[0].epi != EPI_SWIGLU) return launch_tok_typed<TYPE, NU, false, T>(a, st);
        if constexpr (!KQ) return launch_tok_typed<TYPE, NU, true, T>(a, st);
    }
    return hipErrorInvalidValue;
}

template <int TYPE, int NU>
hipError_t launch_tok_nu(const TokArgs & a, hipStream_t st) {
    switch (a.n_tok) {
    case 1: return launch_tok_nu_t<TYPE, NU, 1>(a, st);
    case 2: return launch_tok_nu_t<TYPE, NU, 2>(a, st);
    case 3: return launch_tok_nu_t<TYPE, NU, 3>(a, st);
    case 4: return launch_tok_nu_t<TYPE, NU, 4>(a, st);
    default: return hipErrorInvalidValue;
    }
}

template <int TYPE>
hipError_t launch_tok_type(const TokArgs & a, hipStream_t st) {
    constexpr bool KQ = TYPE == T_Q5_K || TYPE == T_Q6_K;
    switch ((a.cols / (KQ ? 64 : 32) + 63) / 64) {
    case 1: return launch_tok_nu<TYPE, 1>(a, st);
    case 2: return launch_tok_nu<TYPE, 2>(a, st);
    case 3: return launch_tok_nu<TYPE, 3>(a, st);
    case 4: return launch_tok_nu<TYPE, 4>(a, st);
    case 5: return launch_tok_nu<TYPE, 5>(a, st);
    case 6: return launch_tok_nu<TYPE, 6>(a, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace
}  // namespace gq
