// Reference-arithmetic GEMV (see gq_ref.h): the GEMV command and its groups and epilogs with the rows summed as the
// reference's CPU path sums them (gemvq_ref.h:94-265), bit for bit.
//
// The prologue is the canonical kernel's (the activation quantizers are the reference's already; only the folded
// norm's scale comes from ref_norm_value). Each wave then takes batches of RB rows of one member: lane l forms the
// FP32 terms of its blocks l, l + 64, .. (K-quants: of its 64-weight units, the per-index-class integer sums
// reduced over the four lanes of a super-block) and stores them in its wave's LDS rows; then lane j adds row j's
// terms in block order, from 0, as one FP32 chain (K-quants: lanes 16 j .. 16 j + 8 each run one of the row's
// partial chains over the super-blocks, and lane 16 j adds them in order). The epilog runs on the row's lane.
#include "gemvq_hip.h"
#include "gq_gemv_impl.h"
#include "gq_ref.h"
#include "gq_refmath.h"

namespace gq {
namespace {

constexpr int RB = 4;  // rows per batch

// FP32 block terms of row r (Q4_0 / Q8_0: float(sumi) * (d_w * d_x); Q4_1: (d_w * d_x) * float(sumi) + m_w * s_x)
// into t[b] for this lane's blocks.
template <int TYPE, int NU>
__device__ __forceinline__ void row_load(const WeightView & w, int r, int nb, int lane, WB * wb) {
#pragma unroll
    for (int k = 0; k < NU; ++k) {
        const int b = lane + 64 * k, bb = b < nb ? b : nb - 1;
        load_wb<TYPE>(w, size_t(r) * nb + bb, wb[k]);
    }
}
template <int TYPE, int NU>
__device__ __forceinline__ void row_terms_wb(const WB * wb, int nb, int lane, const XB * xb, const float * dx,
                                             const float * sx, float * t) {
#pragma unroll
    for (int k = 0; k < NU; ++k) {
        const int b = lane + 64 * k;
        if (b < nb) {
            const int si = dot_block<TYPE>(wb[k], xb[k]);
            float term;
            if (TYPE == T_Q4_1) {
                const float dw = h2f(wb[k].d & 0xffffu), mw = h2f(wb[k].d >> 16);
                term = (dw * dx[k]) * float(si) + mw * sx[k];
            } else {
                term = float(si) * (h2f(wb[k].d) * dx[k]);
            }
            t[b] = term;
        }
    }
}
template <int TYPE, int NU>
__device__ __forceinline__ void row_terms(const WeightView & w, int r, int nb, int lane, const XB * xb, const float * dx,
                                          const float * sx, float * t) {
    WB wb[NU];
    row_load<TYPE, NU>(w, r, nb, lane, wb);
    row_terms_wb<TYPE, NU>(wb, nb, lane, xb, dx, sx, t);
}

// Batch bi of the members' batches in order: its member and first row.
__device__ __forceinline__ void locate_batch(const GemvArgs & a, int bi, int & mi, int & r0) {
    int b0 = 0;
    mi = 0;
    for (; mi < a.n_members - 1; ++mi) {
        const int nbm = (a.m[mi].rows + RB - 1) / RB;
        if (bi < b0 + nbm) break;
        b0 += nbm;
    }
    r0 = (bi - b0) * RB;
}

// The per-index-class integer sums of one 64-weight unit: aux[l] = sum over its weights i with i % 8 == l of sc *
// (q8_i * q_i) (gemvq_ref.h:116-121, 165-167), and for Q5_K the unit's share of sum over the 16-groups of
// bsum * m (gemvq_ref.h:112-115). The weights are those of the canonical kernel's unit (dot_unit); a product's
// index class is its byte within the word and the word's parity, so it is isolated by a byte mask before the dot.
template <int TYPE>
__device__ __forceinline__ void unit_aux(const WK & w, const XK & x, int part, int * aux, int & sumi) {
#pragma unroll
    for (int l = 0; l < 8; ++l) aux[l] = 0;
    if (TYPE == T_Q6_K) {
        const int scA0 = int(int8_t(w.s0 & 0xff)), scA1 = int(int8_t((w.s0 >> 8) & 0xff));
        const int scB0 = int(int8_t((w.s0 >> 16) & 0xff)), scB1 = int(int8_t(w.s0 >> 24));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t ql = pick(i < 4 ? w.a0 : w.a1, i & 3), qh = pick(w.h0, i & 3);
            const int sh = 2 * (i >> 2);
            const uint32_t ua = (ql & 0x0F0F0F0Fu) | (((qh >> sh) & 0x03030303u) << 4);
            const uint32_t ub = ((ql >> 4) & 0x0F0F0F0Fu) | (((qh >> (sh + 4)) & 0x03030303u) << 4);
            // q = u - 32 in every byte (borrow-free: (u | 0x80) - 0x20 stays in [0x60, 0x9f])
            const uint32_t qa = ((ua | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
            const uint32_t qb = ((ub | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
            const int lb = (i & 1) ? 4 : 0, sa = i < 4 ? scA0 : scA1, sb = i < 4 ? scB0 : scB1;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t m = 0xffu << (8 * t);
                aux[lb + t] += sa * sdot4(qa & m, x.q[i], 0) + sb * sdot4(qb & m, x.q[8 + i], 0);
            }
        }
        sumi = 0;
    } else {
        const int j = part;
        int sc0, m0, sc1, m1;
        scale_min_k4(w, 2 * j, sc0, m0);
        scale_min_k4(w, 2 * j + 1, sc1, m1);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t qs = pick(i < 4 ? w.a0 : w.a1, i & 3), qh = pick(i < 4 ? w.h0 : w.h1, i & 3);
            const uint32_t q0 = (qs & 0x0F0F0F0Fu) | (((qh >> (2 * j)) & 0x01010101u) << 4);
            const uint32_t q1 = ((qs >> 4) & 0x0F0F0F0Fu) | (((qh >> (2 * j + 1)) & 0x01010101u) << 4);
            const int lb = (i & 1) ? 4 : 0;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t m = 0xffu << (8 * t);
                aux[lb + t] += sc0 * sdot4(q0 & m, x.q[i], 0) + sc1 * sdot4(q1 & m, x.q[8 + i], 0);
            }
        }
        sumi = m0 * (x.bs[0] + x.bs[1]) + m1 * (x.bs[2] + x.bs[3]);
    }
}

// K-quant terms of row r: per super-block sb, t[9 sb + l] = d * float(aux[l]) (d = fp16 d_w * the Q8_K d) and for
// Q5_K t[9 sb + 8] = dmin * float(sumi).
template <int TYPE, int NU>
__device__ __forceinline__ void row_load_kq(const WeightView & w, int r, int nu, int lane, WK * wk) {
    const int nsb = nu >> 2;
#pragma unroll
    for (int k = 0; k < NU; ++k) {
        const int u0 = lane + 64 * k, u = u0 < nu ? u0 : nu - 1;
        load_wk<TYPE>(w, size_t(r) * nsb + (u >> 2), u & 3, wk[k]);
    }
}
template <int TYPE, int NU>
__device__ __forceinline__ void row_terms_kq_wk(const WK * wk, int nu, int lane, const XK * xk, const uint32_t * info,
                                                float * t) {
#pragma unroll
    for (int k = 0; k < NU; ++k) {
        const int u = lane + 64 * k;
        int aux[8], sumi;
        unit_aux<TYPE>(wk[k], xk[k], u & 3, aux, sumi);
        const bool in = u < nu;
#pragma unroll
        for (int l = 0; l < 8; ++l) aux[l] = sum_lanes4_i32(in ? aux[l] : 0);
        sumi = sum_lanes4_i32(in ? sumi : 0);
        if (in && (u & 3) == 0) {
            const int sb = u >> 2;
            const float d8 = __uint_as_float(info[sb]);
            const float d = h2f(wk[k].d & 0xffffu) * d8;
#pragma unroll
            for (int l = 0; l < 8; ++l) t[9 * sb + l] = d * float(aux[l]);
            if (TYPE == T_Q5_K) {
                const float dmin = h2f(wk[k].d >> 16) * d8;
                t[9 * sb + 8] = dmin * float(sumi);
            }
        }
    }
}
template <int TYPE, int NU>
__device__ __forceinline__ void row_terms_kq(const WeightView & w, int r, int nu, int lane, const XK * xk,
                                             const uint32_t * info, float * t) {
    WK wk[NU];
    row_load_kq<TYPE, NU>(w, r, nu, lane, wk);
    row_terms_kq_wk<TYPE, NU>(wk, nu, lane, xk, info, t);
}

// Orders this wave's LDS writes before its later LDS reads (another lane's data); LDS keeps a wave's accesses in
// order, so keeping the compiler from moving them is enough.
__device__ __forceinline__ void wave_lds_order() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

template <int TYPE, int NU, bool PAIR>
__global__ __launch_bounds__(NT) void gemv_ref_kernel(GemvArgs a, int total_batches) {
    constexpr bool KQ = TYPE == T_Q5_K || TYPE == T_Q6_K;
    constexpr int TPR = KQ ? 16 * NU * 9 : 64 * NU;  // terms per row at most
    // a row of terms, padded against bank conflicts (K-quants: one float; Q4_0 / Q4_1 / Q8_0: four, so that each
    // row's chain reads its terms 16 bytes at a time)
    constexpr int STR = KQ ? TPR + 1 : TPR + 4;
    __shared__ Lds s;
    __shared__ __attribute__((aligned(16))) float tm[NWAVES][PAIR ? 2 : 1][RB][STR];
    __shared__ double red[NWAVES];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cols = a.cols, nb = cols / 32, nu = cols / 64, nsb = cols / 256;
    // ---- the wave's first batch of rows (Q4_0 / Q4_1 / Q8_0 up to 4096 columns) is requested before the
    // prologue, so its weights stream while the activation is quantized
    constexpr bool PRE = !KQ && NU <= 2;
    const int bi0 = blockIdx.x * NWAVES + wave;
    WB pre[PRE ? RB : 1][PRE ? NU : 1], pre2[PRE && PAIR ? RB : 1][PRE && PAIR ? NU : 1];
    if constexpr (PRE) {
        int mi = 0, r0 = 0;
        locate_batch(a, bi0 < total_batches ? bi0 : 0, mi, r0);
        const GemvMember & m = a.m[mi];
        const int n = min(RB, m.rows - r0);
        // a pair kernel's members other than the SwiGLU pair have no second matrix (w2 is not set for them here):
        // they read their own matrix again, whose terms are not used
        const WeightView & w2 = m.epi == EPI_SWIGLU ? m.w2 : m.w;
#pragma unroll
        for (int j = 0; j < RB; ++j) {
            row_load<TYPE, NU>(m.w, r0 + min(j, n - 1), nb, lane, pre[j]);
            if constexpr (PAIR) row_load<TYPE, NU>(w2, r0 + min(j, n - 1), nb, lane, pre2[j]);
        }
    }
    // ---- Q6_K of one unit per lane (up to 4096 columns; the output head's shape): each batch's rows are requested
    // before the previous batch's terms are formed (the first batch's before the prologue), the registers holding
    // two batches (head 166 -> 158 us at 151936 x 4096)
    constexpr bool KPRE = TYPE == T_Q6_K && NU == 1;
    const int bstride = gridDim.x * NWAVES;
    WK kcur[KPRE ? RB : 1][1], knext[KPRE ? RB : 1][1];
    if constexpr (KPRE) {
        if (bi0 < total_batches) {
            int mi = 0, r0 = 0;
            locate_batch(a, bi0, mi, r0);
            const GemvMember & m = a.m[mi];
            const int n = min(RB, m.rows - r0);
#pragma unroll
            for (int j = 0; j < RB; ++j) row_load_kq<TYPE, 1>(m.w, r0 + min(j, n - 1), cols / 64, lane, kcur[j]);
        }
    }
    // ---- prologue: the activation, with the folded norm in the reference's arithmetic, quantized into LDS
    const bool norm = a.xsrc == XSRC_NORM;
    float scale = 1.0f;
    if constexpr (KQ) {
        if (norm) {
            const float v = ref_norm_value(a.x, cols, a.norm_l2, red);
            scale = a.norm_l2 ? 1.0f / fmaxf(sqrtf(v), a.norm_eps) : 1.0f / sqrtf(v + a.norm_eps);
        }
        quantize_q8_K(a.x, cols, norm, a.norm_w, scale, s.xq, s.bs, s.info);
    } else {
        // thread t's items t + NT g (16 floats each) are loaded once, for the norm's share and the quantization
        constexpr int R = (NU + 1) / 2;  // rounds: cols <= 2048 NU = 16 NT R
        const int n16 = cols / 16;
        float xv[R][16], wv[R][16];
        const bool normw = norm && a.norm_w;
#pragma unroll
        for (int g = 0; g < R; ++g) {
            const int i = item_of(g, n16);
            load16(a.x + size_t(i) * 16, xv[g]);
            load16(normw ? a.norm_w + size_t(i) * 16 : a.x + size_t(i) * 16, wv[g]);
        }
        if (norm) {
            double p = 0.0;
#pragma unroll
            for (int g = 0; g < R; ++g) {
                if (tid + NT * g < n16) {
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        const float sq = xv[g][j] * xv[g][j];
                        p += double(sq);
                    }
                }
            }
            const float v = ref_norm_reduce(p, a.x, cols, a.norm_l2, red);
            scale = a.norm_l2 ? 1.0f / fmaxf(sqrtf(v), a.norm_eps) : 1.0f / sqrtf(v + a.norm_eps);
        }
#pragma unroll
        for (int g = 0; g < R; ++g) {
            float * v = xv[g];
            if (norm) {
                if (normw) {
#pragma unroll
                    for (int j = 0; j < 16; ++j) v[j] = (v[j] * scale) * wv[g][j];
                } else {
#pragma unroll
                    for (int j = 0; j < 16; ++j) v[j] = v[j] * scale;
                }
            }
            quantize_half(v, tid + NT * g, tid + NT * g < n16, s);
        }
    }
    __syncthreads();
    // ---- this lane's activation blocks (units), kept in registers
    XB xb[KQ ? 1 : NU];
    XK xk[KQ ? NU : 1];
    float dx[KQ ? 1 : NU], sx[KQ ? 1 : NU];
    if constexpr (KQ) {
#pragma unroll
        for (int k = 0; k < NU; ++k) load_xk<TYPE>(s, lane + 64 * k, nu, xk[k]);
    } else {
#pragma unroll
        for (int k = 0; k < NU; ++k) {
            const int b = lane + 64 * k, bb = b < nb ? b : nb - 1;
            load_xb<TYPE>(s, b, nb, xb[k]);
            dx[k] = h2f(s.info[bb] & 0xffffu);
            sx[k] = TYPE == T_Q4_1 ? h2f(s.s1[bb]) : 0.0f;
        }
    }
    // ---- batches of RB rows of one member: batch bi of the members' batches in order
    unsigned long long best = 0;
    const bool argmax = a.argmax_key != nullptr;
    for (int bi = bi0; bi < total_batches; bi += gridDim.x * NWAVES) {
        int mi = 0, r0 = 0;
        locate_batch(a, bi, mi, r0);
        const GemvMember & m = a.m[mi];
        const int n = min(RB, m.rows - r0);
        const bool pair = PAIR && m.epi == EPI_SWIGLU;
        if (PRE && bi == bi0) {  // the rows requested before the prologue
#pragma unroll
            for (int j = 0; j < RB; ++j) {
                row_terms_wb<TYPE, NU>(pre[j], nb, lane, xb, dx, sx, tm[wave][0][j]);
                if (pair) row_terms_wb<TYPE, NU>(pre2[PAIR ? j : 0], nb, lane, xb, dx, sx, tm[wave][PAIR ? 1 : 0][j]);
            }
        } else if constexpr (KPRE) {
            const int bn = bi + bstride;
            if (bn < total_batches) {
                int mn = 0, rn = 0;
                locate_batch(a, bn, mn, rn);
                const GemvMember & mb = a.m[mn];
                const int nn = min(RB, mb.rows - rn);
#pragma unroll
                for (int j = 0; j < RB; ++j) row_load_kq<TYPE, 1>(mb.w, rn + min(j, nn - 1), nu, lane, knext[j]);
            }
#pragma unroll
            for (int j = 0; j < RB; ++j) row_terms_kq_wk<TYPE, 1>(kcur[j], nu, lane, xk, s.info, tm[wave][0][j]);
            if (bn < total_batches) {
#pragma unroll
                for (int j = 0; j < RB; ++j) kcur[j][0] = knext[j][0];
            }
        } else {
#pragma unroll
            for (int j = 0; j < RB; ++j) {
                const int r = r0 + min(j, n - 1);
                if constexpr (KQ) {
                    row_terms_kq<TYPE, NU>(m.w, r, nu, lane, xk, s.info, tm[wave][0][j]);
                } else {
                    row_terms<TYPE, NU>(m.w, r, nb, lane, xb, dx, sx, tm[wave][0][j]);
                    if (pair) row_terms<TYPE, NU>(m.w2, r, nb, lane, xb, dx, sx, tm[wave][PAIR ? 1 : 0][j]);
                }
            }
        }
        wave_lds_order();
        float v = 0.0f, u = 0.0f;
        if constexpr (KQ) {
            // lane 16 j + l: partial chain l (< 8) of row j over the super-blocks; Q5_K lane 16 j + 8: the dmin chain
            const int j = lane >> 4, l = lane & 15;
            const float * t = tm[wave][0][j];
            float acc = 0.0f;
            if (l < 8) {
                for (int sb = 0; sb < nsb; ++sb) acc += t[9 * sb + l];
            } else if (TYPE == T_Q5_K && l == 8) {
                for (int sb = 0; sb < nsb; ++sb) acc -= t[9 * sb + 8];
            }
            const int g0 = lane & ~15;
            float sumf = TYPE == T_Q5_K ? __shfl(acc, g0 + 8, WAVE) : 0.0f;
#pragma unroll
            for (int l2 = 0; l2 < 8; ++l2) sumf += __shfl(acc, g0 + l2, WAVE);
            v = __shfl(sumf, (lane & (RB - 1)) * 16, WAVE);  // lane j < RB: row j
        } else {
            // lane j < RB: row j (of g for a pair); lane RB + j: row j of u
            const int j = lane & (RB - 1), w2 = lane / RB;
            float acc = 0.0f;
            if (lane < (pair ? 2 * RB : RB)) {
                // the row's terms in block order, read 16 bytes at a time, two reads ahead of their additions
                const float * tf = tm[wave][PAIR ? w2 : 0][j];
                const float4 * t = reinterpret_cast<const float4 *>(tf);
                const int n4 = nb >> 2;
                int b = 0;
                for (; b + 2 <= n4; b += 2) {
                    const float4 x0 = t[b], x1 = t[b + 1];
                    acc += x0.x;
                    acc += x0.y;
                    acc += x0.z;
                    acc += x0.w;
                    acc += x1.x;
                    acc += x1.y;
                    acc += x1.z;
                    acc += x1.w;
                }
                if (b < n4) {
                    const float4 x0 = t[b];
                    acc += x0.x;
                    acc += x0.y;
                    acc += x0.z;
                    acc += x0.w;
                }
                for (int e = n4 * 4; e < nb; ++e) acc += tf[e];
            }
            v = __shfl(acc, j, WAVE);
            u = __shfl(acc, RB + j, WAVE);
        }
        if (lane < n) {
            const int r = r0 + lane;
            float out = v;
            switch (m.epi) {
            case EPI_SWIGLU: out = v / (1.0f + cr::expf(-v)) * u; break;  // gemvq_ref.h:303-307
            case EPI_ADD: out = v + m.res[r]; break;
            case EPI_SILU: out = cr::silu(v); break;
            case EPI_CONV: {  // gemvq_ref.h:344-358 on the row result
                const float s0 = m.conv_src[3 * r], s1 = m.conv_src[3 * r + 1], s2 = m.conv_src[3 * r + 2];
                float sum = 0.0f;
                sum += s0 * m.conv_w[4 * r];
                sum += s1 * m.conv_w[4 * r + 1];
                sum += s2 * m.conv_w[4 * r + 2];
                sum += v * m.conv_w[4 * r + 3];
                out = m.conv_silu ? cr::silu(sum) : sum;
                m.conv_dst[3 * r] = s1;
                m.conv_dst[3 * r + 1] = s2;
                m.conv_dst[3 * r + 2] = v;
                break;
            }
            default: break;
            }
            m.y[r] = out;
            if (argmax && mi == 0) {
                const unsigned long long key = argmax_key(out, uint32_t(r));
                best = key > best ? key : best;
            }
        }
        wave_lds_order();  // the next batch's terms overwrite these rows after every lane has read them
    }
    if (argmax) {
#pragma unroll
        for (int st = 1; st < 64; st <<= 1) {
            const unsigned long long o = (unsigned long long)shfl_xor_i64((long long)best, st);
            best = o > best ? o : best;
        }
        if (lane == 0 && best) atomicMax(a.argmax_key, best);
    }
}

template <int TYPE, int NU, bool PAIR>
hipError_t launch_ref_typed(const GemvArgs & a, hipStream_t st) {
    static const int cap = resident_blocks(gemv_ref_kernel<TYPE, NU, PAIR>);
    int batches = 0;
    for (int i = 0; i < a.n_members; ++i) batches += (a.m[i].rows + RB - 1) / RB;
    int grid = (batches + NWAVES - 1) / NWAVES;
    grid = grid < cap ? grid : cap;
    GQ_LAUNCH((gemv_ref_kernel<TYPE, NU, PAIR>), dim3(grid > 0 ? grid : 1), dim3(NT), 0, st, a, batches);
    return hipGetLastError();
}

template <int TYPE, int NU>
hipError_t launch_ref_pair(const GemvArgs & a, hipStream_t st) {
    bool pair = false;
    for (int i = 0; i < a.n_members; ++i) pair = pair || a.m[i].epi == EPI_SWIGLU;
    if constexpr (TYPE == T_Q5_K || TYPE == T_Q6_K) {
        if (pair) return hipErrorInvalidValue;
        return launch_ref_typed<TYPE, NU, false>(a, st);
    } else {
        return pair ? launch_ref_typed<TYPE, NU, true>(a, st) : launch_ref_typed<TYPE, NU, false>(a, st);
    }
}

template <int TYPE>
hipError_t launch_ref_nu(const GemvArgs & a, hipStream_t st) {
    constexpr bool KQ = TYPE == T_Q5_K || TYPE == T_Q6_K;
    const int nu = (a.cols / (KQ ? 64 : 32) + 63) / 64;
    switch (nu) {
    case 1: return launch_ref_pair<TYPE, 1>(a, st);
    case 2: return launch_ref_pair<TYPE, 2>(a, st);
    case 3: return launch_ref_pair<TYPE, 3>(a, st);
    case 4: return launch_ref_pair<TYPE, 4>(a, st);
    default: break;
    }
    if constexpr (!KQ) {
        switch (nu) {
        case 5: return launch_ref_pair<TYPE, 5>(a, st);
        case 6: return launch_ref_pair<TYPE, 6>(a, st);
        case 7: return launch_ref_pair<TYPE, 7>(a, st);
        case 8: return launch_ref_pair<TYPE, 8>(a, st);
        default: break;
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_gemv_ref(const GemvArgs & a, int type, hipStream_t s) {
    if (a.xsrc != XSRC_RAW && a.xsrc != XSRC_NORM) return hipErrorInvalidValue;
    switch (type) {
    case T_Q4_0: return launch_ref_nu<T_Q4_0>(a, s);
    case T_Q4_1: return launch_ref_nu<T_Q4_1>(a, s);
    case T_Q8_0: return launch_ref_nu<T_Q8_0>(a, s);
    case T_Q5_K: return launch_ref_nu<T_Q5_K>(a, s);
    case T_Q6_K: return launch_ref_nu<T_Q6_K>(a, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace gq
