// The Gated DeltaNet step fused with its gated output norm, the ssm_out product and its residual sum (GdnOutArgs in
// gq_kernels.h; the reference's GDN_WITH_OUT, gemvqc16.h:75-81 and gemvqc16.cpp:872-903, which streams ssm_out
// while the heads finish).
//
// One launch of rows / 16 workgroups of 256 threads. Every workgroup owns 16 rows of ssm_out (16 lanes a row, lane
// l16 holding the row's 32-blocks l16 + 16 i) and holds them in registers while the heads are stepped. Workgroup
// h < hv also runs value head h's step; it requests the head's state rows and inputs before its weights, and the
// other workgroups request their weights about two microseconds after they start, so that the step's inputs are
// not queued behind the 9 MB of weights:
//   1. the head's 128 state rows (16 lanes a row, 8 rows a lane group) are stepped once;
//   2. the gated output norm of the head's 128 outputs and their Q8_0 quantization (element e in thread e, the
//      canonical pairwise sums), the gated output stored to y;
//   3. the head's 32 words of quants and 4 block words are published to the exchange area as 64-bit agent-scope
//      stores (coherent across the XCDs' L2 caches without a write-back), each word beside a nonzero tag: a word
//      and its tag arrive together, so no counter or store-completion wait is needed. The words go to 8 copies of
//      the area, one per XCD, so that the polls below spread over 8 times the cache lines;
//   4. the new state rows are written back where they were read.
// Every workgroup then polls its XCD's copy of the exchange words (agent-scope 64-bit loads, a word again only
// while its tag is unset, at most `polls` rounds) until every tag is set, puts the words in LDS, and forms its rows:
// each block term exact and floored to 2^-40 as in the GEMV, a row's terms summed in int64 across its 16 lanes
// (integer addition is order-free, so the sums are the GEMV's), rounded to FP32 once and added to the residual.
//
// The exchange area has two slots; the fused launches of a command list use them in turn, and each launch clears
// the other slot's tags once its own words are loaded (the launch before it, which used that slot, has ended; the
// next launch on it starts after this one ends). A list with an odd number of fused launches ends with a fill of
// slot 0.
//
// Workgroups are dispatched in index order, so the head workgroups (the lowest indices) run before any workgroup
// that waits for them can hold their place; the wait is still bounded, and a wait that runs out of polls sets the
// fault word (host memory, read by the host after the stream has finished) instead of the output.
#include "gq_gdn.h"
#include "gq_gemv_impl.h"

#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__) && !defined(__gfx942__)
#error "the exchange relies on gfx9 store counting (vmcnt); build for gfx950 (or gfx942)"
#endif

namespace gq {
namespace {

constexpr int GX_T = 256;   // threads per workgroup: 16 rows of 16 lanes
constexpr int GX_NBT = GDN_OUT_MAX_HEADS / 4;  // 32-blocks per lane at most (hv / 4)

constexpr unsigned long long XCH_TAG = 1ull << 32;  // an exchange word published in this launch: tag | word
constexpr int XCH_PER = (GDN_XCH_SLOT + GX_T - 1) / GX_T;  // exchange words a thread polls

__device__ __forceinline__ void xch_store(unsigned long long * p, unsigned long long v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long xch_load(const unsigned long long * p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Q8_0 of one value per thread (the quantize_half_core arithmetic spread over a 32-lane block): returns the quant.
// The block's largest magnitude: the DPP swaps within 16 lanes (every lane of a 16-lane row ends with the row's
// maximum), then one exchange between the two rows.
__device__ __forceinline__ int go_quant(float v, float & d) {
    float amax = fabsf(v);
    amax = fmaxf(amax, dpp_f32<DPP_XOR1>(amax));
    amax = fmaxf(amax, dpp_f32<DPP_XOR2>(amax));
    amax = fmaxf(amax, dpp_f32<DPP_HALF_MIRROR>(amax));
    amax = fmaxf(amax, dpp_f32<DPP_MIRROR>(amax));
    amax = fmaxf(amax, __shfl_xor(amax, 16, WAVE));
    d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const float y = v * id;
    return int(y + copysignf(0.49999997f, y));
}

// This workgroup's ssm_out rows, every lane's GX_NBT blocks requested in one straight run (blocks past hv / 4 re-read
// the row's first block and are not used).
template <int TYPE>
__device__ __forceinline__ void load_rows(const GdnOutArgs & a, int row, int nb, int nbt, WB (&wr)[GX_NBT]) {
    const int l16 = threadIdx.x & 15;
#pragma unroll
    for (int i = 0; i < GX_NBT; ++i) load_wb<TYPE>(a.w, size_t(row) * nb + (i < nbt ? l16 + 16 * i : 0), wr[i]);
}

// Value head h's step, gated norm and quantization; publishes the quants and block words and writes the new state
// rows (steps 1-4 above). The weights are requested after the step's inputs.
template <int TYPE>
__device__ __forceinline__ void head_step(const GdnOutArgs & a, int h, float * ys, float * hsum, int8_t * q8,
                                          uint32_t * qinfo, int row, int nb, int nbt, WB (&wr)[GX_NBT]) {
    const GdnArgs & g = a.g;
    const int t = threadIdx.x, l16 = t & 15, rg = t >> 4, lane = t & 63, kh = h % g.hk;
    const int e = t & 127;  // the element this thread gates (threads below 128)
    const float zv = a.z[h * 128 + e], wv = a.nw[e];  // first: the gate is formed while the state arrives
    float x[8][8];
#pragma unroll
    for (int it = 0; it < 8; ++it) {
        const float4 * p = reinterpret_cast<const float4 *>(g.src + (size_t(h) * 128 + rg + 16 * it) * 128 + 8 * l16);
        const float4 s0 = p[0], s1 = p[1];
        x[it][0] = s0.x; x[it][1] = s0.y; x[it][2] = s0.z; x[it][3] = s0.w;
        x[it][4] = s1.x; x[it][5] = s1.y; x[it][6] = s1.z; x[it][7] = s1.w;
    }
    float q[8], k[8], v[8];
    {
        const float4 * qp = reinterpret_cast<const float4 *>(g.q + kh * 128 + 8 * l16);
        const float4 * kp = reinterpret_cast<const float4 *>(g.k + kh * 128 + 8 * l16);
        const float4 q0 = qp[0], q1 = qp[1], k0 = kp[0], k1 = kp[1];
        q[0] = q0.x; q[1] = q0.y; q[2] = q0.z; q[3] = q0.w; q[4] = q1.x; q[5] = q1.y; q[6] = q1.z; q[7] = q1.w;
        k[0] = k0.x; k[1] = k0.y; k[2] = k0.z; k[3] = k0.w; k[4] = k1.x; k[5] = k1.y; k[6] = k1.z; k[7] = k1.w;
    }
#pragma unroll
    for (int it = 0; it < 8; ++it) v[it] = g.v[h * 128 + rg + 16 * it];
    const bool gates = g.flags & 8;
    const float gr = g.g[h], br = g.beta[h], dtv = gates ? g.dt[h] : 0.0f, av = gates ? g.a[h] : 0.0f;
    __builtin_amdgcn_sched_barrier(0);
    load_rows<TYPE>(a, row, nb, nbt, wr);
    __builtin_amdgcn_sched_barrier(0);
    const float zg = a.z_silu ? zv : silu_(zv);
    // 1. the step (the arithmetic of gdn_kernel)
    if (g.flags & 2) gdn_l2_qk(q, k, g.l2_eps);
    float bt;
    const float decay = gdn_gates(gates, gr, br, dtv, av, bt);
    float out[8];
    gdn_step_rows<8>(q, k, v, decay, bt, x, out);
    if (l16 == 0) {
#pragma unroll
        for (int it = 0; it < 8; ++it) ys[rg + 16 * it] = out[it] * g.scale;
    }
    __syncthreads();
    // 2. the gated output norm (gemvqc_gdn.h:284-346) and Q8_0 of the 128 values, element e in thread e: the sum of
    //    squares is the pairwise tree over the elements (64 lanes, then the two halves)
    if (t < 128) {
        const float yv = ys[e];
        const float half = pair_sum_lanes<64>(yv * yv);
        if (lane == 0) hsum[t >> 6] = half;
    }
    __syncthreads();
    if (t < 128) {
        const float sc = 1.0f / sqrtf((hsum[0] + hsum[1]) / 128.0f + a.rms_eps);
        const float gv = zg * ((ys[e] * sc) * wv);
        a.y[h * 128 + e] = gv;  // the gated output (the GDN command's y)
        float d;
        const int qv = go_quant(gv, d);
        q8[e] = int8_t(qv);
        int sum = qv;  // the block's quant sum (integer: any order)
        sum += dpp_i32<DPP_XOR1>(sum);
        sum += dpp_i32<DPP_XOR2>(sum);
        sum += dpp_i32<DPP_HALF_MIRROR>(sum);
        sum += dpp_i32<DPP_MIRROR>(sum);
        sum += __shfl_xor(sum, 16, WAVE);
        if ((e & 31) == 0) qinfo[e >> 5] = f2h(d) | (uint32_t(sum & 0xffff) << 16);
    }
    __syncthreads();
    // 3. publish: the head's 32 quant words, then its 4 block words, each beside the tag, in each XCD's copy
    for (int i = t; i < 36 * GDN_XCH_COPIES; i += GX_T) {
        const int j = i % 36, cp = i / 36;
        const uint32_t w = j < 32 ? reinterpret_cast<const uint32_t *>(q8)[j] : qinfo[j - 32];
        xch_store(a.xch + (size_t(a.slot) * GDN_XCH_COPIES + cp) * GDN_XCH_SLOT + h * 36 + j, XCH_TAG | w);
    }
    // 4. the new state rows
#pragma unroll
    for (int it = 0; it < 8; ++it) {
        float4 * p = reinterpret_cast<float4 *>(g.dst + (size_t(h) * 128 + rg + 16 * it) * 128 + 8 * l16);
        p[0] = make_float4(x[it][0], x[it][1], x[it][2], x[it][3]);
        p[1] = make_float4(x[it][4], x[it][5], x[it][6], x[it][7]);
    }
}

template <int TYPE>
__global__ __launch_bounds__(GX_T) void gdn_out_kernel(GdnOutArgs a) {
    __shared__ __align__(16) uint32_t xq[GDN_OUT_MAX_HEADS * 32];  // every head's quants
    __shared__ uint32_t xinfo[GDN_OUT_MAX_HEADS * 4];              // per block: fp16 d | sum of its quants << 16
    __shared__ float ys[128];
    __shared__ float hsum[2];
    __shared__ __align__(16) int8_t q8[128];
    __shared__ uint32_t qinfo[4];
    const int t = threadIdx.x, l16 = t & 15, b = int(blockIdx.x);
    const int hv = a.g.hv, nb = hv * 4, nbt = hv / 4, row = b * 16 + (t >> 4);
    WB wr[GX_NBT];
    float res;
    if (b < hv) {
        head_step<TYPE>(a, b, ys, hsum, q8, qinfo, row, nb, nbt, wr);
        res = a.res[row];
    } else {
        __builtin_amdgcn_s_sleep(64);  // about two microseconds: the heads' inputs go first
        load_rows<TYPE>(a, row, nb, nbt, wr);
        res = a.res[row];
        __builtin_amdgcn_s_waitcnt(0);  // polling starts once the weights are in
    }
    // this thread's exchange words t + 256 k (of this XCD's copy), polled until every tag is set
    const unsigned long long * area = a.xch + (size_t(a.slot) * GDN_XCH_COPIES + (b & (GDN_XCH_COPIES - 1))) * GDN_XCH_SLOT;
    const int nw = hv * 36;
    unsigned long long v[XCH_PER];
#pragma unroll
    for (int k = 0; k < XCH_PER; ++k) v[k] = 0;
    bool have = false;
    for (unsigned n = 0; n < a.polls && !have; ++n) {
#pragma unroll
        for (int k = 0; k < XCH_PER; ++k)
            if ((v[k] >> 32) != 1u) v[k] = xch_load(area + min(t + GX_T * k, nw - 1));
        have = true;
#pragma unroll
        for (int k = 0; k < XCH_PER; ++k) have = have && (v[k] >> 32) == 1u;
        if (!have) __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int k = 0; k < XCH_PER; ++k) {
        const int w = t + GX_T * k, h = w / 36, j = w % 36;
        if (w < nw) {
            if (j < 32) xq[h * 32 + j] = uint32_t(v[k]);
            else xinfo[h * 4 + j - 32] = uint32_t(v[k]);
        }
    }
    const int missing = __syncthreads_or(!have);
    if (missing && t == 0) __hip_atomic_store(a.fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    {  // this workgroup's share of the other slot's words (all copies), cleared for the launch after this one
        constexpr int all = GDN_XCH_COPIES * GDN_XCH_SLOT;
        unsigned long long * other = a.xch + size_t(1 - a.slot) * all;
        const int per = (all + int(gridDim.x) - 1) / int(gridDim.x), w0 = b * per;
        for (int w = w0 + t; w < min(w0 + per, all); w += GX_T) xch_store(other + w, 0ull);
    }
    if (missing) return;
    // every block term is an integer-valued double below 2^63 in magnitude: its high and low 32-bit parts are summed
    // in two FP64 accumulators (exact for GX_NBT terms), then joined into int64 once; blocks past hv / 4 add zero
    double acc_hi = 0.0, acc_lo = 0.0;
#pragma unroll
    for (int i = 0; i < GX_NBT; ++i) {
        const int blk = i < nbt ? l16 + 16 * i : l16;
        XB xb;
        const uint4 * p = reinterpret_cast<const uint4 *>(xq + blk * 8);
        const uint4 lo = p[0], hi = p[1];
        xb.q[0] = lo.x; xb.q[1] = lo.y; xb.q[2] = lo.z; xb.q[3] = lo.w;
        xb.q[4] = hi.x; xb.q[5] = hi.y; xb.q[6] = hi.z; xb.q[7] = hi.w;
        const uint32_t inf = xinfo[blk];
        xb.dx40 = h2f(inf & 0xffffu) * 1099511627776.0f;  // * 2^40, exact
        xb.sum = int(int16_t(inf >> 16));
        xb.sx40 = 0.0f;
        const double tv = i < nbt ? block_term<TYPE>(dot_block<TYPE>(wr[i], xb), wr[i].d, xb) : 0.0;
        const double th = floor(tv * 2.3283064365386963e-10);  // tv / 2^32
        acc_hi += th;
        acc_lo += __builtin_fma(-th, 4294967296.0, tv);  // 0 <= tv - th 2^32 < 2^32, exact
    }
    long long acc = (long long)(((unsigned long long)(long long)acc_hi << 32) + (unsigned long long)(long long)acc_lo);
    acc += dpp_i64<DPP_XOR1>(acc);  // the row's 16 lanes: every lane ends with the total
    acc += dpp_i64<DPP_XOR2>(acc);
    acc += dpp_i64<DPP_HALF_MIRROR>(acc);
    acc += dpp_i64<DPP_MIRROR>(acc);
    if (l16 == 0) a.out[row] = fixed_to_float(acc) + res;  // gemvqc16.cpp:282-301 (the ADD epilog)
}

}  // namespace

bool gdn_out_fits(int hv, int rows) {
    return hv >= 4 && hv <= GDN_OUT_MAX_HEADS && hv % 4 == 0 && rows % 16 == 0 && rows / 16 >= hv &&
           rows <= GDN_OUT_MAX_ROWS;
}

hipError_t launch_gdn_out(const GdnOutArgs & a, int type, hipStream_t s) {
    if (a.g.hk < 1 || a.g.hv % a.g.hk || a.g.n_tok > 1 || !gdn_out_fits(a.g.hv, a.rows) || !a.xch || !a.fault)
        return hipErrorInvalidValue;
    const dim3 grid(a.rows / 16);
    if (type == T_Q4_0) {
        GQ_LAUNCH(gdn_out_kernel<T_Q4_0>, grid, dim3(GX_T), 0, s, a);
    } else if (type == T_Q8_0) {
        GQ_LAUNCH(gdn_out_kernel<T_Q8_0>, grid, dim3(GX_T), 0, s, a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace gq
