// The Gated DeltaNet step fused with its gated output norm and the ssm_out product (GdnOutArgs in gq_kernels.h; the
// reference's GDN_WITH_OUT, gemvqc16.h:75-81 and gemvqc16.cpp:872-903, which streams ssm_out in column blocks as
// heads finish).
//
// `parts` workgroups of 1024 threads per value head (go_place). Every workgroup of the head
//   1. requests the head's state rows, q, k, v and gates, then its own rows / parts rows of the head's ssm_out
//      columns, 4 lanes per row and one 32-block per lane (the weights do not depend on the step, so they arrive
//      while it runs);
//   2. runs the step on all 128 state rows (two rows per 16-lane group, the arithmetic of the step kernel) and
//      stores its own 128 / parts new rows to the shadow rows (the others of the head still read the old ones);
//   3. forms the gated output norm of the head's 128 outputs and their Q8_0 quantization, one element per thread
//      over 128 threads, with the canonical pairwise sums;
//   4. multiplies them with its ssm_out rows: every block term exact and floored to 2^-40 as in the GEMV, a row's 4
//      terms summed exactly across its lanes and added into acc[row] with a 64-bit integer atomic. Integer addition
//      is order-free, so after the launch acc holds exactly the fixed-point sums of the whole ssm_out GEMV. The
//      launch that reads acc converts it (adds the residual) in its prologue and copies the shadow rows back into
//      the state.
#include "gq_gdn.h"
#include "gq_gemv_impl.h"

namespace gq {
namespace {

constexpr int GO_T = 1024;       // 64 groups of 16 lanes, each holding two state rows of the head
constexpr int GO_RR = GO_T / 4;   // ssm_out rows per round
constexpr int GO_RMAX = 4;        // rounds per workgroup (rows <= 1024 parts)

// Workgroup b's head and part: a head's parts run on one XCD (workgroups are dealt to the XCDs in turn), and the
// heads of one XCD are consecutive, so the 64-byte column slices of neighbouring heads, which share 128-byte lines,
// stream through one L2 (placement only affects speed, never what is computed).
__device__ __forceinline__ void go_place(int b, int hv, int & h, int & s) {
    if (hv % 8 == 0) {
        const int per = hv / 8, xcd = b & 7, k = b >> 3;  // k-th workgroup of the XCD: head xcd * per + k % per
        h = xcd * per + k % per;
        s = k / per;
    } else {
        h = b % hv;
        s = b / hv;
    }
}

// Q8_0 of one value per thread (the quantize_half_core arithmetic spread over a 32-lane block): returns the quant.
__device__ __forceinline__ int go_quant(float v, float & d) {
    float amax = fabsf(v);
#pragma unroll
    for (int s = 1; s < 32; s <<= 1) amax = fmaxf(amax, __shfl_xor(amax, s, WAVE));
    d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const float y = v * id;
    return int(y + copysignf(0.49999997f, y));
}

template <int TYPE>
__global__ __launch_bounds__(GO_T) void gdn_out_kernel(GdnOutArgs a) {
    __shared__ float ys[128];
    __shared__ float hsum[2];
    __shared__ __align__(16) int8_t xq8[128];  // the head's 128 quants
    __shared__ uint32_t xinfo[4];              // per block: fp16 d | sum of its quants << 16
    const GdnArgs & g = a.g;
    int h, s;  // head, part
    go_place(int(blockIdx.x), g.hv, h, s);
    const int t = threadIdx.x, l16 = t & 15, rg = t >> 4, lane = t & 63;
    const int nb = g.hv * 4;
    const int rows_per = a.rows / a.parts, r_lo = s * rows_per;  // rows a multiple of 256 parts
    // 1. what the step needs, then this part's weight rows: 4 lanes per row (lane t & 3 holds block 4 h + (t & 3)),
    //    256 rows per round
    const int kh = h % g.hk;
    float x[2][8];
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const float4 * p = reinterpret_cast<const float4 *>(g.src + (size_t(h) * 128 + rg + 64 * it) * 128 + 8 * l16);
        const float4 s0 = p[0], s1 = p[1];
        x[it][0] = s0.x; x[it][1] = s0.y; x[it][2] = s0.z; x[it][3] = s0.w;
        x[it][4] = s1.x; x[it][5] = s1.y; x[it][6] = s1.z; x[it][7] = s1.w;
    }
    float q[8], k[8];
    {
        const float4 * qp = reinterpret_cast<const float4 *>(g.q + kh * 128 + 8 * l16);
        const float4 * kp = reinterpret_cast<const float4 *>(g.k + kh * 128 + 8 * l16);
        const float4 q0 = qp[0], q1 = qp[1], k0 = kp[0], k1 = kp[1];
        q[0] = q0.x; q[1] = q0.y; q[2] = q0.z; q[3] = q0.w; q[4] = q1.x; q[5] = q1.y; q[6] = q1.z; q[7] = q1.w;
        k[0] = k0.x; k[1] = k0.y; k[2] = k0.z; k[3] = k0.w; k[4] = k1.x; k[5] = k1.y; k[6] = k1.z; k[7] = k1.w;
    }
    const float v[2] = {g.v[h * 128 + rg], g.v[h * 128 + rg + 64]};
    const bool gates = g.flags & 8;
    const float gr = g.g[h], br = g.beta[h], dtv = gates ? g.dt[h] : 0.0f, av = gates ? g.a[h] : 0.0f;
    const int e = t & 127;  // the element this thread gates (threads below 128)
    const float zv = a.z[h * 128 + e], wv = a.nw[e];
    __builtin_amdgcn_sched_barrier(0);
    const int blk = t & 3, rt = t >> 2, nr = rows_per / GO_RR;  // block, row within the round, rounds (<= GO_RMAX)
    WB wr[GO_RMAX];
#pragma unroll
    for (int j = 0; j < GO_RMAX; ++j)
        if (j < nr) load_wb<TYPE>(a.w, size_t(r_lo + GO_RR * j + rt) * nb + 4 * h + blk, wr[j]);
    __builtin_amdgcn_sched_barrier(0);
    // 2. the step (the arithmetic of gdn_kernel); this part's rows of the new state go to the shadow rows
    if (g.flags & 2) gdn_l2_qk(q, k, g.l2_eps);
    float bt;
    const float decay = gdn_gates(gates, gr, br, dtv, av, bt);
    float out[2];
    gdn_step_rows<2>(q, k, v, decay, bt, x, out);
    const int own = 128 / a.parts;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int j = rg + 64 * it;
        if (j / own == s) {
            float4 * p = reinterpret_cast<float4 *>(a.shadow + (size_t(h) * 128 + j) * 128 + 8 * l16);
            p[0] = make_float4(x[it][0], x[it][1], x[it][2], x[it][3]);
            p[1] = make_float4(x[it][4], x[it][5], x[it][6], x[it][7]);
        }
    }
    if (l16 == 0) {
        ys[rg] = out[0] * g.scale;
        ys[rg + 64] = out[1] * g.scale;
    }
    __syncthreads();
    // 3. the gated output norm (gemvqc_gdn.h:284-346) and Q8_0 of the 128 values, element e in thread e: the sum of
    //    squares is the pairwise tree over the elements (64 lanes, then the two halves)
    if (t < 128) {
        const float yv = ys[e];
        const float half = pair_sum_lanes<64>(yv * yv);
        if (lane == 0) hsum[t >> 6] = half;
    }
    __syncthreads();
    if (t < 128) {
        const float sc = 1.0f / sqrtf((hsum[0] + hsum[1]) / 128.0f + a.rms_eps);
        const float zg = a.z_silu ? zv : silu_(zv);
        const float gv = zg * ((ys[e] * sc) * wv);
        if (s == 0) a.y[h * 128 + e] = gv;  // the gated output (the GDN command's y)
        float d;
        const int qv = go_quant(gv, d);
        xq8[e] = int8_t(qv);
        int sum = qv;
#pragma unroll
        for (int m = 1; m < 32; m <<= 1) sum += __shfl_xor(sum, m, WAVE);
        if ((e & 31) == 0) xinfo[e >> 5] = f2h(d) | (uint32_t(sum & 0xffff) << 16);
    }
    __syncthreads();
    // 4. this thread's block of its rows: the block terms of a row (4 consecutive lanes) summed exactly and added into
    //    the row's accumulator
    {
        XB xb;
        const uint4 * p = reinterpret_cast<const uint4 *>(xq8 + 32 * blk);
        const uint4 lo = p[0], hi = p[1];
        xb.q[0] = lo.x; xb.q[1] = lo.y; xb.q[2] = lo.z; xb.q[3] = lo.w;
        xb.q[4] = hi.x; xb.q[5] = hi.y; xb.q[6] = hi.z; xb.q[7] = hi.w;
        const uint32_t inf = xinfo[blk];
        xb.dx40 = h2f(inf & 0xffffu) * 1099511627776.0f;  // * 2^40, exact
        xb.sum = int(int16_t(inf >> 16));
        xb.sx40 = 0.0f;
#pragma unroll
        for (int j = 0; j < GO_RMAX; ++j) {
            if (j < nr) {
                long long tv = dint_to_i64(block_term<TYPE>(dot_block<TYPE>(wr[j], xb), wr[j].d, xb));
                tv += dpp_i64<DPP_XOR1>(tv);
                tv += dpp_i64<DPP_XOR2>(tv);
                if (blk == 0) atomicAdd(a.acc + r_lo + GO_RR * j + rt, (unsigned long long)tv);
            }
        }
    }
    // 5. this workgroup's share of the other accumulator is cleared for the next fused step
    const int nwg = g.hv * a.parts, wg = blockIdx.x;
    const int z0 = int((long long)wg * a.rows / nwg), z1 = int((long long)(wg + 1) * a.rows / nwg);
    for (int r = z0 + t; r < z1; r += GO_T) a.zero[r] = 0ull;
}

}  // namespace

// Parts per head: 8 when the rows split into whole rounds, else as few as hold them (0: the shape does not fit).
int gdn_out_parts(int rows) {
    for (int p : {8, 4, 16, 32, 64, 128})
        if (rows % (GO_RR * p) == 0 && rows / p <= GO_RR * GO_RMAX) return p;
    return 0;
}

hipError_t launch_gdn_out(const GdnOutArgs & a, int type, hipStream_t s) {
    // the parts split the rows into whole rounds and the head's 128 state rows evenly
    if (a.g.hv < 1 || a.g.hv > GDN_MAX_HEADS || a.g.hk < 1 || a.g.hv % a.g.hk || a.g.n_tok > 1 || a.rows < 1 ||
        a.parts < 1 || 128 % a.parts || a.rows % (GO_RR * a.parts) || a.rows / a.parts > GO_RR * GO_RMAX)
        return hipErrorInvalidValue;
    const dim3 grid(a.g.hv * a.parts);
    if (type == T_Q4_0) {
        GQ_LAUNCH(gdn_out_kernel<T_Q4_0>, grid, dim3(GO_T), 0, s, a);
    } else if (type == T_Q8_0) {
        GQ_LAUNCH(gdn_out_kernel<T_Q8_0>, grid, dim3(GO_T), 0, s, a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace gq
