// Reference-arithmetic mode (gemvq_set_arith): the reference's CPU arithmetic (fpga/src/gemvq_ref.h, composed as
// ggml's graph composes it) evaluated on the GPU, so that a decode gives the tokens and logits of that CPU path bit
// for bit. Launch descriptors and launchers shared by the host command processor and gq_ref.hip / gq_ref_gemv.hip.
//
// Where the canonical kernels sum in fixed point or by pairwise trees, these follow the reference's order:
//   - GEMV rows: the FP32 block terms float(sumi) * (d_w * d_x) added in block order from 0 (Q4_1: (d_w d_x)
//     float(sumi) + m_w s_x); Q5_K / Q6_K: eight FP32 partial sums over the super-blocks of d * float(aux[l]), aux[l]
//     the integer sum of the products whose index is l modulo 8, then added in order (Q5_K starts from the running
//     difference of its dmin terms) (gemvq_ref.h:94-265);
//   - norms: the FP32 squares summed in double in index order, then float(sum / n) (gemvq_ref.h:309-324);
//   - the DeltaNet step: one thread per state row with its two dots in order (gemvq_ref.h:360-397);
//   - attention: F16 dots of the rounded query summed in double, softmax with a double sum, fp16 probabilities
//     times V summed in double (the reference leaves attention to ggml's CPU path, README.md:77);
//   - exp and log correctly rounded (gq_refmath.h) in SiLU, sigmoid, softplus, the decay and the softmax.
#pragma once
#include "gq_device.h"
#include "gq_kernels.h"

namespace gq {

// The reference's norm value of one row of n floats (n a multiple of 4, x 16-byte aligned), computed by the whole
// workgroup (blockDim.x a multiple of 64, at most 1024; red: shared memory of blockDim.x / 64 doubles): S = sum over
// i of double(x_i * x_i) (FP32 squares) in index order, then float(S / n) (RMS) or float(S) (L2)
// (gemvq_ref.h:309-324). S is first formed as T, the workgroup's sum in its own order (each thread's 4-float pieces,
// then across the lanes and the waves). Any order of adding n non-negative terms in double is within (n - 1) 2^-53 S
// of the exact sum, so the sequential sum lies in [T - E, T + E] with E = (n + 64) 2^-52 T (a factor 2 of margin);
// rounding is monotone, so when both ends give the same float the sequential sum gives it too. Otherwise (about one
// row in 10^5 at n = 4096) thread 0 adds the squares in order. Every thread returns the value.
template <int CTRL>
__device__ inline double dpp_f64(double v) {
    return __builtin_bit_cast(double, dpp_i64<CTRL>(__builtin_bit_cast(long long, v)));
}
// The second half of ref_norm_value: each thread's partial p of T (the double squares of its share of the row, in
// any order; the shares together cover the row once), then the workgroup's sum, the check and the fallback.
// The workgroup's sum of the threads' doubles p (in no particular order), on every thread; red holds a double per
// wave. Ends with the threads' reads of red pending: a following use of red needs a barrier first.
__device__ inline double ref_block_sum(double p, double * red) {
    const int tid = threadIdx.x, nt = blockDim.x;
    // across the wave: within rows of 16 lanes by DPP, then across the rows
    p += dpp_f64<DPP_XOR1>(p);
    p += dpp_f64<DPP_XOR2>(p);
    p += dpp_f64<DPP_HALF_MIRROR>(p);
    p += dpp_f64<DPP_MIRROR>(p);
    p += __shfl_xor(p, 16, 64);
    p += __shfl_xor(p, 32, 64);
    if ((tid & 63) == 0) red[tid >> 6] = p;
    __syncthreads();
    double t = 0.0;
    for (int w = 0; w < nt / 64; ++w) t += red[w];
    return t;
}
__device__ inline float ref_norm_reduce(double p, const float * x, int n, int l2, double * red) {
    const int tid = threadIdx.x;
    const double t = ref_block_sum(p, red);
    const double e = double(n + 64) * 2.220446049250313080847e-16 * t;
    const double lo = t - e, hi = t + e;
    const float vlo = l2 ? float(lo) : float(lo / double(n));
    const float vhi = l2 ? float(hi) : float(hi / double(n));
    float v = vlo;
    if (!(vlo == vhi)) {  // the same on every thread
        __syncthreads();
        if (tid == 0) {
            double q = 0.0;
            for (int i = 0; i < n; ++i) {
                const float sq = x[i] * x[i];
                q += double(sq);
            }
            red[0] = q;
        }
        __syncthreads();
        v = l2 ? float(red[0]) : float(red[0] / double(n));
    }
    __syncthreads();
    return v;
}
__device__ inline float ref_norm_value(const float * x, int n, int l2, double * red) {
    double p = 0.0;
    for (int i = 4 * int(threadIdx.x); i < n; i += 4 * int(blockDim.x)) {
        const float4 q = *reinterpret_cast<const float4 *>(x + i);
        const float s0 = q.x * q.x, s1 = q.y * q.y, s2 = q.z * q.z, s3 = q.w * q.w;
        p += double(s0);
        p += double(s1);
        p += double(s2);
        p += double(s3);
    }
    return ref_norm_reduce(p, x, n, l2, red);
}

hipError_t launch_gemv_ref(const GemvArgs & a, int type, hipStream_t s);
hipError_t launch_norm_ref(const NormArgs & a, hipStream_t s);
hipError_t launch_ew_ref(const EwArgs & a, hipStream_t s);
// One token `tok` of a CONV, GDN or ATTN command with n_tok tokens (the command runs as n_tok such launches in
// order; the sequences forms take token tok's own state, window, KV region and position).
hipError_t launch_conv_ref(const ConvArgs & a, int tok, hipStream_t s);
hipError_t launch_gdn_ref(const GdnArgs & a, int tok, hipStream_t s);
hipError_t launch_attn_ref(const AttnArgs & a, int tok, hipStream_t s);
// hashes[b] (b < 4096): sum mod 2^64 over i < 2^20 of bits(f(x)) (2 i + 1), x the binary32 with bits b 2^20 + i,
// f the correctly rounded exp (fn 0) or log (fn 1), NaN results as 0x7fc00000.
hipError_t launch_crmath_hash(int fn, unsigned long long * hashes, hipStream_t s);

}  // namespace gq
