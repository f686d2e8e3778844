#pragma once
// The Gated DeltaNet step on state rows held in registers (gemvq_ref.h:360-397, gemvqc_gdn.h:73-187), shared by the
// step kernel and the step fused with ssm_out. A row of the 128 x 128 head state is held by 16 consecutive lanes,
// lane l16 holding columns 8 l16 .. 8 l16 + 7; every dot product is the pairwise tree over the 128 columns (the
// lane's 8 in registers, then across the 16 lanes), the canonical order.
#include "gq_device.h"

namespace gq {

// L2 norm of q and k of the key head (ggml_l2_norm: x / max(sqrt(sum x^2), eps)), each lane holding 8 elements.
__device__ __forceinline__ void gdn_l2_qk(float (&q)[8], float (&k)[8], float eps) {
    float sq[8], sk[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        sq[i] = q[i] * q[i];
        sk[i] = k[i] * k[i];
    }
    const float tq = pair_sum_lanes<16>(tree<8>(sq)), tk = pair_sum_lanes<16>(tree<8>(sk));
    const float fq = 1.0f / fmaxf(sqrtf(tq), eps), fk = 1.0f / fmaxf(sqrtf(tk), eps);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        q[i] = q[i] * fq;
        k[i] = k[i] * fk;
    }
}

// The step's gates: with `raw` (GDN gates flag) beta = sigmoid(b) and the log decay g = softplus(a_raw + dt) * a
// (ggml-xrt.cpp:1977-2000), else g and b as given; returns the decay exp(g).
__device__ __forceinline__ float gdn_gates(bool raw, float g, float b, float dtv, float av, float & beta) {
    float gv = g;
    beta = b;
    if (raw) {
        gv = softplus_(g + dtv) * av;
        beta = sigmoid_(b);
    }
    return expf_(gv);
}

// IT rows of one thread: x_j = S_j * decay; delta = (v_j - x_j . k) * beta; S_j' = x_j + k * delta; out_j = S_j' . q
// (before the output scale). Every lane of a row's 16 ends with its out_j.
template <int IT>
__device__ __forceinline__ void gdn_step_rows(const float (&q)[8], const float (&k)[8], const float * v, float decay,
                                              float beta, float (&x)[IT][8], float * out) {
    float dot[IT];
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        float pr[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            x[it][i] = x[it][i] * decay;
            pr[i] = x[it][i] * k[i];
        }
        dot[it] = tree<8>(pr);
    }
    pair_sum_lanes_n<16, IT>(dot);
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const float delta = (v[it] - dot[it]) * beta;
        float pr[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            x[it][i] = x[it][i] + k[i] * delta;
            pr[i] = x[it][i] * q[i];
        }
        out[it] = tree<8>(pr);
    }
    pair_sum_lanes_n<16, IT>(out);
}

}  // namespace gq
