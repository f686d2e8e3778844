// Test infrastructure: exports the reference's own CPU path (fpga/src/gemvq_ref.h, compiled where it lies in the
// reference tree) with a C ABI, so the oracle's restatement can be compared against it. Nothing here is shipped.
#include "gemvq_ref.h"

#include <cstdint>
#include <vector>

extern "C" {

float refshim_half_to_float(uint16_t h) { return gemvq_ref::half_to_float(h); }
uint16_t refshim_float_to_half(float f) { return gemvq_ref::float_to_half(f); }
int refshim_nearest_int(float v) { return gemvq_ref::nearest_int(v); }

void refshim_quantize_q8_k(const float * x, unsigned n, int8_t * q, float * d) {
    std::vector<int8_t> vq;
    std::vector<float> vd;
    gemvq_ref::quantize_q8_k(x, n, vq, vd);
    for (unsigned i = 0; i < n; ++i) q[i] = vq[i];
    for (unsigned i = 0; i < n / 256; ++i) d[i] = vd[i];
}

void refshim_gemv(const uint8_t * w, const float * x, unsigned rows, unsigned cols, unsigned format, float * y,
                  double * mag) {
    std::vector<double> m;
    const std::vector<float> r = gemvq_ref::reference(w, x, rows, cols, format, m);
    for (unsigned i = 0; i < rows; ++i) {
        y[i] = r[i];
        mag[i] = m[i];
    }
}

int refshim_within_tolerance(float got, float ref, double mag) { return gemvq_ref::within_tolerance(got, ref, mag); }
int refshim_within_elementwise(float got, float ref) { return gemvq_ref::within_elementwise(got, ref); }
int refshim_within_swiglu(float got, float g, double gm, float u, double um) {
    return gemvq_ref::within_swiglu(got, g, gm, u, um);
}

void refshim_rmsnorm(const float * x, const float * w, unsigned n, float eps, float * y) {
    const std::vector<float> r = gemvq_ref::rmsnorm(x, w, n, eps);
    for (unsigned i = 0; i < n; ++i) y[i] = r[i];
}

void refshim_rownorm(const float * x, const float * w, unsigned n, unsigned rows, float eps, unsigned flags, float * y) {
    const std::vector<float> r = gemvq_ref::rownorm(x, w, n, rows, eps, flags);
    for (size_t i = 0; i < r.size(); ++i) y[i] = r[i];
}

void refshim_silu_mul(const float * g, const float * u, unsigned n, float * y) {
    const std::vector<float> r = gemvq_ref::silu_mul(g, u, n);
    for (unsigned i = 0; i < n; ++i) y[i] = r[i];
}

void refshim_unary(const float * x, unsigned n, unsigned kind, float * y) {
    const std::vector<float> r = gemvq_ref::unary(x, n, kind);
    for (unsigned i = 0; i < n; ++i) y[i] = r[i];
}

void refshim_conv(const float * state, const float * x, const float * w, unsigned ch, int silu, float * y, float * ns) {
    std::vector<float> s;
    const std::vector<float> r = gemvq_ref::conv(state, x, w, ch, silu != 0, s);
    for (unsigned i = 0; i < ch; ++i) y[i] = r[i];
    for (unsigned i = 0; i < ch * 3; ++i) ns[i] = s[i];
}

void refshim_gdn(float * state, const float * q, const float * k, const float * v, const float * g, const float * beta,
                 unsigned hv, unsigned hk, float scale, float * y, double * y_mag, double * s_mag) {
    std::vector<float> st(state, state + size_t(hv) * 128 * 128);
    std::vector<double> ym, sm;
    const std::vector<float> r = gemvq_ref::gdn(st, q, k, v, g, beta, hv, hk, scale, ym, sm);
    for (size_t i = 0; i < st.size(); ++i) state[i] = st[i];
    for (size_t i = 0; i < r.size(); ++i) {
        y[i] = r[i];
        if (y_mag) y_mag[i] = ym[i];
    }
    if (s_mag)
        for (size_t i = 0; i < sm.size(); ++i) s_mag[i] = sm[i];
}

}  // extern "C"
