// Device-side arithmetic shared by the gfx950 kernels: fp16 conversion, exp/log, reductions, fixed-point terms.
// Every function here evaluates exactly the formula documented next to it, with no fused multiply-add except
// where fmaf is written (the sources are compiled with -ffp-contract=off), so results are reproducible bit for bit.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gq {

constexpr int WAVE = 64;

// IEEE binary16 -> binary32 (gemvq_ref.h:16-30): exact for every half, subnormals included (the hardware
// conversion; fp16 denormals are preserved in the default mode), NaN stays NaN.
__device__ __forceinline__ float h2f(uint32_t h) { return float(__builtin_bit_cast(_Float16, uint16_t(h))); }

// binary32 -> binary16, round to nearest even, subnormal results rounded, overflow to infinity (gemvq_ref.h:32-52):
// the hardware conversion in the default rounding mode, of the binary32 value. The empty asm makes that value exist:
// without it the compiler may fold a product into the conversion (v_fma_mixlo_f16, one rounding of the exact
// product), which differs from rounding the FP32 product first whenever that product lands on an fp16 tie.
__device__ __forceinline__ uint32_t f2h(float f) {
    __asm__("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, _Float16(f));
}

// exp: Cody-Waite reduction x = n ln2 + r (ln2 in a 15-bit and a low part), Taylor series of e^r to r^7/7! by
// Horner with fused multiply-adds, exact scaling by 2^n; results below the normal range flush to +0.
__device__ __forceinline__ float pow2i(int n) { return __uint_as_float(uint32_t(n + 127) << 23); }

__device__ __forceinline__ float expf_(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return __builtin_inff();
    if (x < -87.0f) return 0.0f;
    const float n = __builtin_rintf(x * 1.44269504088896341f);
    float r = __builtin_fmaf(-n, 0.693145751953125f, x);
    r = __builtin_fmaf(-n, 1.42860682030941723212e-6f, r);
    float p = 1.0f / 5040.0f;
    p = __builtin_fmaf(p, r, 1.0f / 720.0f);
    p = __builtin_fmaf(p, r, 1.0f / 120.0f);
    p = __builtin_fmaf(p, r, 1.0f / 24.0f);
    p = __builtin_fmaf(p, r, 1.0f / 6.0f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int ni = int(n);
    if (ni > 127) return (p * 2.0f) * pow2i(ni - 1);
    return p * pow2i(ni);
}

// log for x > 0: x = m 2^e, m in [sqrt(1/2), sqrt(2)), log m = 2 atanh((m - 1) / (m + 1)) to s^9 / 9.
__device__ __forceinline__ float logf_(float x) {
    if (x != x || x < 0.0f) return __builtin_nanf("");
    if (x == 0.0f) return -__builtin_inff();
    if (x == __builtin_inff()) return x;
    uint32_t b = __float_as_uint(x);
    int e;
    if ((b >> 23) == 0) {
        b = __float_as_uint(x * 8388608.0f);
        e = int(b >> 23) - 150;
    } else {
        e = int(b >> 23) - 127;
    }
    float m = __uint_as_float((b & 0x7fffffu) | 0x3f800000u);
    if (m > 1.41421353816986083984f) {
        m = m * 0.5f;
        e += 1;
    }
    const float f = m - 1.0f;
    const float s = f / (2.0f + f);
    const float s2 = s * s;
    float p = 1.0f / 9.0f;
    p = __builtin_fmaf(p, s2, 1.0f / 7.0f);
    p = __builtin_fmaf(p, s2, 1.0f / 5.0f);
    p = __builtin_fmaf(p, s2, 1.0f / 3.0f);
    p = p * s2;
    const float two_s = 2.0f * s;
    const float logm = __builtin_fmaf(two_s, p, two_s);
    const float ef = float(e);
    return __builtin_fmaf(ef, 0.693145751953125f, __builtin_fmaf(ef, 1.42860682030941723212e-6f, logm));
}

// ggml forms (gemvqc_ops.h:64-99): SiLU x / (1 + e^-x), sigmoid 1 / (1 + e^-x), softplus x > 20 ? x : log(1 + e^x).
__device__ __forceinline__ float silu_(float x) { return x / (1.0f + expf_(-x)); }
__device__ __forceinline__ float sigmoid_(float x) { return 1.0f / (1.0f + expf_(-x)); }
__device__ __forceinline__ float softplus_(float x) { return x > 20.0f ? x : logf_(1.0f + expf_(x)); }

// Cross-lane moves through DPP (in-VALU, no LDS round trip). quad_perm [1,0,3,2] and [2,3,0,1] swap neighbours at
// distance 1 and 2; row_half_mirror (lane i <- 7 - i within 8) and row_mirror (i <- 15 - i within 16) act as the
// swaps at distance 4 and 8 once every aligned group below that size holds one value.
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;

template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(dpp_i32<CTRL>(__float_as_int(v)));
}
template <int CTRL>
__device__ __forceinline__ long long dpp_i64(long long v) {
    const int lo = dpp_i32<CTRL>(int(uint32_t(uint64_t(v))));
    const int hi = dpp_i32<CTRL>(int(uint64_t(v) >> 32));
    return (long long)((uint64_t(uint32_t(hi)) << 32) | uint32_t(lo));
}

// Pairwise (adjacent-pair tree) sums. Lane l holds element l of an aligned group of `width` lanes: after the steps
// at distance 1, 2, 4, .. every lane of the group holds the tree sum (a + b == b + a bitwise, so both lanes of a
// pair agree).
template <int WIDTH>
__device__ __forceinline__ float pair_sum_lanes(float v) {
    if (WIDTH > 1) v = v + dpp_f32<DPP_XOR1>(v);
    if (WIDTH > 2) v = v + dpp_f32<DPP_XOR2>(v);
    if (WIDTH > 4) v = v + dpp_f32<DPP_HALF_MIRROR>(v);
    if (WIDTH > 8) v = v + dpp_f32<DPP_MIRROR>(v);
#pragma unroll
    for (int s = 16; s < WIDTH; s <<= 1) v = v + __shfl_xor(v, s, WAVE);
    return v;
}

// The same for N independent values at once (their cross-lane steps interleave instead of waiting in turn).
template <int WIDTH, int N>
__device__ __forceinline__ void pair_sum_lanes_n(float * v) {
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (WIDTH > 1) v[i] = v[i] + dpp_f32<DPP_XOR1>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (WIDTH > 2) v[i] = v[i] + dpp_f32<DPP_XOR2>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (WIDTH > 4) v[i] = v[i] + dpp_f32<DPP_HALF_MIRROR>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (WIDTH > 8) v[i] = v[i] + dpp_f32<DPP_MIRROR>(v[i]);
#pragma unroll
    for (int st = 16; st < WIDTH; st <<= 1) {
        float o[N];
#pragma unroll
        for (int i = 0; i < N; ++i) o[i] = __shfl_xor(v[i], st, WAVE);
#pragma unroll
        for (int i = 0; i < N; ++i) v[i] = v[i] + o[i];
    }
}

// In-register adjacent tree of N (power of two) consecutive elements.
template <int N>
__device__ __forceinline__ float tree(float * v) {
#pragma unroll
    for (int s = 1; s < N; s <<= 1)
#pragma unroll
        for (int i = 0; i < N; i += 2 * s) v[i] = v[i] + v[i + s];
    return v[0];
}

__device__ __forceinline__ long long readlane_i64(long long v, int lane) {
    const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(uint64_t(v))), lane));
    const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(uint64_t(v) >> 32), lane));
    return (long long)((uint64_t(hi) << 32) | lo);
}

// Exact integer sum over the wave (any order gives the same result); uniform result.
__device__ __forceinline__ long long wave_sum_i64(long long v) {
    v += dpp_i64<DPP_XOR1>(v);
    v += dpp_i64<DPP_XOR2>(v);
    v += dpp_i64<DPP_HALF_MIRROR>(v);
    v += dpp_i64<DPP_MIRROR>(v);
    return (readlane_i64(v, 0) + readlane_i64(v, 16)) + (readlane_i64(v, 32) + readlane_i64(v, 48));
}

__device__ __forceinline__ long long shfl_xor_i64(long long v, int m) {
    const int lo = __shfl_xor(int(uint32_t(uint64_t(v))), m, WAVE);
    const int hi = __shfl_xor(int(uint64_t(v) >> 32), m, WAVE);
    return (long long)((uint64_t(uint32_t(hi)) << 32) | uint32_t(lo));
}

// Exact int64 totals of G rows (G = 1, 2 or 4) held as per-lane partials p[0..G-1]: afterwards every lane of lane
// group g (64 / G consecutive lanes) holds the total of row g. The halving exchanges give each half of the wave half
// of the rows, so the cross-lane steps are shared by the rows instead of repeated for each.
template <int G>
__device__ __forceinline__ long long reduce_rows(const long long * p) {
    const int lane = threadIdx.x & 63;
    long long v;
    if constexpr (G == 4) {
        const bool up = lane & 32;
        const long long k0 = up ? p[2] : p[0], k1 = up ? p[3] : p[1];
        const long long g0 = up ? p[0] : p[2], g1 = up ? p[1] : p[3];
        const long long a0 = k0 + shfl_xor_i64(g0, 32), a1 = k1 + shfl_xor_i64(g1, 32);
        const bool up16 = lane & 16;
        v = (up16 ? a1 : a0) + shfl_xor_i64(up16 ? a0 : a1, 16);
    } else if constexpr (G == 2) {
        const bool up = lane & 32;
        v = (up ? p[1] : p[0]) + shfl_xor_i64(up ? p[0] : p[1], 32);
        v += shfl_xor_i64(v, 16);
    } else {
        v = p[0] + shfl_xor_i64(p[0], 32);
        v += shfl_xor_i64(v, 16);
    }
    v += dpp_i64<DPP_XOR1>(v);
    v += dpp_i64<DPP_XOR2>(v);
    v += dpp_i64<DPP_HALF_MIRROR>(v);
    v += dpp_i64<DPP_MIRROR>(v);
    return v;
}

__device__ __forceinline__ int sum_lanes4_i32(int v) {
    v += dpp_i32<DPP_XOR1>(v);
    v += dpp_i32<DPP_XOR2>(v);
    return v;
}

// An integer-valued double with |d| < 2^63 as int64 (exact: the split at 2^32 and the difference are exact).
__device__ __forceinline__ long long dint_to_i64(double d) {
    const double hi = floor(d * 2.3283064365386963e-10);  // d / 2^32
    const double lo = d - hi * 4294967296.0;              // 0 <= lo < 2^32, exact
    return (long long)((uint64_t(uint32_t(int(hi))) << 32) + uint64_t(uint32_t(lo)));
}

// Fixed-point term of the reference kernel (gemvqw_engine.h:352-445): floor(s * m * 2^(e + 40)) for the signed
// integer s times the significand product m and the power of two e; LSB of the accumulator is 2^-40.
__device__ __forceinline__ long long fixed_term(long long p, int e) {
    const int sh = e + 40;
    return sh >= 0 ? (long long)((unsigned long long)p << (sh < 63 ? sh : 63)) : (p >> (-sh < 63 ? -sh : 63));
}

// fp16 bits -> (significand, exponent): value = m * 2^e (subnormals: raw fraction, e = -24).
__device__ __forceinline__ void half_parts(uint32_t h, int & m, int & e) {
    const int ex = (h >> 10) & 31, f = h & 1023;
    m = ex == 0 ? f : (f | 1024);
    e = ex == 0 ? -24 : ex - 25;
}

// FP32 -> (significand, exponent); FP32 subnormals count as zero (gemvqw_engine.h:385-394).
__device__ __forceinline__ void float_parts(float v, int & m, int & e) {
    const uint32_t b = __float_as_uint(v);
    const int ex = (b >> 23) & 255;
    m = ex == 0 ? 0 : int((b & 0x7fffffu) | 0x800000u);
    e = ex - 150;
}

// The accumulator (LSB 2^-40) rounded to FP32 once (int64 -> FP32 rounds to nearest even; the scaling is exact).
__device__ __forceinline__ float fixed_to_float(long long acc) { return float(acc) * 9.094947017729282379e-13f; }

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(int(a), int(b), c, false);
}

// Orderable key of (value, index): larger value wins, then the smaller index (ggml argmax keeps the first).
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
    uint32_t b = __float_as_uint(v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)b << 32) | (0xffffffffu - idx);
}

}  // namespace gq
