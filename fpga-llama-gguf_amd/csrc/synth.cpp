// Synthetic weights and activations: portable counter RNG and ggml's reference weight quantizers (host only).
// The quantizers restate ggml's quantize_row_*_ref (ggml-quants.c of the llama.cpp revision the reference pins,
// c92e806d; the reference itself receives GGUF bytes and never quantizes weights). Built with -ffp-contract=off.
#include "gemvq_synth.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ULL;

uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

uint64_t stream_key(uint64_t seed, uint64_t stream) { return mix64(mix64(seed + kGamma) ^ (stream * 0xD1B54A32D192ED03ULL)); }

// (0, 1]: never zero, so log() is finite.
double unit(uint64_t z) { return double((z >> 11) + 1) * (1.0 / 9007199254740992.0); }

uint16_t f2h(float f) {  // IEEE half, round to nearest even (ggml GGML_FP32_TO_FP16 for finite values)
    uint32_t b;
    std::memcpy(&b, &f, 4);
    const uint16_t sign = uint16_t((b >> 16) & 0x8000u);
    const int e = int((b >> 23) & 0xff) - 127 + 15;
    uint32_t m = b & 0x7fffffu;
    if (e >= 31) return sign | 0x7c00u;
    if (e <= 0) {
        if (e < -10) return sign;
        m |= 0x800000u;
        const int sh = 14 - e;
        uint32_t r = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return sign | uint16_t(r);
    }
    uint32_t out = (uint32_t(e) << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (out & 1u))) ++out;
    return sign | uint16_t(out);
}

float h2f(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; ++sh; }
            bits = sign | (uint32_t(113 - sh) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

int nearest_int(float v) {  // round half to even through 1.5 * 2^23
    const float biased = v + 12582912.f;
    int32_t b;
    std::memcpy(&b, &biased, 4);
    return (b & 0x007fffff) - 0x00400000;
}

void put16(uint8_t * p, uint16_t v) {
    p[0] = uint8_t(v);
    p[1] = uint8_t(v >> 8);
}

// ggml quantize_row_q4_0_ref: d = max / -8 with max the signed value of largest magnitude.
void q4_0_row(const float * x, int64_t cols, uint8_t * out) {
    for (int64_t b = 0; b < cols / 32; ++b, x += 32, out += 18) {
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 32; ++j) {
            if (amax < std::fabs(x[j])) {
                amax = std::fabs(x[j]);
                max = x[j];
            }
        }
        const float d = max / -8.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
        put16(out, f2h(d));
        for (int j = 0; j < 16; ++j) {
            const float x0 = x[j] * id, x1 = x[16 + j] * id;
            const uint8_t xi0 = uint8_t(std::min(15, int(int8_t(x0 + 8.5f))));
            const uint8_t xi1 = uint8_t(std::min(15, int(int8_t(x1 + 8.5f))));
            out[2 + j] = uint8_t(xi0 | (xi1 << 4));
        }
    }
}

// ggml quantize_row_q4_1_ref: d = (max - min) / 15, m = min, q = min(15, (int8)((x - min) / d + 0.5)).
void q4_1_row(const float * x, int64_t cols, uint8_t * out) {
    for (int64_t b = 0; b < cols / 32; ++b, x += 32, out += 20) {
        float mn = 3.402823466e38f, mx = -3.402823466e38f;
        for (int j = 0; j < 32; ++j) {
            if (x[j] < mn) mn = x[j];
            if (x[j] > mx) mx = x[j];
        }
        const float d = (mx - mn) / 15.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
        put16(out, f2h(d));
        put16(out + 2, f2h(mn));
        for (int j = 0; j < 16; ++j) {
            const float x0 = (x[j] - mn) * id, x1 = (x[16 + j] - mn) * id;
            const uint8_t xi0 = uint8_t(std::min(15, int(int8_t(x0 + 0.5f))));
            const uint8_t xi1 = uint8_t(std::min(15, int(int8_t(x1 + 0.5f))));
            out[4 + j] = uint8_t(xi0 | (xi1 << 4));
        }
    }
}

// ggml quantize_row_q8_0_ref: d = amax / 127, q = roundf(x / d).
void q8_0_row(const float * x, int64_t cols, uint8_t * out) {
    for (int64_t b = 0; b < cols / 32; ++b, x += 32, out += 34) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(x[j]));
        const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
        put16(out, f2h(d));
        for (int j = 0; j < 32; ++j) out[2 + j] = uint8_t(int8_t(std::roundf(x[j] * id)));
    }
}

constexpr float kGroupMaxEps = 1e-15f;

// ggml make_qx_quants (rmse_type 1, no importance weights).
float make_qx_quants(int n, int nmax, const float * x, int8_t * L) {
    float max = 0.0f, amax = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float ax = std::fabs(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax < kGroupMaxEps) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.0f;
    }
    float iscale = -nmax / max;
    float sumlx = 0.0f, suml2 = 0.0f;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = std::max(-nmax, std::min(nmax - 1, l));
        L[i] = int8_t(l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 != 0.0f ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / max;
        sumlx = suml2 = 0.0f;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * x[i]);
            l = std::max(-nmax, std::min(nmax - 1, l));
            const float w = x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0.0f && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                const int l = nearest_int(iscale * x[i]);
                L[i] = int8_t(nmax + std::max(-nmax, std::min(nmax - 1, l)));
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

// ggml quantize_row_q6_K_ref: 16 scales per super-block (int8), 6-bit quants, d = 1 / iscale.
void q6_K_row(const float * x, int64_t cols, uint8_t * out) {
    int8_t L[256];
    float scales[16];
    for (int64_t i = 0; i < cols / 256; ++i, x += 256, out += 210) {
        float max_scale = 0.0f, max_abs_scale = 0.0f;
        for (int ib = 0; ib < 16; ++ib) {
            const float scale = make_qx_quants(16, 32, x + 16 * ib, L + 16 * ib);
            scales[ib] = scale;
            const float abs_scale = std::fabs(scale);
            if (abs_scale > max_abs_scale) {
                max_abs_scale = abs_scale;
                max_scale = scale;
            }
        }
        uint8_t * ql = out, * qh = out + 128;
        int8_t * sc = reinterpret_cast<int8_t *>(out + 192);
        if (max_abs_scale < kGroupMaxEps) {
            std::memset(out, 0, 210);
            continue;
        }
        const float iscale = -128.0f / max_scale;
        put16(out + 208, f2h(1.0f / iscale));
        for (int ib = 0; ib < 16; ++ib) sc[ib] = int8_t(std::min(127, nearest_int(iscale * scales[ib])));
        for (int j = 0; j < 16; ++j) {
            const float d = h2f(uint16_t(out[208] | (out[209] << 8))) * sc[j];
            if (d == 0.0f) continue;
            for (int ii = 0; ii < 16; ++ii) {
                int l = nearest_int(x[16 * j + ii] / d);
                l = std::max(-32, std::min(31, l));
                L[16 * j + ii] = int8_t(l + 32);
            }
        }
        for (int j = 0; j < 256; j += 128) {
            for (int l = 0; l < 32; ++l) {
                const uint8_t q1 = L[j + l] & 0xF, q2 = L[j + l + 32] & 0xF, q3 = L[j + l + 64] & 0xF,
                              q4 = L[j + l + 96] & 0xF;
                ql[l] = uint8_t(q1 | (q3 << 4));
                ql[l + 32] = uint8_t(q2 | (q4 << 4));
                qh[l] = uint8_t((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) |
                                ((L[j + l + 96] >> 4) << 6));
            }
            ql += 64;
            qh += 32;
        }
    }
}

// ggml make_qkx2_quants: scale and min of one sub-block with a weighted least-squares refinement.
float make_qkx2_quants(int n, int nmax, const float * x, const float * weights, uint8_t * L, float * the_min,
                       uint8_t * Laux, float rmin, float rdelta, int nstep) {
    float min = x[0], max = x[0];
    float sum_w = weights[0], sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -min;
        return 0.0f;
    }
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < n; ++i) {
        const int l = nearest_int(iscale * (x[i] - min));
        L[i] = uint8_t(std::max(0, std::min(nmax, l)));
        float diff = scale * L[i] + min - x[i];
        diff = diff * diff;
        best_error += weights[i] * diff;
    }
    if (nstep < 1) {
        *the_min = -min;
        return scale;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = std::max(0, std::min(nmax, l));
            Laux[i] = uint8_t(l);
            const float w = weights[i];
            sum_l += w * l;
            sum_l2 += w * l * l;
            sum_xl += w * l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float cur_error = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = diff * diff;
                cur_error += weights[i] * diff;
            }
            if (cur_error < best_error) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_error = cur_error;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

void get_scale_min_k4(int j, const uint8_t * q, uint8_t * d, uint8_t * m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4);
    }
}

// ggml quantize_row_q5_K_ref: 8 sub-blocks of 32 with 6-bit scales and mins, 5-bit quants.
void q5_K_row(const float * x, int64_t cols, uint8_t * out) {
    uint8_t L[256], Laux[32];
    float mins[8], scales[8], weights[32];
    for (int64_t i = 0; i < cols / 256; ++i, x += 256, out += 176) {
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < 8; ++j) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
            const float av_x = std::sqrt(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) weights[l] = av_x + std::fabs(x[32 * j + l]);
            scales[j] = make_qkx2_quants(32, 31, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, -0.5f, 0.1f, 15);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        uint8_t * sc = out + 4;
        std::memset(sc, 0, 12);
        const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
        for (int j = 0; j < 8; ++j) {
            uint8_t ls = uint8_t(nearest_int(inv_scale * scales[j]));
            uint8_t lm = uint8_t(nearest_int(inv_min * mins[j]));
            ls = std::min<uint8_t>(63, ls);
            lm = std::min<uint8_t>(63, lm);
            if (j < 4) {
                sc[j] = ls;
                sc[j + 4] = lm;
            } else {
                sc[j + 4] = uint8_t((ls & 0xF) | ((lm & 0xF) << 4));
                sc[j - 4] |= uint8_t((ls >> 4) << 6);
                sc[j - 0] |= uint8_t((lm >> 4) << 6);
            }
        }
        put16(out, f2h(max_scale / 63.f));
        put16(out + 2, f2h(max_min / 63.f));
        const float dd = h2f(uint16_t(out[0] | (out[1] << 8))), dm = h2f(uint16_t(out[2] | (out[3] << 8)));
        for (int j = 0; j < 8; ++j) {
            uint8_t s, m;
            get_scale_min_k4(j, sc, &s, &m);
            const float d = dd * s;
            if (d == 0.0f) continue;
            const float dmn = dm * m;
            for (int ii = 0; ii < 32; ++ii) {
                int l = nearest_int((x[32 * j + ii] + dmn) / d);
                l = std::max(0, std::min(31, l));
                L[32 * j + ii] = uint8_t(l);
            }
        }
        uint8_t * qh = out + 16, * ql = out + 48;
        std::memset(qh, 0, 32);
        uint8_t m1 = 1, m2 = 2;
        for (int n = 0; n < 256; n += 64) {
            for (int j = 0; j < 32; ++j) {
                int l1 = L[n + j];
                if (l1 > 15) {
                    l1 -= 16;
                    qh[j] |= m1;
                }
                int l2 = L[n + j + 32];
                if (l2 > 15) {
                    l2 -= 16;
                    qh[j] |= m2;
                }
                ql[j] = uint8_t(l1 | (l2 << 4));
            }
            m1 <<= 2;
            m2 <<= 2;
            ql += 32;
        }
    }
}

}  // namespace

extern "C" {

uint64_t gqs_u64(uint64_t seed, uint64_t stream, uint64_t i) { return mix64(stream_key(seed, stream) + (i + 1) * kGamma); }

void gqs_normal(uint64_t seed, uint64_t stream, uint64_t first, size_t n, float mean, float stddev, float * out) {
    const uint64_t key = stream_key(seed, stream);
    for (size_t k = 0; k < n; ++k) {
        const uint64_t i = first + k, p = i / 2;
        const double u1 = unit(mix64(key + (2 * p + 1) * kGamma)), u2 = unit(mix64(key + (2 * p + 2) * kGamma));
        const double r = std::sqrt(-2.0 * std::log(u1)), t = 6.283185307179586476925 * u2;
        const double z = (i & 1) ? r * std::sin(t) : r * std::cos(t);
        out[k] = float(double(mean) + double(stddev) * z);
    }
}

void gqs_uniform(uint64_t seed, uint64_t stream, uint64_t first, size_t n, float lo, float hi, float * out) {
    const uint64_t key = stream_key(seed, stream);
    for (size_t k = 0; k < n; ++k) {
        const double u = unit(mix64(key + (first + k + 1) * kGamma));
        out[k] = float(double(lo) + (double(hi) - double(lo)) * u);
    }
}

size_t gqs_row_bytes(int type, int64_t cols) {
    switch (type) {
    case 2: return cols % 32 ? 0 : size_t(cols / 32) * 18;
    case 3: return cols % 32 ? 0 : size_t(cols / 32) * 20;
    case 8: return cols % 32 ? 0 : size_t(cols / 32) * 34;
    case 13: return cols % 256 ? 0 : size_t(cols / 256) * 176;
    case 14: return cols % 256 ? 0 : size_t(cols / 256) * 210;
    default: return 0;
    }
}

size_t gqs_quantize(int type, const float * x, int64_t rows, int64_t cols, uint8_t * out) {
    const size_t rb = gqs_row_bytes(type, cols);
    if (rb == 0) return 0;
    for (int64_t r = 0; r < rows; ++r) {
        const float * xr = x + r * cols;
        uint8_t * o = out + size_t(r) * rb;
        switch (type) {
        case 2: q4_0_row(xr, cols, o); break;
        case 3: q4_1_row(xr, cols, o); break;
        case 8: q8_0_row(xr, cols, o); break;
        case 13: q5_K_row(xr, cols, o); break;
        case 14: q6_K_row(xr, cols, o); break;
        }
    }
    return rb * size_t(rows);
}

size_t gqs_matrix(int type, int64_t rows, int64_t cols, uint64_t seed, uint64_t stream, float mean, float stddev,
                  uint8_t * out, int n_threads) {
    const size_t rb = gqs_row_bytes(type, cols);
    if (rb == 0 || rows <= 0) return 0;
    n_threads = std::max(1, n_threads);
    const int64_t chunk = 64;
    const int64_t nchunks = (rows + chunk - 1) / chunk;
    auto work = [&](int t) {
        std::vector<float> buf(size_t(chunk * cols));
        for (int64_t c = t; c < nchunks; c += n_threads) {
            const int64_t r0 = c * chunk, nr = std::min(chunk, rows - r0);
            gqs_normal(seed, stream, uint64_t(r0 * cols), size_t(nr * cols), mean, stddev, buf.data());
            gqs_quantize(type, buf.data(), nr, cols, out + size_t(r0) * rb);
        }
    };
    std::vector<std::thread> th;
    for (int t = 1; t < n_threads; ++t) th.emplace_back(work, t);
    work(0);
    for (auto & x : th) x.join();
    return rb * size_t(rows);
}

}  // extern "C"
