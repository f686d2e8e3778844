// GEMV dispatch by weight type (the instances live in gq_gemv_q4_0 / _q4_1 / _q8_0 / _kq.hip, compiled apart).
#include "gq_kernels.h"

namespace gq {

hipError_t launch_gemv_q4_0(const GemvArgs & a, hipStream_t st);
hipError_t launch_gemv_q4_1(const GemvArgs & a, hipStream_t st);
hipError_t launch_gemv_q8_0(const GemvArgs & a, hipStream_t st);
hipError_t launch_gemv_q5_k(const GemvArgs & a, hipStream_t st);
hipError_t launch_gemv_q6_k(const GemvArgs & a, hipStream_t st);

hipError_t launch_gemv_tok_q4_0(const TokArgs & a, hipStream_t st);
hipError_t launch_gemv_tok_q8_0(const TokArgs & a, hipStream_t st);
hipError_t launch_gemv_tok_q5_k(const TokArgs & a, hipStream_t st);
hipError_t launch_gemv_tok_q6_k(const TokArgs & a, hipStream_t st);

// The instances of gq_gemv_tok_impl.h: Q4_0 / Q8_0 with 2-4 tokens up to 4096 columns and 2 up to 12288 (SwiGLU
// pairs included); Q5_K / Q6_K with 1-4 tokens up to 4096 columns and 1-2 up to 12288 (no pairs).
bool gemv_tok_ok(int type, int cols, int n_tok, bool pair) {
    if (cols <= 0 || cols > GEMV_MAXK || n_tok < 1 || n_tok > TOK_MAX) return false;
    if (type == T_Q5_K || type == T_Q6_K) {
        if (pair || cols % 256) return false;
        const int nu = (cols / 64 + 63) / 64;
        return nu == 1 || (nu <= 3 && n_tok <= 2);
    }
    if ((type != T_Q4_0 && type != T_Q8_0) || cols % 32) return false;
    const int nu = (cols / 32 + 63) / 64;
    return n_tok >= 2 && (nu <= 2 || (nu <= 6 && n_tok == 2));
}

hipError_t launch_gemv_tok(const TokArgs & a, int type, hipStream_t st) {
    bool pair = false;
    for (int i = 0; i < a.n_members; ++i) pair = pair || a.m[i].epi == EPI_SWIGLU;
    if (!gemv_tok_ok(type, a.cols, a.n_tok, pair) || a.n_members < 1 || a.n_members > 4 || (pair && a.n_members != 1))
        return hipErrorInvalidValue;
    switch (type) {
    case T_Q4_0: return launch_gemv_tok_q4_0(a, st);
    case T_Q8_0: return launch_gemv_tok_q8_0(a, st);
    case T_Q5_K: return launch_gemv_tok_q5_k(a, st);
    default: return launch_gemv_tok_q6_k(a, st);
    }
}

hipError_t launch_gemv(const GemvArgs & a, int type, hipStream_t st) {
    if (a.cols <= 0 || a.cols > GEMV_MAXK || a.total_tasks <= 0) return hipErrorInvalidValue;
    switch (type) {
    case T_Q4_0: return launch_gemv_q4_0(a, st);
    case T_Q4_1: return launch_gemv_q4_1(a, st);
    case T_Q8_0: return launch_gemv_q8_0(a, st);
    case T_Q5_K: return a.cols % 256 ? hipErrorInvalidValue : launch_gemv_q5_k(a, st);
    case T_Q6_K: return a.cols % 256 ? hipErrorInvalidValue : launch_gemv_q6_k(a, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace gq
