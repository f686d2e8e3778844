// GEMV dispatch by weight type (the instances live in gq_gemv_q4_0 / _q4_1 / _q8_0 / _kq.hip, compiled apart).
#include "gq_kernels.h"

namespace gq {

hipError_t launch_gemv_q4_0(const GemvArgs & a, hipStream_t st);
hipError_t launch_gemv_q4_1(const GemvArgs & a, hipStream_t st);
hipError_t launch_gemv_q8_0(const GemvArgs & a, hipStream_t st);
hipError_t launch_gemv_q5_k(const GemvArgs & a, hipStream_t st);
hipError_t launch_gemv_q6_k(const GemvArgs & a, hipStream_t st);

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
