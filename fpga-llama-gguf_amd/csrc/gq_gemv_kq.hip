// GEMV instances for Q5_K and Q6_K weights (the kernel is in gq_gemv_impl.h).
#include "gq_gemv_impl.h"

namespace gq {

hipError_t launch_gemv_q5_k(const GemvArgs & a, hipStream_t st) { return launch_nu<T_Q5_K>(a, st); }
hipError_t launch_gemv_q6_k(const GemvArgs & a, hipStream_t st) { return launch_nu<T_Q6_K>(a, st); }

}  // namespace gq
