// GEMV instances for Q4_1 weights (the kernel is in gq_gemv_impl.h).
#include "gq_gemv_impl.h"

namespace gq {

hipError_t launch_gemv_q4_1(const GemvArgs & a, hipStream_t st) { return launch_nu<T_Q4_1>(a, st); }

}  // namespace gq
