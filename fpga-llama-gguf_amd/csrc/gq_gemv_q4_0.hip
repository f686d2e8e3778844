// GEMV instances for Q4_0 weights (the kernel is in gq_gemv_impl.h).
#include "gq_gemv_impl.h"

namespace gq {

hipError_t launch_gemv_q4_0(const GemvArgs & a, hipStream_t st) { return launch_nu<T_Q4_0>(a, st); }

}  // namespace gq
