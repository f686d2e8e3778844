// Small-token GEMV instances for Q8_0 weights (the kernel is in gq_gemv_tok_impl.h).
#include "gq_gemv_tok_impl.h"

namespace gq {

hipError_t launch_gemv_tok_q8_0(const TokArgs & a, hipStream_t st) { return launch_tok_type<T_Q8_0>(a, st); }

}  // namespace gq
