// Small-token GEMV instances for Q5_K and Q6_K weights (the kernel is in gq_gemv_tok_impl.h).
#include "gq_gemv_tok_impl.h"

namespace gq {

hipError_t launch_gemv_tok_q5_k(const TokArgs & a, hipStream_t st) { return launch_tok_type<T_Q5_K>(a, st); }
hipError_t launch_gemv_tok_q6_k(const TokArgs & a, hipStream_t st) { return launch_tok_type<T_Q6_K>(a, st); }

}  // namespace gq
