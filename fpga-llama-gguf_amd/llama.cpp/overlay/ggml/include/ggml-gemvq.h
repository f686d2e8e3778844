// ggml backend for AMD Instinct MI355X (gfx950): a translation layer over libgemvq_hip.so's ggml-facing C ABI
// (gemvq_ggml.h), registered by ggml-backend-reg.cpp when ggml is configured with -DGGML_GEMVQ=ON.
// Counterpart of the reference's ggml-xrt.h:11-16.
#ifndef GGML_GEMVQ_H
#define GGML_GEMVQ_H

#include "ggml-backend.h"

#ifdef __cplusplus
extern "C" {
#endif

GGML_BACKEND_API ggml_backend_reg_t ggml_backend_gemvq_reg(void);

// Buffer type for llama.cpp's recurrent-state caches (cache_r_l*, cache_s_l*) of the layers on `dev`: the states
// stay in HBM, where the backend's DeltaNet commands update them in place. NULL when `dev` is another device or no
// gemvq backend has been created yet.
GGML_BACKEND_API ggml_backend_buffer_type_t ggml_backend_gemvq_rs_buffer_type(ggml_backend_dev_t dev);

// Buffer type for the attention layers' KV caches (cache_k_l*, cache_v_l*) on `dev`, read and appended by the
// backend's ATTN command. Same NULL rule. Without it the caches stay in host memory and attention runs on the CPU.
GGML_BACKEND_API ggml_backend_buffer_type_t ggml_backend_gemvq_kv_buffer_type(ggml_backend_dev_t dev);

#ifdef __cplusplus
}
#endif

#endif  // GGML_GEMVQ_H
