// Host-side launchers of the HIP kernels (one declaration per kernel family).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace qwen {

// ---- ORDERED (bit-exact) kernels: kernels_ordered.hip ----
void launch_rmsnorm_ordered(const float* x, const float* w, float* y, int tokens, bool prefill, hipStream_t st);
void launch_project_ordered(const float* x, int tokens, int in_dim, const uint8_t* W, const float* scale,
                            const float* bias, int out_dim, float* y, const float* residual, hipStream_t st);
void launch_silu_mul(const float* g, const float* u, float* s, size_t n, bool prefill, hipStream_t st);
void launch_rope_append_decode(float* q, const float* k, const float* v, const int* pos, const float* rope,
                               bool rope_rows_are_tokens, float* k_cache, float* v_cache, size_t cache_stride,
                               int tokens, hipStream_t st);
void launch_rope_prefill(float* q, float* k_rows, const float* rope, int tokens, hipStream_t st);
void launch_rope_table_prefill(float* rope, int first, int count, hipStream_t st);
void launch_attention_ordered(const float* q, const float* k_cache, const float* v_cache, size_t cache_stride,
                              const int* pos, int tokens, bool prefill, float* ctx, hipStream_t st);

}  // namespace qwen
