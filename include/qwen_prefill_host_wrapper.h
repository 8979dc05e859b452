/*
 * Prefill-side C ABI exported by the MI355X build (libqwen_prefill_stub.so).
 *
 * Symbol names, argument order, argument meaning and status codes follow the reference host
 * wrapper each entry point replaces (hls/prefill_only/qwen_prefill_host_wrapper.h:9-169), so the
 * reference's ctypes callers (verification/real_host_top_backend.py:83-114 and the prefill
 * validators) load this library unchanged.  All pointers are caller-owned HOST buffers; each call
 * stages the spans it reads on the GPU, runs the HIP kernels and copies every output back.
 * The eleven tile integers are validated exactly as the reference validates them and then only
 * select error codes: the result never depends on them.
 * Return value: 0 on success, the reference's error code (1, 2, 20, 21, 22), or 90 when the HIP
 * runtime fails (no counterpart in the reference).
 *
 * Numerics: bit-exact with the reference.  The matrix-core kernels are reached through the
 * device-resident model API (qwen_hip_model.h, QWEN_MODE_FAST).
 */
#ifndef QWEN_PREFILL_HOST_WRAPPER_H
#define QWEN_PREFILL_HOST_WRAPPER_H

#include <stdint.h>

#include "qwen_layout.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces qwen_prefill_host_wrapper.h:9-23 (impl .cpp:205-298): prefill layer with zero weights,
 * unit scales and unit norm weights. */
int qwen_prefill_stub_forward(
    const float* input_sequence, int seq_len, int attention_seq_tile, int attention_query_tile,
    int attention_key_tile, int attention_hidden_proj_tile, int attention_kv_proj_tile,
    int attention_head_dim_tile, int attention_query_heads_parallel, int attention_kv_heads_parallel,
    int mlp_seq_tile, int mlp_hidden_tile, int mlp_ff_tile, float* output_sequence);

/* Replaces qwen_prefill_host_wrapper.h:25-50 (impl .cpp:300-356, kernel
 * qwen_prefill_attention_kernel.cpp:2232-2367): per token RMSNorm, K/V projections + RoPE written
 * to k_cache/v_cache rows 0..seq_len-1, Q projection + RoPE, causal GQA attention, O projection. */
int qwen_prefill_attention_smoke_forward(
    const float* input_sequence, int seq_len, int attention_seq_tile, int attention_query_tile,
    int attention_key_tile, int attention_hidden_proj_tile, int attention_kv_proj_tile,
    int attention_head_dim_tile, int attention_query_heads_parallel, int attention_kv_heads_parallel,
    const float* input_layernorm_weight, const uint8_t* q_packed_weights, const uint8_t* k_packed_weights,
    const uint8_t* v_packed_weights, const uint8_t* o_packed_weights, const float* q_bias, const float* k_bias,
    const float* v_bias, const float* q_scales, const float* k_scales, const float* v_scales,
    const float* o_scales, float* k_cache, float* v_cache, float* output_sequence);

/* Replaces qwen_prefill_host_wrapper.h:52-65 (impl .cpp:358-387, kernel
 * qwen_prefill_mlp_kernel.cpp:264-337). */
int qwen_prefill_mlp_smoke_forward(
    const float* attention_residual_sequence, int seq_len, int mlp_seq_tile, int mlp_hidden_tile,
    int mlp_ff_tile, const float* post_attention_layernorm_weight, const uint8_t* gate_packed_weights,
    const uint8_t* up_packed_weights, const uint8_t* down_packed_weights, const float* gate_scales,
    const float* up_scales, const float* down_scales, float* output_sequence);

/* Replaces qwen_prefill_host_wrapper.h:67-102 (impl .cpp:389-476): attention then MLP. */
int qwen_prefill_layer_smoke_forward(
    const float* input_sequence, int seq_len, int attention_seq_tile, int attention_query_tile,
    int attention_key_tile, int attention_hidden_proj_tile, int attention_kv_proj_tile,
    int attention_head_dim_tile, int attention_query_heads_parallel, int attention_kv_heads_parallel,
    int mlp_seq_tile, int mlp_hidden_tile, int mlp_ff_tile, const float* input_layernorm_weight,
    const float* post_attention_layernorm_weight, const uint8_t* q_packed_weights,
    const uint8_t* k_packed_weights, const uint8_t* v_packed_weights, const uint8_t* o_packed_weights,
    const uint8_t* gate_packed_weights, const uint8_t* up_packed_weights, const uint8_t* down_packed_weights,
    const float* q_bias, const float* k_bias, const float* v_bias, const float* q_scales,
    const float* k_scales, const float* v_scales, const float* o_scales, const float* gate_scales,
    const float* up_scales, const float* down_scales, float* k_cache, float* v_cache, float* output_sequence);

/* Replaces qwen_prefill_host_wrapper.h:104-139 (impl .cpp:478-637): the Catapult glue-top dataflow.
 * On the host it is numerically the layer path; it accepts only the default tiles with
 * head_dim 128 (else 2).  seq_len > 128 also returns 2 here (the reference reads an empty
 * channel in that case). */
int qwen_prefill_glue_smoke_forward(
    const float* input_sequence, int seq_len, int attention_seq_tile, int attention_query_tile,
    int attention_key_tile, int attention_hidden_proj_tile, int attention_kv_proj_tile,
    int attention_head_dim_tile, int attention_query_heads_parallel, int attention_kv_heads_parallel,
    int mlp_seq_tile, int mlp_hidden_tile, int mlp_ff_tile, const float* input_layernorm_weight,
    const float* post_attention_layernorm_weight, const uint8_t* q_packed_weights,
    const uint8_t* k_packed_weights, const uint8_t* v_packed_weights, const uint8_t* o_packed_weights,
    const uint8_t* gate_packed_weights, const uint8_t* up_packed_weights, const uint8_t* down_packed_weights,
    const float* q_bias, const float* k_bias, const float* v_bias, const float* q_scales,
    const float* k_scales, const float* v_scales, const float* o_scales, const float* gate_scales,
    const float* up_scales, const float* down_scales, float* k_cache, float* v_cache, float* output_sequence);

/* Replaces qwen_prefill_host_wrapper.h:141-169 (impl .cpp:639-705, top wrapper
 * qwen_prefill_top_wrapper.cpp:7-18, core qwen_prefill_top_core.cpp:84-183).  The attention
 * scratch is output_sequence_addr + seq_len*1536*4 inside activation_ddr and is written too. */
int qwen_prefill_top_smoke_forward(
    int layer_id, int seq_len, int attention_seq_tile, int attention_query_tile, int attention_key_tile,
    int attention_hidden_proj_tile, int attention_kv_proj_tile, int attention_head_dim_tile,
    int attention_query_heads_parallel, int attention_kv_heads_parallel, int mlp_seq_tile,
    int mlp_hidden_tile, int mlp_ff_tile, uint64_t input_sequence_addr, uint64_t output_sequence_addr,
    uint64_t layer_weights_base_addr, uint64_t layer_scales_base_addr, uint64_t k_cache_base_addr,
    uint64_t v_cache_base_addr, const uint8_t* weight_ddr, const float* scale_ddr, float* kv_cache_ddr,
    float* activation_ddr, uint8_t* weight_sram, float* kv_sram, int32_t* partial_sum_sram,
    float* softmax_sram, float* control_sram);

/* Replaces llm_accel::qwen_prefill_dispatch_layers (qwen_prefill_top_wrapper.cpp:20-35), which the
 * reference only exposes to C++: runs the descriptors in order, stopping at the first failure;
 * *completed_layer_count receives the number of layers that finished. */
int qwen_prefill_dispatch_layers_forward(
    const qwen_prefill_descriptor* descriptors, int layer_count, const uint8_t* weight_ddr,
    const float* scale_ddr, float* kv_cache_ddr, float* activation_ddr, uint8_t* weight_sram, float* kv_sram,
    int32_t* partial_sum_sram, float* softmax_sram, float* control_sram, int* completed_layer_count);

/* Replace qwen_prefill_host_wrapper.h:171-215 (impl qwen_prefill_layer0_reference_wrapper.cpp:60-347):
 * the unquantized layer over seq_len tokens at positions 0..seq_len-1 with fp32 weights (biases may
 * be null), double-accumulated linears rounded to bf16, bf16-rounded RoPE, causal double softmax,
 * attention residual kept; _with_cache also writes the bf16-rounded K/V as HF head-major
 * [2][seq_len][128].  Return 1 for a null input/output, seq_len outside [1, 32768], or exactly one
 * null cache pointer (as the reference), and also for null weights. */
int qwen_prefill_layer0_reference_forward(
    const float* input_sequence, int seq_len, const float* input_layernorm_weight, const float* q_weight,
    const float* q_bias, const float* k_weight, const float* k_bias, const float* v_weight, const float* v_bias,
    const float* o_weight, const float* o_bias, const float* post_attention_layernorm_weight, const float* gate_weight,
    const float* gate_bias, const float* up_weight, const float* up_bias, const float* down_weight,
    const float* down_bias, float rms_eps, float* output_sequence);
int qwen_prefill_layer0_reference_forward_with_cache(
    const float* input_sequence, int seq_len, const float* input_layernorm_weight, const float* q_weight,
    const float* q_bias, const float* k_weight, const float* k_bias, const float* v_weight, const float* v_bias,
    const float* o_weight, const float* o_bias, const float* post_attention_layernorm_weight, const float* gate_weight,
    const float* gate_bias, const float* up_weight, const float* up_bias, const float* down_weight,
    const float* down_bias, float rms_eps, float* output_sequence, float* k_cache, float* v_cache);

#ifdef __cplusplus
}
#endif

#endif /* QWEN_PREFILL_HOST_WRAPPER_H */
