/*
 * Decode-side C ABI exported by the MI355X build (libqwen_decode_stub.so).
 *
 * Each entry point has the symbol name, argument order, argument meaning and status codes of
 * the reference host wrapper it replaces, so a ctypes caller written against the reference
 * (verification/real_host_top_backend.py:78-136 and the decode validators) loads this library
 * unchanged.  All pointers are caller-owned HOST buffers (C-contiguous); every call copies the
 * spans it needs to the GPU, runs the HIP kernels and copies the outputs back before returning.
 * Return value: 0 on success, otherwise the reference's error code (1, 10, 11), or 90 when the
 * HIP runtime fails (no counterpart in the reference).
 *
 * Numerics: bit-exact with the reference (every fp32/f64 operation in the reference's serial
 * order).  The reordered, roofline-oriented kernels are reached through the device-resident model
 * API (qwen_hip_model.h, QWEN_MODE_FAST).
 */
#ifndef QWEN_DECODE_HOST_WRAPPER_H
#define QWEN_DECODE_HOST_WRAPPER_H

#include <stdint.h>

#include "qwen_layout.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces hls/decode_only/qwen_decode_host_wrapper.h:9-12 (impl .cpp:12-71):
 * one decode layer with zero weights, unit scales and unit norm weights. */
int qwen_decode_stub_forward(const float* input_token, int past_seq_len, float* output_token);

/* Replaces qwen_decode_host_wrapper.h:14-31 (impl .cpp:73-111): RMSNorm, INT4 Q/K/V projections
 * with bias, RoPE at position past_seq_len, KV append at row past_seq_len, GQA attention over
 * past_seq_len+1 rows, INT4 O projection.  k_cache/v_cache hold (past_seq_len+1) token-major rows
 * of 256 fp32. */
int qwen_decode_attention_smoke_forward(
    const float* input_token, int past_seq_len, const float* input_layernorm_weight,
    const uint8_t* q_packed_weights, const uint8_t* k_packed_weights, const uint8_t* v_packed_weights,
    const uint8_t* o_packed_weights, const float* q_bias, const float* k_bias, const float* v_bias,
    const float* q_scales, const float* k_scales, const float* v_scales, const float* o_scales,
    float* k_cache, float* v_cache, float* output_token);

/* Replaces qwen_decode_host_wrapper.h:33-42 (impl .cpp:220-242): RMSNorm, gate/up INT4
 * projections, SiLU(gate)*up, INT4 down projection, plus the attention residual. */
int qwen_decode_mlp_smoke_forward(
    const float* attention_residual_token, const float* post_attention_layernorm_weight,
    const uint8_t* gate_packed_weights, const uint8_t* up_packed_weights, const uint8_t* down_packed_weights,
    const float* gate_scales, const float* up_scales, const float* down_scales, float* output_token);

/* Replaces qwen_decode_host_wrapper.h:44-61 (impl .cpp:113-155, top wrapper
 * qwen_decode_top_wrapper.cpp:28-113): descriptor + DDR/SRAM ports.  Addresses are byte offsets
 * into the DDR ports (fp32 ports are indexed by offset/4).  SRAM ports are only null-checked. */
int qwen_decode_top_smoke_forward(
    int layer_id, int past_seq_len, uint64_t input_token_addr, uint64_t output_token_addr,
    uint64_t layer_weights_base_addr, uint64_t layer_scales_base_addr, uint64_t k_cache_base_addr,
    uint64_t v_cache_base_addr, const uint8_t* weight_ddr, const float* scale_ddr, float* kv_cache_ddr,
    float* activation_ddr, uint8_t* weight_sram, float* kv_sram, int32_t* partial_sum_sram,
    float* softmax_sram, float* control_sram);

/* Replaces qwen_decode_host_wrapper.h:63-87 (impl .cpp:157-218): attention then MLP. */
int qwen_decode_layer_smoke_forward(
    const float* input_token, int past_seq_len, const float* input_layernorm_weight,
    const float* post_attention_layernorm_weight, const uint8_t* q_packed_weights,
    const uint8_t* k_packed_weights, const uint8_t* v_packed_weights, const uint8_t* o_packed_weights,
    const uint8_t* gate_packed_weights, const uint8_t* up_packed_weights, const uint8_t* down_packed_weights,
    const float* q_bias, const float* k_bias, const float* v_bias, const float* q_scales,
    const float* k_scales, const float* v_scales, const float* o_scales, const float* gate_scales,
    const float* up_scales, const float* down_scales, float* k_cache, float* v_cache, float* output_token);

/* Replaces llm_accel::qwen_decode_dispatch_layers (qwen_decode_top_wrapper.cpp:115-130), which the
 * reference only exposes to C++: runs descriptors[0..layer_count) in order against one set of
 * ports, stopping at the first failure.  Returns the status; *completed_layer_count receives the
 * number of layers that finished (the failing index on error). */
int qwen_decode_dispatch_layers_forward(
    const qwen_decode_descriptor* descriptors, int layer_count, const uint8_t* weight_ddr,
    const float* scale_ddr, float* kv_cache_ddr, float* activation_ddr, uint8_t* weight_sram, float* kv_sram,
    int32_t* partial_sum_sram, float* softmax_sram, float* control_sram, int* completed_layer_count);

/* Replaces qwen_decode_host_wrapper.h:89-113 (impl qwen_decode_layer0_reference_wrapper.cpp:75-209):
 * the unquantized layer with fp32 weights [out][in] (biases may be null), every linear accumulated in
 * double and rounded to bf16, double softmax, attention residual kept.  Caches are HF head-major:
 * past_k/v_cache [2][past_seq_len][128] in, next_k/v_cache [2][past_seq_len+1][128] out.  Returns 1
 * for a null input/output/cache pointer or a negative past length (as the reference), and also for
 * null weights or past caches the reference would dereference. */
int qwen_decode_layer0_reference_forward(
    const float* input_token, int past_seq_len, const float* past_k_cache, const float* past_v_cache,
    const float* input_layernorm_weight, const float* q_weight, const float* q_bias, const float* k_weight,
    const float* k_bias, const float* v_weight, const float* v_bias, const float* o_weight, const float* o_bias,
    const float* post_attention_layernorm_weight, const float* gate_weight, const float* gate_bias,
    const float* up_weight, const float* up_bias, const float* down_weight, const float* down_bias, float rms_eps,
    float* output_token, float* next_k_cache, float* next_v_cache);

#ifdef __cplusplus
}
#endif

#endif /* QWEN_DECODE_HOST_WRAPPER_H */
