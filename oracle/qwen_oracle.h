/*
 * CPU oracle for the quantized Qwen2.5-1.5B decoder-layer hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load or call this library, and only as the checker (or the timed CPU baseline).  The
 * product path (work_llm_accelerator_amd) never links, loads or falls back to it.
 *
 * The oracle restates, in plain C11 built with -O2 -ffp-contract=off (no FMA, no fast-math), the
 * reference host arithmetic op for op.  Every entry point takes the same arguments in the same
 * order as the reference C ABI it restates (prefixed oracle_), so a test can feed identical
 * buffers to the oracle and to the HIP build.  Citations are relative to the reference root.
 *
 * Pinning (see tests/test_oracle_*.py):
 *   decode layer, decode top, quantizer, bf16 rounding, layout: bit-exact against the reference
 *     decode library compiled from its own sources (oracle/_ref) and the reference's KATs;
 *   prefill layer: the reference's closed-form KATs (atol 1e-5) plus the identity
 *     "prefill projections == decode projections" (both restate the same serial loop);
 *   approx_exp / approx_sqrt / approx_sincos: structural identities (exact values, the halving
 *     ladder, the pi folding) and error bounds against long-double evaluation of the same series,
 *     chosen so that a dropped term, a wrong sign or a wrong constant fails.  The exact rounding
 *     sequence of these three prefill-only helpers cannot be pinned against a reference binary:
 *     the prefill library needs Catapult's ac_channel.h and is unbuildable here.
 */
#ifndef QWEN_ORACLE_H
#define QWEN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/qwen_layout.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- elementwise helpers ---- */
float oracle_approx_sqrt(float v);                     /* qwen_prefill_attention_kernel.cpp:47-57 */
float oracle_wrap_angle(float a);                      /* :59-67 */
void oracle_approx_sincos(float a, float* s, float* c);/* :69-85 */
float oracle_approx_exp(float v);                      /* :87-110 (= qwen_prefill_mlp_kernel.cpp:158-181) */
float oracle_silu_decode(float v);                     /* qwen_decode_mlp_kernel.cpp:79-81 (libm expf) */
float oracle_silu_prefill(float v);                    /* qwen_prefill_mlp_kernel.cpp:256-258 */
float oracle_libm_expf(float v);                       /* the host expf both decode sites call */
void oracle_round_bf16(float* x, size_t n);            /* verification/reference_wrapper_backend.py:40-46 */
void oracle_quantize_int4(const float* w, int out_dim, int in_dim, uint8_t* packed, float* scales);
                                                       /* verification/real_host_top_backend.py:31-41 */
void oracle_decode_rope_row(int position, float* cos_out, float* sin_out);  /* decode kernel :29-42 */
void oracle_prefill_rope_row(int position, float* cos_out, float* sin_out); /* prefill kernel :128-143 */
void oracle_layer_offsets(uint64_t offsets[20]);      /* llm_memory_layout.h:84-128 (+ total) */

/* ---- decode (hls/decode_only/qwen_decode_host_wrapper.cpp) ---- */
int oracle_decode_stub_forward(const float* input_token, int past_seq_len, float* output_token);
int oracle_decode_attention_smoke_forward(
    const float* input_token, int past_seq_len, const float* input_layernorm_weight,
    const uint8_t* q_packed_weights, const uint8_t* k_packed_weights, const uint8_t* v_packed_weights,
    const uint8_t* o_packed_weights, const float* q_bias, const float* k_bias, const float* v_bias,
    const float* q_scales, const float* k_scales, const float* v_scales, const float* o_scales,
    float* k_cache, float* v_cache, float* output_token);
int oracle_decode_mlp_smoke_forward(
    const float* attention_residual_token, const float* post_attention_layernorm_weight,
    const uint8_t* gate_packed_weights, const uint8_t* up_packed_weights, const uint8_t* down_packed_weights,
    const float* gate_scales, const float* up_scales, const float* down_scales, float* output_token);
int oracle_decode_layer_smoke_forward(
    const float* input_token, int past_seq_len, const float* input_layernorm_weight,
    const float* post_attention_layernorm_weight, const uint8_t* q_packed_weights,
    const uint8_t* k_packed_weights, const uint8_t* v_packed_weights, const uint8_t* o_packed_weights,
    const uint8_t* gate_packed_weights, const uint8_t* up_packed_weights, const uint8_t* down_packed_weights,
    const float* q_bias, const float* k_bias, const float* v_bias, const float* q_scales,
    const float* k_scales, const float* v_scales, const float* o_scales, const float* gate_scales,
    const float* up_scales, const float* down_scales, float* k_cache, float* v_cache, float* output_token);
int oracle_decode_top_smoke_forward(
    int layer_id, int past_seq_len, uint64_t input_token_addr, uint64_t output_token_addr,
    uint64_t layer_weights_base_addr, uint64_t layer_scales_base_addr, uint64_t k_cache_base_addr,
    uint64_t v_cache_base_addr, const uint8_t* weight_ddr, const float* scale_ddr, float* kv_cache_ddr,
    float* activation_ddr, uint8_t* weight_sram, float* kv_sram, int32_t* partial_sum_sram,
    float* softmax_sram, float* control_sram);

/* ---- prefill (hls/prefill_only/qwen_prefill_host_wrapper.cpp) ---- */
int oracle_prefill_stub_forward(
    const float* input_sequence, int seq_len, int a_seq, int a_query, int a_key, int a_hidden_proj,
    int a_kv_proj, int a_head_dim, int a_qhp, int a_kvhp, int m_seq, int m_hidden, int m_ff,
    float* output_sequence);
int oracle_prefill_attention_smoke_forward(
    const float* input_sequence, int seq_len, int a_seq, int a_query, int a_key, int a_hidden_proj,
    int a_kv_proj, int a_head_dim, int a_qhp, int a_kvhp, const float* input_layernorm_weight,
    const uint8_t* q_packed_weights, const uint8_t* k_packed_weights, const uint8_t* v_packed_weights,
    const uint8_t* o_packed_weights, const float* q_bias, const float* k_bias, const float* v_bias,
    const float* q_scales, const float* k_scales, const float* v_scales, const float* o_scales,
    float* k_cache, float* v_cache, float* output_sequence);
int oracle_prefill_mlp_smoke_forward(
    const float* attention_residual_sequence, int seq_len, int m_seq, int m_hidden, int m_ff,
    const float* post_attention_layernorm_weight, const uint8_t* gate_packed_weights,
    const uint8_t* up_packed_weights, const uint8_t* down_packed_weights, const float* gate_scales,
    const float* up_scales, const float* down_scales, float* output_sequence);
int oracle_prefill_layer_smoke_forward(
    const float* input_sequence, int seq_len, int a_seq, int a_query, int a_key, int a_hidden_proj,
    int a_kv_proj, int a_head_dim, int a_qhp, int a_kvhp, int m_seq, int m_hidden, int m_ff,
    const float* input_layernorm_weight, const float* post_attention_layernorm_weight,
    const uint8_t* q_packed_weights, const uint8_t* k_packed_weights, const uint8_t* v_packed_weights,
    const uint8_t* o_packed_weights, const uint8_t* gate_packed_weights, const uint8_t* up_packed_weights,
    const uint8_t* down_packed_weights, const float* q_bias, const float* k_bias, const float* v_bias,
    const float* q_scales, const float* k_scales, const float* v_scales, const float* o_scales,
    const float* gate_scales, const float* up_scales, const float* down_scales, float* k_cache,
    float* v_cache, float* output_sequence);
int oracle_prefill_glue_smoke_forward(
    const float* input_sequence, int seq_len, int a_seq, int a_query, int a_key, int a_hidden_proj,
    int a_kv_proj, int a_head_dim, int a_qhp, int a_kvhp, int m_seq, int m_hidden, int m_ff,
    const float* input_layernorm_weight, const float* post_attention_layernorm_weight,
    const uint8_t* q_packed_weights, const uint8_t* k_packed_weights, const uint8_t* v_packed_weights,
    const uint8_t* o_packed_weights, const uint8_t* gate_packed_weights, const uint8_t* up_packed_weights,
    const uint8_t* down_packed_weights, const float* q_bias, const float* k_bias, const float* v_bias,
    const float* q_scales, const float* k_scales, const float* v_scales, const float* o_scales,
    const float* gate_scales, const float* up_scales, const float* down_scales, float* k_cache,
    float* v_cache, float* output_sequence);
int oracle_prefill_top_smoke_forward(
    int layer_id, int seq_len, int a_seq, int a_query, int a_key, int a_hidden_proj, int a_kv_proj,
    int a_head_dim, int a_qhp, int a_kvhp, int m_seq, int m_hidden, int m_ff, uint64_t input_sequence_addr,
    uint64_t output_sequence_addr, uint64_t layer_weights_base_addr, uint64_t layer_scales_base_addr,
    uint64_t k_cache_base_addr, uint64_t v_cache_base_addr, const uint8_t* weight_ddr, const float* scale_ddr,
    float* kv_cache_ddr, float* activation_ddr, uint8_t* weight_sram, float* kv_sram, int32_t* partial_sum_sram,
    float* softmax_sram, float* control_sram);

/* Prefill layer over one layer block with the 128-token cap lifted (any 1 <= seq_len <= 32768).
 * Same per-token arithmetic as the capped path; used for sequences longer than the reference can
 * take in one call.  weight_ddr/scale_ddr are one layer block (base 0); k_cache/v_cache receive
 * seq_len rows; output_sequence receives the layer output; returns 0 or 1. */
int oracle_prefill_layer_uncapped(
    const float* input_sequence, int seq_len, const uint8_t* weight_ddr, const float* scale_ddr,
    float* k_cache, float* v_cache, float* output_sequence);

/* Decode layer over one layer block (base 0) with a caller-sized KV cache of past_seq_len+1 rows. */
int oracle_decode_layer_block(
    const float* input_token, int past_seq_len, const uint8_t* weight_ddr, const float* scale_ddr,
    float* k_cache, float* v_cache, float* output_token);

/* ---- model head of the greedy driver (verification/real_host_top_backend.py:138-146 on the bf16 model
 * of verification/torch_reference_backend.py:67; verification/qwen_full_model_validation.py:128,159).
 * bf16 values travel as uint16 bit patterns.
 *   oracle_head_norm: Qwen2RMSNorm on bf16 tensors: v = bf16(x), var = fp32(sum v^2) / 1536 (the sum
 *     correctly rounded to fp32), r = 1 / sqrtf(var + 1e-6), out = bf16(w * bf16(v * r)).
 *   oracle_lm_head: logits[t][j] = bf16(fp32(sum_k n[t][k] * E[j][k])), the products exact and the
 *     sum accumulated in double, then rounded to fp32 and to bf16.
 *   oracle_argmax: first index of the maximum of each row; a NaN is the maximum (torch.argmax).
 * Pinning: tests/test_oracle_head.py (transformers' Qwen2RMSNorm, torch bf16 linear and
 * torch.argmax on the CPU). */
void oracle_head_norm(const float* x, int count, const uint16_t* w, uint16_t* out);
void oracle_lm_head(const uint16_t* xn, int count, const uint16_t* table, int vocab, float* logits);
void oracle_argmax(const float* logits, int count, int vocab, int* ids);

/* Mismatch count of y[i] against the host expf of bit pattern first + i*stride (NaN == NaN). */
uint64_t oracle_count_expf_mismatches(uint32_t first, uint32_t stride, uint64_t n, const float* y,
                                      uint32_t* first_bad);

#ifdef __cplusplus
}
#endif

#endif /* QWEN_ORACLE_H */
