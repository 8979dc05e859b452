/*
 * Device-resident multi-layer API of the MI355X build (exported by libqwen_mi355x.so).
 *
 * The reference has no device-resident interface: its 28-layer drivers
 * (verification/real_host_top_backend.py:208-351) re-quantize and re-pack every layer and call
 * the per-layer host wrappers with host buffers, and its C++ layer loops
 * (llm_accel::qwen_decode_dispatch_layers, qwen_decode_top_wrapper.cpp:115-130;
 * llm_accel::qwen_prefill_dispatch_layers, qwen_prefill_top_wrapper.cpp:20-35) run layer after
 * layer over one DDR image.  This API keeps the same per-layer DDR image format
 * (include/qwen_layout.h, llm_memory_layout.h:84-128) and the same layer semantics, but uploads
 * the images once and runs every layer of a step on the GPU with all activations and the KV cache
 * resident in HBM.
 *
 * All buffer arguments of the step functions are DEVICE pointers.  Work is queued on the model's
 * own HIP stream (qwen_hip_model_stream) and the functions return once it is queued; call
 * qwen_hip_model_synchronize (or synchronize that stream) before reading results on the host.
 * Calls on one model are serialized by the model; different models are independent.
 * Return value: 0 on success, 1 for an invalid argument, 90 for a HIP runtime failure
 * (qwen_hip_last_error() then holds the message).
 *
 * Modes:
 *   QWEN_MODE_ORDERED  every fp32 operation in the reference order: per layer bit-exact with the
 *                      reference host libraries, and the bf16 rounding between layers of
 *                      verification/real_host_top_backend.py:260,334.
 *   QWEN_MODE_FAST     int8-MFMA projections with two-limb activations, split-KV decode attention,
 *                      reordered reductions; every layer output within 1e-3 of its max of the
 *                      ORDERED result.
 */
#ifndef QWEN_HIP_MODEL_H
#define QWEN_HIP_MODEL_H

#include <stdint.h>

#include "qwen_layout.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct qwen_hip_model qwen_hip_model;

#define QWEN_MODE_ORDERED 0
#define QWEN_MODE_FAST 1
/* OR-ed into `mode`: skip the bf16 rounding between layers (the layer outputs stay fp32). */
#define QWEN_FLAG_NO_BF16_ROUND 0x100
/* OR-ed into `mode` (FAST decode of one sequence): run the small row steps as launches of their own
 * rather than in the prologue of every block of the projection that follows them: the decode
 * attention's split merge + context quantization (fused into O), the O projection's
 * reduce (fused into gate/up), the SiLU·up quantization (fused into down) and the down projection's
 * reduce + next RMSNorm + quantization (fused into the next layer's Q/K/V).  The same arithmetic except
 * the context row's code: the fused O projection quantizes it per head range (two scales), the
 * separate form with one scale for the row, so the two agree within the FAST tolerance, not bit for
 * bit.  It exists to check the fused forms. */
#define QWEN_FLAG_SEPARATE_REDUCE 0x200
/* OR-ed into `mode` (FAST decode of one sequence with at most 1280 keys): run the decode attention as
 * a launch of its own rather than in the blocks of the Q/K/V projection (the fused form attends over
 * the history keys there and adds the new key's term in the O projection's merge).  The two forms
 * round differently; both are within the FAST tolerance.  QWEN_FLAG_SEPARATE_REDUCE implies it. */
#define QWEN_FLAG_SEPARATE_ATTN 0x400

/* Kernels that qwen_hip_model_time_kernel can re-run in isolation. */
#define QWEN_KERNEL_ATTN_DECODE 1   /* split-KV decode attention partials (FAST) */
#define QWEN_KERNEL_GEMM_GATE_UP 2  /* gate/up projection + SiLU*up (FAST) */
#define QWEN_KERNEL_GEMM_DOWN 3     /* down projection + residual (FAST) */
#define QWEN_KERNEL_GEMM_QKV 4      /* fused Q/K/V projection (FAST) */
#define QWEN_KERNEL_GEMM_O 5        /* O projection (FAST) */
#define QWEN_KERNEL_ATTN_PREFILL 6  /* causal prefill attention (FAST) */

/* Uploads `layers` per-layer DDR images.  weight_ddr holds layer l at byte l*QWEN_LAYER_BYTES
 * and scale_ddr holds layer l at word l*QWEN_LAYER_BYTES/4 (the global weight/scale images of
 * python/layer_descriptor_builder.py:205-277 with base 0).  Host pointers. */
int qwen_hip_model_create(int layers, const uint8_t* weight_ddr, const float* scale_ddr, qwen_hip_model** out);

/* Builds `layers` synthetic layers on the device: every weight matrix N(0, 0.02) rounded to bf16
 * and quantized with the reference scheme (verification/real_host_top_backend.py:31-41), biases
 * N(0, 0.02) rounded to bf16, norm weights 1.0, and a bf16 N(0, 0.02) embedding table of
 * QWEN_VOCAB rows.  Normals are Irwin-Hall sums of 12 counter-hashed 24-bit uniforms keyed by
 * (seed, layer, tensor, index). */
int qwen_hip_model_create_synthetic(int layers, uint64_t seed, qwen_hip_model** out);

int qwen_hip_model_destroy(qwen_hip_model* m);
int qwen_hip_model_layers(const qwen_hip_model* m);

/* Copies layer `layer`'s DDR images back to host memory: weight_ddr receives QWEN_LAYER_BYTES bytes
 * and scale_ddr QWEN_LAYER_BYTES/4 words (the per-layer block of llm_memory_layout.h:84-128), e.g. to
 * run a synthetic model's layers through the reference host library.  Synchronizes the model. */
int qwen_hip_model_layer_images(qwen_hip_model* m, int layer, uint8_t* weight_ddr, float* scale_ddr);

/* Copies the tied bf16 embedding / lm_head table [vocab][1536] and the bf16 final RMSNorm weight
 * [1536] back to host memory (raw bf16 bit patterns).  Synchronizes the model. */
int qwen_hip_model_head_tables(qwen_hip_model* m, uint16_t* embed_bf16, uint16_t* norm_bf16);
/* The model's hipStream_t. */
void* qwen_hip_model_stream(qwen_hip_model* m);
int qwen_hip_model_synchronize(qwen_hip_model* m);

/* One decode step through every layer for `batch` independent sequences, one new token each.
 *   hidden     [batch][1536] fp32: input hidden states; receives the last layer's output
 *              (bf16-rounded after every layer, as the reference driver does)
 *   positions  [batch] int32: past length of each sequence (the new token's position)
 *   max_keys   host int >= max(positions) + 1 (sizes the split over the KV length)
 *   k_cache, v_cache: token-major fp32 rows of 256 (llm_memory_layout.h:130-149); sequence b of
 *              layer l starts at l*layer_stride + b*seq_stride floats; row positions[b] is written */
int qwen_hip_model_decode(qwen_hip_model* m, int mode, int batch, float* hidden, const int* positions, int max_keys,
                          float* k_cache, float* v_cache, uint64_t seq_stride, uint64_t layer_stride);

/* Prefill of `batch` independent sequences of seq_len tokens at positions 0..seq_len-1 through
 * every layer (causal attention; no past KV, as qwen_prefill_attention_kernel.cpp:2232-2367).
 *   hidden [batch][seq_len][1536] fp32 in/out; caches as for decode, rows 0..seq_len-1 written.
 * There is no 128-token cap (the reference's qwen_prefill_top_core.h:10 limit is a property of
 * its SRAM windows, not of the arithmetic). */
int qwen_hip_model_prefill(qwen_hip_model* m, int mode, int batch, int seq_len, float* hidden, float* k_cache,
                           float* v_cache, uint64_t seq_stride, uint64_t layer_stride);

/* Chunked prefill: seq_len new tokens per sequence at positions past..past+seq_len-1 of sequences
 * whose cache rows 0..past-1 already hold the earlier tokens (a previous prefill or chunk).  Query
 * past+i attends keys 0..past+i; rows past..past+seq_len-1 are written.  The reference has no
 * continuation entry (its prefill starts at position 0); the arithmetic per token is the reference
 * prefill's, so splitting a prompt into chunks reproduces the single prefill: bit-exactly in
 * QWEN_MODE_ORDERED.  seq_stride must hold past + seq_len rows. */
int qwen_hip_model_prefill_chunk(qwen_hip_model* m, int mode, int batch, int seq_len, int past, float* hidden,
                                 float* k_cache, float* v_cache, uint64_t seq_stride, uint64_t layer_stride);

/* The two step functions above over layers first_layer..first_layer+layer_count-1 only, with the same
 * arguments and semantics; k_cache / v_cache hold the caches of those layers (layer first_layer+i at
 * i*layer_stride floats).  hidden is the input of layer first_layer and receives the output of the
 * range's last layer (bf16-rounded after every layer unless QWEN_FLAG_NO_BF16_ROUND).  Inside a range
 * FAST fuses each layer boundary (the next layer's RMSNorm and quantization run in the down
 * projection's reduce step); at the range's ends they run as steps of their own.  A caller can inspect
 * or replace the hidden state between layers, e.g. to compare two modes layer by layer on the same
 * inputs. */
int qwen_hip_model_decode_layers(qwen_hip_model* m, int mode, int first_layer, int layer_count, int batch,
                                 float* hidden, const int* positions, int max_keys, float* k_cache, float* v_cache,
                                 uint64_t seq_stride, uint64_t layer_stride);
int qwen_hip_model_prefill_layers(qwen_hip_model* m, int mode, int first_layer, int layer_count, int batch,
                                  int seq_len, int past, float* hidden, float* k_cache, float* v_cache,
                                  uint64_t seq_stride, uint64_t layer_stride);

/* Embedding lookup from the model's bf16 table: hidden[i] = fp32(table[token_ids[i]]) (ids outside
 * [0, vocab) read row 0).  token_ids and hidden are device pointers. */
int qwen_hip_model_embed(qwen_hip_model* m, const int* token_ids, int count, float* hidden);

/* Model head of the reference's greedy driver (verification/real_host_top_backend.py:138-146 on the
 * bf16 model of verification/torch_reference_backend.py:67; the argmax of
 * verification/qwen_full_model_validation.py:128,159).  Synthetic models carry a head: their
 * embedding table (tied lm_head) and a final norm weight of 1.0 (HF init).
 *
 * set_head uploads a tied bf16 embedding / lm_head table [vocab][1536] (vocab a positive multiple
 * of 128) and the bf16 final RMSNorm weight [1536] (host pointers, raw bf16 bit patterns). */
int qwen_hip_model_set_head(qwen_hip_model* m, int vocab, const uint16_t* embed_bf16, const uint16_t* norm_bf16);
int qwen_hip_model_vocab(const qwen_hip_model* m);

/* logits[i][v] for `count` hidden rows [count][1536] fp32: Qwen2RMSNorm on bf16 tensors
 * (n = bf16(w * bf16(x * 1/sqrt(mean(x^2) + 1e-6))), x = bf16(hidden)), then the bf16 lm_head with
 * fp32 accumulation, rounded to bf16 and stored as fp32 [count][vocab].  Device pointers. */
int qwen_hip_model_logits(qwen_hip_model* m, const float* hidden, int count, float* logits);

/* Greedy next tokens: token_ids[i] = the first index of the maximal logit of row i (torch.argmax;
 * a NaN counts as the maximum), the logits being those of qwen_hip_model_logits (not stored).
 * Device pointers. */
int qwen_hip_model_greedy(qwen_hip_model* m, const float* hidden, int count, int* token_ids);

/* Re-runs one kernel of the most recent decode/prefill call `reps` times in isolation, on the
 * model's stream between two HIP events, with that call's shapes and the weights of `layer` (one of
 * that call's layers);
 * *avg_ms receives the mean duration of one launch (the decode attention takes the layers' caches in
 * turn from `layer` on, so that no launch re-reads rows a recent launch left in the last-level cache,
 * as in a decode step).  The re-run reads that call's positions and K/V
 * caches through the pointers it was given, so the caller must keep those buffers allocated until
 * time_kernel returns (their contents may have changed: only the timing is reported). */
int qwen_hip_model_time_kernel(qwen_hip_model* m, int kernel, int layer, int reps, float* avg_ms);

/* Device INT4 quantizer (verification/real_host_top_backend.py:31-41): per row
 * scale = max|w| / 7 (1 for an all-zero row), q = clip(rint(w / scale), -8, 7), two nibbles per
 * byte with the even flat index in the low nibble.  Device pointers; queued on `stream`
 * (a hipStream_t, 0 for the null stream). */
int qwen_hip_quantize_int4(const float* w, int out_dim, int in_dim, uint8_t* packed, float* scales, void* stream);

/* Fills `rows` token-major KV rows of 256 fp32 with N(0,1) values quantized per row to INT4
 * (max|x|/7) and dequantized, keyed by seed.  Device pointer. */
int qwen_hip_fill_kv_synthetic(float* cache, uint64_t rows, uint64_t seed, void* stream);

/* Test hook (no counterpart in the reference): y[i] = the device's host-compatible expf, the
 * function the ORDERED decode softmax and SiLU use in place of glibc's expf
 * (qwen_decode_attention_kernel.cpp:149, qwen_decode_mlp_kernel.cpp:80), of the float whose bit
 * pattern is first_bits + i*stride (mod 2^32), for i < n.  Device pointer; queued on `stream`. */
int qwen_hip_eval_expf(uint32_t first_bits, uint32_t stride, uint64_t n, float* y, void* stream);

/* Message of the last failure on this thread (empty when none). */
const char* qwen_hip_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* QWEN_HIP_MODEL_H */
