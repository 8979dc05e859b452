/*
 * Device-resident layer dispatch over the global DDR map (exported by libqwen_mi355x.so).
 *
 * These entry points run the reference's layer loops llm_accel::qwen_decode_dispatch_layers
 * (hls/decode_only/qwen_decode_top_wrapper.cpp:115-130) and llm_accel::qwen_prefill_dispatch_layers
 * (hls/prefill_only/qwen_prefill_top_wrapper.cpp:20-35) over DDR images that already live in HBM:
 * weight_ddr (uint8), scale_ddr (fp32 words, a byte address a names word a/4), kv_cache_ddr and
 * activation_ddr (fp32) are DEVICE pointers, laid out as python/layer_descriptor_builder.py:205-277
 * lays out the global map (or any other map the descriptors describe).  The descriptors themselves
 * are a host array of the structs of qwen_layout.h (llm_layer_dispatch.h:19-42).
 *
 * Per descriptor, in order, the layer runs exactly as the reference's top wrapper runs it (every
 * fp32/f64 operation in the reference order: bit-exact with the reference host library), with the
 * reference's validation and status codes:
 *   decode:  10 invalid descriptor (layer id outside [0, 28) or a negative past length), 11 a null
 *            DDR port; K/V rows 0..past are read at the descriptor's K/V bases and row `past` is
 *            written; the layer output goes to output_token_addr.
 *   prefill: 20 invalid descriptor (seq_len outside [1, 128], layer id, tile configuration), 21 a null
 *            DDR port, 22 an address outside the per-layer windows of qwen_prefill_top_core.h:10-18
 *            (so the global builder's addresses, whose layer bases grow by a layer per descriptor,
 *            are rejected from the first descriptor on: the reference's own behaviour), 1 / 2 the
 *            attention kernel's tile checks; the attention output goes to scratch_base_addr, as
 *            qwen_prefill_top_core.cpp:103,155 writes it.
 * The loop stops at the first failure; *completed_layer_count (when not null) receives the number of
 * descriptors that finished (the failing index).  A null descriptor array or layer_count <= 0 gives
 * 10 (decode) or 20 (prefill) and 0 completed.
 *
 * The SRAM ports of the host wrappers are not taken: they are only null-checked by the reference.
 * Work is queued on `stream` (a hipStream_t, 0 for the null stream); both calls return after
 * synchronizing it.  90 reports a HIP runtime failure (qwen_hip_last_error()).
 */
#ifndef QWEN_HIP_DISPATCH_H
#define QWEN_HIP_DISPATCH_H

#include <stdint.h>

#include "qwen_layout.h"

#ifdef __cplusplus
extern "C" {
#endif

int qwen_hip_decode_dispatch_layers(const qwen_decode_descriptor* descriptors, int layer_count,
                                    const uint8_t* weight_ddr, const float* scale_ddr, float* kv_cache_ddr,
                                    float* activation_ddr, void* stream, int* completed_layer_count);

int qwen_hip_prefill_dispatch_layers(const qwen_prefill_descriptor* descriptors, int layer_count,
                                     const uint8_t* weight_ddr, const float* scale_ddr, float* kv_cache_ddr,
                                     float* activation_ddr, void* stream, int* completed_layer_count);

/* No counterpart in the reference (its host wrappers run on the CPU and have no device memory to
 * allocate).  For callers that cannot allocate device memory: code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  Same descriptors, DDR ports, validation, status
 * codes, completed count and results (bit for bit) as qwen_hip_decode_dispatch_layers, except that it
 * calls no allocating routine (no hipMalloc / hipFree, no allocating library call) and does not
 * synchronize: every layer is queued on `stream` and the call returns.  The intermediates of the layer
 * being run live in one static device array of 147,456 bytes per GPU (one token's workspace, the
 * attention output row, the descriptor's RoPE row and position), held until the process ends; one
 * token per descriptor fixes that need, so no argument can exceed it.  The array keeps the last
 * call's contents, and every value a layer reads from it is written earlier in the same call.  Calls
 * that overlap on one GPU (other streams, other threads) race on the array. */
int qwen_hip_decode_dispatch_layers_noalloc(const qwen_decode_descriptor* descriptors, int layer_count,
                                            const uint8_t* weight_ddr, const float* scale_ddr, float* kv_cache_ddr,
                                            float* activation_ddr, void* stream, int* completed_layer_count);

#ifdef __cplusplus
}
#endif

#endif /* QWEN_HIP_DISPATCH_H */
