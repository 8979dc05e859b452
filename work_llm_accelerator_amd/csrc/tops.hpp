// Validation of the reference's top-level wrappers and kernels, shared by the host-buffer C ABI
// (abi.hip) and the device-resident descriptor dispatch (dispatch.hip).  Every check returns the
// reference's status code in the reference's order.
#pragma once

#include <stdint.h>

#include "qwen_layout.h"

namespace qwen {

// qwen_decode_top_wrapper.cpp:31-35: the descriptor (10); the ports are checked next (11).
inline int decode_descriptor_status(const qwen_decode_descriptor& d) {
  return (!qwen_valid_layer_id(d.layer_id) || d.past_seq_len < 0) ? QWEN_ERR_DECODE_DESC : QWEN_OK;
}

// qwen_prefill_attention_kernel.cpp:2252-2268 (pointer checks done by the caller).
inline int check_prefill_attention_tiles(int S, const qwen_prefill_attention_tiles& t) {
  if (S <= 0 || t.seq <= 0 || t.query <= 0 || t.key <= 0 || t.hidden_proj <= 0 || t.kv_proj <= 0 ||
      t.head_dim != QWEN_HEAD_DIM || t.query_heads_parallel <= 0 || t.kv_heads_parallel <= 0)
    return QWEN_ERR_KERNEL;
  if (S > QWEN_PREFILL_CAPACITY || t.seq > QWEN_PREFILL_CAPACITY || t.query > QWEN_PREFILL_QUERY_CAPACITY ||
      t.key > QWEN_PREFILL_KEY_CAPACITY || t.hidden_proj > QWEN_PREFILL_PROJ_CAPACITY ||
      t.kv_proj > QWEN_PREFILL_PROJ_CAPACITY || t.query_heads_parallel > QWEN_Q_HEADS ||
      t.kv_heads_parallel > QWEN_KV_HEADS)
    return QWEN_ERR_CAPACITY;
  return QWEN_OK;
}

// qwen_prefill_mlp_kernel.cpp:277-283 (pointer checks done by the caller).
inline int check_prefill_mlp_tiles(int S, const qwen_prefill_mlp_tiles& t) {
  if (S <= 0 || t.seq <= 0 || t.hidden <= 0 || t.ff <= 0 || t.hidden > QWEN_PREFILL_MLP_HIDDEN_CAPACITY ||
      t.ff > QWEN_PREFILL_MLP_FF_CAPACITY)
    return QWEN_ERR_KERNEL;
  return QWEN_OK;
}

// valid_memory_windows: qwen_prefill_top_core.cpp:42-80.  Every address is a byte offset inside the
// per-layer windows of qwen_prefill_top_core.h:10-18, 4-byte aligned, and in, out, scratch and the
// K/V spans must not overlap.
inline bool range_fits(uint64_t off, uint64_t count, uint64_t cap) { return off <= cap && count <= cap - off; }
inline bool ranges_overlap(uint64_t a, uint64_t as, uint64_t b, uint64_t bs) { return a < b + bs && b < a + as; }

inline bool prefill_windows_ok(const qwen_prefill_descriptor& d) {
  if (d.seq_len <= 0 || d.seq_len > QWEN_PREFILL_CAPACITY) return false;
  const uint64_t seq_bytes = (uint64_t)d.seq_len * QWEN_HIDDEN * 4u;
  const uint64_t kvb = (uint64_t)d.seq_len * QWEN_KV_WIDTH * 4u;
  const uint64_t packed = QWEN_OFF_DOWN_W + QWEN_DOWN_WEIGHT_BYTES - QWEN_OFF_Q_W;
  const uint64_t scale_bytes = QWEN_OFF_DOWN_S + 4ull * QWEN_HIDDEN;
  if (d.input_sequence_addr % 4 || d.output_sequence_addr % 4 || d.k_cache_base_addr % 4 || d.v_cache_base_addr % 4 ||
      d.scratch_base_addr % 4 || d.layer_scales_base_addr % 4)
    return false;
  if (!range_fits(d.input_sequence_addr, seq_bytes, QWEN_PREFILL_ACT_WINDOW_BYTES) ||
      !range_fits(d.output_sequence_addr, seq_bytes, QWEN_PREFILL_ACT_WINDOW_BYTES) ||
      !range_fits(d.scratch_base_addr, seq_bytes, QWEN_PREFILL_ACT_WINDOW_BYTES) ||
      !range_fits(d.k_cache_base_addr, kvb, QWEN_PREFILL_KV_WINDOW_BYTES) ||
      !range_fits(d.v_cache_base_addr, kvb, QWEN_PREFILL_KV_WINDOW_BYTES) ||
      !range_fits(d.layer_weights_base_addr + QWEN_OFF_Q_W, packed, QWEN_PREFILL_WEIGHT_WINDOW) ||
      !range_fits(d.layer_scales_base_addr, scale_bytes, QWEN_PREFILL_SCALE_WINDOW_BYTES))
    return false;
  if (ranges_overlap(d.input_sequence_addr, seq_bytes, d.output_sequence_addr, seq_bytes) ||
      ranges_overlap(d.input_sequence_addr, seq_bytes, d.scratch_base_addr, seq_bytes) ||
      ranges_overlap(d.output_sequence_addr, seq_bytes, d.scratch_base_addr, seq_bytes) ||
      ranges_overlap(d.k_cache_base_addr, kvb, d.v_cache_base_addr, kvb))
    return false;
  return true;
}

// qwen_prefill_top_wrapper.cpp:7-18 then qwen_prefill_top_core.cpp:84-98: the descriptor (20), the
// ports (21, `ports_null`), the windows (22), then the attention kernel's tile checks (1, 2).  On 0
// the layer runs; *mlp_status receives the MLP kernel's tile check, which the reference evaluates
// after the attention has already written its outputs.
inline int prefill_top_status(const qwen_prefill_descriptor& d, bool ports_null, int* mlp_status) {
  *mlp_status = QWEN_OK;
  if (d.seq_len <= 0 || d.seq_len > QWEN_MAX_SEQ) return QWEN_ERR_PREFILL_DESC;
  if (d.seq_len > QWEN_PREFILL_CAPACITY) return QWEN_ERR_PREFILL_DESC;
  if (!qwen_valid_layer_id(d.layer_id) || !qwen_valid_prefill_tiles(&d.tiles)) return QWEN_ERR_PREFILL_DESC;
  if (ports_null) return QWEN_ERR_PREFILL_PORT;
  if (!prefill_windows_ok(d)) return QWEN_ERR_PREFILL_WINDOW;
  const int ast = check_prefill_attention_tiles(d.seq_len, d.tiles.attention);
  if (ast) return ast;
  *mlp_status = check_prefill_mlp_tiles(d.seq_len, d.tiles.mlp);
  return QWEN_OK;
}

}  // namespace qwen
