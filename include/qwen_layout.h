/*
 * Qwen2.5-1.5B decoder-layer constants and the per-layer DDR parameter layout.
 *
 * This header is plain C99 so that the CPU oracle (C), the HIP host runtime (C++) and
 * the HIP device code share one definition of every shape and byte offset.
 *
 * Reference interfaces mirrored here:
 *   hls/common/qwen2_model_config.h:7-32   model constants, eps, rope theta, default tiles
 *   hls/common/llm_accel_types.h:7-37      tile-config structs, KernelStatus
 *   hls/common/llm_memory_layout.h:17-149  LayerParameterLayout / KvCacheLayout offsets
 *   hls/common/llm_layer_dispatch.h:10-61  layer descriptors and their validity checks
 *   python/layer_descriptor_builder.py:100-277  Python twin of the layout and descriptors
 */
#ifndef QWEN_LAYOUT_H
#define QWEN_LAYOUT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- model shape (qwen2_model_config.h:7-14) ---- */
#define QWEN_HIDDEN 1536
#define QWEN_INTERMEDIATE 8960
#define QWEN_LAYERS 28
#define QWEN_Q_HEADS 12
#define QWEN_KV_HEADS 2
#define QWEN_HEAD_DIM 128
#define QWEN_VOCAB 151936
#define QWEN_MAX_SEQ 32768
#define QWEN_KV_WIDTH (QWEN_KV_HEADS * QWEN_HEAD_DIM) /* 256 fp32 per token per K or V */
#define QWEN_GROUPS (QWEN_Q_HEADS / QWEN_KV_HEADS)    /* 6 query heads share a KV head */
#define QWEN_QKV_ROWS (QWEN_HIDDEN + 2 * QWEN_KV_WIDTH) /* 2048 */

/* ---- default tiles (qwen2_model_config.h:16-30) ---- */
#define QWEN_TILE_N 128
#define QWEN_ATTN_MAC_ROWS 32
#define QWEN_ATTN_MAC_COLS 64
#define QWEN_PREFILL_SEQ_TILE 128
#define QWEN_PREFILL_MLP_HIDDEN_TILE 256
#define QWEN_PREFILL_MLP_FF_TILE 640
#define QWEN_PREFILL_QHEADS_PARALLEL 2
#define QWEN_PREFILL_KVHEADS_PARALLEL 1

/* eps 1e-6f and theta 1e6f (qwen2_model_config.h:31-32) */
#define QWEN_RMS_EPS 1.0e-6f
#define QWEN_ROPE_THETA 1000000.0f

/* ---- status codes (kernels, decode top, prefill top) ---- */
#define QWEN_OK 0
#define QWEN_ERR_KERNEL 1            /* null pointer / bad argument in a kernel */
#define QWEN_ERR_CAPACITY 2          /* prefill capacity or glue tile mismatch */
#define QWEN_ERR_DECODE_DESC 10      /* qwen_decode_top_wrapper.cpp:11 */
#define QWEN_ERR_DECODE_PORT 11      /* qwen_decode_top_wrapper.cpp:12 */
#define QWEN_ERR_PREFILL_DESC 20     /* qwen_prefill_top_core.h:7 */
#define QWEN_ERR_PREFILL_PORT 21     /* qwen_prefill_top_core.h:8 */
#define QWEN_ERR_PREFILL_WINDOW 22   /* qwen_prefill_top_core.h:9 */
#define QWEN_ERR_DEVICE 90           /* HIP runtime failure (no counterpart in the reference) */

/* ---- per-layer parameter block (llm_memory_layout.h:17-128) ---- */
#define QWEN_Q_WEIGHT_BYTES ((uint64_t)QWEN_HIDDEN * QWEN_HIDDEN / 2)
#define QWEN_K_WEIGHT_BYTES ((uint64_t)QWEN_HIDDEN * QWEN_KV_WIDTH / 2)
#define QWEN_V_WEIGHT_BYTES QWEN_K_WEIGHT_BYTES
#define QWEN_O_WEIGHT_BYTES QWEN_Q_WEIGHT_BYTES
#define QWEN_GATE_WEIGHT_BYTES ((uint64_t)QWEN_HIDDEN * QWEN_INTERMEDIATE / 2)
#define QWEN_UP_WEIGHT_BYTES QWEN_GATE_WEIGHT_BYTES
#define QWEN_DOWN_WEIGHT_BYTES ((uint64_t)QWEN_INTERMEDIATE * QWEN_HIDDEN / 2)

/* Byte offsets inside one layer block.  weight_ddr (uint8) and scale_ddr (fp32 words at
 * offset/4) share the same offsets; the INT4 matrices live in weight_ddr, the fp32 norms,
 * biases and per-row scales in scale_ddr. */
#define QWEN_OFF_INPUT_LN 0ull
#define QWEN_OFF_Q_W (QWEN_OFF_INPUT_LN + 4ull * QWEN_HIDDEN)              /* 6144 */
#define QWEN_OFF_K_W (QWEN_OFF_Q_W + QWEN_Q_WEIGHT_BYTES)                  /* 1185792 */
#define QWEN_OFF_V_W (QWEN_OFF_K_W + QWEN_K_WEIGHT_BYTES)                  /* 1382400 */
#define QWEN_OFF_O_W (QWEN_OFF_V_W + QWEN_V_WEIGHT_BYTES)                  /* 1579008 */
#define QWEN_OFF_POST_LN (QWEN_OFF_O_W + QWEN_O_WEIGHT_BYTES)              /* 2758656 */
#define QWEN_OFF_GATE_W (QWEN_OFF_POST_LN + 4ull * QWEN_HIDDEN)            /* 2764800 */
#define QWEN_OFF_UP_W (QWEN_OFF_GATE_W + QWEN_GATE_WEIGHT_BYTES)           /* 9646080 */
#define QWEN_OFF_DOWN_W (QWEN_OFF_UP_W + QWEN_UP_WEIGHT_BYTES)             /* 16527360 */
#define QWEN_OFF_Q_B (QWEN_OFF_DOWN_W + QWEN_DOWN_WEIGHT_BYTES)            /* 23408640 */
#define QWEN_OFF_K_B (QWEN_OFF_Q_B + 4ull * QWEN_HIDDEN)                   /* 23414784 */
#define QWEN_OFF_V_B (QWEN_OFF_K_B + 4ull * QWEN_KV_WIDTH)                 /* 23415808 */
#define QWEN_OFF_Q_S (QWEN_OFF_V_B + 4ull * QWEN_KV_WIDTH)                 /* 23416832 */
#define QWEN_OFF_K_S (QWEN_OFF_Q_S + 4ull * QWEN_HIDDEN)                   /* 23422976 */
#define QWEN_OFF_V_S (QWEN_OFF_K_S + 4ull * QWEN_KV_WIDTH)                 /* 23424000 */
#define QWEN_OFF_O_S (QWEN_OFF_V_S + 4ull * QWEN_KV_WIDTH)                 /* 23425024 */
#define QWEN_OFF_GATE_S (QWEN_OFF_O_S + 4ull * QWEN_HIDDEN)                /* 23431168 */
#define QWEN_OFF_UP_S (QWEN_OFF_GATE_S + 4ull * QWEN_INTERMEDIATE)         /* 23467008 */
#define QWEN_OFF_DOWN_S (QWEN_OFF_UP_S + 4ull * QWEN_INTERMEDIATE)         /* 23502848 */
#define QWEN_LAYER_BYTES (QWEN_OFF_DOWN_S + 4ull * QWEN_HIDDEN)            /* 23508992 */
#define QWEN_LAYER_SCALE_WORDS ((QWEN_LAYER_BYTES + 3ull) / 4ull)          /* 5877248 */
#define QWEN_PACKED_WEIGHT_BYTES (QWEN_OFF_Q_B - QWEN_OFF_Q_W - 4ull * QWEN_HIDDEN)

/* ---- KV cache (llm_memory_layout.h:50-53, 130-149): token-major fp32, one row of
 * QWEN_KV_WIDTH floats per token for K and another for V. ---- */
#define QWEN_KV_TOKEN_BYTES (4ull * QWEN_KV_WIDTH)                          /* 1024 */
#define QWEN_KV_LAYER_STRIDE ((uint64_t)QWEN_MAX_SEQ * QWEN_KV_TOKEN_BYTES) /* 32 MiB */
#define QWEN_KV_V_BASE ((uint64_t)QWEN_LAYERS * QWEN_KV_LAYER_STRIDE)

/* ---- prefill top windows (qwen_prefill_top_core.h:10-18) ---- */
#define QWEN_PREFILL_CAPACITY 128
#define QWEN_PREFILL_WEIGHT_WINDOW QWEN_LAYER_BYTES
#define QWEN_PREFILL_SCALE_WINDOW_BYTES (QWEN_LAYER_SCALE_WORDS * 4ull)
#define QWEN_PREFILL_KV_WINDOW_BYTES (2ull * QWEN_PREFILL_CAPACITY * QWEN_KV_WIDTH * 4ull)
#define QWEN_PREFILL_ACT_WINDOW_BYTES (3ull * QWEN_PREFILL_CAPACITY * QWEN_HIDDEN * 4ull)

/* Prefill attention capacities (qwen_prefill_attention_kernel.cpp:18-24) and MLP tile
 * capacities (qwen_prefill_mlp_kernel.cpp:11-14). */
#define QWEN_PREFILL_QUERY_CAPACITY QWEN_ATTN_MAC_ROWS   /* 32 */
#define QWEN_PREFILL_KEY_CAPACITY QWEN_ATTN_MAC_COLS     /* 64 */
#define QWEN_PREFILL_PROJ_CAPACITY QWEN_ATTN_MAC_COLS    /* 64 */
#define QWEN_PREFILL_MLP_HIDDEN_CAPACITY QWEN_PREFILL_MLP_HIDDEN_TILE
#define QWEN_PREFILL_MLP_FF_CAPACITY QWEN_PREFILL_MLP_FF_TILE

/* Tile configuration (llm_accel_types.h:11-31). */
typedef struct {
  int seq, query, key, hidden_proj, kv_proj, head_dim, query_heads_parallel, kv_heads_parallel;
} qwen_prefill_attention_tiles;

typedef struct {
  int seq, hidden, ff;
} qwen_prefill_mlp_tiles;

typedef struct {
  qwen_prefill_attention_tiles attention;
  qwen_prefill_mlp_tiles mlp;
} qwen_prefill_tiles;

/* Layer descriptors (llm_layer_dispatch.h:19-42). */
typedef struct {
  int layer_id;
  int past_seq_len;
  uint64_t input_token_addr, output_token_addr, layer_weights_base_addr, layer_scales_base_addr;
  uint64_t k_cache_base_addr, v_cache_base_addr, scratch_base_addr;
} qwen_decode_descriptor;

typedef struct {
  int layer_id;
  int seq_len;
  qwen_prefill_tiles tiles;
  uint64_t input_sequence_addr, output_sequence_addr, layer_weights_base_addr, layer_scales_base_addr;
  uint64_t k_cache_base_addr, v_cache_base_addr, scratch_base_addr;
} qwen_prefill_descriptor;

/* valid_layer_id (llm_layer_dispatch.h:50-52). */
static inline int qwen_valid_layer_id(int layer_id) { return layer_id >= 0 && layer_id < QWEN_LAYERS; }

/* valid_prefill_tile_config (llm_layer_dispatch.h:54-65): the only accepted attention tiles are
 * query 32, key 64, hidden_proj 64, kv_proj 64 with head_dim 64 or 128. */
static inline int qwen_valid_prefill_tiles(const qwen_prefill_tiles* t) {
  const int head_ok = t->attention.head_dim == QWEN_ATTN_MAC_COLS || t->attention.head_dim == QWEN_HEAD_DIM;
  return t->attention.seq > 0 && t->attention.query == QWEN_ATTN_MAC_ROWS && t->attention.key == QWEN_ATTN_MAC_COLS &&
         t->attention.hidden_proj == QWEN_ATTN_MAC_COLS && t->attention.kv_proj == QWEN_ATTN_MAC_COLS && head_ok &&
         t->attention.query_heads_parallel > 0 && t->attention.kv_heads_parallel > 0 && t->mlp.seq > 0 &&
         t->mlp.hidden > 0 && t->mlp.ff > 0;
}

/* default_prefill_tile_config (qwen2_model_config.h:34-52). */
static inline qwen_prefill_tiles qwen_default_prefill_tiles(void) {
  qwen_prefill_tiles t;
  t.attention.seq = QWEN_PREFILL_SEQ_TILE;
  t.attention.query = QWEN_ATTN_MAC_ROWS;
  t.attention.key = QWEN_ATTN_MAC_COLS;
  t.attention.hidden_proj = QWEN_ATTN_MAC_COLS;
  t.attention.kv_proj = QWEN_ATTN_MAC_COLS;
  t.attention.head_dim = QWEN_ATTN_MAC_COLS;
  t.attention.query_heads_parallel = QWEN_PREFILL_QHEADS_PARALLEL;
  t.attention.kv_heads_parallel = QWEN_PREFILL_KVHEADS_PARALLEL;
  t.mlp.seq = QWEN_PREFILL_SEQ_TILE;
  t.mlp.hidden = QWEN_PREFILL_MLP_HIDDEN_TILE;
  t.mlp.ff = QWEN_PREFILL_MLP_FF_TILE;
  return t;
}

#ifdef __cplusplus
}
#endif

#endif /* QWEN_LAYOUT_H */
