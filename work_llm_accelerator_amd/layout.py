"""Per-layer DDR layout, KV layout, tile configs and layer descriptors.

Python twin of include/qwen_layout.h, mirroring the reference's
python/layer_descriptor_builder.py:16-277 (dataclasses, build_layer_parameter_layout,
build_kv_cache_layout, build_decode_descriptors, build_prefill_descriptors) and
hls/common/llm_memory_layout.h:55-149.  The model constants come from
hls/common/qwen2_model_config.h:7-14 (the reference reads them from a config.json that is not
available here).
"""

from __future__ import annotations

import ctypes
from dataclasses import asdict, dataclass

HIDDEN = 1536
INTERMEDIATE = 8960
LAYERS = 28
Q_HEADS = 12
KV_HEADS = 2
HEAD_DIM = 128
VOCAB = 151936
MAX_SEQ = 32768
KV_WIDTH = KV_HEADS * HEAD_DIM
RMS_EPS = 1.0e-6
ROPE_THETA = 1.0e6

SRAM_BUDGET_BYTES = 1 << 20
WEIGHT_BUFFER_BYTES = 256 << 10
KV_WORKING_SET_BYTES = 256 << 10
PARTIAL_SUM_BYTES = 128 << 10
SOFTMAX_SCRATCH_BYTES = 128 << 10
CONTROL_SCRATCH_BYTES = (SRAM_BUDGET_BYTES - WEIGHT_BUFFER_BYTES - KV_WORKING_SET_BYTES - PARTIAL_SUM_BYTES
                         - SOFTMAX_SCRATCH_BYTES)


@dataclass(frozen=True)
class LayerParameterLayout:
    input_layernorm_weight_offset_bytes: int
    q_weight_offset_bytes: int
    k_weight_offset_bytes: int
    v_weight_offset_bytes: int
    o_weight_offset_bytes: int
    post_attention_layernorm_weight_offset_bytes: int
    gate_weight_offset_bytes: int
    up_weight_offset_bytes: int
    down_weight_offset_bytes: int
    q_bias_offset_bytes: int
    k_bias_offset_bytes: int
    v_bias_offset_bytes: int
    q_scale_offset_bytes: int
    k_scale_offset_bytes: int
    v_scale_offset_bytes: int
    o_scale_offset_bytes: int
    gate_scale_offset_bytes: int
    up_scale_offset_bytes: int
    down_scale_offset_bytes: int
    total_parameter_bytes: int


@dataclass(frozen=True)
class KvCacheLayout:
    k_base_offset_bytes: int
    v_base_offset_bytes: int
    layer_stride_bytes: int
    token_stride_bytes: int


@dataclass(frozen=True)
class PrefillAttentionTileConfig:
    seq: int
    query: int
    key: int
    hidden_proj: int
    kv_proj: int
    head_dim: int
    query_heads_parallel: int
    kv_heads_parallel: int


@dataclass(frozen=True)
class PrefillMLPTileConfig:
    seq: int
    hidden: int
    ff: int


@dataclass(frozen=True)
class PrefillTileConfig:
    attention: PrefillAttentionTileConfig
    mlp: PrefillMLPTileConfig

    def as_args(self) -> tuple[int, ...]:
        a, m = self.attention, self.mlp
        return (a.seq, a.query, a.key, a.hidden_proj, a.kv_proj, a.head_dim, a.query_heads_parallel,
                a.kv_heads_parallel, m.seq, m.hidden, m.ff)


def default_prefill_tile_config() -> PrefillTileConfig:
    """The Python default of the reference (layer_descriptor_builder.py:100-117).

    The C++ check (llm_layer_dispatch.h:54-65) rejects it (status 20); it is kept because the
    reference's RealHostTopBackend passes exactly these values.
    """
    return PrefillTileConfig(PrefillAttentionTileConfig(128, 128, 128, 256, 256, 128, 2, 1),
                             PrefillMLPTileConfig(128, 256, 640))


def valid_prefill_tile_config() -> PrefillTileConfig:
    """The one tile configuration the C++ top accepts, with head_dim 128 so the attention kernel
    runs (validate_prefill_top_wrapper_regression.py:28-38)."""
    return PrefillTileConfig(PrefillAttentionTileConfig(128, 32, 64, 64, 64, 128, 2, 1),
                             PrefillMLPTileConfig(128, 256, 640))


def build_layer_parameter_layout() -> LayerParameterLayout:
    """layer_descriptor_builder.py:120-191 / llm_memory_layout.h:84-128."""
    kvw = KV_WIDTH
    sizes = [
        ("input_layernorm_weight_offset_bytes", HIDDEN * 4),
        ("q_weight_offset_bytes", HIDDEN * HIDDEN // 2),
        ("k_weight_offset_bytes", HIDDEN * kvw // 2),
        ("v_weight_offset_bytes", HIDDEN * kvw // 2),
        ("o_weight_offset_bytes", HIDDEN * HIDDEN // 2),
        ("post_attention_layernorm_weight_offset_bytes", HIDDEN * 4),
        ("gate_weight_offset_bytes", HIDDEN * INTERMEDIATE // 2),
        ("up_weight_offset_bytes", HIDDEN * INTERMEDIATE // 2),
        ("down_weight_offset_bytes", INTERMEDIATE * HIDDEN // 2),
        ("q_bias_offset_bytes", HIDDEN * 4),
        ("k_bias_offset_bytes", kvw * 4),
        ("v_bias_offset_bytes", kvw * 4),
        ("q_scale_offset_bytes", HIDDEN * 4),
        ("k_scale_offset_bytes", kvw * 4),
        ("v_scale_offset_bytes", kvw * 4),
        ("o_scale_offset_bytes", HIDDEN * 4),
        ("gate_scale_offset_bytes", INTERMEDIATE * 4),
        ("up_scale_offset_bytes", INTERMEDIATE * 4),
        ("down_scale_offset_bytes", HIDDEN * 4),
    ]
    offsets, off = {}, 0
    for name, size in sizes:
        offsets[name] = off
        off += size
    return LayerParameterLayout(**offsets, total_parameter_bytes=off)


LAYOUT = build_layer_parameter_layout()


def build_kv_cache_layout() -> KvCacheLayout:
    """layer_descriptor_builder.py:194-202 / llm_memory_layout.h:130-139."""
    token_stride = KV_WIDTH * 4
    layer_stride = MAX_SEQ * token_stride
    return KvCacheLayout(0, LAYERS * layer_stride, layer_stride, token_stride)


@dataclass(frozen=True)
class DecodeLayerDescriptor:
    layer_id: int
    past_seq_len: int
    input_token_addr: int
    output_token_addr: int
    layer_weights_base_addr: int
    layer_scales_base_addr: int
    k_cache_base_addr: int
    v_cache_base_addr: int
    scratch_base_addr: int


@dataclass(frozen=True)
class PrefillLayerDescriptor:
    layer_id: int
    seq_len: int
    tile_config: PrefillTileConfig
    input_sequence_addr: int
    output_sequence_addr: int
    layer_weights_base_addr: int
    layer_scales_base_addr: int
    k_cache_base_addr: int
    v_cache_base_addr: int
    scratch_base_addr: int


def build_decode_descriptors(past_seq_len: int, activation_base_addr: int, weight_base_addr: int,
                             scale_base_addr: int, kv_cache_base_addr: int,
                             scratch_base_addr: int) -> list[DecodeLayerDescriptor]:
    """layer_descriptor_builder.py:205-238: one descriptor per layer over the global DDR map."""
    p, kv = LAYOUT, build_kv_cache_layout()
    stride = HIDDEN * 4
    return [
        DecodeLayerDescriptor(
            layer_id=i, past_seq_len=past_seq_len,
            input_token_addr=activation_base_addr + i * stride,
            output_token_addr=activation_base_addr + (i + 1) * stride,
            layer_weights_base_addr=weight_base_addr + i * p.total_parameter_bytes,
            layer_scales_base_addr=scale_base_addr + i * p.total_parameter_bytes,
            k_cache_base_addr=kv_cache_base_addr + kv.k_base_offset_bytes + i * kv.layer_stride_bytes,
            v_cache_base_addr=kv_cache_base_addr + kv.v_base_offset_bytes + i * kv.layer_stride_bytes,
            scratch_base_addr=scratch_base_addr)
        for i in range(LAYERS)
    ]


def build_prefill_descriptors(seq_len: int, activation_base_addr: int, weight_base_addr: int, scale_base_addr: int,
                              kv_cache_base_addr: int, scratch_base_addr: int,
                              tile_config: PrefillTileConfig | None = None) -> list[PrefillLayerDescriptor]:
    """layer_descriptor_builder.py:241-277."""
    tile_config = default_prefill_tile_config() if tile_config is None else tile_config
    p, kv = LAYOUT, build_kv_cache_layout()
    stride = seq_len * HIDDEN * 4
    return [
        PrefillLayerDescriptor(
            layer_id=i, seq_len=seq_len, tile_config=tile_config,
            input_sequence_addr=activation_base_addr + i * stride,
            output_sequence_addr=activation_base_addr + (i + 1) * stride,
            layer_weights_base_addr=weight_base_addr + i * p.total_parameter_bytes,
            layer_scales_base_addr=scale_base_addr + i * p.total_parameter_bytes,
            k_cache_base_addr=kv_cache_base_addr + kv.k_base_offset_bytes + i * kv.layer_stride_bytes,
            v_cache_base_addr=kv_cache_base_addr + kv.v_base_offset_bytes + i * kv.layer_stride_bytes,
            scratch_base_addr=scratch_base_addr)
        for i in range(LAYERS)
    ]


def summary_dict() -> dict[str, object]:
    """layer_descriptor_builder.py:280-293."""
    return {
        "sram": {
            "budget_bytes": SRAM_BUDGET_BYTES, "weight_buffer_bytes": WEIGHT_BUFFER_BYTES,
            "kv_working_set_bytes": KV_WORKING_SET_BYTES, "partial_sum_bytes": PARTIAL_SUM_BYTES,
            "softmax_scratch_bytes": SOFTMAX_SCRATCH_BYTES, "control_scratch_bytes": CONTROL_SCRATCH_BYTES,
        },
        "parameter_layout": asdict(LAYOUT),
        "kv_layout": asdict(build_kv_cache_layout()),
    }


# ---- C structs of include/qwen_layout.h (for the dispatch entry points) ----
class CDecodeDescriptor(ctypes.Structure):
    _fields_ = [("layer_id", ctypes.c_int), ("past_seq_len", ctypes.c_int),
                ("input_token_addr", ctypes.c_uint64), ("output_token_addr", ctypes.c_uint64),
                ("layer_weights_base_addr", ctypes.c_uint64), ("layer_scales_base_addr", ctypes.c_uint64),
                ("k_cache_base_addr", ctypes.c_uint64), ("v_cache_base_addr", ctypes.c_uint64),
                ("scratch_base_addr", ctypes.c_uint64)]


class CPrefillDescriptor(ctypes.Structure):
    _fields_ = [("layer_id", ctypes.c_int), ("seq_len", ctypes.c_int), ("tiles", ctypes.c_int * 11),
                ("input_sequence_addr", ctypes.c_uint64), ("output_sequence_addr", ctypes.c_uint64),
                ("layer_weights_base_addr", ctypes.c_uint64), ("layer_scales_base_addr", ctypes.c_uint64),
                ("k_cache_base_addr", ctypes.c_uint64), ("v_cache_base_addr", ctypes.c_uint64),
                ("scratch_base_addr", ctypes.c_uint64)]


def to_c_decode(descs: list[DecodeLayerDescriptor]):
    arr = (CDecodeDescriptor * len(descs))()
    for c, d in zip(arr, descs):
        for f, _ in CDecodeDescriptor._fields_:
            setattr(c, f, getattr(d, f))
    return arr


def to_c_prefill(descs: list[PrefillLayerDescriptor]):
    arr = (CPrefillDescriptor * len(descs))()
    for c, d in zip(arr, descs):
        for f, _ in CPrefillDescriptor._fields_:
            if f == "tiles":
                c.tiles[:] = list(d.tile_config.as_args())
            else:
                setattr(c, f, getattr(d, f))
    return arr


def kv_to_head_major(flat_cache, seq_len: int):
    """ABI token-major KV rows [seq_len][kv_head][128] (flat fp32) -> HF cache layout
    [kv_head][seq_len][128] (verification/real_host_top_backend.py:199-201)."""
    import numpy as np

    token_major = np.asarray(flat_cache, dtype=np.float32).reshape(seq_len, KV_HEADS, HEAD_DIM)
    return np.ascontiguousarray(np.transpose(token_major, (1, 0, 2)))


def kv_to_token_major(head_major, seq_len: int):
    """HF cache layout [kv_head][seq_len][128] -> flat ABI token-major rows
    (verification/real_host_top_backend.py:203-206)."""
    import numpy as np

    hm = np.asarray(head_major, dtype=np.float32).reshape(KV_HEADS, seq_len, HEAD_DIM)
    return np.ascontiguousarray(np.transpose(hm, (1, 0, 2)).reshape(-1))
