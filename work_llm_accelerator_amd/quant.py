"""INT4 per-row quantizer, bf16 rounding and layer-image packing (host side, numpy).

Mirrors the reference caller verification/real_host_top_backend.py:31-41 (quantize),
:148-188 (_pack_layer_parameters) and verification/reference_wrapper_backend.py:40-46
(round_bfloat16_array) with the same numpy semantics (fp32 arithmetic throughout).
"""

from __future__ import annotations

import numpy as np

from .layout import HIDDEN, INTERMEDIATE, KV_WIDTH, LAYOUT


def quantize_int4_per_channel(matrix: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric per-output-row INT4: scale = max|w|/7 (1.0 for an all-zero row),
    q = clip(rint(w/scale), -8, 7), two nibbles per byte, even flat index in the low nibble."""
    m = np.ascontiguousarray(matrix, dtype=np.float32)
    max_abs = np.max(np.abs(m), axis=1)
    scales = np.where(max_abs > 0.0, max_abs / np.float32(7.0), np.float32(1.0)).astype(np.float32)
    q = np.clip(np.rint(m / scales[:, None]).astype(np.int32), -8, 7)
    nib = np.where(q < 0, q + 16, q).astype(np.uint8).reshape(-1)
    if nib.size % 2:
        nib = np.concatenate([nib, np.zeros(1, np.uint8)])
    packed = np.bitwise_or(nib[0::2], np.left_shift(nib[1::2], 4)).astype(np.uint8)
    return np.ascontiguousarray(packed), np.ascontiguousarray(scales)


def round_bfloat16_array(array: np.ndarray) -> np.ndarray:
    """bits += 0x7FFF + ((bits >> 16) & 1); bits &= 0xFFFF0000 (uint32 wrap-around)."""
    out = np.ascontiguousarray(array, dtype=np.float32).copy()
    bits = out.view(np.uint32)
    bits += np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1))
    bits &= np.uint32(0xFFFF0000)
    return out


# (name, out_dim, in_dim, weight offset attribute, scale offset attribute)
MATRICES = (
    ("q", HIDDEN, HIDDEN, "q_weight_offset_bytes", "q_scale_offset_bytes"),
    ("k", KV_WIDTH, HIDDEN, "k_weight_offset_bytes", "k_scale_offset_bytes"),
    ("v", KV_WIDTH, HIDDEN, "v_weight_offset_bytes", "v_scale_offset_bytes"),
    ("o", HIDDEN, HIDDEN, "o_weight_offset_bytes", "o_scale_offset_bytes"),
    ("gate", INTERMEDIATE, HIDDEN, "gate_weight_offset_bytes", "gate_scale_offset_bytes"),
    ("up", INTERMEDIATE, HIDDEN, "up_weight_offset_bytes", "up_scale_offset_bytes"),
    ("down", HIDDEN, INTERMEDIATE, "down_weight_offset_bytes", "down_scale_offset_bytes"),
)
VECTORS = (
    ("input_layernorm", HIDDEN, "input_layernorm_weight_offset_bytes"),
    ("post_attention_layernorm", HIDDEN, "post_attention_layernorm_weight_offset_bytes"),
    ("q_bias", HIDDEN, "q_bias_offset_bytes"),
    ("k_bias", KV_WIDTH, "k_bias_offset_bytes"),
    ("v_bias", KV_WIDTH, "v_bias_offset_bytes"),
)


def pack_layer_parameters(float_weights: dict[str, np.ndarray]) -> tuple[np.ndarray, np.ndarray]:
    """Builds (weight_ddr uint8, scale_ddr fp32) for one layer (real_host_top_backend.py:148-188).

    float_weights holds fp32 [out, in] matrices "q","k","v","o","gate","up","down" and fp32
    vectors "input_layernorm","post_attention_layernorm","q_bias","k_bias","v_bias".
    """
    total = LAYOUT.total_parameter_bytes
    weight_ddr = np.zeros(total, dtype=np.uint8)
    scale_ddr = np.zeros((total + 3) // 4, dtype=np.float32)
    for name, out_dim, in_dim, w_attr, s_attr in MATRICES:
        packed, scales = quantize_int4_per_channel(np.asarray(float_weights[name]).reshape(out_dim, in_dim))
        off = getattr(LAYOUT, w_attr)
        weight_ddr[off:off + packed.size] = packed
        so = getattr(LAYOUT, s_attr) // 4
        scale_ddr[so:so + out_dim] = scales
    for name, size, attr in VECTORS:
        so = getattr(LAYOUT, attr) // 4
        scale_ddr[so:so + size] = np.asarray(float_weights[name], dtype=np.float32).reshape(-1)
    return weight_ddr, scale_ddr


def layer_views(weight_ddr: np.ndarray, scale_ddr: np.ndarray) -> dict[str, np.ndarray]:
    """Named views of the 19 segments of one layer block (base 0)."""
    views: dict[str, np.ndarray] = {}
    for name, out_dim, in_dim, w_attr, s_attr in MATRICES:
        off = getattr(LAYOUT, w_attr)
        views[name + "_w"] = weight_ddr[off:off + out_dim * in_dim // 2]
        so = getattr(LAYOUT, s_attr) // 4
        views[name + "_s"] = scale_ddr[so:so + out_dim]
    for name, size, attr in VECTORS:
        so = getattr(LAYOUT, attr) // 4
        views[name] = scale_ddr[so:so + size]
    return views
