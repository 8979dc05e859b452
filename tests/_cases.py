"""Test cases shared by the oracle and GPU parity tests.

* sparse known-answer layers built the way the reference validators build them
  (verification/validate_decode_*.py, validate_prefill_*.py: single +-1 nibbles, unit scales);
* dense random layers: N(0, 0.02) weights rounded to bf16 and quantized with the reference
  scheme (verification/real_host_top_backend.py:31-41), N(0, 0.02) bf16 biases and, unless
  `unit_norms`, norm weights 1 + N(0, 0.1) so the norm multiply is exercised;
* callers that pass one case to any library exposing the reference ABI (the HIP build, the
  oracle with its `oracle_` prefix, or the reference decode library).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from work_llm_accelerator_amd.layout import HIDDEN, INTERMEDIATE, KV_WIDTH, LAYOUT, PrefillTileConfig
from work_llm_accelerator_amd.quant import pack_layer_parameters, layer_views, round_bfloat16_array

SRAM = lambda: (np.zeros(1, np.uint8), np.zeros(1, np.float32), np.zeros(1, np.int32),  # noqa: E731
                np.zeros(1, np.float32), np.zeros(1, np.float32))


def set_packed_weight(packed: np.ndarray, out_dim: int, in_dim: int, o: int, i: int, value: int) -> None:
    """Same convention as the reference validators (validate_decode_attention_smoke.py:20-28)."""
    flat = o * in_dim + i
    nib = value & 0xF
    if flat % 2 == 0:
        packed[flat // 2] = (packed[flat // 2] & 0xF0) | nib
    else:
        packed[flat // 2] = (packed[flat // 2] & 0x0F) | (nib << 4)


@dataclass
class LayerCase:
    weight_ddr: np.ndarray
    scale_ddr: np.ndarray
    v: dict = field(default_factory=dict)

    @classmethod
    def from_images(cls, weight_ddr, scale_ddr):
        return cls(weight_ddr, scale_ddr, layer_views(weight_ddr, scale_ddr))

    def attention_args(self):
        v = self.v
        return [v["input_layernorm"], v["q_w"], v["k_w"], v["v_w"], v["o_w"], v["q_bias"], v["k_bias"],
                v["v_bias"], v["q_s"], v["k_s"], v["v_s"], v["o_s"]]

    def mlp_args(self):
        v = self.v
        return [v["post_attention_layernorm"], v["gate_w"], v["up_w"], v["down_w"], v["gate_s"], v["up_s"],
                v["down_s"]]

    def layer_args(self):
        v = self.v
        return [v["input_layernorm"], v["post_attention_layernorm"], v["q_w"], v["k_w"], v["v_w"], v["o_w"],
                v["gate_w"], v["up_w"], v["down_w"], v["q_bias"], v["k_bias"], v["v_bias"], v["q_s"], v["k_s"],
                v["v_s"], v["o_s"], v["gate_s"], v["up_s"], v["down_s"]]


def empty_layer() -> LayerCase:
    """All-zero INT4 weights, unit scales and norms, zero biases."""
    w = np.zeros(LAYOUT.total_parameter_bytes, np.uint8)
    s = np.zeros((LAYOUT.total_parameter_bytes + 3) // 4, np.float32)
    case = LayerCase.from_images(w, s)
    for k in ("input_layernorm", "post_attention_layernorm", "q_s", "k_s", "v_s", "o_s", "gate_s", "up_s", "down_s"):
        case.v[k][:] = 1.0
    return case


def random_layer(seed: int, unit_norms: bool = False) -> LayerCase:
    rng = np.random.default_rng(seed)

    def normal(shape, sigma):
        return round_bfloat16_array((rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma)))

    fw = {
        "q": normal((HIDDEN, HIDDEN), 0.02), "k": normal((KV_WIDTH, HIDDEN), 0.02),
        "v": normal((KV_WIDTH, HIDDEN), 0.02), "o": normal((HIDDEN, HIDDEN), 0.02),
        "gate": normal((INTERMEDIATE, HIDDEN), 0.02), "up": normal((INTERMEDIATE, HIDDEN), 0.02),
        "down": normal((HIDDEN, INTERMEDIATE), 0.02),
        "q_bias": normal(HIDDEN, 0.02), "k_bias": normal(KV_WIDTH, 0.02), "v_bias": normal(KV_WIDTH, 0.02),
    }
    if unit_norms:
        fw["input_layernorm"] = np.ones(HIDDEN, np.float32)
        fw["post_attention_layernorm"] = np.ones(HIDDEN, np.float32)
    else:
        fw["input_layernorm"] = round_bfloat16_array(1.0 + normal(HIDDEN, 0.1))
        fw["post_attention_layernorm"] = round_bfloat16_array(1.0 + normal(HIDDEN, 0.1))
    w, s = pack_layer_parameters(fw)
    return LayerCase.from_images(w, s)


def random_hidden(seed: int, tokens: int, scale: float = 1.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((tokens, HIDDEN), dtype=np.float32) * np.float32(scale)).reshape(-1).copy()


def quantized_kv_history(seed: int, rows: int) -> tuple[np.ndarray, np.ndarray]:
    """K/V rows N(0,1), each 256-wide row quantized to INT4 (absmax/7) and dequantized to fp32."""
    from work_llm_accelerator_amd.quant import quantize_int4_per_channel

    rng = np.random.default_rng(seed)
    out = []
    for _ in range(2):
        m = rng.standard_normal((rows, KV_WIDTH), dtype=np.float32)
        packed, scales = quantize_int4_per_channel(m)
        nib = np.stack([packed & 0xF, packed >> 4], axis=1).reshape(rows, KV_WIDTH).astype(np.int32)
        q = np.where(nib >= 8, nib - 16, nib).astype(np.float32)
        out.append((q * scales[:, None]).astype(np.float32).reshape(-1))
    return out[0], out[1]


# ---- callers (fn is any library's function with the reference signature) ----
def decode_layer(fn, case: LayerCase, x, past, k_cache, v_cache):
    out = np.zeros(HIDDEN, np.float32)
    st = fn(x, past, *case.layer_args(), k_cache, v_cache, out)
    return st, out


def decode_attention(fn, case: LayerCase, x, past, k_cache, v_cache):
    out = np.zeros(HIDDEN, np.float32)
    st = fn(x, past, *case.attention_args(), k_cache, v_cache, out)
    return st, out


def decode_mlp(fn, case: LayerCase, a):
    out = np.zeros(HIDDEN, np.float32)
    st = fn(a, *case.mlp_args(), out)
    return st, out


def prefill_layer(fn, case: LayerCase, x, seq_len, tiles: PrefillTileConfig):
    kc = np.zeros(seq_len * KV_WIDTH, np.float32)
    vc = np.zeros(seq_len * KV_WIDTH, np.float32)
    out = np.zeros(seq_len * HIDDEN, np.float32)
    st = fn(x, seq_len, *tiles.as_args(), *case.layer_args(), kc, vc, out)
    return st, out, kc, vc


def prefill_attention(fn, case: LayerCase, x, seq_len, tiles: PrefillTileConfig):
    kc = np.zeros(seq_len * KV_WIDTH, np.float32)
    vc = np.zeros(seq_len * KV_WIDTH, np.float32)
    out = np.zeros(seq_len * HIDDEN, np.float32)
    st = fn(x, seq_len, *tiles.as_args()[:8], *case.attention_args(), kc, vc, out)
    return st, out, kc, vc


def prefill_mlp(fn, case: LayerCase, a, seq_len, tiles: PrefillTileConfig):
    out = np.zeros(seq_len * HIDDEN, np.float32)
    st = fn(a, seq_len, *tiles.as_args()[8:], *case.mlp_args(), out)
    return st, out


def bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    return np.array_equal(np.ascontiguousarray(a).view(np.uint32), np.ascontiguousarray(b).view(np.uint32))


def first_mismatch(a: np.ndarray, b: np.ndarray) -> str:
    ua = np.ascontiguousarray(a).view(np.uint32)
    ub = np.ascontiguousarray(b).view(np.uint32)
    idx = np.nonzero(ua != ub)[0]
    if idx.size == 0:
        return "identical"
    i = int(idx[0])
    return f"{idx.size} mismatches; first at {i}: {a[i]!r} vs {b[i]!r}; max|d|={np.max(np.abs(a - b)):.3g}"


def raw_function(lib_path, name: str, prefix: str = ""):
    """The entry point with every pointer argument declared as c_void_p, so a test can pass None
    (a null pointer) where the reference checks for one.  Arrays are passed as their data address."""
    import ctypes

    from work_llm_accelerator_amd.abi import SIGNATURES

    fn = getattr(ctypes.CDLL(str(lib_path)), prefix + name)
    argtypes = [a if a in (ctypes.c_int, ctypes.c_uint64) else ctypes.c_void_p for a in SIGNATURES[name]]
    fn.argtypes = argtypes
    fn.restype = ctypes.c_int

    def call(*args):
        conv = [a.ctypes.data if isinstance(a, np.ndarray) else a for a in args]
        return fn(*conv)

    return call
