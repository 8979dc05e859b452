"""Device-resident multi-layer model (include/qwen_hip_model.h) driven from Python.

This is the host side of the 28-layer drivers of the reference
(verification/real_host_top_backend.py:208-351: per-layer DDR images, layer loop, bf16 rounding
between layers) on top of the HIP library's device-resident API.  torch is used only to own
device memory and to wrap the model's HIP stream; every layer runs in the HIP library.  There is
no CPU fallback: without the built library or a GPU the constructor raises.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import abi
from .layout import HIDDEN, KV_WIDTH, LAYOUT

MODE_ORDERED = 0
MODE_FAST = 1
FLAG_NO_BF16_ROUND = 0x100  # skip the driver's bf16 rounding between layers
FLAG_SEPARATE_REDUCE = 0x200  # FAST decode of one sequence: the row steps fused into projections as own launches
FLAG_SEPARATE_ATTN = 0x400  # FAST decode of one sequence: the attention as its own launch (not in the Q/K/V blocks)

KERNEL_ATTN_DECODE = 1
KERNEL_GEMM_GATE_UP = 2
KERNEL_GEMM_DOWN = 3
KERNEL_GEMM_QKV = 4
KERNEL_GEMM_O = 5
KERNEL_ATTN_PREFILL = 6


def _ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _check(lib, status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what} failed with status {status}: {abi.last_error(lib)}")


@dataclass
class KvCache:
    """Token-major fp32 K and V caches, [layers][sequences][positions][256] each."""

    k: "object"  # torch.Tensor on the GPU
    v: "object"
    layers: int
    sequences: int
    positions: int

    @property
    def seq_stride(self) -> int:
        return self.positions * KV_WIDTH

    @property
    def layer_stride(self) -> int:
        return self.sequences * self.seq_stride

    @classmethod
    def allocate(cls, layers: int, sequences: int, positions: int, device="cuda:0"):
        import torch

        shape = (layers, sequences, positions, KV_WIDTH)
        return cls(torch.zeros(shape, dtype=torch.float32, device=device),
                   torch.zeros(shape, dtype=torch.float32, device=device), layers, sequences, positions)


class DeviceModel:
    """A stack of quantized decoder layers resident in HBM."""

    def __init__(self, layers: int, weight_ddr: np.ndarray | None = None, scale_ddr: np.ndarray | None = None,
                 synthetic_seed: int | None = None):
        import torch

        if not torch.cuda.is_available():
            raise RuntimeError("DeviceModel needs a GPU (the HIP path has no CPU fallback)")
        self.lib = abi.load()
        handle = ctypes.c_void_p()
        if synthetic_seed is not None:
            st = self.lib.qwen_hip_model_create_synthetic(layers, synthetic_seed, ctypes.byref(handle))
        else:
            if weight_ddr is None or scale_ddr is None:
                raise ValueError("weight_ddr and scale_ddr are required unless synthetic_seed is given")
            if weight_ddr.size != layers * LAYOUT.total_parameter_bytes or scale_ddr.size * 4 != weight_ddr.size:
                raise ValueError("images must hold `layers` blocks of QWEN_LAYER_BYTES each")
            st = self.lib.qwen_hip_model_create(layers, np.ascontiguousarray(weight_ddr),
                                                np.ascontiguousarray(scale_ddr), ctypes.byref(handle))
        _check(self.lib, st, "qwen_hip_model_create")
        self.handle = handle
        self.layers = layers
        self.stream = torch.cuda.ExternalStream(self.lib.qwen_hip_model_stream(handle))

    def close(self) -> None:
        if getattr(self, "handle", None) is not None and self.handle.value:
            self.lib.qwen_hip_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def synchronize(self) -> None:
        _check(self.lib, self.lib.qwen_hip_model_synchronize(self.handle), "synchronize")

    def _enter(self):
        """Orders the model's stream after work already queued on torch's current stream."""
        import torch

        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream())
        self.stream.wait_event(ev)

    def _range(self, cache: KvCache, layers) -> tuple[int, int, int]:
        """(first layer, layer count, cache offset in floats) of a `layers` range: None for every layer,
        an int for one layer, or (first, count).  A cache of fewer layers than the model holds the
        range's own layers from its layer 0; a whole-model cache holds every layer."""
        if layers is None:
            first, count = 0, self.layers
        elif isinstance(layers, int):
            first, count = layers, 1
        else:
            first, count = int(layers[0]), int(layers[1])
        if cache.layers == self.layers:
            return first, count, first * cache.layer_stride
        if cache.layers < count:
            raise ValueError(f"cache holds {cache.layers} layers, the range {count}")
        return first, count, 0

    def decode(self, mode: int, hidden, positions, max_keys: int, cache: KvCache, order: bool = True,
               layers=None) -> None:
        """hidden [B,1536] fp32 (in/out), positions [B] int32 on the GPU; `layers` as in _range."""
        if order:
            self._enter()
        B = hidden.shape[0]
        first, count, off = self._range(cache, layers)
        st = self.lib.qwen_hip_model_decode_layers(self.handle, mode, first, count, B, _ptr(hidden), _ptr(positions),
                                                   int(max_keys), ctypes.c_void_p(cache.k.data_ptr() + 4 * off),
                                                   ctypes.c_void_p(cache.v.data_ptr() + 4 * off), cache.seq_stride,
                                                   cache.layer_stride)
        _check(self.lib, st, "qwen_hip_model_decode_layers")

    def prefill(self, mode: int, hidden, cache: KvCache, order: bool = True, past: int = 0, layers=None) -> None:
        """hidden [B,S,1536] fp32 (in/out) at positions past..past+S-1; cache rows past..past+S-1 of
        sequences 0..B-1 are written (rows 0..past-1 hold the earlier tokens); `layers` as in _range."""
        if order:
            self._enter()
        B, S = hidden.shape[0], hidden.shape[1]
        first, count, off = self._range(cache, layers)
        st = self.lib.qwen_hip_model_prefill_layers(self.handle, mode, first, count, B, S, int(past), _ptr(hidden),
                                                    ctypes.c_void_p(cache.k.data_ptr() + 4 * off),
                                                    ctypes.c_void_p(cache.v.data_ptr() + 4 * off), cache.seq_stride,
                                                    cache.layer_stride)
        _check(self.lib, st, "qwen_hip_model_prefill_layers")

    def embed(self, token_ids, hidden, order: bool = True) -> None:
        if order:
            self._enter()
        st = self.lib.qwen_hip_model_embed(self.handle, _ptr(token_ids), int(token_ids.numel()), _ptr(hidden))
        _check(self.lib, st, "qwen_hip_model_embed")

    @property
    def vocab(self) -> int:
        """Rows of the tied embedding / lm_head table (0 when the model has no head)."""
        return int(self.lib.qwen_hip_model_vocab(self.handle))

    def set_head(self, embed_bf16: np.ndarray, norm_bf16: np.ndarray) -> None:
        """Uploads a tied bf16 embedding / lm_head table [vocab, 1536] and the bf16 final RMSNorm
        weight [1536], both as uint16 bit patterns (vocab a multiple of 128)."""
        embed = np.ascontiguousarray(embed_bf16, dtype=np.uint16)
        norm = np.ascontiguousarray(norm_bf16, dtype=np.uint16)
        if embed.ndim != 2 or embed.shape[1] != 1536 or norm.shape != (1536,):
            raise ValueError("embed must be [vocab, 1536] and norm [1536] (bf16 bit patterns)")
        st = self.lib.qwen_hip_model_set_head(self.handle, embed.shape[0], embed.ctypes.data_as(ctypes.c_void_p),
                                              norm.ctypes.data_as(ctypes.c_void_p))
        _check(self.lib, st, "qwen_hip_model_set_head")

    def logits(self, hidden, logits, order: bool = True) -> None:
        """Final RMSNorm + tied bf16 lm_head of hidden [N,1536] fp32 into logits [N,vocab] fp32
        (bf16-rounded values, verification/real_host_top_backend.py:138-146)."""
        if order:
            self._enter()
        n = hidden.numel() // 1536
        st = self.lib.qwen_hip_model_logits(self.handle, _ptr(hidden), n, _ptr(logits))
        _check(self.lib, st, "qwen_hip_model_logits")

    def greedy(self, hidden, token_ids, order: bool = True) -> None:
        """Greedy next token ids [N] int32 of hidden [N,1536] (torch.argmax of the logits)."""
        if order:
            self._enter()
        n = hidden.numel() // 1536
        st = self.lib.qwen_hip_model_greedy(self.handle, _ptr(hidden), n, _ptr(token_ids))
        _check(self.lib, st, "qwen_hip_model_greedy")

    def time_kernel(self, kernel: int, layer: int = 0, reps: int = 20) -> float:
        """Mean milliseconds of one launch of `kernel`, re-run in isolation with the shapes of the
        last FAST call (HIP events on the model's stream)."""
        ms = ctypes.c_float(0.0)
        st = self.lib.qwen_hip_model_time_kernel(self.handle, kernel, layer, reps, ctypes.byref(ms))
        _check(self.lib, st, "qwen_hip_model_time_kernel")
        return float(ms.value)


def fill_kv_synthetic(cache: KvCache, seed: int) -> None:
    """N(0,1) K/V rows quantized per row to INT4 and dequantized, generated on the device."""
    lib = abi.load()
    rows = cache.layers * cache.sequences * cache.positions
    _check(lib, lib.qwen_hip_fill_kv_synthetic(_ptr(cache.k), rows, seed, None), "fill K")
    _check(lib, lib.qwen_hip_fill_kv_synthetic(_ptr(cache.v), rows, seed + 0x5bd1e995, None), "fill V")


def quantize_int4_device(w) -> tuple:
    """Device INT4 quantizer (verification/real_host_top_backend.py:31-41) of an fp32 [out,in]
    torch tensor on the GPU; returns (packed uint8 [out*in/2], scales fp32 [out])."""
    import torch

    out_dim, in_dim = w.shape
    packed = torch.empty(out_dim * in_dim // 2, dtype=torch.uint8, device=w.device)
    scales = torch.empty(out_dim, dtype=torch.float32, device=w.device)
    lib = abi.load()
    st = lib.qwen_hip_quantize_int4(_ptr(w.contiguous()), out_dim, in_dim, _ptr(packed), _ptr(scales),
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _check(lib, st, "qwen_hip_quantize_int4")
    return packed, scales


__all__ = ["DeviceModel", "KvCache", "fill_kv_synthetic", "quantize_int4_device", "MODE_ORDERED", "MODE_FAST",
           "HIDDEN"]
