"""ctypes bindings of the MI355X C ABI.

`load()` opens the in-tree HIP library and declares every entry point with the argument types
the reference's own callers use (verification/real_host_top_backend.py:78-136 and the decode /
prefill validators), so code written against the reference host libraries can switch to this
build by changing only the library path.  The library is never replaced by a CPU fallback: if it
is missing, `load()` raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB_DIR = Path(__file__).resolve().parent / "_lib"
LIB_PATH = LIB_DIR / "libqwen_mi355x.so"
DECODE_STUB_PATH = LIB_DIR / "libqwen_decode_stub.so"
PREFILL_STUB_PATH = LIB_DIR / "libqwen_prefill_stub.so"

F32P = np.ctypeslib.ndpointer(dtype=np.float32, ndim=1, flags="C_CONTIGUOUS")
U8P = np.ctypeslib.ndpointer(dtype=np.uint8, ndim=1, flags="C_CONTIGUOUS")
I32P = np.ctypeslib.ndpointer(dtype=np.int32, ndim=1, flags="C_CONTIGUOUS")
c_int, c_u64, c_void_p, c_f64 = ctypes.c_int, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_double

# Argument lists in reference order (hls/decode_only/qwen_decode_host_wrapper.h:9-87,
# hls/prefill_only/qwen_prefill_host_wrapper.h:9-169).
_TILES_ATT = [c_int] * 8
_TILES_MLP = [c_int] * 3
_SRAM = [U8P, F32P, I32P, F32P, F32P]

SIGNATURES: dict[str, list] = {
    "qwen_decode_stub_forward": [F32P, c_int, F32P],
    "qwen_decode_attention_smoke_forward": [F32P, c_int, F32P] + [U8P] * 4 + [F32P] * 7 + [F32P] * 3,
    "qwen_decode_mlp_smoke_forward": [F32P, F32P] + [U8P] * 3 + [F32P] * 3 + [F32P],
    "qwen_decode_layer_smoke_forward": [F32P, c_int, F32P, F32P] + [U8P] * 7 + [F32P] * 10 + [F32P] * 3,
    "qwen_decode_top_smoke_forward": [c_int, c_int] + [c_u64] * 6 + [U8P, F32P, F32P, F32P] + _SRAM,
    "qwen_prefill_stub_forward": [F32P, c_int] + _TILES_ATT + _TILES_MLP + [F32P],
    "qwen_prefill_attention_smoke_forward": [F32P, c_int] + _TILES_ATT + [F32P] + [U8P] * 4 + [F32P] * 7
    + [F32P] * 3,
    "qwen_prefill_mlp_smoke_forward": [F32P, c_int] + _TILES_MLP + [F32P] + [U8P] * 3 + [F32P] * 3 + [F32P],
    "qwen_prefill_layer_smoke_forward": [F32P, c_int] + _TILES_ATT + _TILES_MLP + [F32P, F32P] + [U8P] * 7
    + [F32P] * 10 + [F32P] * 3,
    "qwen_prefill_glue_smoke_forward": [F32P, c_int] + _TILES_ATT + _TILES_MLP + [F32P, F32P] + [U8P] * 7
    + [F32P] * 10 + [F32P] * 3,
    "qwen_prefill_top_smoke_forward": [c_int, c_int] + _TILES_ATT + _TILES_MLP + [c_u64] * 6
    + [U8P, F32P, F32P, F32P] + _SRAM,
    "qwen_decode_dispatch_layers_forward": [c_void_p, c_int, U8P, F32P, F32P, F32P] + _SRAM + [c_void_p],
    "qwen_prefill_dispatch_layers_forward": [c_void_p, c_int, U8P, F32P, F32P, F32P] + _SRAM + [c_void_p],
    # unquantized layer-0 reference wrappers: 16 weight / bias pointers (biases may be None)
    "qwen_decode_layer0_reference_forward": [F32P, c_int, c_void_p, c_void_p] + [c_void_p] * 16
    + [ctypes.c_float, F32P, F32P, F32P],
    "qwen_prefill_layer0_reference_forward": [F32P, c_int] + [c_void_p] * 16 + [ctypes.c_float, F32P],
    "qwen_prefill_layer0_reference_forward_with_cache": [F32P, c_int] + [c_void_p] * 16
    + [ctypes.c_float, F32P, c_void_p, c_void_p],
}

# Additive entry points of this build (no counterpart in the reference): the device-resident
# model API of include/qwen_hip_model.h.  Device pointers are passed as c_void_p.
P = ctypes.c_void_p
EXTRA_SIGNATURES: dict[str, tuple[list, object]] = {
    "qwen_hip_last_error": ([], ctypes.c_char_p),
    "qwen_hip_model_create": ([c_int, U8P, F32P, ctypes.POINTER(P)], c_int),
    "qwen_hip_model_create_synthetic": ([c_int, c_u64, ctypes.POINTER(P)], c_int),
    "qwen_hip_model_destroy": ([P], c_int),
    "qwen_hip_model_layers": ([P], c_int),
    "qwen_hip_model_stream": ([P], P),
    "qwen_hip_model_synchronize": ([P], c_int),
    "qwen_hip_model_decode": ([P, c_int, c_int, P, P, c_int, P, P, c_u64, c_u64], c_int),
    "qwen_hip_model_prefill": ([P, c_int, c_int, c_int, P, P, P, c_u64, c_u64], c_int),
    "qwen_hip_model_prefill_chunk": ([P, c_int, c_int, c_int, c_int, P, P, P, c_u64, c_u64], c_int),
    "qwen_hip_model_decode_layers": ([P, c_int, c_int, c_int, c_int, P, P, c_int, P, P, c_u64, c_u64], c_int),
    "qwen_hip_model_prefill_layers": ([P, c_int, c_int, c_int, c_int, c_int, c_int, P, P, P, c_u64, c_u64], c_int),
    "qwen_hip_model_embed": ([P, P, c_int, P], c_int),
    "qwen_hip_model_set_head": ([P, c_int, P, P], c_int),
    "qwen_hip_model_vocab": ([P], c_int),
    "qwen_hip_model_logits": ([P, P, c_int, P], c_int),
    "qwen_hip_model_greedy": ([P, P, c_int, P], c_int),
    "qwen_hip_model_time_kernel": ([P, c_int, c_int, c_int, ctypes.POINTER(ctypes.c_float)], c_int),
    "qwen_hip_quantize_int4": ([P, c_int, c_int, P, P, P], c_int),
    "qwen_hip_fill_kv_synthetic": ([P, c_u64, c_u64, P], c_int),
    "qwen_hip_eval_expf": ([ctypes.c_uint32, ctypes.c_uint32, c_u64, P, P], c_int),
    "qwen_hip_model_layer_images": ([P, c_int, U8P, F32P], c_int),
    "qwen_hip_model_head_tables": ([P, np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS"),
                                    np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")], c_int),
    # FAST operators (include/qwen_hip_ops.h)
    "qwen_hip_fast_quantize_rows": ([P, c_int, c_int, P, P, P, P], c_int),
    "qwen_hip_fast_project": ([P, P, P, c_int, c_int, P, c_int, c_int, P, P], c_int),
    "qwen_hip_fast_silu_mul_grouped": ([P, P, P, P, P, c_int, P, P, P, P, P], c_int),
    "qwen_hip_fast_project_grouped": ([P, P, c_int, P, P, P, c_int, P, P], c_int),
    # device-resident descriptor dispatch (include/qwen_hip_dispatch.h): descriptors on the host,
    # DDR images on the device
    "qwen_hip_decode_dispatch_layers": ([c_void_p, c_int, P, P, P, P, P, c_void_p], c_int),
    "qwen_hip_prefill_dispatch_layers": ([c_void_p, c_int, P, P, P, P, P, c_void_p], c_int),
    "qwen_hip_decode_dispatch_layers_noalloc": ([c_void_p, c_int, P, P, P, P, P, c_void_p], c_int),
}

_LIB: ctypes.CDLL | None = None


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Loads the HIP library (default: the in-tree build) and declares every entry point."""
    global _LIB
    if path is None and _LIB is not None:
        return _LIB
    lib_path = Path(path) if path is not None else LIB_PATH
    if not lib_path.exists():
        raise FileNotFoundError(
            f"{lib_path} is missing: build it with `python -m work_llm_accelerator_amd.build` "
            "(there is no CPU fallback for the HIP path)")
    lib = ctypes.CDLL(str(lib_path))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = c_int
    for name, (argtypes, restype) in EXTRA_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    if path is None:
        _LIB = lib
    return lib


def last_error(lib: ctypes.CDLL | None = None) -> str:
    lib = lib or load()
    msg = lib.qwen_hip_last_error()
    return msg.decode() if msg else ""
