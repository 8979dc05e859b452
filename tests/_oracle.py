"""ctypes binding of the CPU oracle (oracle/build/libqwen_oracle.so) and of the reference decode
library compiled from the reference sources (oracle/_ref/libqwen_decode_ref.so).

Test infrastructure only: the oracle is the checker, never the thing under test.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

from work_llm_accelerator_amd.abi import F32P, SIGNATURES, U8P, c_int

ROOT = Path(__file__).resolve().parents[1]
ORACLE_LIB = ROOT / "oracle" / "build" / "libqwen_oracle.so"
REF_DECODE_LIB = ROOT / "oracle" / "_ref" / "libqwen_decode_ref.so"
REF_PREFILL_L0_LIB = ROOT / "oracle" / "_ref" / "libqwen_prefill_layer0_ref.so"

_oracle = None


def oracle() -> ctypes.CDLL:
    global _oracle
    if _oracle is not None:
        return _oracle
    if not ORACLE_LIB.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle"), "oracle"], check=True, capture_output=True)
    lib = ctypes.CDLL(str(ORACLE_LIB))
    for name, argtypes in SIGNATURES.items():
        if "dispatch" in name or "layer0" in name:  # layer-0 wrappers: pinned by the compiled reference
            continue
        fn = getattr(lib, "oracle_" + name.removeprefix("qwen_"))
        fn.argtypes = argtypes
        fn.restype = c_int
    f = ctypes.c_float
    for name in ("oracle_approx_sqrt", "oracle_wrap_angle", "oracle_approx_exp", "oracle_silu_decode",
                 "oracle_silu_prefill", "oracle_libm_expf"):
        fn = getattr(lib, name)
        fn.argtypes = [f]
        fn.restype = f
    lib.oracle_approx_sincos.argtypes = [f, ctypes.POINTER(f), ctypes.POINTER(f)]
    lib.oracle_approx_sincos.restype = None
    lib.oracle_round_bf16.argtypes = [F32P, ctypes.c_size_t]
    lib.oracle_round_bf16.restype = None
    lib.oracle_quantize_int4.argtypes = [F32P, c_int, c_int, U8P, F32P]
    lib.oracle_quantize_int4.restype = None
    for name in ("oracle_decode_rope_row", "oracle_prefill_rope_row"):
        fn = getattr(lib, name)
        fn.argtypes = [c_int, F32P, F32P]
        fn.restype = None
    lib.oracle_layer_offsets.argtypes = [np.ctypeslib.ndpointer(dtype=np.uint64, ndim=1, flags="C_CONTIGUOUS")]
    lib.oracle_layer_offsets.restype = None
    lib.oracle_prefill_layer_uncapped.argtypes = [F32P, c_int, U8P, F32P, F32P, F32P, F32P]
    lib.oracle_prefill_layer_uncapped.restype = c_int
    lib.oracle_decode_layer_block.argtypes = [F32P, c_int, U8P, F32P, F32P, F32P, F32P]
    lib.oracle_decode_layer_block.restype = c_int
    U16P = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
    I32P = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
    F32A = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
    lib.oracle_head_norm.argtypes = [F32A, c_int, U16P, U16P]
    lib.oracle_head_norm.restype = None
    lib.oracle_lm_head.argtypes = [U16P, c_int, U16P, c_int, F32A]
    lib.oracle_lm_head.restype = None
    lib.oracle_argmax.argtypes = [F32A, c_int, c_int, I32P]
    lib.oracle_argmax.restype = None
    _oracle = lib
    return lib


def ref_prefill_layer0() -> ctypes.CDLL | None:
    """The reference's unquantized prefill layer-0 wrapper built from its own source, or None."""
    if not REF_PREFILL_L0_LIB.exists():
        return None
    lib = ctypes.CDLL(str(REF_PREFILL_L0_LIB))
    for name in ("qwen_prefill_layer0_reference_forward", "qwen_prefill_layer0_reference_forward_with_cache"):
        fn = getattr(lib, name)
        fn.argtypes = SIGNATURES[name]
        fn.restype = c_int
    return lib


def ref_decode() -> ctypes.CDLL | None:
    """The reference decode host library built from its own sources, or None when absent."""
    if not REF_DECODE_LIB.exists():
        return None
    lib = ctypes.CDLL(str(REF_DECODE_LIB))
    for name, argtypes in SIGNATURES.items():
        if name.startswith("qwen_decode") and "dispatch" not in name:
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = c_int
    return lib


def head_logits(hidden: np.ndarray, norm_bf16: np.ndarray, table_bf16: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Oracle final RMSNorm + lm_head: (normalized rows as bf16 bits [N,1536], logits [N,vocab] fp32)."""
    lib = oracle()
    x = np.ascontiguousarray(hidden, dtype=np.float32).reshape(-1, 1536)
    n = x.shape[0]
    xn = np.zeros((n, 1536), dtype=np.uint16)
    lib.oracle_head_norm(x, n, np.ascontiguousarray(norm_bf16, dtype=np.uint16), xn)
    vocab = table_bf16.shape[0]
    logits = np.zeros((n, vocab), dtype=np.float32)
    lib.oracle_lm_head(xn, n, np.ascontiguousarray(table_bf16, dtype=np.uint16), vocab, logits)
    return xn, logits


def argmax_rows(logits: np.ndarray) -> np.ndarray:
    lib = oracle()
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    ids = np.zeros(lg.shape[0], dtype=np.int32)
    lib.oracle_argmax(lg, lg.shape[0], lg.shape[1], ids)
    return ids
