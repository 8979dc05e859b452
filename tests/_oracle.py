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

_oracle = None


def oracle() -> ctypes.CDLL:
    global _oracle
    if _oracle is not None:
        return _oracle
    if not ORACLE_LIB.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle"), "oracle"], check=True, capture_output=True)
    lib = ctypes.CDLL(str(ORACLE_LIB))
    for name, argtypes in SIGNATURES.items():
        if "dispatch" in name:
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
    _oracle = lib
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
