"""The device's host-compatible expf (used by the ORDERED decode softmax and SiLU in place of
glibc's expf, qwen_decode_attention_kernel.cpp:149 and qwen_decode_mlp_kernel.cpp:80) against the
host expf, bit for bit, on every third float bit pattern (1.43 G inputs: every sign, exponent and
mantissa region including denormals, infinities and NaNs), in chunks of 2^26."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from _oracle import oracle

pytestmark = pytest.mark.gpu

STRIDE = 3          # coprime with 2^32: the sweep visits distinct bit patterns
CHUNK = 1 << 26


def test_device_expf_matches_host_expf_strided_sweep():
    import torch

    from work_llm_accelerator_amd import abi

    lib = abi.load()
    o = oracle()
    o.oracle_count_expf_mismatches.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64,
                                               np.ctypeslib.ndpointer(dtype=np.float32, ndim=1,
                                                                      flags="C_CONTIGUOUS"),
                                               ctypes.POINTER(ctypes.c_uint32)]
    o.oracle_count_expf_mismatches.restype = ctypes.c_uint64
    total = (1 << 32) // STRIDE + 1
    dev = torch.empty(CHUNK, dtype=torch.float32, device="cuda")
    host = torch.empty(CHUNK, dtype=torch.float32, pin_memory=True)
    done, mismatches = 0, 0
    first_bad = ctypes.c_uint32(0)
    while done < total:
        n = min(CHUNK, total - done)
        first = (done * STRIDE) & 0xFFFFFFFF
        st = lib.qwen_hip_eval_expf(first, STRIDE, n, ctypes.c_void_p(dev.data_ptr()),
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert st == 0, abi.last_error(lib)
        host[:n].copy_(dev[:n])
        torch.cuda.synchronize()
        fb = ctypes.c_uint32(0)
        bad = o.oracle_count_expf_mismatches(first, STRIDE, n, host[:n].numpy(), ctypes.byref(fb))
        if bad and not mismatches:
            first_bad = fb
        mismatches += bad
        done += n
    print(f"expf sweep: {done} inputs, {mismatches} mismatches", flush=True)
    assert mismatches == 0, f"first mismatching input bits 0x{first_bad.value:08x}"
