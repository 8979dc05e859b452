"""The allocation-free decode dispatch (qwen_hip_decode_dispatch_layers_noalloc) against the
allocating device dispatch it varies (qwen_hip_decode_dispatch_layers), bit for bit, through the C ABI.

Two calls in a row on the same GPU (the second with a smaller input: fewer layers, a shorter KV
history), each compared with the allocating entry point run on copies of the same buffers; the
scratch keeps the first call's contents, so the second call also shows that nothing stale is read.
Status codes and completed counts of a failing descriptor and a null port match too.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from _cases import bits_equal, first_mismatch, quantized_kv_history, random_hidden, random_layer
from work_llm_accelerator_amd import abi
from work_llm_accelerator_amd import layout as L
from work_llm_accelerator_amd.layout import HIDDEN, KV_WIDTH

pytestmark = pytest.mark.gpu

NL = 3
KV_LAYER = L.build_kv_cache_layout().layer_stride_bytes
V_BASE = L.build_kv_cache_layout().v_base_offset_bytes


@pytest.fixture(scope="module")
def torch():
    import torch as t

    return t


@pytest.fixture(scope="module")
def lib():
    return abi.load()


def dptr(t):
    return ctypes.c_void_p(t.data_ptr())


def setup(torch, past, layers):
    imgs = [random_layer(seed=41 + i) for i in range(layers)]
    w = torch.from_numpy(np.concatenate([c.weight_ddr for c in imgs])).cuda()
    s = torch.from_numpy(np.concatenate([c.scale_ddr for c in imgs])).cuda()
    kv = torch.zeros((V_BASE + layers * KV_LAYER) // 4, dtype=torch.float32, device="cuda")
    for l in range(layers):
        k, v = quantized_kv_history(500 + 7 * past + l, past)
        kv[(l * KV_LAYER) // 4:(l * KV_LAYER) // 4 + past * KV_WIDTH] = torch.from_numpy(k)
        kv[(V_BASE + l * KV_LAYER) // 4:(V_BASE + l * KV_LAYER) // 4 + past * KV_WIDTH] = torch.from_numpy(v)
    act = torch.zeros((layers + 1) * HIDDEN, dtype=torch.float32, device="cuda")
    act[:HIDDEN] = torch.from_numpy(random_hidden(77 + past, 1))
    torch.cuda.synchronize()
    return w, s, kv, act


def call(fn, descs, w, s, kv, act):
    arr = L.to_c_decode(descs)
    done = ctypes.c_int(-1)
    st = fn(ctypes.cast(arr, ctypes.c_void_p), len(descs), dptr(w), dptr(s), dptr(kv), dptr(act), None,
            ctypes.byref(done))
    return st, done.value


@pytest.mark.parametrize("calls", [((40, 3), (6, 2))])
def test_noalloc_matches_allocating_dispatch(torch, lib, calls):
    for past, layers in calls:
        print(f"no-alloc decode dispatch: {layers} layers, past {past}", flush=True)
        w, s, kv, act = setup(torch, past, layers)
        kv2, act2 = kv.clone(), act.clone()
        torch.cuda.synchronize()
        descs = L.build_decode_descriptors(past, 0, 0, 0, 0, 0)[:layers]
        assert call(lib.qwen_hip_decode_dispatch_layers_noalloc, descs, w, s, kv, act) == (0, layers), \
            abi.last_error(lib)
        torch.cuda.synchronize()  # the no-alloc entry point returns without synchronizing
        assert call(lib.qwen_hip_decode_dispatch_layers, descs, w, s, kv2, act2) == (0, layers)
        a, b = act.cpu().numpy(), act2.cpu().numpy()
        assert bits_equal(a, b), first_mismatch(a, b)
        for l in range(layers):
            for base in ((l * KV_LAYER) // 4, (V_BASE + l * KV_LAYER) // 4):
                g = kv[base:base + (past + 1) * KV_WIDTH].cpu().numpy()
                r = kv2[base:base + (past + 1) * KV_WIDTH].cpu().numpy()
                assert bits_equal(g, r), f"layer {l}: " + first_mismatch(g, r)


def test_noalloc_status_codes(torch, lib):
    from dataclasses import replace

    w, s, kv, act = setup(torch, 4, 2)
    descs = L.build_decode_descriptors(4, 0, 0, 0, 0, 0)[:2]
    bad = [descs[0], replace(descs[1], layer_id=-1)]
    assert call(lib.qwen_hip_decode_dispatch_layers_noalloc, bad, w, s, kv, act) == (10, 1)
    torch.cuda.synchronize()
    arr = L.to_c_decode(descs)
    done = ctypes.c_int(-1)
    assert lib.qwen_hip_decode_dispatch_layers_noalloc(ctypes.cast(arr, ctypes.c_void_p), 2, dptr(w), dptr(s), None,
                                                       dptr(act), None, ctypes.byref(done)) == 11
    assert done.value == 0
    assert lib.qwen_hip_decode_dispatch_layers_noalloc(None, 2, dptr(w), dptr(s), dptr(kv), dptr(act), None,
                                                       ctypes.byref(done)) == 10
