"""Layer dispatch over descriptors, on the GPU.

The reference's C++ layer loops qwen_decode_dispatch_layers / qwen_prefill_dispatch_layers
(hls/decode_only/qwen_decode_top_wrapper.cpp:115-130, hls/prefill_only/qwen_prefill_top_wrapper.cpp:
20-35) run the top wrapper per descriptor and stop at the first failure with
completed_layer_count = its index.  Both exports of this build are checked here:

* qwen_{decode,prefill}_dispatch_layers_forward, the host-buffer C ABI (drop-in library);
* qwen_hip_{decode,prefill}_dispatch_layers, the same loop over DDR images resident in HBM.

Decode descriptors come from the global map builder (work_llm_accelerator_amd.layout, the twin of
python/layer_descriptor_builder.py:205-238: weights at a 23,508,992-byte stride, K at 0 and V at
28 x 32 MiB, activations chained); every layer output and appended K/V row must equal the reference
decode library built from its own sources (oracle/_ref, or the oracle where it is absent) run
descriptor by descriptor, bit for bit.  Prefill descriptors from the global builder are rejected at
the first descriptor with 22 (qwen_prefill_top_core.cpp:42-80 only accepts per-layer windows), and
with the builder's Python default tiles with 20; a chain of descriptors inside the windows equals the
oracle's prefill top run per descriptor.  Mid-list failures give the failing status and index, and
the layers before them keep their outputs.
"""

from __future__ import annotations

import ctypes
from dataclasses import replace

import numpy as np
import pytest

from _cases import SRAM, bits_equal, first_mismatch, quantized_kv_history, random_hidden, random_layer
from _oracle import oracle, ref_decode
from work_llm_accelerator_amd import abi
from work_llm_accelerator_amd import layout as L
from work_llm_accelerator_amd.layout import HIDDEN, KV_WIDTH

pytestmark = pytest.mark.gpu

LAYER_BLOCK = L.LAYOUT.total_parameter_bytes
NL = 3      # layers of the global images
PAST = 6
KV_LAYER = L.build_kv_cache_layout().layer_stride_bytes
V_BASE = L.build_kv_cache_layout().v_base_offset_bytes


@pytest.fixture(scope="module")
def torch():
    import torch as t

    return t


@pytest.fixture(scope="module")
def images():
    layers = [random_layer(seed=21 + i) for i in range(NL)]
    w = np.concatenate([c.weight_ddr for c in layers])
    s = np.concatenate([c.scale_ddr for c in layers])
    return w, s


@pytest.fixture(scope="module")
def lib():
    return abi.load()


def reference_top():
    """The reference's decode top wrapper (compiled from its sources) or the oracle's restatement."""
    ref = ref_decode()
    if ref is not None:
        return ref.qwen_decode_top_smoke_forward
    return oracle().oracle_decode_top_smoke_forward


def global_kv():
    """K/V DDR of the global map up to V of layer NL-1 (zero pages stay unallocated) with PAST history
    rows of quantized N(0,1) values at every layer's K and V base."""
    floats = (V_BASE + NL * KV_LAYER) // 4
    kv = np.zeros(floats, np.float32)
    for l in range(NL):
        k, v = quantized_kv_history(300 + l, PAST)
        kv[(l * KV_LAYER) // 4:(l * KV_LAYER) // 4 + PAST * KV_WIDTH] = k
        kv[(V_BASE + l * KV_LAYER) // 4:(V_BASE + l * KV_LAYER) // 4 + PAST * KV_WIDTH] = v
    return kv


def run_reference_decode(descs, w, s, kv, act):
    top = reference_top()
    for d in descs:
        st = top(d.layer_id, d.past_seq_len, d.input_token_addr, d.output_token_addr, d.layer_weights_base_addr,
                 d.layer_scales_base_addr, d.k_cache_base_addr, d.v_cache_base_addr, w, s, kv, act, *SRAM())
        if st:
            return st
    return 0


def kv_rows(kv, l):
    """The appended K and V rows of layer l (row PAST at its bases)."""
    k0 = (l * KV_LAYER) // 4 + PAST * KV_WIDTH
    v0 = (V_BASE + l * KV_LAYER) // 4 + PAST * KV_WIDTH
    return kv[k0:k0 + KV_WIDTH], kv[v0:v0 + KV_WIDTH]


def decode_inputs():
    act = np.zeros((NL + 1) * HIDDEN, np.float32)
    act[:HIDDEN] = random_hidden(55, 1)
    return act


def dropin_decode(lib, descs, w, s, kv, act, sram=None):
    arr = L.to_c_decode(descs)
    done = ctypes.c_int(-1)
    sram = SRAM() if sram is None else sram
    st = lib.qwen_decode_dispatch_layers_forward(ctypes.cast(arr, ctypes.c_void_p), len(descs), w, s, kv, act, *sram,
                                                 ctypes.byref(done))
    return st, done.value


def test_dropin_decode_dispatch_global_map(lib, images):
    w, s = images
    descs = L.build_decode_descriptors(PAST, 0, 0, 0, 0, 0)[:NL]
    print(f"drop-in decode dispatch: {NL} layers of the global map, past {PAST}", flush=True)
    kv_g, act_g = global_kv(), decode_inputs()
    kv_r, act_r = kv_g.copy(), act_g.copy()
    st, done = dropin_decode(lib, descs, w, s, kv_g, act_g)
    assert (st, done) == (0, NL), abi.last_error(lib)
    assert run_reference_decode(descs, w, s, kv_r, act_r) == 0
    assert bits_equal(act_g, act_r), first_mismatch(act_g, act_r)
    for l in range(NL):
        for g, r in zip(kv_rows(kv_g, l), kv_rows(kv_r, l)):
            assert bits_equal(g, r), f"layer {l}: " + first_mismatch(g, r)


def test_dropin_decode_dispatch_stops_at_first_failure(lib, images):
    w, s = images
    descs = L.build_decode_descriptors(PAST, 0, 0, 0, 0, 0)[:NL]
    bad = replace(descs[1], layer_id=28)  # valid_layer_id fails: 10
    kv_g, act_g = global_kv(), decode_inputs()
    st, done = dropin_decode(lib, [descs[0], bad, descs[2]], w, s, kv_g, act_g)
    assert (st, done) == (10, 1)
    kv_r, act_r = global_kv(), decode_inputs()
    assert run_reference_decode(descs[:1], w, s, kv_r, act_r) == 0
    assert bits_equal(act_g, act_r), "layer 0 output kept, nothing after it"
    assert not act_g[2 * HIDDEN:].any()
    # a null SRAM port: 11 at the first descriptor; no descriptors: 10 with nothing completed
    sram = list(SRAM())
    sram[2] = None
    arr = L.to_c_decode(descs)
    done_c = ctypes.c_int(-1)
    fn = lib.qwen_decode_dispatch_layers_forward
    argtypes = list(fn.argtypes)
    raw = getattr(ctypes.CDLL(str(abi.LIB_PATH)), "qwen_decode_dispatch_layers_forward")
    raw.argtypes = argtypes[:6] + [ctypes.c_void_p] * 5 + [ctypes.c_void_p]
    raw.restype = ctypes.c_int
    ptrs = [None if a is None else a.ctypes.data for a in sram]
    assert raw(ctypes.cast(arr, ctypes.c_void_p), NL, w, s, global_kv(), decode_inputs(), *ptrs,
               ctypes.byref(done_c)) == 11 and done_c.value == 0
    assert lib.qwen_decode_dispatch_layers_forward(ctypes.cast(arr, ctypes.c_void_p), 0, w, s, global_kv(),
                                                   decode_inputs(), *SRAM(), ctypes.byref(done_c)) == 10
    assert done_c.value == 0


# ---------------------------------------------------------------------------------------------
# prefill
# ---------------------------------------------------------------------------------------------
S = 24
A = S * HIDDEN * 4  # bytes of one activation sequence


def prefill_chain(t):
    """Two descriptors over one layer block (base 0) inside the per-layer windows: layer 0 reads
    [2A, 3A) and writes [0, A) with scratch [A, 2A); layer 1 reads [0, A) and writes [A, 2A) with scratch
    [2A, 3A).  Scratch = out + A, the address qwen_prefill_host_wrapper.cpp:639-705 derives."""
    kvb = S * KV_WIDTH * 4
    d0 = L.PrefillLayerDescriptor(0, S, t, 2 * A, 0, 0, 0, 0, kvb, A)
    d1 = L.PrefillLayerDescriptor(1, S, t, 0, A, 0, 0, 0, kvb, 2 * A)
    return [d0, d1]


def prefill_act():
    act = np.zeros(3 * S * HIDDEN, np.float32)
    act[2 * S * HIDDEN:] = random_hidden(66, S)
    return act


def run_oracle_prefill(descs, w, s, kv, act):
    o = oracle()
    for d in descs:
        st = o.oracle_prefill_top_smoke_forward(d.layer_id, d.seq_len, *d.tile_config.as_args(), d.input_sequence_addr,
                                                d.output_sequence_addr, d.layer_weights_base_addr,
                                                d.layer_scales_base_addr, d.k_cache_base_addr, d.v_cache_base_addr, w,
                                                s, kv, act, *SRAM())
        if st:
            return st
    return 0


def dropin_prefill(lib, descs, w, s, kv, act):
    arr = L.to_c_prefill(descs)
    done = ctypes.c_int(-1)
    st = lib.qwen_prefill_dispatch_layers_forward(ctypes.cast(arr, ctypes.c_void_p), len(descs), w, s, kv, act, *SRAM(),
                                                  ctypes.byref(done))
    return st, done.value


def test_dropin_prefill_dispatch_global_map_is_rejected(lib, images):
    w, s = images
    kv = np.zeros(2 * S * KV_WIDTH, np.float32)
    act = np.zeros(3 * S * HIDDEN, np.float32)
    valid = L.build_prefill_descriptors(S, 0, 0, 0, 0, 2 * A, L.valid_prefill_tile_config())[:2]
    assert dropin_prefill(lib, valid, w, s, kv, act) == (22, 0)  # V base 28 x 32 MiB is outside the KV window
    default = L.build_prefill_descriptors(S, 0, 0, 0, 0, 2 * A)[:2]
    assert dropin_prefill(lib, default, w, s, kv, act) == (20, 0)  # the Python default tiles
    assert run_oracle_prefill(valid[:1], w, s, kv.copy(), act.copy()) == 22
    assert run_oracle_prefill(default[:1], w, s, kv.copy(), act.copy()) == 20


def test_dropin_prefill_dispatch_window_chain(lib, images):
    w, s = images
    descs = prefill_chain(L.valid_prefill_tile_config())
    print(f"drop-in prefill dispatch: two chained descriptors, S={S}", flush=True)
    kv_g, act_g = np.zeros(2 * S * KV_WIDTH, np.float32), prefill_act()
    kv_r, act_r = kv_g.copy(), act_g.copy()
    assert dropin_prefill(lib, descs, w, s, kv_g, act_g) == (0, 2), abi.last_error(lib)
    assert run_oracle_prefill(descs, w, s, kv_r, act_r) == 0
    assert bits_equal(act_g, act_r), first_mismatch(act_g, act_r)
    assert bits_equal(kv_g, kv_r), first_mismatch(kv_g, kv_r)
    # a misaligned input address in the second descriptor: 22 at index 1, layer 0's outputs kept
    bad = replace(descs[1], input_sequence_addr=2)
    kv_g, act_g = np.zeros(2 * S * KV_WIDTH, np.float32), prefill_act()
    assert dropin_prefill(lib, [descs[0], bad], w, s, kv_g, act_g) == (22, 1)
    kv_r, act_r = np.zeros(2 * S * KV_WIDTH, np.float32), prefill_act()
    assert run_oracle_prefill(descs[:1], w, s, kv_r, act_r) == 0
    assert bits_equal(act_g, act_r) and bits_equal(kv_g, kv_r)


# ---------------------------------------------------------------------------------------------
# device-resident dispatch (DDR images in HBM)
# ---------------------------------------------------------------------------------------------
def dptr(t):
    return ctypes.c_void_p(t.data_ptr())


def test_device_decode_dispatch_global_map(torch, lib, images):
    w, s = images
    descs = L.build_decode_descriptors(PAST, 0, 0, 0, 0, 0)[:NL]
    print(f"device decode dispatch: {NL} layers of the global map in HBM, past {PAST}", flush=True)
    kv_h, act_h = global_kv(), decode_inputs()
    wd, sd = torch.from_numpy(w).cuda(), torch.from_numpy(s).cuda()
    kvd, actd = torch.from_numpy(kv_h).cuda(), torch.from_numpy(act_h).cuda()
    arr = L.to_c_decode(descs)
    done = ctypes.c_int(-1)
    torch.cuda.synchronize()
    st = lib.qwen_hip_decode_dispatch_layers(ctypes.cast(arr, ctypes.c_void_p), NL, dptr(wd), dptr(sd), dptr(kvd),
                                             dptr(actd), None, ctypes.byref(done))
    assert (st, done.value) == (0, NL), abi.last_error(lib)
    kv_r, act_r = kv_h.copy(), act_h.copy()
    assert run_reference_decode(descs, w, s, kv_r, act_r) == 0
    act_g = actd.cpu().numpy()
    assert bits_equal(act_g, act_r), first_mismatch(act_g, act_r)
    for l in range(NL):
        k0 = (l * KV_LAYER) // 4
        v0 = (V_BASE + l * KV_LAYER) // 4
        for base in (k0, v0):
            g = kvd[base:base + (PAST + 1) * KV_WIDTH].cpu().numpy()
            r = kv_r[base:base + (PAST + 1) * KV_WIDTH]
            assert bits_equal(g, r), f"layer {l}: " + first_mismatch(g, r)
    # mid-list failure: a negative past length in descriptor 2 gives 10 with 2 layers completed
    bad = replace(descs[2], past_seq_len=-1)
    arr = L.to_c_decode([descs[0], descs[1], bad])
    assert lib.qwen_hip_decode_dispatch_layers(ctypes.cast(arr, ctypes.c_void_p), 3, dptr(wd), dptr(sd), dptr(kvd),
                                               dptr(actd), None, ctypes.byref(done)) == 10
    assert done.value == 2
    assert lib.qwen_hip_decode_dispatch_layers(ctypes.cast(arr, ctypes.c_void_p), 3, None, dptr(sd), dptr(kvd),
                                               dptr(actd), None, ctypes.byref(done)) == 11
    assert done.value == 0


def test_device_prefill_dispatch(torch, lib, images):
    w, s = images
    wd, sd = torch.from_numpy(w).cuda(), torch.from_numpy(s).cuda()
    descs = prefill_chain(L.valid_prefill_tile_config())
    print(f"device prefill dispatch: two chained descriptors in HBM, S={S}", flush=True)
    kv_h, act_h = np.zeros(2 * S * KV_WIDTH, np.float32), prefill_act()
    kvd, actd = torch.from_numpy(kv_h).cuda(), torch.from_numpy(act_h).cuda()
    arr = L.to_c_prefill(descs)
    done = ctypes.c_int(-1)
    torch.cuda.synchronize()
    st = lib.qwen_hip_prefill_dispatch_layers(ctypes.cast(arr, ctypes.c_void_p), 2, dptr(wd), dptr(sd), dptr(kvd),
                                              dptr(actd), None, ctypes.byref(done))
    assert (st, done.value) == (0, 2), abi.last_error(lib)
    kv_r, act_r = kv_h.copy(), act_h.copy()
    assert run_oracle_prefill(descs, w, s, kv_r, act_r) == 0
    assert bits_equal(actd.cpu().numpy(), act_r), first_mismatch(actd.cpu().numpy(), act_r)
    assert bits_equal(kvd.cpu().numpy(), kv_r)
    # the global builder's descriptors: 22 at the first descriptor, nothing completed
    glob = L.to_c_prefill(L.build_prefill_descriptors(S, 0, 0, 0, 0, 2 * A, L.valid_prefill_tile_config())[:2])
    assert lib.qwen_hip_prefill_dispatch_layers(ctypes.cast(glob, ctypes.c_void_p), 2, dptr(wd), dptr(sd), dptr(kvd),
                                                dptr(actd), None, ctypes.byref(done)) == 22
    assert done.value == 0
    # invalid MLP tiles: the attention of that descriptor still writes K/V and scratch, then status 1
    t = L.valid_prefill_tile_config()
    bad_tiles = L.PrefillTileConfig(t.attention, L.PrefillMLPTileConfig(128, 512, 640))
    d = replace(descs[0], tile_config=bad_tiles)
    kvd.zero_()
    actd.copy_(torch.from_numpy(prefill_act()))
    torch.cuda.synchronize()
    one = L.to_c_prefill([d])
    assert lib.qwen_hip_prefill_dispatch_layers(ctypes.cast(one, ctypes.c_void_p), 1, dptr(wd), dptr(sd), dptr(kvd),
                                                dptr(actd), None, ctypes.byref(done)) == 1
    assert done.value == 0
    kv_r, act_r = np.zeros(2 * S * KV_WIDTH, np.float32), prefill_act()
    assert run_oracle_prefill([d], w, s, kv_r, act_r) == 1
    assert bits_equal(kvd.cpu().numpy(), kv_r) and bits_equal(actd.cpu().numpy(), act_r)


def test_device_decode_dispatch_past_beyond_32768(torch, lib, images):
    """A position past 32,767 (the length of the model API's decode RoPE table): the reference builds
    each RoPE row from libm at the position (qwen_decode_attention_kernel.cpp:29-42) and sets no bound,
    so both device dispatch entry points (the allocating one and qwen_hip_decode_dispatch_layers_noalloc)
    take per-descriptor host rows too.  Layers 0 and 1 at past 33,000 and 6: both entry points return
    (0, 2) and equal the reference top wrapper bit for bit."""
    w, s = images
    big = 33000
    k, v = quantized_kv_history(901, big + 1)
    k[big * KV_WIDTH:] = 0.0
    v[big * KV_WIDTH:] = 0.0
    kv_h = np.zeros(2 * (big + 1) * KV_WIDTH + 2 * (PAST + 1) * KV_WIDTH, np.float32)
    kv_h[:k.size] = k
    kv_h[k.size:2 * k.size] = v
    k2, v2 = quantized_kv_history(902, PAST + 1)
    k2[PAST * KV_WIDTH:] = 0.0
    v2[PAST * KV_WIDTH:] = 0.0
    o2 = 2 * k.size
    kv_h[o2:o2 + k2.size] = k2
    kv_h[o2 + k2.size:] = v2
    d0 = replace(L.build_decode_descriptors(big, 0, 0, 0, 0, 0)[0], k_cache_base_addr=0,
                 v_cache_base_addr=k.size * 4)
    d1 = replace(L.build_decode_descriptors(PAST, 0, 0, 0, 0, 0)[1], k_cache_base_addr=o2 * 4,
                 v_cache_base_addr=(o2 + k2.size) * 4)
    descs = [d0, d1]
    print(f"device decode dispatch at past {big} and {PAST}: allocating and allocation-free entry points", flush=True)
    act_h = decode_inputs()
    kv_r, act_r = kv_h.copy(), act_h.copy()
    assert run_reference_decode(descs, w, s, kv_r, act_r) == 0
    wd, sd = torch.from_numpy(w).cuda(), torch.from_numpy(s).cuda()
    arr = L.to_c_decode(descs)
    for fn in (lib.qwen_hip_decode_dispatch_layers, lib.qwen_hip_decode_dispatch_layers_noalloc):
        kvd, actd = torch.from_numpy(kv_h).cuda(), torch.from_numpy(act_h).cuda()
        torch.cuda.synchronize()
        done = ctypes.c_int(-1)
        st = fn(ctypes.cast(arr, ctypes.c_void_p), 2, dptr(wd), dptr(sd), dptr(kvd), dptr(actd), None,
                ctypes.byref(done))
        torch.cuda.synchronize()  # the allocation-free entry point returns without synchronizing
        assert (st, done.value) == (0, 2), abi.last_error(lib)
        act_g, kv_g = actd.cpu().numpy(), kvd.cpu().numpy()
        assert bits_equal(act_g, act_r), first_mismatch(act_g, act_r)
        assert bits_equal(kv_g, kv_r), first_mismatch(kv_g, kv_r)
