"""Chunked prefill with past KV on the GPU (qwen_hip_model_prefill_chunk).

The reference prefill starts at position 0 (qwen_prefill_attention_kernel.cpp:2232-2367); a chunk at
positions past..past+S-1 runs the same per-token arithmetic with its queries over keys 0..position.
The query at position p depends only on tokens 0..p, so a prompt prefilled in chunks must give the
rows of a single prefill of the whole prompt: the oracle's single prefill is the reference for every
chunk.  ORDERED: bit-exact, outputs and K/V rows.  FAST: within the per-layer tolerance."""

from __future__ import annotations

import numpy as np
import pytest

from _cases import bits_equal, first_mismatch, random_hidden, random_layer
from test_gpu_model import FAST_TOL, images, oracle_prefill, rel_err
from work_llm_accelerator_amd.layout import HIDDEN
from work_llm_accelerator_amd.quant import round_bfloat16_array

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t

    return t


@pytest.fixture(scope="module")
def layers2():
    return [random_layer(seed=71), random_layer(seed=72)]


def run_chunks(torch, m, mode, x_seqs, chunks, positions, n_layers):
    """Prefills each sequence of x_seqs [B][S*1536] in `chunks`; returns outputs [B][S*1536] and the cache."""
    from work_llm_accelerator_amd.model import KvCache

    B = len(x_seqs)
    cache = KvCache.allocate(n_layers, B, positions)
    outs = [[] for _ in range(B)]
    past = 0
    for c in chunks:
        print(f"prefill chunk past={past} len={c} B={B}", flush=True)
        h = np.stack([x[past * HIDDEN:(past + c) * HIDDEN] for x in x_seqs]).reshape(B, c, HIDDEN)
        hd = torch.from_numpy(np.ascontiguousarray(h)).cuda()
        m.prefill(mode, hd, cache, past=past)
        m.synchronize()
        got = hd.cpu().numpy().reshape(B, -1)
        for b in range(B):
            outs[b].append(got[b])
        past += c
    return [np.concatenate(o) for o in outs], cache


def test_chunked_prefill_ordered_bitexact(torch, layers2):
    from work_llm_accelerator_amd.model import MODE_ORDERED, DeviceModel

    S, chunks = 70, [30, 1, 39]
    w, s = images(layers2)
    m = DeviceModel(2, w, s)
    try:
        x = round_bfloat16_array(random_hidden(4242, S))
        got, cache = run_chunks(torch, m, MODE_ORDERED, [x], chunks, S, 2)
        ref, ks, vs = oracle_prefill(layers2, x, S)
        assert bits_equal(got[0], ref), first_mismatch(got[0], ref)
        for l in range(2):
            gk = cache.k[l, 0, :S].cpu().numpy().reshape(-1)
            gv = cache.v[l, 0, :S].cpu().numpy().reshape(-1)
            assert bits_equal(gk, ks[l]), first_mismatch(gk, ks[l])
            assert bits_equal(gv, vs[l]), first_mismatch(gv, vs[l])
    finally:
        m.close()


def test_chunked_prefill_fast_within_tolerance(torch, layers2):
    """Two sequences of 300 tokens in chunks of 128, 100, 72 (pasts 0, 128, 228: the last is not a
    multiple of the 32-key tile), FAST without bf16 rounding, against the oracle's single prefill."""
    from work_llm_accelerator_amd.model import FLAG_NO_BF16_ROUND, MODE_FAST, DeviceModel

    S, chunks = 300, [128, 100, 72]
    m = DeviceModel(1, layers2[0].weight_ddr, layers2[0].scale_ddr)
    try:
        xs = [round_bfloat16_array(random_hidden(5000 + b, S)) for b in range(2)]
        got, cache = run_chunks(torch, m, MODE_FAST | FLAG_NO_BF16_ROUND, xs, chunks, S, 1)
        for b in range(2):
            ref, ks, vs = oracle_prefill(layers2[:1], xs[b], S, rounding=False)
            for c0, c1 in ((0, 128), (128, 228), (228, 300)):
                sl = slice(c0 * HIDDEN, c1 * HIDDEN)
                assert rel_err(got[b][sl], ref[sl]) <= FAST_TOL, (b, c0, rel_err(got[b][sl], ref[sl]))
            gk = cache.k[0, b, :S].cpu().numpy().reshape(-1)
            gv = cache.v[0, b, :S].cpu().numpy().reshape(-1)
            assert rel_err(gk, ks[0]) <= FAST_TOL and rel_err(gv, vs[0]) <= FAST_TOL
    finally:
        m.close()


def test_chunk_arguments_rejected(torch):
    """A chunk that does not fit the cache rows, or a negative past, is refused with status 1."""
    from work_llm_accelerator_amd.model import MODE_FAST, DeviceModel, KvCache

    m = DeviceModel(1, synthetic_seed=3)
    try:
        cache = KvCache.allocate(1, 1, 40)
        h = torch.zeros(1, 16, HIDDEN, dtype=torch.float32, device="cuda")
        with pytest.raises(RuntimeError):
            m.prefill(MODE_FAST, h, cache, past=30)   # rows 30..45 > 40
        with pytest.raises(RuntimeError):
            m.prefill(MODE_FAST, h, cache, past=-1)
        m.prefill(MODE_FAST, h, cache, past=24)       # rows 24..39 fit
        m.synchronize()
    finally:
        m.close()


def test_chunked_prefill_fast_wide_chunks(torch, layers2):
    """Chunks of more than 256 tokens take the pipelined GEMMs with RoPE and the K/V append in the
    Q/K/V projection's epilogue: three sequences of 200 tokens in two chunks of 100 (300 tokens per
    launch; the second at past 100, inside a 32-key tile), FAST without bf16 rounding, against the
    oracle's single prefill of each sequence (the three run in threads: the oracle releases the GIL)."""
    from concurrent.futures import ThreadPoolExecutor

    from work_llm_accelerator_amd.model import FLAG_NO_BF16_ROUND, MODE_FAST, DeviceModel

    B, S, chunks = 3, 200, [100, 100]
    m = DeviceModel(1, layers2[1].weight_ddr, layers2[1].scale_ddr)
    try:
        xs = [round_bfloat16_array(random_hidden(6000 + b, S)) for b in range(B)]
        got, cache = run_chunks(torch, m, MODE_FAST | FLAG_NO_BF16_ROUND, xs, chunks, S, 1)
        with ThreadPoolExecutor(B) as ex:
            refs = list(ex.map(lambda x: oracle_prefill(layers2[1:], x, S, rounding=False), xs))
        for b, (ref, ks, vs) in enumerate(refs):
            for c0, c1 in ((0, 100), (100, 200)):
                sl = slice(c0 * HIDDEN, c1 * HIDDEN)
                assert rel_err(got[b][sl], ref[sl]) <= FAST_TOL, (b, c0, rel_err(got[b][sl], ref[sl]))
            gk = cache.k[0, b, :S].cpu().numpy().reshape(-1)
            gv = cache.v[0, b, :S].cpu().numpy().reshape(-1)
            assert rel_err(gk, ks[0]) <= FAST_TOL and rel_err(gv, vs[0]) <= FAST_TOL
    finally:
        m.close()
