"""GPU parity of the device-resident model API (include/qwen_hip_model.h).

* ORDERED decode/prefill over several layers and sequences equals the oracle bit for bit: per
  layer oracle_decode_layer_block / oracle_prefill_layer_uncapped (the reference host arithmetic)
  followed by the driver's bf16 rounding (verification/real_host_top_backend.py:260,334).
* FAST decode/prefill agrees with the oracle within the stated tolerance:
      max |y - y_ref| <= 1e-3 * max |y_ref|   per layer output and per K/V cache tensor
  (checked on one layer without the inter-layer bf16 rounding, which would otherwise quantize a
  1e-6 difference into a whole bf16 step), and within 1e-2 * max over two rounded layers.
* The device INT4 quantizer equals the reference scheme (verification/real_host_top_backend.py:31-41,
  restated in work_llm_accelerator_amd.quant) bit for bit, including all-zero rows and exact ties.
"""

from __future__ import annotations

import numpy as np
import pytest

from _cases import bits_equal, first_mismatch, quantized_kv_history, random_hidden, random_layer
from _oracle import oracle
from work_llm_accelerator_amd.layout import HIDDEN, KV_WIDTH
from work_llm_accelerator_amd.quant import quantize_int4_per_channel, round_bfloat16_array

pytestmark = pytest.mark.gpu

FAST_TOL = 1e-3        # one layer, fp32 output: |y - y_ref| <= FAST_TOL * max|y_ref|
FAST_TOL_ROUNDED = 1e-2  # two layers with bf16 rounding between them


@pytest.fixture(scope="module")
def torch():
    import torch as t

    return t


@pytest.fixture(scope="module")
def layers2():
    return [random_layer(seed=61), random_layer(seed=62)]


def images(layers):
    w = np.concatenate([c.weight_ddr for c in layers])
    s = np.concatenate([c.scale_ddr for c in layers])
    return w, s


@pytest.fixture(scope="module")
def model2(torch, layers2):
    from work_llm_accelerator_amd.model import DeviceModel

    w, s = images(layers2)
    m = DeviceModel(2, w, s)
    yield m
    m.close()


def oracle_decode(layers, x, past, k_hist, v_hist, rounding=True):
    """Per-layer oracle decode of one sequence; k_hist/v_hist[l] hold past+1 rows (row `past` is written)."""
    o = oracle()
    h = x.copy()
    for l, case in enumerate(layers):
        out = np.zeros(HIDDEN, np.float32)
        assert o.oracle_decode_layer_block(h, past, case.weight_ddr, case.scale_ddr, k_hist[l], v_hist[l], out) == 0
        h = round_bfloat16_array(out) if rounding else out
    return h


def oracle_prefill(layers, x, S, rounding=True):
    o = oracle()
    h = x.copy()
    ks, vs = [], []
    for case in layers:
        kc = np.zeros(S * KV_WIDTH, np.float32)
        vc = np.zeros(S * KV_WIDTH, np.float32)
        out = np.zeros(S * HIDDEN, np.float32)
        assert o.oracle_prefill_layer_uncapped(h, S, case.weight_ddr, case.scale_ddr, kc, vc, out) == 0
        h = round_bfloat16_array(out) if rounding else out
        ks.append(kc)
        vs.append(vc)
    return h, ks, vs


def rel_err(got, ref):
    scale = float(np.max(np.abs(ref)))
    return float(np.max(np.abs(got.astype(np.float64) - ref.astype(np.float64)))) / max(scale, 1e-30)


def decode_setup(torch, n_layers, pasts, positions_cap, seed):
    from work_llm_accelerator_amd.model import KvCache

    B = len(pasts)
    cache = KvCache.allocate(n_layers, B, positions_cap)
    hist = {}
    for l in range(n_layers):
        for b, past in enumerate(pasts):
            k, v = quantized_kv_history(seed + 10 * l + b, past + 1)
            k = k.reshape(past + 1, KV_WIDTH)
            v = v.reshape(past + 1, KV_WIDTH)
            k[past] = 0.0
            v[past] = 0.0
            cache.k[l, b, :past + 1] = torch.from_numpy(k)
            cache.v[l, b, :past + 1] = torch.from_numpy(v)
            hist[(l, b)] = (k.reshape(-1).copy(), v.reshape(-1).copy())
    x = np.stack([round_bfloat16_array(random_hidden(seed + 100 + b, 1)) for b in range(B)])
    return cache, hist, x


@pytest.mark.parametrize("mode_name", ["ordered", "fast"])
def test_model_decode(torch, layers2, model2, mode_name):
    from work_llm_accelerator_amd.model import FLAG_NO_BF16_ROUND, MODE_FAST, MODE_ORDERED

    pasts = [0, 5, 300]
    print(f"model decode {mode_name} pasts={pasts}", flush=True)
    cache, hist, x = decode_setup(torch, 2, pasts, 320, seed=7)
    hidden = torch.from_numpy(x).cuda()
    pos = torch.tensor(pasts, dtype=torch.int32, device="cuda")
    if mode_name == "ordered":
        model2.decode(MODE_ORDERED, hidden, pos, max(pasts) + 1, cache)
        model2.synchronize()
        got = hidden.cpu().numpy()
        for b, past in enumerate(pasts):
            kl = [hist[(l, b)][0].copy() for l in range(2)]
            vl = [hist[(l, b)][1].copy() for l in range(2)]
            ref = oracle_decode(layers2, x[b], past, kl, vl)
            assert bits_equal(got[b], ref), f"seq {b}: " + first_mismatch(got[b], ref)
            for l in range(2):
                gk = cache.k[l, b, :past + 1].cpu().numpy().reshape(-1)
                gv = cache.v[l, b, :past + 1].cpu().numpy().reshape(-1)
                assert bits_equal(gk, kl[l]), first_mismatch(gk, kl[l])
                assert bits_equal(gv, vl[l]), first_mismatch(gv, vl[l])
    else:
        # one layer without rounding: the per-layer tolerance
        from work_llm_accelerator_amd.model import DeviceModel

        m1 = DeviceModel(1, layers2[0].weight_ddr, layers2[0].scale_ddr)
        try:
            cache1, hist1, _ = decode_setup(torch, 1, pasts, 320, seed=7)
            h1 = torch.from_numpy(x).cuda()
            m1.decode(MODE_FAST | FLAG_NO_BF16_ROUND, h1, pos, max(pasts) + 1, cache1)
            m1.synchronize()
            got = h1.cpu().numpy()
            for b, past in enumerate(pasts):
                kl = [hist1[(0, b)][0].copy()]
                vl = [hist1[(0, b)][1].copy()]
                ref = oracle_decode(layers2[:1], x[b], past, kl, vl, rounding=False)
                assert rel_err(got[b], ref) <= FAST_TOL, (b, rel_err(got[b], ref))
                gk = cache1.k[0, b, past].cpu().numpy()
                gv = cache1.v[0, b, past].cpu().numpy()
                rk = kl[0].reshape(past + 1, KV_WIDTH)[past]
                rv = vl[0].reshape(past + 1, KV_WIDTH)[past]
                assert rel_err(gk, rk) <= FAST_TOL and rel_err(gv, rv) <= FAST_TOL
                # untouched history rows stay bit-identical
                assert bits_equal(cache1.k[0, b, :past].cpu().numpy().reshape(-1), kl[0][:past * KV_WIDTH])
        finally:
            m1.close()
        # two layers with the driver's rounding
        model2.decode(MODE_FAST, hidden, pos, max(pasts) + 1, cache)
        model2.synchronize()
        got = hidden.cpu().numpy()
        for b, past in enumerate(pasts):
            kl = [hist[(l, b)][0].copy() for l in range(2)]
            vl = [hist[(l, b)][1].copy() for l in range(2)]
            ref = oracle_decode(layers2, x[b], past, kl, vl)
            assert rel_err(got[b], ref) <= FAST_TOL_ROUNDED, (b, rel_err(got[b], ref))


def test_model_decode_fast_many_splits(torch, layers2):
    """Two sequences with long histories (700 and 1100 keys): the decode attention plan gives them
    18 key splits of 64, so the merge launch combines 11 and 18 splits in batches of 8 (two and three
    batches).  One layer without rounding, within the per-layer tolerance of the oracle."""
    from work_llm_accelerator_amd.model import FLAG_NO_BF16_ROUND, MODE_FAST, DeviceModel

    pasts = [700, 1100]
    print(f"model decode fast many splits pasts={pasts}", flush=True)
    m1 = DeviceModel(1, layers2[0].weight_ddr, layers2[0].scale_ddr)
    try:
        cache1, hist1, x = decode_setup(torch, 1, pasts, 1120, seed=11)
        h1 = torch.from_numpy(x).cuda()
        pos = torch.tensor(pasts, dtype=torch.int32, device="cuda")
        m1.decode(MODE_FAST | FLAG_NO_BF16_ROUND, h1, pos, max(pasts) + 1, cache1)
        m1.synchronize()
        got = h1.cpu().numpy()
        for b, past in enumerate(pasts):
            ref = oracle_decode(layers2[:1], x[b], past, [hist1[(0, b)][0].copy()], [hist1[(0, b)][1].copy()],
                                rounding=False)
            err = rel_err(got[b], ref)
            print(f"  seq {b} past {past}: rel err {err:.2e}", flush=True)
            assert err <= FAST_TOL, (b, err)
    finally:
        m1.close()


@pytest.mark.parametrize("mode_name", ["ordered", "fast"])
def test_model_prefill(torch, layers2, model2, mode_name):
    from work_llm_accelerator_amd.model import FLAG_NO_BF16_ROUND, MODE_FAST, MODE_ORDERED, DeviceModel, KvCache

    B, S = 2, 37
    print(f"model prefill {mode_name} B={B} S={S}", flush=True)
    xs = [round_bfloat16_array(random_hidden(900 + b, S)) for b in range(B)]
    if mode_name == "ordered":
        cache = KvCache.allocate(2, B, 48)
        hidden = torch.from_numpy(np.stack(xs).reshape(B, S, HIDDEN)).cuda()
        model2.prefill(MODE_ORDERED, hidden, cache)
        model2.synchronize()
        got = hidden.cpu().numpy().reshape(B, -1)
        for b in range(B):
            ref, ks, vs = oracle_prefill(layers2, xs[b], S)
            assert bits_equal(got[b], ref), f"seq {b}: " + first_mismatch(got[b], ref)
            for l in range(2):
                gk = cache.k[l, b, :S].cpu().numpy().reshape(-1)
                gv = cache.v[l, b, :S].cpu().numpy().reshape(-1)
                assert bits_equal(gk, ks[l]), first_mismatch(gk, ks[l])
                assert bits_equal(gv, vs[l]), first_mismatch(gv, vs[l])
    else:
        m1 = DeviceModel(1, layers2[0].weight_ddr, layers2[0].scale_ddr)
        try:
            cache = KvCache.allocate(1, B, 48)
            hidden = torch.from_numpy(np.stack(xs).reshape(B, S, HIDDEN)).cuda()
            m1.prefill(MODE_FAST | FLAG_NO_BF16_ROUND, hidden, cache)
            m1.synchronize()
            got = hidden.cpu().numpy().reshape(B, -1)
            for b in range(B):
                ref, ks, vs = oracle_prefill(layers2[:1], xs[b], S, rounding=False)
                assert rel_err(got[b], ref) <= FAST_TOL, (b, rel_err(got[b], ref))
                gk = cache.k[0, b, :S].cpu().numpy().reshape(-1)
                gv = cache.v[0, b, :S].cpu().numpy().reshape(-1)
                assert rel_err(gk, ks[0]) <= FAST_TOL and rel_err(gv, vs[0]) <= FAST_TOL
        finally:
            m1.close()


def test_model_prefill_ordered_uncapped(torch, layers2):
    """S = 133 > 128 (the reference's per-call cap): the per-token arithmetic is unchanged."""
    from work_llm_accelerator_amd.model import FLAG_NO_BF16_ROUND, MODE_ORDERED, DeviceModel, KvCache

    S = 133
    print(f"model prefill ordered uncapped S={S}", flush=True)
    x = round_bfloat16_array(random_hidden(77, S))
    m1 = DeviceModel(1, layers2[1].weight_ddr, layers2[1].scale_ddr)
    try:
        cache = KvCache.allocate(1, 1, S)
        hidden = torch.from_numpy(x.reshape(1, S, HIDDEN)).cuda()
        m1.prefill(MODE_ORDERED | FLAG_NO_BF16_ROUND, hidden, cache)
        m1.synchronize()
        got = hidden.cpu().numpy().reshape(-1)
        ref, ks, vs = oracle_prefill(layers2[1:], x, S, rounding=False)
        assert bits_equal(got, ref), first_mismatch(got, ref)
        assert bits_equal(cache.k[0, 0].cpu().numpy().reshape(-1), ks[0])
    finally:
        m1.close()


def test_device_quantizer_bitexact(torch):
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((64, 1536), dtype=np.float32) * np.float32(0.02))
    w[3] = 0.0                       # all-zero row -> scale 1, all nibbles 0
    w[5, :8] = [7.0, 3.5, -3.5, 2.5, -0.5, 0.5, 1.5, -8.0]  # exact ties of rint (half to even)
    w = round_bfloat16_array(w).reshape(64, 1536)
    packed_ref, scales_ref = quantize_int4_per_channel(w)
    packed, scales = __import__("work_llm_accelerator_amd.model", fromlist=["x"]).quantize_int4_device(
        torch.from_numpy(w).cuda())
    torch.cuda.synchronize()
    assert bits_equal(scales.cpu().numpy(), scales_ref)
    assert np.array_equal(packed.cpu().numpy(), packed_ref)


def test_synthetic_model_runs(torch):
    """A synthetic 2-layer model decodes and prefills without error and gives finite outputs in
    both modes; FAST stays within the rounded tolerance of ORDERED on the same synthetic model."""
    from work_llm_accelerator_amd.model import MODE_FAST, MODE_ORDERED, DeviceModel, KvCache, fill_kv_synthetic

    m = DeviceModel(2, synthetic_seed=4)
    try:
        cache = KvCache.allocate(2, 4, 600)
        fill_kv_synthetic(cache, 11)
        ids = torch.randint(0, 151936, (4,), dtype=torch.int32, device="cuda")
        h0 = torch.empty(4, HIDDEN, dtype=torch.float32, device="cuda")
        m.embed(ids, h0)
        pos = torch.tensor([512, 513, 100, 599], dtype=torch.int32, device="cuda")
        outs = []
        for mode in (MODE_ORDERED, MODE_FAST):
            c = KvCache(cache.k.clone(), cache.v.clone(), 2, 4, 600)
            h = h0.clone()
            m.decode(mode, h, pos, 600, c)
            m.synchronize()
            outs.append(h.cpu().numpy())
        assert np.all(np.isfinite(outs[0])) and np.all(np.isfinite(outs[1]))
        assert rel_err(outs[1], outs[0]) <= FAST_TOL_ROUNDED
        assert m.time_kernel(1, 0, 3) > 0.0
    finally:
        m.close()


@pytest.mark.parametrize("batch", [2, 5, 20, 64, 100, 300])
def test_model_decode_fast_batched(torch, layers2, batch):
    """Every sequence of the batch stays within the per-layer tolerance of the oracle, on each of
    the batched paths: 2..64 sequences take the skinny GEMMs (activations staged in LDS, weights
    in registers) with the RoPE/append and RMSNorm/quantization steps fused into their reduce
    kernels and the SiLU·up rows passed to the down projection as a grouped code (2..16: the Q/K/V
    projection in one K wave group, 17..64 in two); 65..256 the pipelined GEMMs split over K, with
    the same fused reduce steps; above 256 the unfused path (separate RMSNorm/quantization, RoPE and
    append launches)."""
    from work_llm_accelerator_amd.model import FLAG_NO_BF16_ROUND, MODE_FAST, DeviceModel

    rng = np.random.default_rng(batch)
    pasts = [int(p) for p in rng.integers(0, 40, batch)]
    print(f"model decode fast batch={batch}", flush=True)
    m1 = DeviceModel(1, layers2[1].weight_ddr, layers2[1].scale_ddr)
    try:
        cache, hist, x = decode_setup(torch, 1, pasts, 48, seed=31)
        hidden = torch.from_numpy(x).cuda()
        pos = torch.tensor(pasts, dtype=torch.int32, device="cuda")
        m1.decode(MODE_FAST | FLAG_NO_BF16_ROUND, hidden, pos, max(pasts) + 1, cache)
        m1.synchronize()
        got = hidden.cpu().numpy()
        for b, past in enumerate(pasts):
            kl = [hist[(0, b)][0].copy()]
            vl = [hist[(0, b)][1].copy()]
            ref = oracle_decode(layers2[1:], x[b], past, kl, vl, rounding=False)
            assert rel_err(got[b], ref) <= FAST_TOL, (b, rel_err(got[b], ref))
    finally:
        m1.close()


@pytest.mark.skip(reason="split decode on CU-masked streams switched off: on MI355X both cases passed, then "
                  "the process hung while the model and its CU-masked streams were torn down (cause not found)")
@pytest.mark.parametrize("pcus", [4, 8])
def test_model_decode_fast_split(torch, layers2, model2, monkeypatch, pcus):
    """A batch decoded as two concurrent halves on CU-masked streams (projections on `pcus` CUs of
    every XCD, attention on the rest): every sequence of both halves stays within the per-layer
    tolerance of the oracle over two layers (the second layer's input RMSNorm + quantization fused
    into the first layer's down projection), and so do the appended K/V rows."""
    from work_llm_accelerator_amd.model import FLAG_NO_BF16_ROUND, MODE_FAST

    batch = 32
    rng = np.random.default_rng(900 + pcus)
    pasts = [int(p) for p in rng.integers(0, 60, batch)]
    print(f"model decode fast split batch={batch} pcus={pcus}", flush=True)
    monkeypatch.setenv("QWEN_SPLIT_CUS", str(pcus))
    cache, hist, x = decode_setup(torch, 2, pasts, 64, seed=53)
    hidden = torch.from_numpy(x).cuda()
    pos = torch.tensor(pasts, dtype=torch.int32, device="cuda")
    model2.decode(MODE_FAST | FLAG_NO_BF16_ROUND, hidden, pos, max(pasts) + 1, cache)
    model2.synchronize()
    got = hidden.cpu().numpy()
    for b, past in enumerate(pasts):
        kl = [hist[(l, b)][0].copy() for l in range(2)]
        vl = [hist[(l, b)][1].copy() for l in range(2)]
        ref = oracle_decode(layers2, x[b], past, kl, vl, rounding=False)
        assert rel_err(got[b], ref) <= FAST_TOL, (b, rel_err(got[b], ref))
        for l in range(2):
            gk = cache.k[l, b, past].cpu().numpy().reshape(-1)
            rk = kl[l].reshape(-1, KV_WIDTH)[past]
            assert rel_err(gk, rk) <= FAST_TOL, (b, l, rel_err(gk, rk))


@pytest.mark.parametrize("S", [1, 16, 40, 150, 300])
def test_model_prefill_fast_mid(torch, layers2, S):
    """1 token: a one-token prompt (one key, a one-query attention block); 16 tokens: exactly one
    token tile of the skinny GEMMs; 40 tokens: the 17..64-token GEMM path on prefill shapes; 150 tokens: the 65..256-token GEMM
    path and five causal 32-key tiles of the prefill attention (partial last tile); 300 tokens: the
    many-token GEMM (4-wave blocks: four full 64-token tiles and a partial one), ten key tiles and a
    partial last 16-query attention block."""
    from work_llm_accelerator_amd.model import FLAG_NO_BF16_ROUND, MODE_FAST, DeviceModel, KvCache

    print(f"model prefill fast S={S}", flush=True)
    x = round_bfloat16_array(random_hidden(444 + S, S))
    m1 = DeviceModel(1, layers2[0].weight_ddr, layers2[0].scale_ddr)
    try:
        cache = KvCache.allocate(1, 1, S)
        hidden = torch.from_numpy(x.reshape(1, S, HIDDEN)).cuda()
        m1.prefill(MODE_FAST | FLAG_NO_BF16_ROUND, hidden, cache)
        m1.synchronize()
        got = hidden.cpu().numpy().reshape(-1)
        ref, ks, vs = oracle_prefill(layers2[:1], x, S, rounding=False)
        assert rel_err(got, ref) <= FAST_TOL
        assert rel_err(cache.k[0, 0].cpu().numpy().reshape(-1), ks[0]) <= FAST_TOL
    finally:
        m1.close()


def test_model_prefill_fast_many_seqs(torch, layers2):
    """Three sequences of 200 tokens: 600 tokens per projection (the many-token GEMM, a partial last
    64-token tile), three sequences in the attention grid, each with a partial last 16-query block
    and a partial last key tile."""
    from work_llm_accelerator_amd.model import FLAG_NO_BF16_ROUND, MODE_FAST, DeviceModel, KvCache

    B, S = 3, 200
    print(f"model prefill fast B={B} S={S}", flush=True)
    xs = [round_bfloat16_array(random_hidden(777 + b, S)) for b in range(B)]
    m1 = DeviceModel(1, layers2[0].weight_ddr, layers2[0].scale_ddr)
    try:
        cache = KvCache.allocate(1, B, S)
        hidden = torch.from_numpy(np.stack(xs).reshape(B, S, HIDDEN)).cuda()
        m1.prefill(MODE_FAST | FLAG_NO_BF16_ROUND, hidden, cache)
        m1.synchronize()
        got = hidden.cpu().numpy().reshape(B, -1)
        for b in range(B):
            ref, ks, vs = oracle_prefill(layers2[:1], xs[b], S, rounding=False)
            assert rel_err(got[b], ref) <= FAST_TOL, (b, rel_err(got[b], ref))
            gk = cache.k[0, b, :S].cpu().numpy().reshape(-1)
            gv = cache.v[0, b, :S].cpu().numpy().reshape(-1)
            assert rel_err(gk, ks[0]) <= FAST_TOL and rel_err(gv, vs[0]) <= FAST_TOL
    finally:
        m1.close()


# The one-sequence forms against the separate launches, without the bf16 rounding between layers (which
# turns any difference into a whole bf16 step): the O projection's blocks quantize the context row per
# head range (kOneTokenOSplits ranges of 768 columns, each with its own scale) where the separate form
# quantizes the whole row with one scale, so the forms differ by about that code's rounding, not bit for
# bit (measured on MI355X: up to 3.8e-4 of max after two calls of two layers).
ONE_VS_SEPARATE_TOL = 1e-3


@pytest.mark.parametrize("past", [0, 37, 1500])
def test_model_decode_o_reduce_in_gate_up(torch, layers2, model2, past):
    """One sequence: the decode attention's split merge and the context row's quantization run in
    every block of the O projection (each block merging and quantizing one head range), the O
    projection's reduce step (adding the head ranges' partials, RMSNorm, quantization) in every block
    of the gate/up projection, the SiLU·up row's quantization in every block of the down projection,
    and layer 0's down-projection reduce step (residual, bf16 rounding, layer 1's RMSNorm,
    quantization) in every block of layer 1's Q/K/V projection, instead of their own launches.  Over
    both layers without the bf16 rounding: layer 0's new K/V row is bit-identical to the separate
    form's (it precedes the O projection), the hidden row and layer 1's K/V row agree within
    ONE_VS_SEPARATE_TOL of max, for two calls in a row (the second from the first's output).  1500
    keys: 24 attention splits, so the O blocks' merge loads its partials in two batches (16 + 8); its
    first call is also checked against the oracle."""
    from work_llm_accelerator_amd.model import FLAG_NO_BF16_ROUND, FLAG_SEPARATE_ATTN, FLAG_SEPARATE_REDUCE, MODE_FAST

    print(f"model decode fast O reduce in gate/up past={past}", flush=True)
    if past > 1000:
        cache, hist, x = decode_setup(torch, 2, [past], past + 1, seed=61)
        hidden = torch.from_numpy(x).cuda()
        pos = torch.tensor([past], dtype=torch.int32, device="cuda")
        model2.decode(MODE_FAST, hidden, pos, past + 1, cache)
        model2.synchronize()
        kl = [hist[(l, 0)][0].copy() for l in range(2)]
        vl = [hist[(l, 0)][1].copy() for l in range(2)]
        ref = oracle_decode(layers2, x[0], past, kl, vl)
        assert rel_err(hidden.cpu().numpy()[0], ref) <= FAST_TOL_ROUNDED
    outs = {}
    # the attention runs as its own launch in both forms (its fusion into Q/K/V rounds differently,
    # checked by test_model_decode_fused_attention)
    for flag in (FLAG_SEPARATE_ATTN, FLAG_SEPARATE_REDUCE):
        cache, _, x = decode_setup(torch, 2, [past], max(48, past + 1), seed=61)
        hidden = torch.from_numpy(x).cuda()
        pos = torch.tensor([past], dtype=torch.int32, device="cuda")
        calls = []
        for _ in range(2):
            model2.decode(MODE_FAST | FLAG_NO_BF16_ROUND | flag, hidden, pos, past + 1, cache)
            model2.synchronize()
            calls.append((hidden.cpu().numpy()[0], cache.k[:, 0, past].cpu().numpy(), cache.v[:, 0, past].cpu().numpy()))
        outs[flag] = calls
    one, sep = outs[FLAG_SEPARATE_ATTN], outs[FLAG_SEPARATE_REDUCE]
    for i in (1, 2):  # the first call's layer-0 K/V row
        assert bits_equal(one[0][i][0], sep[0][i][0]), first_mismatch(one[0][i][0], sep[0][i][0])
    for c in range(2):
        d_h = rel_err(one[c][0], sep[c][0])
        d_kv = max(rel_err(one[c][i][l], sep[c][i][l]) for i in (1, 2) for l in range(2))
        print(f"  call {c}: hidden {d_h:.3g}, K/V rows {d_kv:.3g} of max", flush=True)
        assert d_h <= ONE_VS_SEPARATE_TOL and d_kv <= ONE_VS_SEPARATE_TOL


# The two attention forms: |y_fused - y_sep| <= 5e-4 * max|y_sep|.  The context rows differ in the last
# fp32 bits, which moves a few elements of its two-limb code by one step, so the forms differ by about
# the code's own rounding (measured on MI355X: up to 9.5e-5, against 1.1e-4 for either vs the oracle).
FUSED_VS_SEPARATE_TOL = 5e-4


@pytest.mark.parametrize("past", [0, 1, 15, 63, 64, 65, 300, 1279])
def test_model_decode_fused_attention(torch, layers2, model2, past):
    """One sequence with at most 1280 keys: the decode attention over the history keys runs in the
    blocks of the Q/K/V projection (one block per query head and 64-key split, its K/V rows staged in
    LDS) and the O projection's merge adds the new key's term.  Checked against the oracle (one layer
    without rounding: FAST_TOL; two layers with the driver's rounding, the second layer's Q/K/V blocks
    also finishing the first layer's down projection: FAST_TOL_ROUNDED) and against the separate
    attention launch (QWEN_FLAG_SEPARATE_ATTN), which rounds differently: within
    FUSED_VS_SEPARATE_TOL, with layer 0's new K/V row bit-identical.  The pasts cover no history
    (0), a partial first split, exact split boundaries (63, 64, 65: the new key opens a split in the
    separate form) and 20 splits (1279: the most the fused form takes)."""
    from work_llm_accelerator_amd.model import DeviceModel, FLAG_NO_BF16_ROUND, FLAG_SEPARATE_ATTN, MODE_FAST

    print(f"model decode fused attention past={past}", flush=True)
    pos = torch.tensor([past], dtype=torch.int32, device="cuda")
    m1 = DeviceModel(1, layers2[0].weight_ddr, layers2[0].scale_ddr)
    try:
        got = {}
        for flag in (0, FLAG_SEPARATE_ATTN):
            cache, hist, x = decode_setup(torch, 1, [past], past + 1, seed=71)
            h = torch.from_numpy(x).cuda()
            m1.decode(MODE_FAST | FLAG_NO_BF16_ROUND | flag, h, pos, past + 1, cache)
            m1.synchronize()
            got[flag] = (h.cpu().numpy()[0], cache.k[0, 0, past].cpu().numpy(), cache.v[0, 0, past].cpu().numpy())
        kl, vl = [hist[(0, 0)][0].copy()], [hist[(0, 0)][1].copy()]
        ref = oracle_decode(layers2[:1], x[0], past, kl, vl, rounding=False)
        e_f, e_s = rel_err(got[0][0], ref), rel_err(got[FLAG_SEPARATE_ATTN][0], ref)
        d = rel_err(got[0][0], got[FLAG_SEPARATE_ATTN][0])
        print(f"  one layer: fused {e_f:.3g}, separate {e_s:.3g} of max vs the oracle; fused vs separate {d:.3g}",
              flush=True)
        assert e_f <= FAST_TOL and e_s <= FAST_TOL
        assert d <= FUSED_VS_SEPARATE_TOL
        for i in (1, 2):
            assert bits_equal(got[0][i], got[FLAG_SEPARATE_ATTN][i]), first_mismatch(got[0][i], got[FLAG_SEPARATE_ATTN][i])
    finally:
        m1.close()
    got2 = {}
    for flag in (0, FLAG_SEPARATE_ATTN):
        cache, hist, x = decode_setup(torch, 2, [past], past + 1, seed=73)
        h = torch.from_numpy(x).cuda()
        model2.decode(MODE_FAST | flag, h, pos, past + 1, cache)
        model2.synchronize()
        got2[flag] = (h.cpu().numpy()[0], cache.k[0, 0, past].cpu().numpy(), cache.v[0, 0, past].cpu().numpy())
    kl = [hist[(l, 0)][0].copy() for l in range(2)]
    vl = [hist[(l, 0)][1].copy() for l in range(2)]
    ref = oracle_decode(layers2, x[0], past, kl, vl)
    e_f, e_s = rel_err(got2[0][0], ref), rel_err(got2[FLAG_SEPARATE_ATTN][0], ref)
    print(f"  two layers: fused {e_f:.3g}, separate {e_s:.3g} of max vs the oracle", flush=True)
    assert e_f <= FAST_TOL_ROUNDED and e_s <= FAST_TOL_ROUNDED
    for i in (1, 2):
        assert bits_equal(got2[0][i], got2[FLAG_SEPARATE_ATTN][i])
