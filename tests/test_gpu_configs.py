"""GPU parity at the shapes of the three full-model workloads.

* 64 x 4096 batched decode (64 sequences, KV histories of 4096 quantized N(0,1) rows, positions
  4096..4127 so the attention reads 4097..4128 keys; synthetic model seed 4, the bench's decode
  workload).  One layer: every sequence's FAST output and appended K/V rows against the oracle
  (oracle_decode_layer_block, the reference decode arithmetic) within FAST_TOL, and the ORDERED
  output and rows bit for bit; this runs the attention plan of the bench (6 splits of 688 keys, the
  steady-state tile loop, the masked last tile and the 64-sequence last-arriving merge).  All 28
  layers: FAST stays within DRIFT_28 of ORDERED with the driver's bf16 rounding after every layer.
* 8 x 2048 prefill: one layer's FAST outputs and K/V rows against the oracle's, committed as the
  golden fixture tests/golden/prefill_c4.npz (sampled rows in every key tile, and every row's max and
  sum).
* 28-layer greedy generation, batch 1, a 512-token prompt then 128 decode steps (synthetic model seed
  2): layer 0 of the prefill and of the first decode step against the oracle (ORDERED bit for bit,
  FAST within FAST_TOL); every greedy id equal to the argmax of the same mode's logits; FAST fed
  ORDERED's token trajectory (teacher forcing) with logits within LOGIT_TOL of ORDERED's and ids equal
  except where ORDERED's top two logits are closer than the logit difference allows.

Tolerances (max |y - y_ref| / max |y_ref| per tensor):
  FAST_TOL = 1e-3   one layer, fp32 output (no bf16 rounding), and each K/V tensor;
  DRIFT_28 = 3e-2   hidden state after 28 FAST layers against 28 ORDERED layers, both bf16-rounded
                    after every layer (a rounding flip is a whole bf16 step, 2^-8 relative);
  LOGIT_TOL = 5e-2  logits after 28 layers and the head.
"""

from __future__ import annotations

import numpy as np
import pytest

from _cases import bits_equal, first_mismatch
from _oracle import head_logits, oracle
from work_llm_accelerator_amd.layout import HIDDEN, KV_WIDTH, LAYOUT

pytestmark = pytest.mark.gpu

FAST_TOL = 1e-3
DRIFT_28 = 3e-2
LOGIT_TOL = 5e-2


@pytest.fixture(scope="module")
def torch():
    import torch as t

    return t


def rel_err(got, ref):
    scale = float(np.max(np.abs(ref)))
    return float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64)))) / max(scale, 1e-30)


def layer_images(model, layer):
    from work_llm_accelerator_amd import abi

    w = np.zeros(LAYOUT.total_parameter_bytes, np.uint8)
    s = np.zeros(LAYOUT.total_parameter_bytes // 4, np.float32)
    assert model.lib.qwen_hip_model_layer_images(model.handle, layer, w, s) == 0, abi.last_error(model.lib)
    return w, s


# ---------------------------------------------------------------------------------------------
# 64 sequences x KV 4097..4128
# ---------------------------------------------------------------------------------------------
B5, HIST5, CYCLE5 = 64, 4096, 32


def c5_inputs(torch, model, layers):
    from work_llm_accelerator_amd.model import KvCache, fill_kv_synthetic

    positions = HIST5 + CYCLE5
    cache = KvCache.allocate(layers, B5, positions)
    fill_kv_synthetic(cache, 4 + 1000)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4)
    ids = torch.randint(0, 151936, (B5,), dtype=torch.int32, device="cuda", generator=gen)
    hidden = torch.empty(B5, HIDDEN, dtype=torch.float32, device="cuda")
    model.embed(ids, hidden)
    pasts = [HIST5 + (b % CYCLE5) for b in range(B5)]
    pos = torch.tensor(pasts, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    return cache, hidden, pos, pasts, positions


def test_decode_64x4096_one_layer(torch):
    from work_llm_accelerator_amd.model import FLAG_NO_BF16_ROUND, MODE_FAST, MODE_ORDERED, DeviceModel, KvCache

    print("decode 64 x 4097..4128 keys, one layer (seed 4): FAST and ORDERED vs oracle", flush=True)
    m = DeviceModel(1, synthetic_seed=4)
    try:
        cache, hidden, pos, pasts, positions = c5_inputs(torch, m, 1)
        w, s = layer_images(m, 0)
        x = hidden.cpu().numpy()
        k_host = cache.k[0].cpu().numpy()  # [64][4128][256]
        v_host = cache.v[0].cpu().numpy()
        outs = {}
        for name, mode in (("fast", MODE_FAST), ("ordered", MODE_ORDERED)):
            c = KvCache(cache.k.clone(), cache.v.clone(), 1, B5, positions)
            h = hidden.clone()
            m.decode(mode | FLAG_NO_BF16_ROUND, h, pos, positions, c)
            m.synchronize()
            outs[name] = (h.cpu().numpy(), c.k[0].cpu().numpy(), c.v[0].cpu().numpy())
            del c
        o = oracle()
        worst = {"fast": 0.0, "fast_k": 0.0, "fast_v": 0.0}
        for b, past in enumerate(pasts):
            kc = np.ascontiguousarray(k_host[b, :past + 1]).reshape(-1)
            vc = np.ascontiguousarray(v_host[b, :past + 1]).reshape(-1)
            ref = np.zeros(HIDDEN, np.float32)
            assert o.oracle_decode_layer_block(x[b].copy(), past, w, s, kc, vc, ref) == 0
            rk = kc.reshape(past + 1, KV_WIDTH)[past]
            rv = vc.reshape(past + 1, KV_WIDTH)[past]
            go, gk, gv = outs["ordered"]
            assert bits_equal(go[b], ref), f"ORDERED seq {b}: " + first_mismatch(go[b], ref)
            assert bits_equal(gk[b, past], rk) and bits_equal(gv[b, past], rv), f"ORDERED K/V row, seq {b}"
            fo, fk, fv = outs["fast"]
            worst["fast"] = max(worst["fast"], rel_err(fo[b], ref))
            worst["fast_k"] = max(worst["fast_k"], rel_err(fk[b, past], rk))
            worst["fast_v"] = max(worst["fast_v"], rel_err(fv[b, past], rv))
            # history rows and rows past the new one are untouched
            for g in (gk, fk):
                assert bits_equal(g[b, :past].reshape(-1), k_host[b, :past].reshape(-1)), f"K history, seq {b}"
                assert bits_equal(g[b, past + 1:].reshape(-1), k_host[b, past + 1:].reshape(-1)), f"K tail, seq {b}"
        print(f"  FAST worst relative error over 64 sequences: out {worst['fast']:.3g}, K row {worst['fast_k']:.3g}, "
              f"V row {worst['fast_v']:.3g}", flush=True)
        assert worst["fast"] <= FAST_TOL and worst["fast_k"] <= FAST_TOL and worst["fast_v"] <= FAST_TOL, worst
    finally:
        m.close()


def test_decode_64x4096_28_layers_fast_vs_ordered(torch):
    from work_llm_accelerator_amd.model import MODE_FAST, MODE_ORDERED, DeviceModel, KvCache

    print("decode 64 x 4097..4128 keys, 28 layers (seed 4): FAST vs ORDERED drift", flush=True)
    m = DeviceModel(28, synthetic_seed=4)
    try:
        cache, hidden, pos, pasts, positions = c5_inputs(torch, m, 28)
        outs = []
        rows = []
        for mode in (MODE_ORDERED, MODE_FAST):
            c = KvCache(cache.k.clone(), cache.v.clone(), 28, B5, positions)
            h = hidden.clone()
            m.decode(mode, h, pos, positions, c)
            m.synchronize()
            outs.append(h.cpu().numpy())
            idx = torch.tensor(pasts, device="cuda", dtype=torch.long)
            rows.append(c.k[27, torch.arange(B5, device="cuda"), idx].cpu().numpy())  # last layer's new K rows
            del c
        assert np.all(np.isfinite(outs[0])) and np.all(np.isfinite(outs[1]))
        drift = max(rel_err(outs[1][b], outs[0][b]) for b in range(B5))
        drift_k = max(rel_err(rows[1][b], rows[0][b]) for b in range(B5))
        print(f"  28-layer drift FAST vs ORDERED: hidden {drift:.3g}, layer-27 K rows {drift_k:.3g}", flush=True)
        assert drift <= DRIFT_28 and drift_k <= DRIFT_28, (drift, drift_k)
    finally:
        m.close()


# ---------------------------------------------------------------------------------------------
# 8 x 2048 prefill against the committed golden fixture
# ---------------------------------------------------------------------------------------------
def test_prefill_8x2048_one_layer_golden(torch):
    import hashlib
    import sys
    from pathlib import Path

    from work_llm_accelerator_amd.model import FLAG_NO_BF16_ROUND, MODE_FAST, DeviceModel, KvCache

    golden_dir = Path(__file__).resolve().parent / "golden"
    sys.path.insert(0, str(golden_dir))
    import make_prefill_c4_golden as gen

    fx = np.load(golden_dir / "prefill_c4.npz")
    nseq, S = int(fx["nseq"]), int(fx["seq_len"])
    print(f"prefill {nseq} x {S}, one layer: FAST vs the oracle's golden rows", flush=True)
    layer = gen.layer_case()
    assert hashlib.sha256(layer.weight_ddr.tobytes()).hexdigest() == str(fx["weight_sha256"]), "layer regenerated differently"
    xs = [gen.hidden_input(b) for b in range(nseq)]
    for b in range(nseq):
        assert hashlib.sha256(xs[b].tobytes()).hexdigest() == str(fx["x_sha256"][b]), f"input {b} regenerated differently"
    m = DeviceModel(1, layer.weight_ddr, layer.scale_ddr)
    try:
        cache = KvCache.allocate(1, nseq, S)
        hidden = torch.from_numpy(np.stack(xs).reshape(nseq, S, HIDDEN)).cuda()
        m.prefill(MODE_FAST | FLAG_NO_BF16_ROUND, hidden, cache)
        m.synchronize()
        got = hidden.cpu().numpy()
        gk = cache.k[0].cpu().numpy()
        gv = cache.v[0].cpu().numpy()
    finally:
        m.close()
    pos = fx["positions"]
    worst = {}
    for b in range(nseq):
        for name, g, rows, amax, sums in (("out", got[b], fx["out_rows"][b], fx["out_amax"][b], fx["out_sum"][b]),
                                          ("k", gk[b], fx["k_rows"][b], fx["k_amax"][b], fx["k_sum"][b]),
                                          ("v", gv[b], fx["v_rows"][b], fx["v_amax"][b], fx["v_sum"][b])):
            scale = float(np.max(amax))  # max |y_ref| over the whole tensor (every row's max is stored)
            e_rows = float(np.max(np.abs(g[pos].astype(np.float64) - rows))) / scale
            # every row: its max |.| and its sum, each within the tolerance of the tensor scale
            # (a sum of n elements each within tol*scale is within n*tol*scale)
            e_amax = float(np.max(np.abs(np.max(np.abs(g), axis=1) - amax))) / scale
            e_sum = float(np.max(np.abs(g.astype(np.float64).sum(axis=1) - sums))) / (scale * g.shape[1])
            worst[name] = max(worst.get(name, 0.0), e_rows, e_amax, e_sum)
    print(f"  worst relative error over {nseq} sequences: {worst}", flush=True)
    for name, e in worst.items():
        assert e <= FAST_TOL, (name, e)


# ---------------------------------------------------------------------------------------------
# 28-layer greedy generation, batch 1: 512-token prompt + 128 steps
# ---------------------------------------------------------------------------------------------
PROMPT3, STEPS3 = 512, 128


def test_greedy_28_layers_prompt512_128_steps(torch):
    from work_llm_accelerator_amd.model import (FLAG_NO_BF16_ROUND, MODE_FAST, MODE_ORDERED, DeviceModel,
                                                KvCache)
    print("greedy 28 layers (seed 2): 512-token prompt + 128 teacher-forced steps, FAST vs ORDERED", flush=True)
    m = DeviceModel(28, synthetic_seed=2)
    vocab = m.vocab
    positions = PROMPT3 + STEPS3 + 1
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2)
    prompt = torch.randint(0, vocab, (PROMPT3,), dtype=torch.int32, device="cuda", generator=gen)
    try:
        x0 = torch.empty(1, PROMPT3, HIDDEN, dtype=torch.float32, device="cuda")
        m.embed(prompt, x0)
        m.synchronize()
        x0_host = x0.cpu().numpy().reshape(-1)

        runs = {}
        pos_all = torch.arange(PROMPT3, PROMPT3 + STEPS3, dtype=torch.int32, device="cuda")
        for name, mode in (("ordered", MODE_ORDERED), ("fast", MODE_FAST)):
            cache = KvCache.allocate(28, 1, positions)
            hp = x0.clone()
            m.prefill(mode, hp, cache)
            logits = torch.empty(STEPS3, vocab, dtype=torch.float32, device="cuda")
            ids = torch.empty(STEPS3, dtype=torch.int32, device="cuda")
            first = torch.empty(1, dtype=torch.int32, device="cuda")
            h = torch.empty(1, HIDDEN, dtype=torch.float32, device="cuda")
            m.greedy(hp[0, PROMPT3 - 1:], first)  # the prompt's next token starts the loop
            # teacher forcing: FAST is fed ORDERED's tokens (step i embeds the id ORDERED chose at step i-1);
            # every operation below is queued on the model's stream, in order
            src_first = first if name == "ordered" else runs["ordered"]["first"]
            src_ids = ids if name == "ordered" else runs["ordered"]["ids"]
            for i in range(STEPS3):
                m.embed(src_first if i == 0 else src_ids[i - 1:i], h, order=False)
                m.decode(mode, h, pos_all[i:i + 1], positions, cache, order=False)
                m.logits(h, logits[i:i + 1], order=False)
                m.greedy(h, ids[i:i + 1], order=False)
                if i == 0:
                    m.synchronize()
                    h0 = h.clone()
                    torch.cuda.synchronize()
            m.synchronize()
            runs[name] = {"ids": ids, "first": first, "logits": logits, "cache": cache, "h0": h0}
        fed = {name: np.concatenate([r["first"].cpu().numpy(), r["ids"].cpu().numpy()[:-1]])
               for name, r in runs.items()}
        fed["fast"] = np.concatenate([runs["ordered"]["first"].cpu().numpy(), runs["ordered"]["ids"].cpu().numpy()[:-1]])

        # every greedy id is the first maximum of the same mode's logits
        for name, r in runs.items():
            am = torch.argmax(r["logits"], dim=1).to(torch.int32)
            assert torch.equal(am, r["ids"]), f"{name}: greedy ids differ from the argmax of the logits"
        assert np.array_equal(fed["fast"], fed["ordered"])

        # layer 0 against the oracle: prefill K/V rows (bit for bit in ORDERED), and the first decode step's
        # new K/V rows at position 512 (the embedded first generated token over the prefilled rows)
        w0, s0 = layer_images(m, 0)
        o = oracle()
        kc = np.zeros(PROMPT3 * KV_WIDTH, np.float32)
        vc = np.zeros(PROMPT3 * KV_WIDTH, np.float32)
        out0 = np.zeros(PROMPT3 * HIDDEN, np.float32)
        assert o.oracle_prefill_layer_uncapped(x0_host, PROMPT3, w0, s0, kc, vc, out0) == 0
        for name, r in runs.items():
            gk = r["cache"].k[0, 0, :PROMPT3].cpu().numpy().reshape(-1)
            gv = r["cache"].v[0, 0, :PROMPT3].cpu().numpy().reshape(-1)
            if name == "ordered":
                assert bits_equal(gk, kc), "ORDERED layer-0 prefill K: " + first_mismatch(gk, kc)
                assert bits_equal(gv, vc), "ORDERED layer-0 prefill V: " + first_mismatch(gv, vc)
            else:
                assert rel_err(gk, kc) <= FAST_TOL and rel_err(gv, vc) <= FAST_TOL, (rel_err(gk, kc), rel_err(gv, vc))
        # layer-0 output of the prompt: a one-layer model of the same images, without the driver's rounding
        m1 = DeviceModel(1, w0, s0)
        try:
            for mode in (MODE_ORDERED, MODE_FAST):
                c1 = KvCache.allocate(1, 1, PROMPT3)
                h1 = x0.clone()
                m1.prefill(mode | FLAG_NO_BF16_ROUND, h1, c1)
                m1.synchronize()
                g1 = h1.cpu().numpy().reshape(-1)
                if mode == MODE_ORDERED:
                    assert bits_equal(g1, out0), "ORDERED layer-0 prefill output: " + first_mismatch(g1, out0)
                else:
                    assert rel_err(g1, out0) <= FAST_TOL, rel_err(g1, out0)
        finally:
            m1.close()
        # first decode step, layer 0: K/V row 512 from the embedded first generated token
        tok = runs["ordered"]["first"]
        e = torch.empty(1, HIDDEN, dtype=torch.float32, device="cuda")
        m.embed(tok, e)
        m.synchronize()
        kd = np.zeros((PROMPT3 + 1) * KV_WIDTH, np.float32)
        vd = np.zeros((PROMPT3 + 1) * KV_WIDTH, np.float32)
        kd[:PROMPT3 * KV_WIDTH] = kc
        vd[:PROMPT3 * KV_WIDTH] = vc
        outd = np.zeros(HIDDEN, np.float32)
        assert o.oracle_decode_layer_block(e.cpu().numpy().reshape(-1), PROMPT3, w0, s0, kd, vd, outd) == 0
        for name, r in runs.items():
            gk = r["cache"].k[0, 0, PROMPT3].cpu().numpy()
            gv = r["cache"].v[0, 0, PROMPT3].cpu().numpy()
            rk, rv = kd[PROMPT3 * KV_WIDTH:], vd[PROMPT3 * KV_WIDTH:]
            if name == "ordered":
                assert bits_equal(gk, rk) and bits_equal(gv, rv), "ORDERED layer-0 decode K/V row 512"
            else:
                assert rel_err(gk, rk) <= FAST_TOL and rel_err(gv, rv) <= FAST_TOL

        # the head of the first step against the oracle (final RMSNorm + tied bf16 lm_head over the vocab)
        embed = np.zeros((vocab, HIDDEN), np.uint16)
        norm = np.zeros(HIDDEN, np.uint16)
        assert m.lib.qwen_hip_model_head_tables(m.handle, embed, norm) == 0
        h0 = runs["ordered"]["h0"].cpu().numpy()
        _, ref_logits = head_logits(h0, norm, embed)
        got0 = runs["ordered"]["logits"][0].cpu().numpy()
        assert bits_equal(got0, ref_logits[0]), "head logits of step 0: " + first_mismatch(got0, ref_logits[0])

        # FAST against ORDERED (same tokens): logits within LOGIT_TOL, ids equal except near-ties
        lo = runs["ordered"]["logits"].cpu().numpy().astype(np.float64)
        lf = runs["fast"]["logits"].cpu().numpy().astype(np.float64)
        io = runs["ordered"]["ids"].cpu().numpy()
        jf = runs["fast"]["ids"].cpu().numpy()
        dl = np.max(np.abs(lf - lo), axis=1)
        worst = float(np.max(dl / np.max(np.abs(lo), axis=1)))
        diff = np.nonzero(io != jf)[0]
        for i in diff:
            gap = lo[i, io[i]] - lo[i, jf[i]]
            assert gap <= 2.0 * dl[i], f"step {i}: ids {io[i]} vs {jf[i]} with ORDERED gap {gap:.4g} > 2 x {dl[i]:.4g}"
        print(f"  logits FAST vs ORDERED: worst {worst:.3g} of max; ids equal at {STEPS3 - diff.size}/{STEPS3} steps "
              f"(the rest are near-ties)", flush=True)
        assert worst <= LOGIT_TOL, worst
    finally:
        m.close()
