"""Layer-by-layer, teacher-forced parity of FAST against ORDERED at the full shapes of the three
28-layer workloads, so that every layer's FAST kernels are checked at every layer, not only layer 0.

For each layer l of a 28-layer synthetic model, FAST layer l and ORDERED layer l run on the SAME
input: ORDERED's output of layer l - 1 rounded to bf16, as the reference driver rounds between
layers (verification/real_host_top_backend.py:260,334).  Both run one layer at a time
(qwen_hip_model_decode_layers / _prefill_layers) with QWEN_FLAG_NO_BF16_ROUND, so their fp32 outputs
are compared before the rounding; FAST runs first and ORDERED then overwrites the K/V rows, so every
later step reads ORDERED's cache.  ORDERED itself is bit-exact with the reference at layer 0 (checked
here against the oracle, and in the other GPU tests against the reference library), and runs the same
kernels at every layer.

Checked for every layer of every workload:
  * per tensor (FAST_TOL): max|y - y_ref| <= 1e-3 max|y_ref|, for the layer output and for the new K
    and V rows (fp32, before rounding);
  * per element, condition-aware (C_ELEM): |y_i - y_ref_i| <= C_ELEM * 2^-15 * A_i, where A_i is the
    absolute-value sum of the projection(s) producing element i (sum_j |x_j||w_ij|, in float64 from the
    layer images, tests/_layer64.py).  The FAST activation code has a step of max|x| / 32512 (~2^-15 of
    the row's largest element), so its error per output is a small multiple of 2^-15 A_i.  C_ELEM = 2;
    measured on MI355X: 0.92 at worst (prefill layer 0), 0.3-0.5 elsewhere (each test prints its
    figures per layer);
  * decode only: ORDERED against the float64 restatement within 1e-4 of max (the decode reference uses
    libm expf and double RMSNorm sums, so float64 differs from it only by fp32 rounding).  The prefill
    reference's approx_sqrt / approx_exp / approx_sincos are not exact functions, so prefill ORDERED is
    checked against the oracle at layer 0 only.

Workloads:
  * 64 x 4096 batched decode (seed 4): 64 sequences, KV histories of 4096 quantized N(0,1) rows,
    positions 4096..4127, one embedded random token per sequence;
  * 8 x 2048 prefill (seed 3): 8 sequences of 2048 embedded random ids, causal;
  * batch-1 generation (seed 2): a 512-token prompt prefilled layer by layer, then 128 decode steps at
    positions 512..639 fed a fixed sequence of uniform random ids (128 ids, so at least 64 distinct),
    every step layer by layer; at every step the layer-0 K/V row of the embedded id is checked against
    the oracle's decode layer (oracle_decode_layer_block): ORDERED bit for bit, FAST within FAST_TOL.
"""

from __future__ import annotations

import time

import numpy as np
import pytest

from _cases import bits_equal, first_mismatch
from _layer64 import Layer64
from _oracle import oracle
from work_llm_accelerator_amd.layout import HIDDEN, KV_WIDTH, LAYOUT

pytestmark = pytest.mark.gpu

FAST_TOL = 1e-3
C_ELEM = 2.0
ORDERED_F64_TOL = 1e-4
LAYERS = 28


@pytest.fixture(scope="module")
def torch():
    import torch as t

    return t


class Worst:
    """Per-layer worst figures, kept on the device until the end (no host sync per layer)."""

    KEYS = ("out", "k", "v", "c_out", "c_k", "c_v", "f64")

    def __init__(self, torch):
        self.t = torch
        self.w = torch.zeros(LAYERS, len(self.KEYS), dtype=torch.float64, device="cuda")

    def rel(self, got, ref):
        """max over sequences of max|got - ref| / max|ref| within the sequence (dim 0 is the sequence)."""
        t = self.t
        r = ref.to(t.float64).flatten(1)
        d = (got.to(t.float64).flatten(1) - r).abs()
        return (d.max(dim=1).values / r.abs().max(dim=1).values).max()

    def add(self, layer, fast, ordered, ref64=None, terms=None):
        """fast / ordered: dicts of tensors out, k, v with the sequence as dim 0; ref64: the float64
        restatement's values; terms: its condition terms (a_out, a_k, a_v)."""
        t = self.t
        row = [self.rel(fast[name], ordered[name]) for name in ("out", "k", "v")]
        for name in ("out", "k", "v"):
            if terms is None:
                row.append(t.zeros((), dtype=t.float64, device="cuda"))
            else:
                d = (fast[name].to(t.float64) - ordered[name].to(t.float64)).abs()
                row.append((d / (terms["a_" + name] * 2.0 ** -15)).max())
        if ref64 is None:
            row.append(t.zeros((), dtype=t.float64, device="cuda"))
        else:
            row.append(t.stack([self.rel(ordered[n], ref64[n]) for n in ("out", "k", "v")]).max())
        self.w[layer] = t.maximum(self.w[layer], t.stack(row))

    def report(self, what):
        w = self.w.cpu().numpy()
        print(f"  {what}: worst per layer (rel. to max: out / K / V; per-element c: out / K / V"
              f"{'; ORDERED vs float64' if np.any(w[:, 6]) else ''})", flush=True)
        for layer in range(LAYERS):
            r = w[layer]
            extra = f"  f64 {r[6]:.2e}" if np.any(w[:, 6]) else ""
            print(f"    layer {layer:2d}: {r[0]:.2e} {r[1]:.2e} {r[2]:.2e} | c {r[3]:.3f} {r[4]:.3f} {r[5]:.3f}{extra}",
                  flush=True)
        print(f"    all layers: out {w[:, 0].max():.3g}, K {w[:, 1].max():.3g}, V {w[:, 2].max():.3g}; "
              f"c {w[:, 3:6].max():.3g}" + (f"; ORDERED vs float64 {w[:, 6].max():.3g}" if np.any(w[:, 6]) else ""),
              flush=True)
        assert np.all(np.isfinite(w)), "non-finite error figures"
        assert w[:, 0:3].max() <= FAST_TOL, ("per-tensor", w[:, 0:3].max(axis=1))
        assert w[:, 3:6].max() <= C_ELEM, ("per-element", w[:, 3:6].max(axis=1))
        assert w[:, 6].max() <= ORDERED_F64_TOL, ("ORDERED vs float64", w[:, 6])
        return w


def bf16(torch, x):
    """Round-to-nearest-even to bf16, held in fp32 (the driver's rounding between layers)."""
    return x.to(torch.bfloat16).to(torch.float32)


# ---------------------------------------------------------------------------------------------
# 64 sequences x KV 4097..4128
# ---------------------------------------------------------------------------------------------
def test_decode_64x4096_every_layer_teacher_forced(torch):
    from work_llm_accelerator_amd.model import (FLAG_NO_BF16_ROUND, MODE_FAST, MODE_ORDERED, DeviceModel, KvCache,
                                                fill_kv_synthetic)

    B, HIST, CYCLE = 64, 4096, 32
    print(f"decode {B} x {HIST + 1}..{HIST + CYCLE} keys, every layer teacher-forced (seed 4)", flush=True)
    t0 = time.time()
    m = DeviceModel(LAYERS, synthetic_seed=4)
    try:
        positions = HIST + CYCLE
        cache = KvCache.allocate(LAYERS, B, positions)
        fill_kv_synthetic(cache, 4 + 1000)
        gen = torch.Generator(device="cuda")
        gen.manual_seed(4)
        ids = torch.randint(0, 151936, (B,), dtype=torch.int32, device="cuda", generator=gen)
        h = torch.empty(B, HIDDEN, dtype=torch.float32, device="cuda")
        m.embed(ids, h)
        pos = torch.tensor([HIST + (b % CYCLE) for b in range(B)], dtype=torch.int32, device="cuda")
        m.synchronize()
        rows = torch.arange(B, device="cuda")
        pl = pos.long()
        worst = Worst(torch)
        with torch.cuda.stream(m.stream):
            for layer in range(LAYERS):
                w64 = Layer64.from_model(torch, m, layer)
                ref64 = w64.decode(h.to(torch.float64), pos, cache.k[layer], cache.v[layer])
                hf = h.clone()
                m.decode(MODE_FAST | FLAG_NO_BF16_ROUND, hf, pos, positions, cache, order=False, layers=layer)
                fast = {"out": hf, "k": cache.k[layer, rows, pl].clone(), "v": cache.v[layer, rows, pl].clone()}
                ho = h.clone()
                m.decode(MODE_ORDERED | FLAG_NO_BF16_ROUND, ho, pos, positions, cache, order=False, layers=layer)
                ordered = {"out": ho, "k": cache.k[layer, rows, pl], "v": cache.v[layer, rows, pl]}
                worst.add(layer, fast, ordered, ref64, ref64)
                h = bf16(torch, ho)
                del w64, ref64
        m.synchronize()
        worst.report("64 x 4096 decode")
        print(f"  ({time.time() - t0:.1f} s)", flush=True)
    finally:
        m.close()


# ---------------------------------------------------------------------------------------------
# 8 x 2048 prefill
# ---------------------------------------------------------------------------------------------
def test_prefill_8x2048_every_layer_teacher_forced(torch):
    from work_llm_accelerator_amd.model import FLAG_NO_BF16_ROUND, MODE_FAST, MODE_ORDERED, DeviceModel, KvCache

    B, S = 8, 2048
    print(f"prefill {B} x {S}, every layer teacher-forced (seed 3)", flush=True)
    t0 = time.time()
    m = DeviceModel(LAYERS, synthetic_seed=3)
    try:
        cache = KvCache.allocate(1, B, S)  # one layer's cache, reused by every layer
        gen = torch.Generator(device="cuda")
        gen.manual_seed(3)
        ids = torch.randint(0, 151936, (B * S,), dtype=torch.int32, device="cuda", generator=gen)
        h = torch.empty(B, S, HIDDEN, dtype=torch.float32, device="cuda")
        m.embed(ids, h)
        m.synchronize()
        worst = Worst(torch)
        with torch.cuda.stream(m.stream):
            for layer in range(LAYERS):
                w64 = Layer64.from_model(torch, m, layer)
                terms = w64.prefill(h.to(torch.float64))
                hf = h.clone()
                m.prefill(MODE_FAST | FLAG_NO_BF16_ROUND, hf, cache, order=False, layers=layer)
                fast = {"out": hf, "k": cache.k[0].clone(), "v": cache.v[0].clone()}
                ho = h.clone()
                m.prefill(MODE_ORDERED | FLAG_NO_BF16_ROUND, ho, cache, order=False, layers=layer)
                worst.add(layer, fast, {"out": ho, "k": cache.k[0], "v": cache.v[0]}, None, terms)
                h = bf16(torch, ho)
                del w64, terms
                if layer % 7 == 6:
                    m.synchronize()
                    print(f"    through layer {layer} ({time.time() - t0:.1f} s)", flush=True)
        m.synchronize()
        worst.report("8 x 2048 prefill")
        print(f"  ({time.time() - t0:.1f} s)", flush=True)
    finally:
        m.close()


# ---------------------------------------------------------------------------------------------
# batch-1 generation: 512-token prompt, then 128 steps fed fixed random ids
# ---------------------------------------------------------------------------------------------
PROMPT3, STEPS3 = 512, 128


def test_generation_prompt512_every_layer_teacher_forced(torch):
    from work_llm_accelerator_amd.model import FLAG_NO_BF16_ROUND, MODE_FAST, MODE_ORDERED, DeviceModel, KvCache

    print(f"generation: {PROMPT3}-token prompt + {STEPS3} steps of fixed random ids, every layer teacher-forced "
          "(seed 2)", flush=True)
    t0 = time.time()
    NR = FLAG_NO_BF16_ROUND
    m = DeviceModel(LAYERS, synthetic_seed=2)
    o = oracle()
    try:
        vocab = m.vocab
        positions = PROMPT3 + STEPS3
        cache = KvCache.allocate(LAYERS, 1, positions)
        gen = torch.Generator(device="cuda")
        gen.manual_seed(2)
        prompt = torch.randint(0, vocab, (PROMPT3,), dtype=torch.int32, device="cuda", generator=gen)
        rng = np.random.default_rng(2)
        step_ids = rng.integers(0, vocab, STEPS3).astype(np.int32)
        assert len(set(step_ids.tolist())) >= 64
        ids_dev = torch.from_numpy(step_ids).cuda()
        h = torch.empty(1, PROMPT3, HIDDEN, dtype=torch.float32, device="cuda")
        m.embed(prompt, h)
        m.synchronize()
        x0 = h.cpu().numpy().reshape(-1)
        w0 = np.zeros(LAYOUT.total_parameter_bytes, np.uint8)
        s0 = np.zeros(LAYOUT.total_parameter_bytes // 4, np.float32)
        assert m.lib.qwen_hip_model_layer_images(m.handle, 0, w0, s0) == 0
        layers64 = [Layer64.from_model(torch, m, layer) for layer in range(LAYERS)]

        # the prompt, layer by layer
        pre = Worst(torch)
        with torch.cuda.stream(m.stream):
            for layer in range(LAYERS):
                terms = layers64[layer].prefill(h.to(torch.float64))
                hf = h.clone()
                m.prefill(MODE_FAST | NR, hf, cache, order=False, layers=layer)
                fast = {"out": hf, "k": cache.k[layer, :, :PROMPT3].clone(), "v": cache.v[layer, :, :PROMPT3].clone()}
                ho = h.clone()
                m.prefill(MODE_ORDERED | NR, ho, cache, order=False, layers=layer)
                pre.add(layer, fast, {"out": ho, "k": cache.k[layer, :, :PROMPT3], "v": cache.v[layer, :, :PROMPT3]},
                        None, terms)
                if layer == 0:
                    out0 = ho.clone()
                h = bf16(torch, ho)
        m.synchronize()
        # layer 0 of the prompt against the oracle, bit for bit
        kc = np.zeros(PROMPT3 * KV_WIDTH, np.float32)
        vc = np.zeros(PROMPT3 * KV_WIDTH, np.float32)
        ref0 = np.zeros(PROMPT3 * HIDDEN, np.float32)
        assert o.oracle_prefill_layer_uncapped(x0, PROMPT3, w0, s0, kc, vc, ref0) == 0
        g0 = out0.cpu().numpy().reshape(-1)
        assert bits_equal(g0, ref0), "ORDERED layer-0 prompt output: " + first_mismatch(g0, ref0)
        gk = cache.k[0, 0, :PROMPT3].cpu().numpy().reshape(-1)
        gv = cache.v[0, 0, :PROMPT3].cpu().numpy().reshape(-1)
        assert bits_equal(gk, kc) and bits_equal(gv, vc), "ORDERED layer-0 prompt K/V rows"
        pre.report(f"{PROMPT3}-token prompt")
        print(f"  ({time.time() - t0:.1f} s)", flush=True)

        # 128 decode steps, each embedding the next fixed id, layer by layer
        dec = Worst(torch)
        worst_l0 = 0.0
        e = torch.empty(1, HIDDEN, dtype=torch.float32, device="cuda")
        for i in range(STEPS3):
            p = PROMPT3 + i
            pos = torch.full((1,), p, dtype=torch.int32, device="cuda")
            with torch.cuda.stream(m.stream):
                m.embed(ids_dev[i:i + 1], e, order=False)
                h = e.clone()
                for layer in range(LAYERS):
                    ref64 = layers64[layer].decode(h.to(torch.float64), pos, cache.k[layer], cache.v[layer])
                    hf = h.clone()
                    m.decode(MODE_FAST | NR, hf, pos, p + 1, cache, order=False, layers=layer)
                    fast = {"out": hf, "k": cache.k[layer, :, p].clone(), "v": cache.v[layer, :, p].clone()}
                    if layer == 0:
                        fast0 = (fast["k"].clone(), fast["v"].clone())
                    ho = h.clone()
                    m.decode(MODE_ORDERED | NR, ho, pos, p + 1, cache, order=False, layers=layer)
                    dec.add(layer, fast, {"out": ho, "k": cache.k[layer, :, p], "v": cache.v[layer, :, p]}, ref64, ref64)
                    h = bf16(torch, ho)
            m.synchronize()
            # layer 0 of this step against the oracle: the embedded id over ORDERED's rows 0..p-1
            x = e.cpu().numpy().reshape(-1)
            kd = cache.k[0, 0, :p + 1].cpu().numpy().reshape(-1).copy()
            vd = cache.v[0, 0, :p + 1].cpu().numpy().reshape(-1).copy()
            got_k, got_v = kd[p * KV_WIDTH:].copy(), vd[p * KV_WIDTH:].copy()
            kd[p * KV_WIDTH:] = 0.0
            vd[p * KV_WIDTH:] = 0.0
            out_ref = np.zeros(HIDDEN, np.float32)
            assert o.oracle_decode_layer_block(x, p, w0, s0, kd, vd, out_ref) == 0
            rk, rv = kd[p * KV_WIDTH:], vd[p * KV_WIDTH:]
            assert bits_equal(got_k, rk) and bits_equal(got_v, rv), f"step {i}: ORDERED layer-0 K/V row {p}"
            fk, fv = fast0[0].cpu().numpy().reshape(-1), fast0[1].cpu().numpy().reshape(-1)
            e_k = float(np.max(np.abs(fk - rk))) / float(np.max(np.abs(rk)))
            e_v = float(np.max(np.abs(fv - rv))) / float(np.max(np.abs(rv)))
            worst_l0 = max(worst_l0, e_k, e_v)
            assert e_k <= FAST_TOL and e_v <= FAST_TOL, (i, e_k, e_v)
            if i % 32 == 31:
                print(f"    through step {i} ({time.time() - t0:.1f} s)", flush=True)
        print(f"  layer-0 K/V row of every step's id vs the oracle: ORDERED bit-exact, FAST worst {worst_l0:.3g}; "
              f"{len(set(step_ids.tolist()))} distinct ids fed", flush=True)
        dec.report(f"{STEPS3} decode steps at positions {PROMPT3}..{PROMPT3 + STEPS3 - 1}")
        print(f"  ({time.time() - t0:.1f} s)", flush=True)
    finally:
        m.close()


# ---------------------------------------------------------------------------------------------
# fused layer boundaries: a two-layer range against two one-layer calls
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("batch", [1, 5, 64])
def test_fused_layer_boundary_matches_separate_layers(torch, batch):
    """Inside a range FAST runs each layer boundary fused (the next layer's RMSNorm and quantization in
    the down projection's reduce step, or at one sequence in the next Q/K/V projection's prologue); a
    range that ends at a layer runs them as steps of their own.  Layers (l, l + 1) as one range and as
    two one-layer calls, with the driver's bf16 rounding between them, must give the same outputs and
    K/V rows up to the order of the RMSNorm's double sum: within 1e-5 of max, and the share of
    bit-identical elements is printed (measured on MI355X: 100% at 1, 5 and 64 sequences).  This ties
    the per-layer checks above to the whole-model path."""
    from work_llm_accelerator_amd.model import MODE_FAST, DeviceModel, KvCache, fill_kv_synthetic

    P = 300
    m = DeviceModel(LAYERS, synthetic_seed=4)
    try:
        base = KvCache.allocate(LAYERS, batch, P + 1)
        fill_kv_synthetic(base, 77)
        gen = torch.Generator(device="cuda")
        gen.manual_seed(batch)
        ids = torch.randint(0, 151936, (batch,), dtype=torch.int32, device="cuda", generator=gen)
        x = torch.empty(batch, HIDDEN, dtype=torch.float32, device="cuda")
        m.embed(ids, x)
        pos = torch.tensor([P - (b % 7) for b in range(batch)], dtype=torch.int32, device="cuda")
        m.synchronize()
        rows, pl = torch.arange(batch, device="cuda"), pos.long()
        worst, same, total = 0.0, 0, 0
        for first in (0, 13, 26):
            got = []
            for split in (False, True):
                c = KvCache(base.k.clone(), base.v.clone(), LAYERS, batch, P + 1)
                h = x.clone()
                if split:
                    m.decode(MODE_FAST, h, pos, P + 1, c, layers=first)
                    m.decode(MODE_FAST, h, pos, P + 1, c, layers=first + 1)
                else:
                    m.decode(MODE_FAST, h, pos, P + 1, c, layers=(first, 2))
                m.synchronize()
                got.append([h.cpu().numpy()] + [t[first + j, rows, pl].cpu().numpy() for t in (c.k, c.v)
                                                for j in (0, 1)])
                del c
            for a, b in zip(*got):
                worst = max(worst, float(np.max(np.abs(a.astype(np.float64) - b))) / float(np.max(np.abs(b))))
                same += int(np.sum(a.view(np.uint32) == b.view(np.uint32)))
                total += a.size
        print(f"  batch {batch}: two-layer range vs two one-layer calls (layers 0-1, 13-14, 26-27): worst "
              f"{worst:.3g} of max, {100.0 * same / total:.2f}% of elements bit-identical", flush=True)
        assert worst <= 1e-5, worst
    finally:
        m.close()
