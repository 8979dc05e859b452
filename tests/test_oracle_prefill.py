"""Pins the prefill half of the oracle (the reference prefill library is not buildable here: its
sources include Catapult's <ac_channel.h>, which this image does not have).

1. Known answer of verification/validate_prefill_attention_smoke.py:62-104 (single +1 nibbles at
   (0,0) of Q, K, V and O; unit scales; token t has x[t][0] = 1, 2, 3, ...): K/V rows, RoPE of
   pair 0 at angle t, causal softmax over the keys, output column 0 = context[head 0][0].  The
   validator writes this closed form with exact sqrt/exp/sin/cos; the reference kernel uses
   approx_sqrt / approx_exp / approx_sincos (qwen_prefill_attention_kernel.cpp:47-110), which at
   these inputs (mean square 6.5e-4, where 6 Newton steps from 1 are still 7.7% off) differ by
   far more than its 1e-5 tolerance, so the closed form here uses those pinned scalar functions.
2. Dense random layers against a float64 matrix-form restatement of the whole prefill layer
   (qwen_prefill_attention_kernel.cpp:2232-2367, qwen_prefill_mlp_kernel.cpp:264-337): batched
   matmuls, GQA head mapping h -> h/6, causal mask, RoPE pairs (p, p+64), biases, no input
   residual, a + down(silu(gate) * up).  The elementwise approximations are the oracle's own
   scalar functions (pinned in test_oracle_math.py), so the only difference left is fp32 serial
   vs float64 accumulation: tolerance 2e-4 of each tensor's max.  A wrong head mapping, a missing
   mask, a swapped RoPE pair, a dropped bias or an added residual fails by orders of magnitude.
"""

from __future__ import annotations

import numpy as np
import pytest

from _cases import (empty_layer, prefill_attention, prefill_layer, random_hidden, random_layer, set_packed_weight)
from _oracle import oracle
from work_llm_accelerator_amd.layout import (HEAD_DIM, HIDDEN, INTERMEDIATE, KV_WIDTH, Q_HEADS,
                                             valid_prefill_tile_config)

TILES = valid_prefill_tile_config()
F32 = np.float32


def _vec(fn):
    return np.vectorize(lambda v: fn(float(v)), otypes=[np.float64])


def _sincos(o, angle):
    import ctypes

    s, c = ctypes.c_float(), ctypes.c_float()
    o.oracle_approx_sincos(float(angle), ctypes.byref(s), ctypes.byref(c))
    return s.value, c.value


def _unpack(packed, out_dim, in_dim, scales):
    nib = np.stack([packed & 0xF, packed >> 4], axis=1).reshape(out_dim, in_dim).astype(np.int64)
    q = np.where(nib >= 8, nib - 16, nib).astype(np.float64)
    return q * scales.astype(np.float64)[:, None]


def float64_prefill_layer(case, x, S):
    o = oracle()
    v = case.v
    asqrt, aexp, silu = _vec(o.oracle_approx_sqrt), _vec(o.oracle_approx_exp), _vec(o.oracle_silu_prefill)
    xs = x.reshape(S, HIDDEN).astype(np.float64)

    def rms(a, w):
        ms = np.mean(a * a, axis=1, keepdims=True)
        return a / asqrt(ms + 1e-6) * w.astype(np.float64)

    Wq = _unpack(v["q_w"], HIDDEN, HIDDEN, v["q_s"])
    Wk = _unpack(v["k_w"], KV_WIDTH, HIDDEN, v["k_s"])
    Wv = _unpack(v["v_w"], KV_WIDTH, HIDDEN, v["v_s"])
    Wo = _unpack(v["o_w"], HIDDEN, HIDDEN, v["o_s"])
    n = rms(xs, v["input_layernorm"])
    q = n @ Wq.T + v["q_bias"]
    k = n @ Wk.T + v["k_bias"]
    val = n @ Wv.T + v["v_bias"]
    # RoPE: pair p of every head rotated by the prefill table of position t
    cos = np.zeros((S, 64))
    sin = np.zeros((S, 64))
    for t in range(S):
        cos_row = np.zeros(64, np.float32)
        sin_row = np.zeros(64, np.float32)
        o.oracle_prefill_rope_row(t, cos_row, sin_row)
        cos[t], sin[t] = cos_row, sin_row

    def rope(m, heads):
        m = m.reshape(S, heads, HEAD_DIM).copy()
        e, od = m[:, :, :64].copy(), m[:, :, 64:].copy()
        m[:, :, :64] = e * cos[:, None, :] - od * sin[:, None, :]
        m[:, :, 64:] = od * cos[:, None, :] + e * sin[:, None, :]
        return m

    qh = rope(q, Q_HEADS)
    kh = rope(k, 2)
    vh = val.reshape(S, 2, HEAD_DIM)
    ctx = np.zeros((S, Q_HEADS, HEAD_DIM))
    scaling = float(F32(0.08838834764831845))
    mask = np.tril(np.ones((S, S), bool))
    for h in range(Q_HEADS):
        kv = h // (Q_HEADS // 2)
        s = (qh[:, h] @ kh[:, kv].T) * scaling
        s = np.where(mask, s, -np.inf)
        m = s.max(axis=1, keepdims=True)
        p = np.where(mask, aexp(np.where(mask, s - m, 0.0)), 0.0)
        ctx[:, h] = (p @ vh[:, kv]) / p.sum(axis=1, keepdims=True)
    a = ctx.reshape(S, HIDDEN) @ Wo.T
    post = rms(a, v["post_attention_layernorm"])
    Wg = _unpack(v["gate_w"], INTERMEDIATE, HIDDEN, v["gate_s"])
    Wu = _unpack(v["up_w"], INTERMEDIATE, HIDDEN, v["up_s"])
    Wd = _unpack(v["down_w"], HIDDEN, INTERMEDIATE, v["down_s"])
    g = post @ Wg.T
    u = post @ Wu.T
    out = a + (silu(g) * u) @ Wd.T
    kv_k = kh.reshape(S, KV_WIDTH)
    return out, kv_k, vh.reshape(S, KV_WIDTH), a


def rel(got, ref):
    return float(np.max(np.abs(got.astype(np.float64) - ref))) / float(np.max(np.abs(ref)))


@pytest.mark.parametrize("S", [1, 5, 24])
def test_prefill_layer_matches_float64_restatement(S):
    case = random_layer(seed=70 + S)
    x = random_hidden(80 + S, S)
    st, out, kc, vc = prefill_layer(oracle().oracle_prefill_layer_smoke_forward, case, x, S, TILES)
    assert st == 0
    ref_out, ref_k, ref_v, _ = float64_prefill_layer(case, x, S)
    assert rel(kc, ref_k.reshape(-1)) < 2e-4
    assert rel(vc, ref_v.reshape(-1)) < 2e-4
    assert rel(out, ref_out.reshape(-1)) < 2e-4


def test_prefill_attention_known_answer():
    o = oracle()
    S = 4
    case = empty_layer()
    for name, rows in (("q_w", HIDDEN), ("k_w", KV_WIDTH), ("v_w", KV_WIDTH), ("o_w", HIDDEN)):
        set_packed_weight(case.v[name], rows, HIDDEN, 0, 0, 1)
    x = np.zeros((S, HIDDEN), np.float32)
    for t in range(S):
        x[t, 0] = float(t + 1)
    st, out, kc, vc = prefill_attention(o.oracle_prefill_attention_smoke_forward, case, x.reshape(-1).copy(), S,
                                        TILES)
    assert st == 0
    kc, vc, out = kc.reshape(S, KV_WIDTH), vc.reshape(S, KV_WIDTH), out.reshape(S, HIDDEN)
    n0 = np.zeros(S)
    for t in range(S):
        ms = F32(F32(x[t, 0] * x[t, 0]) / F32(HIDDEN))
        n0[t] = float(F32(x[t, 0] * F32(F32(1.0) / F32(o.oracle_approx_sqrt(float(F32(ms + F32(1e-6))))))))
    for t in range(S):
        s, c = _sincos(o, float(t))  # pair 0: inv_freq 1, angle t
        assert abs(kc[t, 0] - n0[t] * c) <= 1e-5 * abs(n0[t]) and abs(kc[t, 64] - n0[t] * s) <= 1e-5 * abs(n0[t])
        assert abs(vc[t, 0] - n0[t]) <= 1e-5 * abs(n0[t])
        assert np.count_nonzero(kc[t, 1:64]) == 0 and np.count_nonzero(kc[t, 65:]) == 0
        assert np.count_nonzero(vc[t, 1:]) == 0
    for t in range(S):
        # head 0: q = k pattern, scores q_t . k_j * scale over keys j <= t, approx_exp softmax
        qs, qc = _sincos(o, float(t))
        scores = []
        for j in range(t + 1):
            ks_, kc_ = _sincos(o, float(j))
            dot = (n0[t] * qc) * (n0[j] * kc_) + (n0[t] * qs) * (n0[j] * ks_)
            scores.append(dot * float(F32(0.08838834764831845)))
        m = max(scores)
        p = [o.oracle_approx_exp(float(F32(sv - m))) for sv in scores]
        ctx0 = sum(pj * n0[j] for j, pj in enumerate(p)) / sum(p)
        assert abs(out[t, 0] - ctx0) <= 1e-4 * abs(ctx0)
        assert np.count_nonzero(out[t, 1:]) == 0
