"""Pins the oracle's model head (final RMSNorm, tied bf16 lm_head, greedy argmax) on the CPU against
the library routines the reference's driver calls (verification/real_host_top_backend.py:138-146 on
the bf16 model of verification/torch_reference_backend.py:67): transformers' Qwen2RMSNorm and
torch's bf16 linear and argmax (verification/qwen_full_model_validation.py:128,159).

The oracle fixes one summation order (exact products, double sums rounded once); torch's CPU
kernels sum in their own order, so a bf16 result may differ by one unit in the last place where the
fp32 value sits next to a bf16 rounding boundary.  The bar is: every element within 1 bf16 ulp and
at least 99.5% bit-identical, which a dropped rounding step, a wrong epsilon or a missing weight
fails."""

from __future__ import annotations

import numpy as np
import pytest

from tests._oracle import argmax_rows, head_logits, oracle

torch = pytest.importorskip("torch")


def bf16_bits(t) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def bf16_value(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def ulps_apart(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """Distance in bf16 ulps of two arrays of bf16 bit patterns (same sign assumed for nonzero)."""
    def ordered(b):
        b = b.astype(np.int32)
        return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
    return np.abs(ordered(a_bits) - ordered(b_bits))


def test_head_norm_matches_qwen2_rmsnorm():
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm

    g = torch.Generator().manual_seed(5)
    x = torch.randn(64, 1536, generator=g) * 3.0  # fp32 rows, not yet bf16
    w = (1.0 + 0.1 * torch.randn(1536, generator=g)).to(torch.bfloat16)
    norm = Qwen2RMSNorm(1536, eps=1e-6).to(torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(w)
        ref = bf16_bits(norm(x.to(torch.bfloat16)))
    got = np.zeros((64, 1536), dtype=np.uint16)
    oracle().oracle_head_norm(np.ascontiguousarray(x.numpy()), 64, bf16_bits(w), got)
    d = ulps_apart(got, ref)
    assert d.max() <= 1
    assert np.mean(d == 0) >= 0.995


def test_head_norm_rounds_its_input_and_uses_the_weight():
    """A row of constant value c normalizes to bf16(w * bf16(c / sqrt(c^2 + 1e-6))): closed form."""
    c = np.float32(0.37)
    x = np.full((1, 1536), c, dtype=np.float32)
    w = bf16_bits(torch.linspace(0.5, 2.0, 1536))
    got = np.zeros((1, 1536), dtype=np.uint16)
    oracle().oracle_head_norm(x, 1, w, got)
    cb = np.float32(bf16_value(bf16_bits(torch.tensor([float(c)])))[0])
    var = np.float32(np.float64(cb) * np.float64(cb) * 1536) / np.float32(1536)
    r = np.float32(1.0) / np.sqrt(var + np.float32(1e-6), dtype=np.float32)
    y = bf16_value(bf16_bits(torch.tensor([float(np.float32(cb * r))])))[0]
    want = bf16_bits(torch.from_numpy((bf16_value(w) * np.float32(y)).astype(np.float32)))
    assert np.array_equal(got[0], want)


def test_lm_head_matches_torch_bf16_linear():
    g = torch.Generator().manual_seed(6)
    vocab = 512
    table = (0.02 * torch.randn(vocab, 1536, generator=g)).to(torch.bfloat16)
    hidden = torch.randn(7, 1536, generator=g)
    norm_w = torch.ones(1536, dtype=torch.bfloat16)
    xn, logits = head_logits(hidden.numpy(), bf16_bits(norm_w), bf16_bits(table))
    with torch.no_grad():
        n = torch.from_numpy(xn.view(np.int16)).view(torch.bfloat16)
        ref = torch.nn.functional.linear(n, table)
    d = ulps_apart(bf16_bits(torch.from_numpy(logits)), bf16_bits(ref))
    assert d.max() <= 1
    assert np.mean(d == 0) >= 0.995


def test_argmax_matches_torch_including_ties_and_nan():
    g = torch.Generator().manual_seed(7)
    lg = torch.randn(6, 300, generator=g).to(torch.bfloat16).float()
    lg[1, 17] = lg[1, 200] = 50.0          # tie: the first index wins
    lg[2, :] = 0.0                          # all equal -> 0
    lg[3, 9] = float("nan")                 # NaN is the maximum
    lg[3, 250] = float("inf")
    lg[4, 5] = -0.0
    lg[4, :5] = -1.0
    lg[4, 6:] = -1.0
    lg[4, 100] = 0.0                        # -0 == +0: index 5 first
    lg[5, 299] = 1e30                       # last element
    got = argmax_rows(lg.numpy())
    assert got.tolist() == torch.argmax(lg, dim=-1).tolist()
    assert got.tolist()[1:5] == [17, 0, 9, 5]
