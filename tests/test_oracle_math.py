"""Pins the oracle's elementwise functions by mathematics, not by retyping them.

The prefill-only helpers (approx_exp, approx_sqrt, wrap_angle/approx_sincos,
qwen_prefill_attention_kernel.cpp:47-110) have no reference binary to compare with (the
reference prefill library needs Catapult's ac_channel.h).  Each check below is chosen so that a
plausible mistake -- a dropped Taylor term, a wrong sign, a wrong constant, a wrong halving or
folding rule -- fails it:
  * exact values and exact identities of the algorithm (exp(0) = 1, the squaring ladder,
    odd/even symmetry, the pi folding, sqrt of perfect squares once converged);
  * agreement, within a few ulp, with a double-precision evaluation of the same truncated
    series (pins degree and coefficients), and distance to the true function within the
    analytic truncation bound.
The decode helpers (libm expf, RoPE tables) are pinned against the host libm and the compiled
reference in test_oracle_vs_ref.py; bf16 rounding and the quantizer are pinned here against
independent evaluations (torch's bf16 conversion, numpy restatement, closed forms).
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

from _oracle import oracle
from work_llm_accelerator_amd.quant import quantize_int4_per_channel, round_bfloat16_array

F32 = np.float32


def f(x):
    return float(F32(x))


def ulp(x):
    return float(np.spacing(F32(abs(x)) if x != 0 else F32(1e-38)))


def truncated_exp_series(s: float) -> float:
    return sum(s ** k / math.factorial(k) for k in range(7))


def test_approx_exp_exact_points():
    o = oracle()
    assert o.oracle_approx_exp(0.0) == 1.0
    for v in (-16.0, -16.5, -100.0, -1e30):
        assert o.oracle_approx_exp(v) == 0.0
    assert o.oracle_approx_exp(-15.999) > 0.0


@pytest.mark.parametrize("s", np.linspace(-1.0, 1.0, 41).tolist())
def test_approx_exp_series_without_reduction(s):
    """No halving for s >= -1: the value is the degree-6 Taylor sum (within 4 ulp) and within the
    truncation bound |s|^7/7! * e^|s| of exp(s) (a dropped or wrong term breaks both)."""
    o = oracle()
    s = f(s)
    got = o.oracle_approx_exp(s)
    series = truncated_exp_series(s)
    assert abs(got - series) <= 4 * ulp(series)
    assert abs(got - math.exp(s)) <= abs(s) ** 7 / 5040.0 * math.e + 4 * ulp(series)


@pytest.mark.parametrize("v", [-1.0001, -1.5, -1.999, -2.0, -3.7, -7.9, -8.0, -12.25, -15.5])
def test_approx_exp_halving_ladder(v):
    """For v < -1 the argument is halved until >= -1 and the series squared once per halving:
    approx_exp(v) == fl(approx_exp(v/2)^2) exactly (v/2 is exact)."""
    o = oracle()
    v = f(v)
    half = o.oracle_approx_exp(f(v * 0.5))
    assert o.oracle_approx_exp(v) == f(F32(half) * F32(half))
    k = 0
    s = v
    while s < -1.0:
        s *= 0.5
        k += 1
    # relative truncation error at the reduced argument is <= (1/7!)/e^-1 ~ 5.4e-4; each squaring
    # doubles it
    assert abs(o.oracle_approx_exp(v) - math.exp(v)) <= (2 ** k) * 6e-4 * math.exp(v) + 1e-30


@pytest.mark.parametrize("v", [0.0, 1e-12, 1e-3, 0.1, 0.5, 0.999])
def test_approx_sqrt_small_arguments_follow_newton_from_one(v):
    """v < 1: six Newton steps seeded at 1 (not at v); the float result agrees with the same six
    steps in double to 2 ulp and stays above sqrt(v) (Newton from above)."""
    o = oracle()
    got = o.oracle_approx_sqrt(f(v))
    if v <= 0.0:
        assert got == 0.0
        return
    g = 1.0
    for _ in range(6):
        g = 0.5 * (g + f(v) / g)
    assert abs(got - g) <= 2 * ulp(g)
    assert got >= math.sqrt(f(v)) * (1 - 1e-7)


@pytest.mark.parametrize("v", [1.0, 1.3, 2.0, 4.0, 9.0, 16.0, 2.25, 3.999])
def test_approx_sqrt_converged(v):
    o = oracle()
    got = o.oracle_approx_sqrt(f(v))
    assert abs(got - math.sqrt(v)) <= 1 * ulp(math.sqrt(v))
    if v in (1.0, 4.0, 9.0, 16.0, 2.25):
        assert got == math.sqrt(v)


def sincos(a):
    o = oracle()
    s, c = ctypes.c_float(), ctypes.c_float()
    o.oracle_approx_sincos(f(a), ctypes.byref(s), ctypes.byref(c))
    return s.value, c.value


def test_approx_sincos_exact_points_and_symmetry():
    assert sincos(0.0) == (0.0, 1.0)
    for a in np.linspace(-60.0, 60.0, 601):
        s1, c1 = sincos(a)
        s2, c2 = sincos(-a)
        assert s2 == -s1 and c2 == c1  # odd sine, even cosine, bit for bit


@pytest.mark.parametrize("a", np.linspace(-200.0, 200.0, 801).tolist())
def test_approx_sincos_bounds(a):
    """After reduction to |r| <= pi/2 the truncation bounds are |r|^9/9! (sin) and |r|^8/8! (cos);
    the float wrap loop adds ~k ulp(|a|) for k subtractions of 2*pi."""
    s, c = sincos(a)
    k = int(abs(a) / (2 * math.pi)) + 1
    slack = 4 * k * ulp(a) + 1e-6
    assert abs(s - math.sin(a)) <= (math.pi / 2) ** 9 / math.factorial(9) + slack
    assert abs(c - math.cos(a)) <= (math.pi / 2) ** 8 / math.factorial(8) + slack


def test_approx_sincos_polynomials_inside_half_pi():
    """Inside [-pi/2, pi/2] no folding happens: values equal the degree-7 / degree-6 Taylor
    polynomials evaluated in double to within 4 ulp (pins the coefficients and degrees)."""
    for r in np.linspace(-1.5707, 1.5707, 257):
        r = f(r)
        s, c = sincos(r)
        ps = sum((-1) ** k * r ** (2 * k + 1) / math.factorial(2 * k + 1) for k in range(4))
        pc = sum((-1) ** k * r ** (2 * k) / math.factorial(2 * k) for k in range(4))
        # Horner in float: rounding is relative to the O(1) partial sums, so allow 4 ulp(1).
        assert abs(s - ps) <= 4 * ulp(ps) + 4 * ulp(1.0)
        assert abs(c - pc) <= 4 * ulp(pc) + 4 * ulp(1.0)


def test_approx_sincos_fold_rule():
    """r > pi/2 folds to pi - r with a negated cosine: cos(pi - r) = -cos(r), sin(pi - r) = sin(r)."""
    for r in np.linspace(0.1, 1.5, 15):
        s_in, c_in = sincos(r)
        s_out, c_out = sincos(f(math.pi) - f(r))
        # pi - (pi - r) recovers r only to ulp(pi) in float
        tol = 2 * ulp(math.pi)
        assert abs(s_out - s_in) <= 8 * ulp(s_in) + tol and abs(c_out + c_in) <= 8 * ulp(c_in) + tol


def test_prefill_rope_frequencies():
    """inv_freq chain: pair p uses 0.8058421877614801f^p = theta^(-2p/128) with theta = 1e6."""
    o = oracle()
    cos = np.zeros(64, np.float32)
    sin = np.zeros(64, np.float32)
    o.oracle_prefill_rope_row(1, cos, sin)
    for p in (0, 1, 5, 31, 63):
        inv = 1e6 ** (-2.0 * p / 128.0)
        assert abs(cos[p] - math.cos(inv)) <= 1e-3 and abs(sin[p] - math.sin(inv)) <= 1e-3
    o.oracle_prefill_rope_row(0, cos, sin)
    assert np.all(cos == 1.0) and np.all(sin == 0.0)


def test_decode_rope_matches_libm():
    o = oracle()
    cos = np.zeros(64, np.float32)
    sin = np.zeros(64, np.float32)
    for pos in (0, 1, 77, 4096, 32767):
        o.oracle_decode_rope_row(pos, cos, sin)
        ang = pos * np.power(1e6, -2.0 * np.arange(64) / 128.0)
        assert np.array_equal(cos, np.cos(ang).astype(np.float32))
        assert np.array_equal(sin, np.sin(ang).astype(np.float32))


def test_attention_scaling_constants_agree():
    """Decode uses (float)(1/sqrt(128.0)), prefill the literal 0.08838834764831845f: same float."""
    assert F32(1.0 / math.sqrt(128.0)) == F32(0.08838834764831845)
    assert F32(0.08838834764831845).view(np.uint32) == 0x3DB504F3


def test_silu_both_variants():
    o = oracle()
    for v in (-20.0, -3.0, -0.5, 0.0, 0.25, 2.0, 9.0):
        d = o.oracle_silu_decode(f(v))
        assert d == f(F32(v) / (F32(1.0) + F32(o.oracle_libm_expf(f(-v)))))
        p = o.oracle_silu_prefill(f(v))
        assert abs(p - v / (1 + math.exp(-v))) <= 2e-3 * max(1.0, abs(v))


def test_bf16_rounding_matches_torch_and_numpy():
    import torch

    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 1e3,
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 65504.0, 3.4e38], np.float32)])
    ours = round_bfloat16_array(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))
    y = x.copy()
    oracle().oracle_round_bf16(y, y.size)
    assert np.array_equal(y.view(np.uint32), ours.view(np.uint32))


def test_quantizer_oracle_vs_numpy_restatement_and_closed_forms():
    rng = np.random.default_rng(5)
    m = (rng.standard_normal((64, 96)).astype(np.float32) * F32(0.02))
    m[3] = 0.0  # all-zero row -> scale 1, nibbles 0
    m[5, :4] = [7.0, 2.5, -3.5, 0.5]  # ties at scale 1.0: rint half to even -> 2, -4, 0
    m[5, 4:] = 0.0
    packed, scales = quantize_int4_per_channel(m)
    p2 = np.zeros(m.size // 2, np.uint8)
    s2 = np.zeros(64, np.float32)
    oracle().oracle_quantize_int4(np.ascontiguousarray(m.reshape(-1)), 64, 96, p2, s2)
    assert np.array_equal(packed, p2) and np.array_equal(scales.view(np.uint32), s2.view(np.uint32))
    assert scales[3] == 1.0 and not np.any(packed[3 * 48:4 * 48])
    assert scales[5] == 1.0
    nib = np.stack([packed & 0xF, packed >> 4], 1).reshape(64, 96).astype(np.int32)
    q = np.where(nib >= 8, nib - 16, nib)
    assert list(q[5, :4]) == [7, 2, -4, 0]
    rows_max = np.argmax(np.abs(m), axis=1)
    for r in range(64):
        if r == 3:
            continue
        assert abs(q[r, rows_max[r]]) == 7
        assert scales[r] == F32(np.max(np.abs(m[r])) / F32(7.0))
