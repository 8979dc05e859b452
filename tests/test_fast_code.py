"""Pins the numpy restatement of the FAST two-limb activation code (tests/_fastcode.py) by what the
mathematics fixes, so that a wrong limb split, rounding rule, scale or layout fails here before it is
used as the checker of the GPU code (tests/test_gpu_fast_integer.py)."""

from __future__ import annotations

import numpy as np
import pytest

from _fastcode import CHUNK, QMAX, two_limb_code, unpack_int4


def rows(seed, shape, scale=1.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float32)


@pytest.mark.parametrize("n", [128, 1536, 8960])
def test_limbs_reconstruct_the_code(n):
    x = rows(n, (16, n), 3.0)
    xq, sx, sums, X = two_limb_code(x)
    H = xq[:, :, 0, :].reshape(16, n).astype(np.int32)
    L = xq[:, :, 1, :].reshape(16, n).astype(np.int32)
    assert np.array_equal(256 * H + L, X)
    assert L.min() >= -128 and L.max() <= 127
    assert np.abs(H).max() <= 127
    assert np.array_equal(sums[:, 0], H.sum(axis=1)) and np.array_equal(sums[:, 1], L.sum(axis=1))


def test_scale_and_quantization_error_bound():
    x = rows(7, (32, 1536), 5.0)
    _, sx, _, X = two_limb_code(x)
    amax = np.abs(x).max(axis=1)
    assert np.array_equal(sx, (amax / np.float32(QMAX)).astype(np.float32))
    # the element of largest magnitude codes to +-QMAX, and every element is within half a step
    i = np.abs(x).argmax(axis=1)
    assert np.array_equal(np.abs(X[np.arange(32), i]), np.full(32, QMAX))
    # half a step, plus the rounding of inv, of x * inv and of sx (3 x 2^-24 relative each on values up
    # to QMAX steps: at most 0.006 of a step)
    err = np.abs(x.astype(np.float64) - sx[:, None].astype(np.float64) * X)
    assert np.all(err <= sx[:, None] * (0.5 + 3 * QMAX * 2.0**-24))
    assert np.max(err / sx[:, None]) > 0.45  # the bound is tight: a coarser code would fail it
    assert np.abs(X).max() <= QMAX


def test_ties_round_half_to_even_and_zero_row():
    # amax = QMAX makes inv = 1 and x * inv = x exactly: the halves round to the even neighbour
    x = np.zeros((2, CHUNK), np.float32)
    x[0, :6] = [QMAX, 0.5, 1.5, 2.5, -0.5, -3.5]
    _, sx, sums, X = two_limb_code(x)
    assert sx[0] == np.float32(1.0)
    assert list(X[0, :6]) == [QMAX, 0, 2, 2, 0, -4]
    assert sx[1] == np.float32(1.0) and not X[1].any() and not sums[1].any()


def test_limb_split_at_the_boundaries():
    x = np.zeros((1, CHUNK), np.float32)
    vals = [QMAX, -QMAX, 127, 128, 129, -128, -129, 255, 256, -256, 383, 384]
    x[0, :len(vals)] = vals
    xq, _, _, X = two_limb_code(x)
    H = xq[0, 0, 0, :len(vals)].astype(np.int32)
    L = xq[0, 0, 1, :len(vals)].astype(np.int32)
    # floor((X + 128) / 256): the L limb is the centred remainder in [-128, 127]
    assert list(H) == [127, -127, 0, 1, 1, 0, -1, 1, 1, -1, 1, 2]
    assert list(L) == [0, 0, 127, -128, -127, -128, 127, -1, 0, 0, 127, -128]
    assert np.array_equal(256 * H + L, X[0, :len(vals)])


def test_layout_is_chunk_major():
    x = np.arange(256, dtype=np.float32).reshape(1, 256)  # amax 255 -> inv = 32512/255
    xq, _, _, X = two_limb_code(x)
    assert xq.shape == (1, 2, 2, CHUNK)
    assert np.array_equal(256 * xq[0, 1, 0].astype(np.int32) + xq[0, 1, 1], X[0, 128:])


def test_unpack_int4_matches_the_reference_nibble_order():
    packed = np.array([0x21, 0xF8, 0x7E], np.uint8)  # flat 0,1 = 1,2; 2,3 = -8,-1; 4,5 = -2,7
    assert unpack_int4(packed, 1, 6).tolist() == [[1, 2, -8, -1, -2, 7]]


def test_grouped_code_is_two_limb_code_per_group():
    """The grouped code of a row is two_limb_code applied to each 64-row group on its own (padded with
    zeros to a 128-wide row, which changes neither the maximum nor the sums), and the groups
    partition the rows (each row's limbs come from exactly one group)."""
    from _fastcode import GROUP, group_rows, grouped_code, two_limb_code

    rng = np.random.default_rng(3)
    n = 8960
    y = np.stack([rng.standard_normal(n).astype(np.float32) * np.float32(s) for s in (1.0, 1e-3, 5e3)])
    y[1, group_rows(5)] = 0.0  # an all-zero group: scale 1, zero limbs
    xq, gsx, gcorr = grouped_code(y)
    covered = np.zeros(n, bool)
    for g in range(n // GROUP):
        rows = group_rows(g)
        assert not covered[rows].any()
        covered[rows] = True
        padded = np.concatenate([y[:, rows], np.zeros((y.shape[0], GROUP), np.float32)], axis=1)
        rq, rsx, rsums, _ = two_limb_code(padded)
        assert np.array_equal(xq[:, rows // 128, 0, rows % 128], rq[:, 0, 0, :GROUP])
        assert np.array_equal(xq[:, rows // 128, 1, rows % 128], rq[:, 0, 1, :GROUP])
        assert np.array_equal(gsx[:, g].view(np.uint32), rsx.view(np.uint32))
        assert np.array_equal(gcorr[:, g], 256 * rsums[:, 0] + rsums[:, 1])
    assert covered.all()
    assert gsx[1, 5] == 1.0 and gcorr[1, 5] == 0
