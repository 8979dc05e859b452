"""numpy restatement of the FAST path's integer arithmetic (test infrastructure only).

The FAST layers feed every projection input to the int8 matrix cores as a two-limb code
(include/qwen_hip_ops.h):
    amax = max |x| (fp32),  inv = fp32(32512 / amax) (0 when amax = 0),
    X = clip(rint(fp32(x * inv)), -32512, 32512)    (rint: round half to even),
    H = floor((X + 128) / 256),  L = X - 256 H,  so X = 256 H + L with L in [-128, 127],
    sx = fp32(amax / 32512) (1 when amax = 0),  sums = (sum H, sum L),
laid out per row as [K chunk of 128][H limbs | L limbs].  A projection row o of token t is then
    y = sw[o] * sx[t] * sum_k q(o, k) X(t, k) (+ bias),
whose integer part sum_k q X = 256 (sum_k u H - 8 sum H) + (sum_k u L - 8 sum L) with u = q + 8 is
what the matrix cores accumulate.  tests/test_fast_code.py pins this restatement by closed forms.
"""

from __future__ import annotations

import numpy as np

QMAX = 32512  # 127 * 256: |X| <= QMAX keeps both limbs in int8
CHUNK = 128


def two_limb_code(x: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """(xq int8 [rows][n/128][2][128], sx fp32 [rows], sums int32 [rows][2], X int32 [rows][n])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, n = x.shape
    assert n % CHUNK == 0
    amax = np.max(np.abs(x), axis=1)
    with np.errstate(divide="ignore"):
        inv = np.where(amax > 0, np.float32(QMAX) / amax, np.float32(0.0)).astype(np.float32)
        sx = np.where(amax > 0, amax / np.float32(QMAX), np.float32(1.0)).astype(np.float32)
    prod = (x * inv[:, None]).astype(np.float32)
    X = np.clip(np.rint(prod), -QMAX, QMAX).astype(np.int32)
    H = (X + 128) >> 8
    L = X - (H << 8)
    xq = np.stack([H.reshape(rows, n // CHUNK, CHUNK), L.reshape(rows, n // CHUNK, CHUNK)], axis=2).astype(np.int8)
    sums = np.stack([H.sum(axis=1), L.sum(axis=1)], axis=1).astype(np.int32)
    return xq, sx, sums, X


def unpack_int4(packed: np.ndarray, out_dim: int, in_dim: int) -> np.ndarray:
    """Signed INT4 weights [out][in] of the reference layout (even flat index in the low nibble,
    hls/decode_only/qwen_decode_attention_kernel.cpp:44-60)."""
    p = np.asarray(packed, dtype=np.uint8)
    nib = np.stack([p & 0xF, p >> 4], axis=1).reshape(-1)[: out_dim * in_dim].astype(np.int32)
    return np.where(nib >= 8, nib - 16, nib).reshape(out_dim, in_dim)


GROUP = 64  # rows of one group of the grouped code (the K of one 16x16x64 matrix-core product)


def group_rows(g: int) -> np.ndarray:
    """Rows (down-projection K) of group g: row tiles 8(g//2) + 2j + g%2, j < 4, 16 rows each."""
    tiles = 8 * (g // 2) + 2 * np.arange(4) + (g % 2)
    return (16 * tiles[:, None] + np.arange(16)[None, :]).reshape(-1)


def grouped_code(y: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Grouped two-limb code of rows y [tokens][n] (include/qwen_hip_ops.h): each group of 64 rows
    (group_rows) of a token quantized with the group's own maximum, by two_limb_code's arithmetic.
    Returns (xq int8 [tokens][n/128][2][128], gsx fp32 [tokens][n/64], gcorr int32 [tokens][n/64])."""
    y = np.ascontiguousarray(y, dtype=np.float32)
    tokens, n = y.shape
    ng = n // GROUP
    xq = np.zeros((tokens, n // CHUNK, 2, CHUNK), np.int8)
    gsx = np.zeros((tokens, ng), np.float32)
    gcorr = np.zeros((tokens, ng), np.int32)
    for g in range(ng):
        rows = group_rows(g)
        v = y[:, rows]
        amax = np.max(np.abs(v), axis=1)
        with np.errstate(divide="ignore"):
            inv = np.where(amax > 0, np.float32(QMAX) / amax, np.float32(0.0)).astype(np.float32)
            gsx[:, g] = np.where(amax > 0, amax / np.float32(QMAX), np.float32(1.0)).astype(np.float32)
        X = np.clip(np.rint((v * inv[:, None]).astype(np.float32)), -QMAX, QMAX).astype(np.int32)
        H = (X + 128) >> 8
        L = X - (H << 8)
        xq[:, rows // CHUNK, 0, rows % CHUNK] = H.astype(np.int8)
        xq[:, rows // CHUNK, 1, rows % CHUNK] = L.astype(np.int8)
        gcorr[:, g] = 256 * H.sum(axis=1) + L.sum(axis=1)
    return xq, gsx, gcorr
