"""Bit-exactness of the FAST path's integer arithmetic on the GPU (include/qwen_hip_ops.h).

* The two-limb activation code (limbs, the scale max|x| / 32512, the limb sums) of the device
  quantizer the FAST layers run before every projection equals tests/_fastcode.two_limb_code bit for
  bit, on rows of width 1536 and 8960 with ties, zero rows and extreme magnitudes.
* The grouped code of the decode of 2..64 sequences (the gate/up projection's SiLU·up rows quantized
  per 64-row group): the device's grouped code equals tests/_fastcode.grouped_code of the same
  projection's fp32 output bit for bit, and the down projection of a grouped code with power-of-two
  group scales equals the int64 sum over groups exactly (a group dequantized with another group's
  scale, or rows of one group read into another, changes it).
* Every kernel a FAST projection can take (the skinny decode GEMMs with one K group and with five
  K splits, the direct-load kernel with its in-block K split, the pipelined GEMM with and without a
  cross-block K split, the pipelined GEMM with two blocks per CU) accumulates the weight x activation
  products exactly: with unit row scales and integer inputs whose largest magnitude is 32512 (so the
  token scale is exactly 1 and the code is the input itself) and whose products stay below 2^24, the
  fp32 output is exactly the int64 product sum_k q(o, k) x(t, k), computed here with numpy.  A wrong
  nibble, limb, zero-point correction, K split or reduce order changes an integer and fails the
  bit comparison.
"""

from __future__ import annotations

import numpy as np
import pytest

from _fastcode import GROUP, QMAX, group_rows, grouped_code, two_limb_code, unpack_int4

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t

    return t


@pytest.fixture(scope="module")
def lib():
    from work_llm_accelerator_amd import abi

    return abi.load()


def dptr(t):
    import ctypes

    return ctypes.c_void_p(t.data_ptr())


def quant_rows(seed, n):
    rng = np.random.default_rng(seed)
    r = [rng.standard_normal(n, dtype=np.float32),
         rng.standard_normal(n, dtype=np.float32) * np.float32(1e-6),
         rng.standard_normal(n, dtype=np.float32) * np.float32(3e4),
         np.zeros(n, np.float32),
         np.full(n, -2.5, np.float32),
         np.abs(rng.standard_normal(n, dtype=np.float32)),
         rng.integers(-QMAX, QMAX + 1, n).astype(np.float32)]
    t = np.zeros(n, np.float32)  # amax = QMAX: inv = 1, halves are exact ties
    t[0] = QMAX
    t[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, 127.5, 128.5, -128.5]
    r.append(t)
    return np.stack(r)


@pytest.mark.parametrize("n", [1536, 8960])
def test_quantize_rows_bitexact(torch, lib, n):
    from work_llm_accelerator_amd import abi

    print(f"two-limb code of rows of width {n}", flush=True)
    x = quant_rows(n, n)
    rows = x.shape[0]
    xd = torch.from_numpy(x).cuda()
    xq = torch.zeros(rows * n * 2, dtype=torch.int8, device="cuda")
    sx = torch.zeros(rows, dtype=torch.float32, device="cuda")
    sums = torch.zeros(rows * 2, dtype=torch.int32, device="cuda")
    st = lib.qwen_hip_fast_quantize_rows(dptr(xd), rows, n, dptr(xq), dptr(sx), dptr(sums), None)
    assert st == 0, abi.last_error(lib)
    torch.cuda.synchronize()
    rq, rsx, rsums, _ = two_limb_code(x)
    assert np.array_equal(xq.cpu().numpy(), rq.reshape(-1)), "limbs differ"
    assert np.array_equal(sx.cpu().numpy().view(np.uint32), rsx.view(np.uint32)), "scales differ"
    assert np.array_equal(sums.cpu().numpy().reshape(rows, 2), rsums), "limb sums differ"


def integer_rows(seed, tokens, n, small, large):
    """Integer-valued fp32 rows: |x| <= small mostly, `large` entries up to QMAX, one entry +-QMAX."""
    rng = np.random.default_rng(seed)
    x = rng.integers(-small, small + 1, (tokens, n)).astype(np.float64)
    for t in range(tokens):
        idx = rng.choice(n, large + 1, replace=False)
        x[t, idx[:-1]] = rng.integers(-QMAX, QMAX + 1, large)
        x[t, idx[-1]] = QMAX if rng.integers(0, 2) else -QMAX
    return x.astype(np.float32)


# (tokens, in_dim, out_dim, flags): the kernel each shape takes inside launch_gemm_i8
SHAPES = [
    (1, 1536, 2048, 0),     # skinny, one K group (decode Q/K/V shape)
    (1, 1536, 1536, 0),     # skinny, one token, the O shape (operands of the first loads preloaded)
    (16, 1536, 1536, 0),    # skinny, one token tile (preloaded operands)
    (64, 1536, 1536, 0),    # skinny, four token tiles (preloaded operands)
    (64, 1536, 8960, 0),    # skinny, four token tiles (decode gate/up shape)
    (1, 8960, 1536, 0),     # skinny, 5 K splits of 14 chunks + reduce (decode down; preloaded operands)
    (64, 8960, 1536, 0),    # skinny, 5 K splits, four token tiles (preloaded operands)
    (5, 8960, 1536, 1),     # direct-load kernel, in-block 4-way K split (no split workspace)
    (7, 1536, 1040, 0),     # direct-load kernel (out_dim not a multiple of 64)
    (40, 1536, 1040, 0),    # pipelined 4-stage, cross-block K split over 12 blocks + reduce
    (40, 1536, 1040, 1),    # pipelined 4-stage, no K split, partial row group
    (150, 1536, 2048, 0),   # pipelined, 6 K splits, partial token tile
    (150, 8960, 1536, 0),   # pipelined, 14 K splits
    (300, 8960, 1536, 0),   # pipelined with two blocks per CU (no K split), partial token tile
    (600, 1536, 2048, 0),   # pipelined with two blocks per CU
]


@pytest.mark.parametrize("tokens,in_dim,out_dim,flags", SHAPES)
def test_projection_integer_sums_exact(torch, lib, tokens, in_dim, out_dim, flags):
    from work_llm_accelerator_amd import abi

    print(f"FAST projection integer sums: tokens={tokens} in={in_dim} out={out_dim} flags={flags}", flush=True)
    rng = np.random.default_rng(tokens * 7919 + in_dim + out_dim + flags)
    packed = rng.integers(0, 256, out_dim * in_dim // 2, dtype=np.uint8)
    q = unpack_int4(packed, out_dim, in_dim).astype(np.int64)
    x = integer_rows(tokens + in_dim, tokens, in_dim, small=48, large=6)
    X = x.astype(np.int64)
    # exactness preconditions: the raw u = q + 8 sums of any K split (u <= 15) and the results stay
    # below 2^24 in magnitude, so every fp32 partial and sum is an exact integer
    assert np.all(15 * np.abs(X).sum(axis=1) < 2**24)
    ref = X @ q.T  # [tokens][out] int64
    assert np.abs(ref).max() < 2**24
    wd = torch.from_numpy(packed).cuda()
    sw = torch.ones(out_dim, dtype=torch.float32, device="cuda")
    xd = torch.from_numpy(x).cuda()
    y = torch.full((tokens, out_dim), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    st = lib.qwen_hip_fast_project(dptr(wd), dptr(sw), None, out_dim, in_dim, dptr(xd), tokens, flags, dptr(y), None)
    assert st == 0, abi.last_error(lib)
    got = y.cpu().numpy()
    want = ref.astype(np.float32)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad[0].size == 0, (f"{bad[0].size} outputs differ; first (t={bad[0][0]}, o={bad[1][0]}): "
                              f"{got[bad[0][0], bad[1][0]]!r} vs {want[bad[0][0], bad[1][0]]!r}")


def test_projection_scales_and_bias(torch, lib):
    """Row scales, the token scale and the bias enter after the exact sums: y = sw * sx * S + b with
    sx = max|x| / 32512, checked against that formula in float64 to a few fp32 roundings."""
    from work_llm_accelerator_amd import abi

    tokens, in_dim, out_dim = 3, 1536, 2048
    rng = np.random.default_rng(11)
    packed = rng.integers(0, 256, out_dim * in_dim // 2, dtype=np.uint8)
    q = unpack_int4(packed, out_dim, in_dim).astype(np.int64)
    x = rng.standard_normal((tokens, in_dim), dtype=np.float32)
    sw = (rng.random(out_dim, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    bias = rng.standard_normal(out_dim, dtype=np.float32)
    _, sx, _, X = two_limb_code(x)
    ref = (X.astype(np.int64) @ q.T).astype(np.float64) * sx[:, None].astype(np.float64) * sw[None, :] + bias[None, :]
    y = torch.empty((tokens, out_dim), dtype=torch.float32, device="cuda")
    args = [torch.from_numpy(a).cuda() for a in (packed, sw, bias, x)]
    torch.cuda.synchronize()
    st = lib.qwen_hip_fast_project(dptr(args[0]), dptr(args[1]), dptr(args[2]), out_dim, in_dim, dptr(args[3]),
                                   tokens, 0, dptr(y), None)
    assert st == 0, abi.last_error(lib)
    got = y.cpu().numpy().astype(np.float64)
    assert np.max(np.abs(got - ref) / (np.abs(ref) + np.abs(bias)[None, :] + 1e-30)) < 4 * 2.0**-24


def test_operator_argument_checks(lib):
    """Shapes the kernels cannot take are refused before anything is launched."""
    import ctypes

    p = ctypes.c_void_p(16)
    assert lib.qwen_hip_fast_project(p, p, None, 1000, 1536, p, 1, 0, p, None) == 1  # out % 16
    assert lib.qwen_hip_fast_project(p, p, None, 1024, 1000, p, 1, 0, p, None) == 1  # in % 128
    assert lib.qwen_hip_fast_project(p, p, None, 1024, 9088, p, 1, 0, p, None) == 1  # in > 8960
    assert lib.qwen_hip_fast_project(p, p, None, 1024, 1536, p, 0, 0, p, None) == 1  # no tokens
    assert lib.qwen_hip_fast_quantize_rows(p, 1, 100, p, p, p, None) == 1


@pytest.mark.parametrize("tokens", [1, 2, 17, 64])
def test_grouped_silu_code_bitexact(torch, lib, tokens):
    from work_llm_accelerator_amd import abi

    print(f"grouped SiLU·up code: tokens={tokens}", flush=True)
    rng = np.random.default_rng(tokens + 404)
    out, inp = 8960, 1536
    gate = rng.integers(0, 256, out * inp // 2, dtype=np.uint8)
    up = rng.integers(0, 256, out * inp // 2, dtype=np.uint8)
    swg = (rng.random(out, dtype=np.float32) * np.float32(0.02) + np.float32(1e-3)).astype(np.float32)
    swu = (rng.random(out, dtype=np.float32) * np.float32(0.02) + np.float32(1e-3)).astype(np.float32)
    swg[group_rows(5)] = 0.0  # an all-zero group: scale 1, zero limbs, zero offset term
    x = rng.standard_normal((tokens, inp), dtype=np.float32)
    d = [torch.from_numpy(v).cuda() for v in (gate, swg, up, swu, x)]
    y = torch.zeros((tokens, out), dtype=torch.float32, device="cuda")
    xq = torch.zeros(tokens * out * 2, dtype=torch.int8, device="cuda")
    gsx = torch.zeros((tokens, out // GROUP), dtype=torch.float32, device="cuda")
    gcorr = torch.zeros((tokens, out // GROUP), dtype=torch.int32, device="cuda")
    st = lib.qwen_hip_fast_silu_mul_grouped(*[dptr(v) for v in d], tokens, dptr(y), dptr(xq), dptr(gsx), dptr(gcorr),
                                            None)
    assert st == 0, abi.last_error(lib)
    rq, rsx, rcorr = grouped_code(y.cpu().numpy())
    assert np.array_equal(xq.cpu().numpy(), rq.reshape(-1)), "limbs differ"
    assert np.array_equal(gsx.cpu().numpy().view(np.uint32), rsx.view(np.uint32)), "group scales differ"
    assert np.array_equal(gcorr.cpu().numpy(), rcorr), "group offset terms differ"
    zr = group_rows(5)
    assert np.all(rsx[:, 5] == 1.0) and not np.any(rq[:, zr // 128, :, zr % 128])  # the zero group was exercised


@pytest.mark.parametrize("tokens", [1, 2, 33, 64])
def test_grouped_down_projection_exact(torch, lib, tokens):
    from work_llm_accelerator_amd import abi

    print(f"grouped down projection: tokens={tokens}", flush=True)
    rng = np.random.default_rng(tokens + 505)
    out, inp = 1536, 8960
    ng = inp // GROUP
    packed = rng.integers(0, 256, out * inp // 2, dtype=np.uint8)
    q = unpack_int4(packed, out, inp).astype(np.int64)
    X = rng.integers(-300, 301, (tokens, inp)).astype(np.int64)  # high limbs -1, 0 and 1
    H = (X + 128) >> 8
    L = X - 256 * H
    xq = np.zeros((tokens, inp // 128, 2, 128), np.int8)
    xq[:, np.arange(inp) // 128, 0, np.arange(inp) % 128] = H
    xq[:, np.arange(inp) // 128, 1, np.arange(inp) % 128] = L
    gsx = np.zeros((tokens, ng), np.float32)
    gcorr = np.zeros((tokens, ng), np.int32)
    ref = np.zeros((tokens, out), np.float64)
    bound = np.zeros((tokens, out), np.float64)
    for g in range(ng):
        rows = group_rows(g)
        gsx[:, g] = np.float32(2.0 ** (g % 3))
        gcorr[:, g] = 256 * H[:, rows].sum(axis=1) + L[:, rows].sum(axis=1)
        term = gsx[:, g:g + 1].astype(np.float64) * (X[:, rows] @ q[:, rows].T)
        ref += term
        bound += np.abs(term)
    # every partial sum of the group terms is an integer below 2^24: any order of fp32 addition is exact
    assert bound.max() < 2**24
    sw = torch.ones(out, dtype=torch.float32, device="cuda")
    d = [torch.from_numpy(v).cuda() for v in (packed, xq.reshape(-1), gsx, gcorr)]
    y = torch.full((tokens, out), float("nan"), dtype=torch.float32, device="cuda")
    st = lib.qwen_hip_fast_project_grouped(dptr(d[0]), dptr(sw), out, dptr(d[1]), dptr(d[2]), dptr(d[3]), tokens,
                                           dptr(y), None)
    assert st == 0, abi.last_error(lib)
    got = y.cpu().numpy()
    want = ref.astype(np.float32)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad[0].size == 0, (f"{bad[0].size} outputs differ; first (t={bad[0][0]}, o={bad[1][0]}): "
                              f"{got[bad[0][0], bad[1][0]]!r} vs {want[bad[0][0], bad[1][0]]!r}")
