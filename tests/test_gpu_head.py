"""Model head on the GPU (final RMSNorm, tied bf16 lm_head, greedy argmax) against the oracle
(verification/real_host_top_backend.py:138-146; greedy step of
verification/qwen_full_model_validation.py:128,159).

Tolerance: the normalized rows are computed the same way on both sides (squares of bf16 values
summed in double, the sum rounded once to fp32).  The device sums the 1536 products of a logit in
MFMA order in fp32, the oracle in double, so a bf16 logit may differ by one unit in the last place
where the fp32 sum sits next to a bf16 rounding boundary, and logits near zero (cancelling sums) by
the fp32 accumulation error: every logit within max(1 bf16 ulp, 1e-5 x the row's largest |logit|)
and at least 99% bit-identical.  Greedy ids equal the first index of the maximum of the device's
own logits exactly, and the oracle's argmax wherever the oracle's two best logits are more than
1 ulp apart (no near-tie)."""

from __future__ import annotations

import numpy as np
import pytest

from tests._oracle import argmax_rows, head_logits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t

    return t


def bf16_bits_np(x: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return b.astype(np.uint16)


def ulps(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    def ordered(x):
        bits = (np.ascontiguousarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.int64)
        return np.where(bits & 0x8000, -(bits & 0x7FFF), bits & 0x7FFF)
    return np.abs(ordered(a) - ordered(b))


def first_argmax(x: np.ndarray) -> np.ndarray:
    return np.argmax(x, axis=-1).astype(np.int32)


def near_tie(logits: np.ndarray) -> np.ndarray:
    top2 = np.sort(logits, axis=-1)[:, -2:]
    return ulps(top2[:, 1:], top2[:, :1])[:, 0] <= 1


def check_head(torch, m, vocab, table, norm, count, seed):
    rng = np.random.default_rng(seed)
    hidden = (rng.standard_normal((count, 1536)) * 2.0).astype(np.float32)
    _, ref = head_logits(hidden, norm, table)
    h = torch.from_numpy(hidden).cuda()
    lg = torch.empty(count, vocab, dtype=torch.float32, device="cuda")
    ids = torch.empty(count, dtype=torch.int32, device="cuda")
    print(f"head vocab={vocab} count={count}", flush=True)
    m.logits(h, lg)
    m.greedy(h, ids)
    m.synchronize()
    got = lg.cpu().numpy()
    gid = ids.cpu().numpy()
    d = ulps(got, ref)
    floor = 1e-5 * np.max(np.abs(ref), axis=1, keepdims=True)
    bad = (d > 1) & (np.abs(got - ref) > floor)
    assert not bad.any(), (d.max(), np.abs(got - ref)[bad].max())
    assert np.mean(d == 0) >= 0.99
    assert np.array_equal(gid, first_argmax(got))
    want = argmax_rows(ref)
    ok = ~near_tie(ref)
    assert np.array_equal(gid[ok], want[ok])


@pytest.mark.parametrize("count", [1, 5, 33])
def test_head_small_vocab(torch, count):
    from work_llm_accelerator_amd.model import DeviceModel

    rng = np.random.default_rng(100 + count)
    vocab = 4096
    table = bf16_bits_np(rng.standard_normal((vocab, 1536)) * 0.02)
    norm = bf16_bits_np(1.0 + 0.1 * rng.standard_normal(1536))
    m = DeviceModel(1, synthetic_seed=9)
    try:
        m.set_head(table, norm)
        assert m.vocab == vocab
        check_head(torch, m, vocab, table, norm, count, seed=count)
    finally:
        m.close()


@pytest.mark.parametrize("count", [1, 2])
def test_head_full_vocab(torch, count):
    """count 1: the one-token row-streaming kernel; 2: the MFMA kernel."""
    from work_llm_accelerator_amd.model import DeviceModel

    rng = np.random.default_rng(151936)
    vocab = 151936
    table = bf16_bits_np(rng.standard_normal((vocab, 1536), dtype=np.float32) * np.float32(0.02))
    norm = np.full(1536, 0x3F80, dtype=np.uint16)
    m = DeviceModel(1, synthetic_seed=9)
    try:
        m.set_head(table, norm)
        check_head(torch, m, vocab, table, norm, count, seed=77)
    finally:
        m.close()


def test_synthetic_greedy_decode_loop(torch):
    """Greedy loop of the reference driver on a synthetic 2-layer model (tied table, norm 1.0):
    embed -> FAST decode -> greedy id -> next step; ids stay in range and equal the argmax of the
    logits the model reports for the same hidden rows."""
    from work_llm_accelerator_amd.model import MODE_FAST, DeviceModel, KvCache

    m = DeviceModel(2, synthetic_seed=12)
    try:
        assert m.vocab == 151936
        B, steps = 3, 4
        cache = KvCache.allocate(2, B, 16)
        ids = torch.tensor([5, 151935, 70000], dtype=torch.int32, device="cuda")
        hidden = torch.empty(B, 1536, dtype=torch.float32, device="cuda")
        lg = torch.empty(B, 151936, dtype=torch.float32, device="cuda")
        for step in range(steps):
            print(f"greedy loop step {step}", flush=True)
            m.embed(ids, hidden)
            pos = torch.full((B,), step, dtype=torch.int32, device="cuda")
            m.decode(MODE_FAST, hidden, pos, 16, cache)
            m.logits(hidden, lg)
            m.greedy(hidden, ids)
            m.synchronize()
            got = ids.cpu().numpy()
            assert np.all((got >= 0) & (got < 151936))
            assert np.array_equal(got, first_argmax(lg.cpu().numpy()))
    finally:
        m.close()
