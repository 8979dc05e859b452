"""KV layout conversion between the ABI's token-major rows (llm_memory_layout.h:130-149) and the
HF cache layout (verification/real_host_top_backend.py:199-206)."""

import numpy as np

from work_llm_accelerator_amd.layout import HEAD_DIM, KV_HEADS, KV_WIDTH, kv_to_head_major, kv_to_token_major


def test_round_trip_and_element_mapping():
    S = 7
    flat = np.arange(S * KV_WIDTH, dtype=np.float32)
    hm = kv_to_head_major(flat, S)
    assert hm.shape == (KV_HEADS, S, HEAD_DIM)
    # token t, head h, dim d lives at flat index t*256 + h*128 + d
    for t, h, d in ((0, 0, 0), (3, 1, 5), (6, 1, 127), (2, 0, 64)):
        assert hm[h, t, d] == flat[t * KV_WIDTH + h * HEAD_DIM + d]
    assert np.array_equal(kv_to_token_major(hm, S), flat)
