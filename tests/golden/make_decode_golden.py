"""Writes tests/golden/decode_c1.npz: one Qwen2.5-1.5B-shaped decode layer (config 1: seed-0
weights N(0,0.02) rounded to bf16 and quantized per row to INT4, unit norm weights, hidden state
N(0,1), a 64-position KV history N(0,1) quantized per row to INT4) run through the REFERENCE
decode host library compiled from the reference's own sources (oracle/_ref, oracle/Makefile).

The fixture holds the inputs that are cheap to store (hidden state, KV history), SHA-256 digests
of the regenerated weight and scale images, and the reference outputs (layer output, appended K
and V rows).  Run in a container where /root/reference is mounted:  python tests/golden/make_decode_golden.py
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE.parents[1]))

from _cases import decode_layer, quantized_kv_history, random_hidden, random_layer  # noqa: E402
from _oracle import ref_decode  # noqa: E402

PAST = 64


def case_inputs():
    layer = random_layer(seed=0, unit_norms=True)
    x = random_hidden(1000, 1)
    k, v = quantized_kv_history(1001, PAST + 1)
    k[PAST * 256:] = 0.0
    v[PAST * 256:] = 0.0
    return layer, x, k, v


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main() -> None:
    ref = ref_decode()
    if ref is None:
        raise SystemExit("oracle/_ref/libqwen_decode_ref.so is missing: run `make -C oracle ref` with the reference mounted")
    layer, x, k, v = case_inputs()
    kc, vc = k.copy(), v.copy()
    st, out = decode_layer(ref.qwen_decode_layer_smoke_forward, layer, x, PAST, kc, vc)
    assert st == 0
    np.savez_compressed(HERE / "decode_c1.npz", x=x, k_hist=k[:PAST * 256], v_hist=v[:PAST * 256], out=out,
                        k_row=kc[PAST * 256:], v_row=vc[PAST * 256:],
                        weight_sha256=np.array(digest(layer.weight_ddr)), scale_sha256=np.array(digest(layer.scale_ddr)))
    print("wrote", HERE / "decode_c1.npz")


if __name__ == "__main__":
    main()
