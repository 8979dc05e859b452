"""The descriptor builders of work_llm_accelerator_amd.layout against the closed forms of the
reference's global DDR map (python/layer_descriptor_builder.py:194-277 over the layer block of
hls/common/llm_memory_layout.h:84-149), and the ctypes descriptor structs against the C structs of
include/qwen_layout.h as a C compiler lays them out."""

from __future__ import annotations

import ctypes
import shutil
import subprocess
import tempfile
from pathlib import Path

import pytest

from work_llm_accelerator_amd import layout as L

ROOT = Path(__file__).resolve().parents[1]

LAYER_BLOCK = 23_508_992      # bytes of one layer's parameters (llm_memory_layout.h:84-128)
KV_LAYER = 32_768 * 1_024     # 32768 positions x 256 fp32 (llm_memory_layout.h:130-139)
V_BASE = 28 * KV_LAYER        # V follows the 28 layers of K


def test_layer_block_and_kv_layout_closed_forms():
    assert L.LAYOUT.total_parameter_bytes == LAYER_BLOCK
    kv = L.build_kv_cache_layout()
    assert (kv.k_base_offset_bytes, kv.v_base_offset_bytes, kv.layer_stride_bytes, kv.token_stride_bytes) == \
        (0, V_BASE, KV_LAYER, 1024)
    assert V_BASE == 939_524_096


@pytest.mark.parametrize("past,act,w,s,kvb,scr", [(0, 0, 0, 0, 0, 0), (64, 4096, 1 << 20, 3 << 20, 1 << 30, 77)])
def test_decode_descriptors_closed_form(past, act, w, s, kvb, scr):
    descs = L.build_decode_descriptors(past, act, w, s, kvb, scr)
    assert len(descs) == 28
    for i, d in enumerate(descs):
        assert d.layer_id == i and d.past_seq_len == past
        assert d.input_token_addr == act + 6144 * i
        assert d.output_token_addr == act + 6144 * (i + 1)  # layer i's output is layer i+1's input
        assert d.layer_weights_base_addr == w + LAYER_BLOCK * i
        assert d.layer_scales_base_addr == s + LAYER_BLOCK * i  # a byte address: fp32 word (s + ...) / 4
        assert d.k_cache_base_addr == kvb + KV_LAYER * i
        assert d.v_cache_base_addr == kvb + V_BASE + KV_LAYER * i
        assert d.scratch_base_addr == scr
    assert descs[-1].v_cache_base_addr + KV_LAYER == kvb + 2 * V_BASE  # the map ends after V of layer 27


@pytest.mark.parametrize("seq_len", [1, 37, 128])
def test_prefill_descriptors_closed_form(seq_len):
    descs = L.build_prefill_descriptors(seq_len, 1000, 0, 0, 0, 5)
    assert len(descs) == 28
    for i, d in enumerate(descs):
        assert d.seq_len == seq_len and d.layer_id == i
        assert d.input_sequence_addr == 1000 + seq_len * 6144 * i
        assert d.output_sequence_addr == 1000 + seq_len * 6144 * (i + 1)
        assert d.layer_weights_base_addr == LAYER_BLOCK * i
        assert d.k_cache_base_addr == KV_LAYER * i and d.v_cache_base_addr == V_BASE + KV_LAYER * i
        assert d.tile_config == L.default_prefill_tile_config()


def test_default_prefill_tiles_are_the_python_defaults():
    # layer_descriptor_builder.py:100-117; the C++ check (llm_layer_dispatch.h:54-65) accepts only
    # query 32 / key 64 / hidden_proj 64 / kv_proj 64, so these defaults give status 20 at the top
    assert L.default_prefill_tile_config().as_args() == (128, 128, 128, 256, 256, 128, 2, 1, 128, 256, 640)
    assert L.valid_prefill_tile_config().as_args() == (128, 32, 64, 64, 64, 128, 2, 1, 128, 256, 640)


def test_c_struct_conversion_round_trip():
    descs = L.build_prefill_descriptors(16, 0, 0, 0, 0, 0, L.valid_prefill_tile_config())
    arr = L.to_c_prefill(descs)
    assert arr[3].layer_id == 3 and arr[3].seq_len == 16 and list(arr[3].tiles) == list(descs[3].tile_config.as_args())
    assert arr[27].v_cache_base_addr == V_BASE + 27 * KV_LAYER
    darr = L.to_c_decode(L.build_decode_descriptors(9, 0, 0, 0, 0, 0))
    assert darr[5].past_seq_len == 9 and darr[5].output_token_addr == 6 * 6144


@pytest.mark.skipif(shutil.which("gcc") is None, reason="no C compiler")
def test_ctypes_structs_match_the_c_layout():
    probe = r'''
#include <stddef.h>
#include <stdio.h>
#include "qwen_layout.h"
int main(void) {
  printf("%zu %zu %zu %zu\n", sizeof(qwen_decode_descriptor), offsetof(qwen_decode_descriptor, input_token_addr),
         offsetof(qwen_decode_descriptor, v_cache_base_addr), offsetof(qwen_decode_descriptor, scratch_base_addr));
  printf("%zu %zu %zu %zu\n", sizeof(qwen_prefill_descriptor), offsetof(qwen_prefill_descriptor, tiles),
         offsetof(qwen_prefill_descriptor, input_sequence_addr), offsetof(qwen_prefill_descriptor, scratch_base_addr));
  return 0;
}
'''
    with tempfile.TemporaryDirectory() as td:
        src = Path(td) / "probe.c"
        exe = Path(td) / "probe"
        src.write_text(probe)
        subprocess.run(["gcc", "-std=c99", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
        lines = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    dec = [int(v) for v in lines[0].split()]
    pre = [int(v) for v in lines[1].split()]
    C, P = L.CDecodeDescriptor, L.CPrefillDescriptor
    assert dec == [ctypes.sizeof(C), C.input_token_addr.offset, C.v_cache_base_addr.offset, C.scratch_base_addr.offset]
    assert pre == [ctypes.sizeof(P), P.tiles.offset, P.input_sequence_addr.offset, P.scratch_base_addr.offset]
