"""The HIP library loads without a GPU and exports every entry point include/*.h declares, and
the drop-in names resolve to it (no compute call is made here)."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from work_llm_accelerator_amd import abi

ROOT = Path(__file__).resolve().parents[1]
DECL = re.compile(r"^\s*(?:int|const char\s*\*|void\s*\*|void)\s*(qwen_[a-z0-9_]+)\s*\(", re.M)


def declared_symbols() -> set[str]:
    names: set[str] = set()
    for header in (ROOT / "include").glob("*.h"):
        names |= set(DECL.findall(header.read_text()))
    return names


def test_headers_declare_reference_entry_points():
    names = declared_symbols()
    for ref_name in ("qwen_decode_stub_forward", "qwen_decode_attention_smoke_forward", "qwen_decode_mlp_smoke_forward",
                     "qwen_decode_top_smoke_forward", "qwen_decode_layer_smoke_forward", "qwen_prefill_stub_forward",
                     "qwen_prefill_attention_smoke_forward", "qwen_prefill_mlp_smoke_forward",
                     "qwen_prefill_layer_smoke_forward", "qwen_prefill_glue_smoke_forward",
                     "qwen_prefill_top_smoke_forward"):
        assert ref_name in names


@pytest.mark.parametrize("path", [abi.LIB_PATH, abi.DECODE_STUB_PATH, abi.PREFILL_STUB_PATH])
def test_library_exports_every_declared_symbol(path):
    assert path.exists(), "build the library first (python -m work_llm_accelerator_amd.build)"
    ctypes.CDLL(str(path))
    out = subprocess.run(["nm", "-D", "--defined-only", str(path)], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = declared_symbols() - exported
    assert not missing, f"missing exports: {sorted(missing)}"


def test_headers_declare_model_api():
    names = declared_symbols()
    for name in abi.EXTRA_SIGNATURES:
        assert name in names, name


def test_bindings_declare_argtypes():
    lib = abi.load()
    for name in list(abi.SIGNATURES) + list(abi.EXTRA_SIGNATURES):
        assert getattr(lib, name).argtypes is not None
