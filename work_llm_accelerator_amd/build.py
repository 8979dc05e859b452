"""Builds the MI355X (gfx950) HIP library in-tree.

Outputs, under work_llm_accelerator_amd/_lib/:
  libqwen_mi355x.so         all HIP kernels, the host runtime and every C-ABI entry point
  libqwen_decode_stub.so    symlink: the drop-in name of the reference decode host library
  libqwen_prefill_stub.so   symlink: the drop-in name of the reference prefill host library

Every .hip source is compiled with hipcc for gfx950 only.  Sources whose name starts with
"kernels_fast" are compiled with -ffp-contract=fast (reordered, tolerance-checked kernels); all
others with -ffp-contract=off so that each written fp32/f64 operation is one IEEE operation.
Packed fp32 instructions are disabled for every source (-packed-fp32-ops).  The "kernels_fast"
sources also have the leading 14 dwords of scalar kernel arguments preloaded into SGPRs at wave
launch (-amdgpu-kernarg-preload-count): the one-token kernels take the operands of their first
loads there, instead of waiting for the argument segment's memory round trip.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB_DIR = PKG / "_lib"
OBJ_DIR = PKG / "_lib" / "obj"
LIB_NAME = "libqwen_mi355x.so"
DROP_IN_NAMES = ("libqwen_decode_stub.so", "libqwen_prefill_stub.so")
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build the HIP library)")


def common_flags() -> list[str]:
    return [
        "-std=c++17",
        "-O3",
        "-fPIC",
        f"--offload-arch={ARCH}",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-fno-fast-math",
        "-Wall",
        "-Wno-unused-function",
        f"-I{ROOT / 'include'}",
        f"-I{CSRC}",
    ]


def compile_one(src: Path) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    fast = src.name.startswith("kernels_fast")
    extra = ["-ffp-contract=fast", "-mllvm", "-amdgpu-kernarg-preload-count=14"] if fast else ["-ffp-contract=off"]
    cmd = [hipcc(), *common_flags(), *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compiles every csrc/*.hip for gfx950 and links the shared library (always rebuilds)."""
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), max(1, int(os.environ.get("MAX_JOBS", "8"))))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(compile_one, sources))
    out = LIB_DIR / LIB_NAME
    tmp = LIB_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp),
           "-Wl,--no-undefined", "-lpthread"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    for name in DROP_IN_NAMES:
        link = LIB_DIR / name
        if link.is_symlink() or link.exists():
            link.unlink()
        link.symlink_to(LIB_NAME)
    if verbose:
        print(f"built {out} from {len(sources)} HIP sources for {ARCH}")
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
