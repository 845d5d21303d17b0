"""Build libcortex_hip.so in-tree with hipcc for gfx950.

Each HIP source is compiled to an object in parallel, then linked into
``cortex/libcortex_hip.so`` next to this file.  Called by ``__graft_entry__.build()``
and usable directly: ``python -m cortex._build``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent  # cortex-engine_amd/
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"
BUILD = ROOT / "_build"
LIB = PKG_DIR / "libcortex_hip.so"

SOURCES = ["abi.cpp", "tokenize_pack.hip", "quant.hip", "norm_gemm.hip", "gemm_bf16.hip", "rowops.hip", "attention.hip", "attention_fast.hip", "block_mask.hip", "pages.hip", "head.hip", "gemm_rowln.hip", "block_attn.hip", "page_table.cpp", "splitk.hip"]
ARCH = os.environ.get("CORTEX_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 vector ops stay off on this target
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the Cortex HIP library needs ROCm's hipcc")


def _compile(src: str, verbose: bool) -> Path:
    hipcc = _hipcc()
    obj = BUILD / (src.rsplit(".", 1)[0] + ".o")
    cmd = [hipcc, *HIP_FLAGS, f"-I{CSRC}", f"-I{INCLUDE}", "-c", str(CSRC / src), "-o", str(obj)]
    if src.endswith(".cpp"):
        cmd.insert(1, "-x")
        cmd.insert(2, "hip")
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
    noise = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln]
    if verbose and noise:
        print("\n".join(noise), flush=True)
    return obj


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
