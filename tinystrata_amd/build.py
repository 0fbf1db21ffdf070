"""Build libtsx_moe.so in-tree with hipcc for gfx950.

    python -m tinystrata_amd.build        (or tinystrata_amd.build.build())

Every translation unit is compiled separately (in parallel) and linked into tinystrata_amd/libtsx_moe.so.
The library has no PyTorch dependency: it is plain HIP behind the C ABI of include/tsx_moe.h.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIB = PKG / "libtsx_moe.so"
ARCH = os.environ.get("TSX_OFFLOAD_ARCH", "gfx950")

SOURCES = [
    "tsx_abi.cpp",
    "tsx_weights.cpp",
    "tsx_gguf.cpp",
    "tsx_cpu_rows.cpp",
    "tsx_pool.cpp",
    "strata_kernels.hip",
    "tsx_decode.hip",
    "tsx_layer.hip",
    "tsx_route.hip",
    "tsx_prefill.hip",
]

COMMON = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 arithmetic stays off on this pool (its packed forms have given wrong results)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # no merging of narrow loads into misaligned wide ones: GGUF fields sit on 2-byte boundaries, and a misaligned
    # ds_read_b32/b64 measured ~1000 cycles per dependent read with 16 waves on gfx950 against ~130 for the aligned
    # 16-bit reads it replaces
    "-Xclang", "-target-feature", "-Xclang", "-unaligned-access-mode",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libtsx_moe.so)")


def _compile(src: str, objdir: Path) -> Path:
    obj = objdir / (Path(src).name + ".o")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", *COMMON, "-c", str(CSRC / src), "-o", str(obj)]
    if not src.endswith(".hip"):
        cmd = [_hipcc(), *COMMON, "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(lambda s: _compile(s, objdir), SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
