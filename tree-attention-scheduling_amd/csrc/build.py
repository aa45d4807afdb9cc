"""Build ``libtree_attn.so`` (gfx950) next to the ``tree_attention`` package.

    python tree-attention-scheduling_amd/csrc/build.py

Uses hipcc directly; no CMake, no JIT cache.  The library is placed in-tree so
it travels with the source snapshot to the GPU machine.
"""
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent / "tree_attention"
INCLUDE = HERE.parent.parent / "include"
LIB = PKG / "libtree_attn.so"
SOURCES = [HERE / "tree_attn.hip"]

FLAGS = [
    "-O3", "-std=c++20", "--offload-arch=gfx950", "-fPIC", "-shared",
    "-mcode-object-version=5",
    # packed-FP32 VALU forms are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: every kernel fits in 256 VGPRs, and the
    # AGPR form made the allocator copy O between register files each step
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; ROCm is required to build the tree_attn library")
    return found


def build(verbose: bool = False) -> Path:
    tmp = LIB.with_name(LIB.name + f".tmp{os.getpid()}")
    cmd = [hipcc(), *FLAGS, f"-I{INCLUDE}", *map(str, SOURCES), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    if verbose and res.stderr.strip():
        print(res.stderr, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
